"""The HIP depthwise convolution (fused_attention.Depthwise) against the
oracle (oracle/eager.py, float64, autograd gradients) on the same inputs.
Tolerances as in test_softmax_gpu.py."""

import pytest
import torch

import problems
from gm_attention_amd.nn import fused_attention
from oracle import eager

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-5, atol=1e-6), torch.float64: dict(rtol=1e-12, atol=1e-13)}

CASES = [
    (16, 32, 2, {0: 32, 1: 32, 2: 32}, "hard"),
    (12, 24, 1, {0: 3, 1: 2}, "quartic"),
    (12, 24, 1, {1: 2, 2: 1}, "hard"),
    (10, 20, 1, {0: 70, 1: 30, 2: 20}, "quartic"),  # more copies than lanes
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("case", CASES)
def test_depthwise_matches_the_oracle(case, dtype, cuda):
    nlat, nlon, batch, field, window = case
    print(f"depthwise case {case} {dtype}", flush=True)
    t = problems.tables(nlat, nlon, batch=batch, window=window)
    p, desc = problems.depthwise_layout(field)
    E = t.source.shape[0]
    v64 = problems.normal((t.n_nodes, p.width), 1).to(dtype).double()
    rc64 = problems.normal((1, E, p.a_0), 2).to(dtype).double()
    cc64 = problems.normal((1, E, p.complex_width), 3).to(dtype).double()
    g64 = problems.normal((t.n_nodes, p.width), 4).to(dtype).double()
    tabs = [x.to(dtype).double() for x in (t.transport, t.angular, t.rho, t.weights)]
    vo, rco, cco = (x.clone().requires_grad_(True) for x in (v64, rc64, cc64))
    out_o = eager.conv_op(vo, rco, cco, *tabs, p.rows, t.row_ptr, t.source)
    grads_o = torch.autograd.grad(out_o, (vo, rco, cco), g64, allow_unused=True, materialize_grads=True)

    dev = lambda x: x.to(dtype).to(cuda)
    v, rc, cc = (dev(x).requires_grad_(True) for x in (v64, rc64, cc64))
    out = fused_attention.Depthwise.apply(v, rc, cc, *(dev(x) for x in tabs), desc.to(cuda), t.row_ptr.to(cuda),
                                          t.source.to(cuda), p.a_0, p.complex_width)
    grads = torch.autograd.grad(out, (v, rc, cc), dev(g64), allow_unused=True, materialize_grads=True)
    torch.testing.assert_close(out.double().cpu(), out_o.detach(), **TOL[dtype], msg="out")
    for name, g, w in zip(("dv", "drc", "dcc"), grads, grads_o):
        torch.testing.assert_close(g.double().cpu(), w, **TOL[dtype], msg=name)
