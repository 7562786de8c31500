"""The HIP scores-and-softmax op (fused_attention.Softmax) against the oracle
(oracle/eager.py, float64, autograd gradients) on the same seeded inputs.

Tolerances: float32 within rtol 1e-5 / atol 1e-6 of the float64 oracle on the
float32 inputs (the north star's fp32 bar); float64 within 1e-12 / 1e-13.
"""

import pytest
import torch

import problems
from gm_attention_amd import _native
from gm_attention_amd.nn import fused_attention
from oracle import eager

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-5, atol=1e-6), torch.float64: dict(rtol=1e-12, atol=1e-13)}

CASES = [
    # nlat, nlon, batch, field, heads, window: fast path (chunked head segments) ...
    (32, 64, 1, {0: 16, 1: 16, 2: 16}, 4, "hard"),
    (16, 32, 2, {0: 32, 1: 32, 2: 32}, 8, "quartic"),
    (12, 24, 1, {0: 4, 1: 4}, 1, "quartic"),
    (12, 24, 1, {0: 8, 2: 8}, 2, "hard"),
    (16, 32, 1, {0: 128, 1: 128, 2: 128}, 16, "hard"),  # D = 640, 16 heads of ten chunks
    (12, 24, 1, {0: 64, 1: 64, 2: 64}, 8, "quartic"),
    # the batched kernels (four copies of frequencies 0..2 a head) at every slot count: S = 16 and 8 above,
    # S = 4 (sixteen heads) and S = 32 (two heads) here
    (12, 24, 1, {0: 64, 1: 64, 2: 64}, 16, "hard"),
    (12, 24, 2, {0: 8, 1: 8, 2: 8}, 2, "quartic"),
    # rows of more than 256 edges (the polar caps of these grids: up to 4 nlon edges), which the
    # batched forward shares among a workgroup's waves, at every slot count
    (48, 96, 1, {0: 32, 1: 32, 2: 32}, 8, "hard"),
    (40, 80, 1, {0: 16, 1: 16, 2: 16}, 4, "quartic"),
    (40, 80, 1, {0: 64, 1: 64, 2: 64}, 16, "hard"),
    (40, 80, 1, {0: 8, 1: 8, 2: 8}, 2, "quartic"),
    # ... and the generic path (odd segments, three heads; sixteen heads of 20 chunks)
    (12, 24, 1, {0: 6, 1: 4, 2: 2}, 2, "quartic"),
    (10, 20, 1, {0: 3, 1: 3, 2: 3}, 3, "hard"),
    (10, 20, 1, {0: 256, 1: 128, 2: 128}, 16, "hard"),  # D = 768
]


def _run(case, dtype, device, seed=0):
    nlat, nlon, batch, field, heads, window = case
    print(f"softmax case {case} {dtype}", flush=True)
    t = problems.tables(nlat, nlon, batch=batch, window=window)
    p, desc, scale = problems.attention_layout(field, heads)
    q64 = problems.normal((t.n_nodes, p.width), seed).to(dtype).double()
    k64 = problems.normal((t.n_nodes, p.width), seed + 1).to(dtype).double()
    dalpha64 = problems.normal((t.source.shape[0], heads), seed + 2).to(dtype).double()
    # oracle, float64 on the same (rounded) inputs
    qo, ko = q64.clone().requires_grad_(True), k64.clone().requires_grad_(True)
    tr64 = t.transport.to(dtype).double()
    bias64 = t.bias.to(dtype).double()
    alpha_o = eager.softmax_op(qo, ko, tr64, bias64, t.inside, p.rows, t.row_ptr, t.source, heads, scale)
    dq_o, dk_o = torch.autograd.grad(alpha_o, (qo, ko), dalpha64)
    # HIP
    dev = lambda x: x.to(device)
    q = dev(q64.to(dtype)).requires_grad_(True)
    k = dev(k64.to(dtype)).requires_grad_(True)
    alpha = fused_attention.Softmax.apply(q, k, dev(t.transport.to(dtype)), dev(t.bias.to(dtype)), dev(t.inside),
                                          dev(desc), dev(t.row_ptr), dev(t.source), heads, scale, 1)
    dq, dk = torch.autograd.grad(alpha, (q, k), dev(dalpha64.to(dtype)))
    return (alpha, dq, dk), (alpha_o.detach(), dq_o, dk_o)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("case", CASES)
def test_softmax_matches_the_oracle(case, dtype, cuda):
    got, want = _run(case, dtype, cuda)
    for name, g, w in zip(("alpha", "dq", "dk"), got, want):
        torch.testing.assert_close(g.double().cpu(), w, **TOL[dtype], msg=name)


def test_the_library_is_the_path_that_runs(cuda):
    """The op reaches libgmhip.so (loaded, not a fallback)."""
    _run(CASES[2], torch.float32, cuda)
    import ctypes

    assert isinstance(_native.library(), ctypes.CDLL)
    assert "libgmhip.so" in open("/proc/self/maps").read()


@pytest.mark.parametrize("field", [{0: 8, 1: 8, 2: 8}, {0: 16, 1: 16, 2: 16}])  # per-step and batched kernels
def test_nodes_without_edges_and_empty_graphs(field, cuda):
    """A graph where some targets have no edges and some nodes are nobody's
    source: alpha only on real edges, dq and dk exactly zero on the bare rows."""
    t = problems.tables(12, 24, window="hard")
    keep = (t.source % 3 != 0) & (torch.repeat_interleave(torch.arange(t.n_nodes), t.row_ptr[1:] - t.row_ptr[:-1]) % 5 != 0)
    target = torch.repeat_interleave(torch.arange(t.n_nodes), t.row_ptr[1:] - t.row_ptr[:-1])[keep]
    source = t.source[keep].contiguous()
    row_ptr = torch.zeros(t.n_nodes + 1, dtype=torch.int64)
    row_ptr[1:] = torch.cumsum(torch.bincount(target, minlength=t.n_nodes), 0)
    p, desc, scale = problems.attention_layout(field, 4)
    q = problems.normal((t.n_nodes, p.width), 5).float().to(cuda).requires_grad_(True)
    k = problems.normal((t.n_nodes, p.width), 6).float().to(cuda).requires_grad_(True)
    tr, bias, inside = t.transport[keep].float(), t.bias[keep].float(), t.inside[keep]
    alpha = fused_attention.Softmax.apply(q, k, tr.to(cuda), bias.to(cuda), inside.to(cuda), desc.to(cuda),
                                          row_ptr.to(cuda), source.to(cuda), 4, scale, 1)
    dalpha = problems.normal(alpha.shape, 7).float().to(cuda)
    dq, dk = torch.autograd.grad(alpha, (q, k), dalpha)
    qo = q.detach().double().cpu().requires_grad_(True)
    ko = k.detach().double().cpu().requires_grad_(True)
    ao = eager.softmax_op(qo, ko, tr.double(), bias.double(), inside, p.rows, row_ptr, source, 4, scale)
    dqo, dko = torch.autograd.grad(ao, (qo, ko), dalpha.double().cpu())
    torch.testing.assert_close(alpha.double().cpu(), ao.detach(), **TOL[torch.float32])
    torch.testing.assert_close(dq.double().cpu(), dqo, **TOL[torch.float32])
    torch.testing.assert_close(dk.double().cpu(), dko, **TOL[torch.float32])
    bare_targets = (row_ptr[1:] == row_ptr[:-1]).to(cuda)
    bare_sources = torch.bincount(source, minlength=t.n_nodes).to(cuda) == 0
    assert bool(bare_targets.any()) and bool(bare_sources.any())
    assert bool((dq[bare_targets] == 0).all()) and bool((dk[bare_sources] == 0).all())
    # no edges at all
    empty = torch.zeros(0, dtype=torch.int64, device=cuda)
    a0 = fused_attention.Softmax.apply(q, k, tr[:0].to(cuda), bias[:0].to(cuda), inside[:0].to(cuda), desc.to(cuda),
                                       torch.zeros(t.n_nodes + 1, dtype=torch.int64, device=cuda), empty, 4, scale, 1)
    assert a0.shape == (0, 4)
    dq0, dk0 = torch.autograd.grad(a0.sum() * 0 + (q * 0).sum(), (q, k), allow_unused=True, materialize_grads=True)
    assert bool((dk0 == 0).all())


def test_checks_raise_the_reference_messages(cuda):
    t = problems.tables(8, 16)
    p, desc, scale = problems.attention_layout({0: 4, 1: 4}, 2)
    q = torch.zeros(t.n_nodes, p.width, device=cuda)
    ext = fused_attention.extension()
    with pytest.raises(RuntimeError, match="q and k must share a shape"):
        ext.softmax_forward(q, q[:, :4].contiguous(), t.transport.float().to(cuda), t.bias.float().to(cuda),
                            t.inside.to(cuda), desc.to(cuda), t.row_ptr.to(cuda), t.source.to(cuda), 2, scale, 1)
    with pytest.raises(RuntimeError, match="at most 16 heads"):
        ext.softmax_forward(q, q, t.transport.float().to(cuda), t.bias.float().to(cuda), t.inside.to(cuda),
                            desc.to(cuda), t.row_ptr.to(cuda), t.source.to(cuda), 17, scale, 1)
    with pytest.raises(RuntimeError, match="GPU only"):
        ext.softmax_forward(q.cpu(), q.cpu(), t.transport.float(), t.bias.float(), t.inside, desc, t.row_ptr,
                            t.source, 2, scale, 1)
