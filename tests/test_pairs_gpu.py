"""The fused pair terms (the general kernel's per-edge readout) on the HIP path.

* the op (``_native.pairs().forward/backward``) against ``oracle.eager.pair_term``
  under every flag combination, with and without the optional phases, scale
  and bias, in float32 and float64: the accumulated output, the input and
  trunk gradients, and the coefficient gradient through the weight and bias
  gradients it gives (``grad_k @ [hidden, 1]``);
* ``SO2SteerableKernel.forward`` on an edge-shaped field against the oracle's
  per-edge readout, with the input's and every parameter's gradient;
* the layers under ``GM_FACTORED_KERNEL=0`` (the per-edge readout path):
  ``SO2MHSA`` batched and per head, ``SO2Convolution``, against the oracle.
Tolerances as test_attention_gpu.close."""

import itertools

import pytest
import torch

import problems
from gm_attention_amd import _native
from gm_attention_amd.nn import kernels
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import eager, modules
from test_attention_gpu import close

pytestmark = pytest.mark.gpu

CX = {torch.float32: torch.complex64, torch.float64: torch.complex128}


def _r(t):
    return torch.view_as_real(t.resolve_conj()) if t.is_complex() else t


def _unit_phase(E, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.polar(torch.ones(E, dtype=torch.float64), torch.rand(E, generator=g, dtype=torch.float64) * 6.283)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("flags", range(16))
@pytest.mark.parametrize("optional", [True, False])
def test_term_op_matches_the_oracle(flags, optional, dtype, cuda):
    E, a, b, trunk = 777, 5, 3, 11
    print(f"pair term flags={flags} optional={optional} {dtype}", flush=True)
    width = (2 if flags & 1 else 1) * a * b
    hidden = problems.normal((E, trunk), 1).to(dtype).double()
    weight = problems.normal((width, trunk), 2).to(dtype).double()
    bias = problems.normal((width,), 3).to(dtype).double() if optional else None
    if flags & 2:
        u = problems.normal((E, a), 4).to(dtype).double()
    else:
        u = torch.view_as_complex(problems.normal((E, a, 2), 4).to(dtype).double())
    pre = _unit_phase(E, 5).to(CX[dtype]).to(torch.complex128) if optional else None
    post = _unit_phase(E, 6).to(CX[dtype]).to(torch.complex128) if optional else None
    scale = problems.normal((E,), 7).abs().to(dtype).double() if optional else None
    out_real = bool(flags & 8)
    g = problems.normal((E, b), 8) if out_real else torch.view_as_complex(problems.normal((E, b, 2), 8))
    g = g.to(dtype if out_real else CX[dtype]).to(torch.float64 if out_real else torch.complex128)
    start = problems.normal((E, b), 9) if out_real else torch.view_as_complex(problems.normal((E, b, 2), 9))

    leaves = [t.clone().requires_grad_(True) for t in (hidden, weight, u)] + (
        [bias.clone().requires_grad_(True)] if bias is not None else [])
    want = eager.pair_term(leaves[0], leaves[1], leaves[3] if bias is not None else None, leaves[2], pre, post, scale,
                           a, b, flags)
    loss = (want.conj() * g).real.sum() if not out_real else (want * g).sum()
    grads = torch.autograd.grad(loss, leaves)

    dev = lambda t: None if t is None else t.to(cuda, CX[dtype] if t.is_complex() else dtype).contiguous()
    empty = torch.empty(0, device=cuda, dtype=dtype)
    ext = _native.pairs()
    out = dev(start.to(torch.float64 if out_real else torch.complex128))
    ext.forward(dev(hidden), dev(weight), dev(bias) if bias is not None else empty, dev(u),
                dev(pre) if pre is not None else empty, dev(post) if post is not None else empty,
                dev(scale) if scale is not None else empty, out, a, b, flags)
    # scaled: grad_hidden measured at up to 3.1x the unscaled bound (entries up to 73)
    close(_r(out - dev(start)), _r(want), dtype, "out", scaled=True)

    grad_u = torch.zeros_like(dev(u))
    grad_hidden = torch.zeros_like(dev(hidden))
    grad_k = torch.empty(width, E + 5, dtype=dtype, device=cuda)[:, :E]  # a row stride beyond n_edges
    ext.backward(dev(hidden), dev(weight), dev(bias) if bias is not None else empty, dev(u),
                 dev(pre) if pre is not None else empty, dev(post) if post is not None else empty,
                 dev(scale) if scale is not None else empty, dev(g), grad_u, grad_hidden, grad_k, a, b, flags)
    close(grad_hidden, grads[0], dtype, "grad_hidden", scaled=True)
    close(_r(grad_u), _r(grads[2]), dtype, "grad_u", scaled=True)
    close(grad_k @ dev(hidden), grads[1], dtype, "grad_weight", reduction=True)
    if bias is not None:
        close(grad_k.sum(1), grads[3], dtype, "grad_bias", reduction=True)


FIELDS = [({0: 4, 1: 3, 2: 2}, {0: 3, 1: 2, 2: 2}), ({0: 4}, {0: 5, 1: 3, 2: 2}), ({1: 3}, {2: 2}),
          ({0: 16, 1: 16, 2: 16}, {0: 8, 1: 8, 2: 8})]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("fin,fout", FIELDS)
def test_kernel_forward_matches_the_readout_oracle(fin, fout, dtype, cuda):
    print(f"pairs kernel {fin}->{fout} {dtype}", flush=True)
    torch.manual_seed(0)
    disc = problems.discretization(10, 20)
    edges = disc.edge_geometry
    k = SO2SteerableKernel(SO2FieldType(fin), SO2FieldType(fout), cutoff=disc.coverage_radius, n_radial_basis=6,
                           dtype=torch.float64)
    with torch.no_grad():
        for p in k.parameters():
            p.add_(0.1 * torch.randn_like(p))
    k.load_state_dict({n: v.to(dtype).double() for n, v in k.state_dict().items()})
    n = edges.row_ptr.shape[0] - 1
    x = problems.normal((n, k.field_type_in.dimension), 1).to(dtype).double()
    probe = problems.normal((edges.n_edges, k.field_type_out.dimension), 2)
    edges_o = edges.to(None, dtype).to(None, torch.float64)

    xo = x.clone().requires_grad_(True)
    want = modules.flat(modules.readout_messages(k, SO2FeatureField.from_flat(k.field_type_in, xo).coefficients,
                                                 edges_o.source_index, edges_o.distances, edges_o.angular_phases,
                                                 edges_o.transport_phases))
    (want * probe).sum().backward()
    want_p = {name: p.grad.clone() for name, p in k.named_parameters()}

    gk = SO2SteerableKernel(k.field_type_in, k.field_type_out, cutoff=k.radial_basis.cutoff, n_radial_basis=6,
                            dtype=dtype, device=cuda)
    gk.load_state_dict({name: v.to(dtype) for name, v in k.state_dict().items()})
    xg = x.to(cuda, dtype).requires_grad_(True)
    e = edges.to(cuda, dtype)
    source = SO2FeatureField.from_flat(gk.field_type_in, xg.index_select(0, e.source_index))
    got = gk(source, e).to_flat()
    (got * probe.to(cuda, dtype)).sum().backward()
    # scaled: dx measured at up to 5.4x the unscaled bound (entries up to 49)
    close(got, want.detach(), dtype, "messages", scaled=True)
    close(xg.grad, xo.grad, dtype, "dx", scaled=True)
    for name, p in gk.named_parameters():
        close(p.grad, want_p[name], dtype, f"d{name}", reduction=True)


@pytest.mark.parametrize("batched", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_mhsa_on_the_per_edge_readout_matches_the_oracle(batched, dtype, cuda, monkeypatch):
    import test_attention_gpu

    monkeypatch.setattr(kernels, "FACTORED", False)
    test_attention_gpu.test_mhsa_matches_the_oracle(({0: 8, 1: 8, 2: 8}, 4, "hard", 2), dtype, batched, cuda)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_convolution_on_the_per_edge_readout_matches_the_oracle(dtype, cuda, monkeypatch):
    import test_convolution_gpu

    monkeypatch.setattr(kernels, "FACTORED", False)
    test_convolution_gpu.test_convolution_matches_the_oracle(({0: 4, 1: 3, 2: 2}, False, "quartic", True, "linear", 1),
                                                            dtype, cuda)


def test_term_op_rejects_bad_shapes(cuda):
    ext = _native.pairs()
    h = torch.zeros(10, 4, device=cuda)
    w = torch.zeros(2 * 3 * 2, 4, device=cuda)
    u = torch.zeros(10, 3, dtype=torch.complex64, device=cuda)
    out = torch.zeros(10, 2, dtype=torch.complex64, device=cuda)
    e = torch.empty(0, device=cuda)
    for bad in itertools.product((17,), (2,)):
        with pytest.raises(RuntimeError):
            ext.forward(h, w, e, u, e, e, e, out, bad[0], bad[1], 1)
    with pytest.raises(RuntimeError):  # u complex under U_REAL
        ext.forward(h, w, e, u, e, e, e, out, 3, 2, 1 | 2)
    with pytest.raises(RuntimeError):  # weight rows for a real matrix
        ext.forward(h, w, e, u, e, e, e, out, 3, 2, 0)
