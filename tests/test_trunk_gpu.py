"""The HIP radial trunk (nn.radial.RadialTrunk: every head's Gaussian basis,
Linear and SiLU in one pass) against the oracle's trunk (oracle.modules._trunk,
the reference's _GaussianRadialBasis + apply_radial_trunk, float64 on the
float32-rounded parameters), features and the weights' and biases' gradients.
Tolerance: rtol 1e-5 with atol 1e-6 times the tensor's largest magnitude for
the features; the gradients (sums over every edge) within 1e-5 of their norm."""

import pytest
import torch

import problems
from gm_attention_amd.nn import radial
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.representations.field_type import SO2FieldType
from oracle import modules

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("n_basis,bias", [(8, True), (8, False), (6, True), (6, False), (4, True), (4, False)])
def test_trunk_matches_the_oracle(n_basis, bias, offset, cuda):
    """offset 1: the distances start one element into their storage (not 16-byte
    aligned) and number no multiple of the 16-edge tiles."""
    disc = problems.discretization(16, 32)
    edges = disc.edge_geometry.tile(3, n_sources=disc.n_nodes)
    torch.manual_seed(1)
    kernels = [SO2SteerableKernel(SO2FieldType({0: 2, 1: 2}), SO2FieldType({0: 1, 1: 1}), cutoff=disc.coverage_radius,
                                  n_radial_basis=n_basis, bias=bias, dtype=torch.float32) for _ in range(5)]
    d32 = edges.distances.float()[offset:]
    probe = problems.normal((5, d32.shape[0], 16), 4)
    # oracle: float64 on the rounded parameters and distances
    want, want_grads = [], []
    for k, pr in zip(kernels, probe):
        k64 = SO2SteerableKernel(k.field_type_in, k.field_type_out, cutoff=disc.coverage_radius, n_radial_basis=n_basis,
                                 bias=bias, dtype=torch.float64)
        k64.load_state_dict({n: v.double() for n, v in k.state_dict().items()})
        h = modules._trunk(k64, d32.double())
        lin = list(k64.radial_trunk)[0]
        grads = torch.autograd.grad((h * pr).sum(), [lin.weight] + ([lin.bias] if bias else []))
        want.append(h.detach())
        want_grads.append(grads)
    gk = [SO2SteerableKernel(k.field_type_in, k.field_type_out, cutoff=disc.coverage_radius, n_radial_basis=n_basis,
                             bias=bias, dtype=torch.float32, device=cuda) for k in kernels]
    for g, k in zip(gk, kernels):
        g.load_state_dict(k.state_dict())
    assert radial.eligible(gk, torch.float32, cuda)
    rho_all = (edges.distances.float() / disc.coverage_radius).to(cuda)
    rho = rho_all[offset:]
    if offset:
        assert rho.data_ptr() % 16 != 0 and rho.shape[0] % 16 != 0
    h = radial.trunk_hidden_heads(gk, rho)
    (h * probe.float().to(cuda)).sum().backward()
    for head in range(5):
        w = want[head]
        problems.report_strict(h[head].detach(), w, f"h[{head}]")
        torch.testing.assert_close(h[head].detach().double().cpu(), w, rtol=1e-5, atol=1e-6 * float(w.abs().max()))
        lin = list(gk[head].radial_trunk)[0]
        got = [lin.weight.grad] + ([lin.bias.grad] if bias else [])
        for a, b in zip(got, want_grads[head]):
            a = a.double().cpu()
            assert float((a - b).norm() / b.norm()) <= 1e-5
            assert float((a - b).abs().max() / b.abs().max()) <= 1e-5
