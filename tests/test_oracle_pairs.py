"""Pins the pair-term oracle and the plan (CPU only).

The per-edge readout (``oracle.modules.readout_messages``, pinned to the
factored order and to the compiled reference in test_oracle_factored.py)
must equal the sum of ``oracle.eager.pair_term`` over the product's plan
(``fused_pairs.plan``), each term fed the tables ``forward_general`` feeds the
op: so the plan's flags, rows, phase orders and radial powers, and the term
restatement, are checked together against an independent derivation.  The
plan's order is the reference's pair loop (nn/fused_pairs.py:96-123): output
frequency outer, input frequency inner, the antilinear term after the linear
one.
"""

import pytest
import torch

import problems
from gm_attention_amd.nn import fused_pairs
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import eager, modules

CONFIGS = [
    ({0: 4, 1: 3, 2: 2}, {0: 3, 1: 2, 2: 2}),
    ({0: 4}, {0: 5, 1: 3, 2: 2}),
    ({0: 4, 1: 3, 2: 2}, {0: 3}),
    ({1: 3}, {2: 2}),
    ({0: 16, 1: 16, 2: 16}, {0: 16, 1: 16, 2: 16}),
]


def _kernel(fin, fout, seed=0):
    torch.manual_seed(seed)
    k = SO2SteerableKernel(SO2FieldType(fin), SO2FieldType(fout), cutoff=problems.discretization(10, 20).coverage_radius,
                           n_radial_basis=6, dtype=torch.float64)
    with torch.no_grad():
        for p in k.parameters():
            p.add_(0.2 * torch.randn_like(p))
    return k


@pytest.mark.parametrize("fin,fout", CONFIGS)
def test_terms_sum_to_the_per_edge_readout(fin, fout):
    kernel = _kernel(fin, fout)
    edges = problems.discretization(10, 20).edge_geometry
    n = edges.row_ptr.shape[0] - 1
    x = SO2FeatureField.from_flat(kernel.field_type_in, problems.normal((n, kernel.field_type_in.dimension), 1))
    want = modules.readout_messages(kernel, x.coefficients, edges.source_index, edges.distances, edges.angular_phases,
                                    edges.transport_phases)
    hidden = modules._trunk(kernel, edges.distances)
    rho = edges.distances / kernel.radial_basis.cutoff
    got = {}
    for t in fused_pairs.plan(kernel):
        head = kernel.real_head if t.real_head else kernel.complex_head
        w, bias = head.weight[t.rows], head.bias[t.rows]
        u = x[t.n].index_select(0, edges.source_index)
        if t.n != 0:
            u = edges.transport_phases[:, t.n].unsqueeze(-1) * torch.view_as_complex(u.contiguous())
        pre = edges.angular_harmonic(t.pre_order) if t.pre_order is not None else None
        post = edges.angular_harmonic(t.post_order) if t.post_order is not None else None
        scale = rho ** t.power if t.power is not None else None
        term = eager.pair_term(hidden, w, bias, u, pre, post, scale, t.a, t.b, t.flags)
        got[t.m] = term if t.m not in got else got[t.m] + term
    for m in want:
        g = got[m] if m == 0 else torch.view_as_real(got[m])
        torch.testing.assert_close(g, want[m], rtol=1e-12, atol=1e-12)


def test_plan_order_and_flags():
    kernel = _kernel({0: 2, 1: 1, 2: 1}, {0: 1, 1: 2})
    terms = fused_pairs.plan(kernel)
    assert [(t.m, t.n, t.role) for t in terms] == [
        (0, 0, "real"), (0, 1, "linear"), (0, 2, "linear"),
        (1, 0, "linear"), (1, 1, "linear"), (1, 1, "antilinear"), (1, 2, "linear"), (1, 2, "antilinear")]
    by = {(t.n, t.m, t.role): t for t in terms}
    assert by[(0, 0, "real")].flags == fused_pairs.U_REAL | fused_pairs.OUT_REAL
    assert by[(1, 0, "linear")].flags == fused_pairs.MATRIX_COMPLEX | fused_pairs.CONJ_U | fused_pairs.OUT_REAL
    assert (by[(1, 0, "linear")].pre_order, by[(1, 0, "linear")].power) == (1, 1)
    assert (by[(0, 1, "linear")].post_order, by[(0, 1, "linear")].flags) == (1, fused_pairs.MATRIX_COMPLEX | fused_pairs.U_REAL)
    assert (by[(2, 1, "linear")].pre_order, by[(2, 1, "antilinear")].pre_order) == (-1, 3)
    assert (by[(2, 1, "linear")].power, by[(2, 1, "antilinear")].power) == (1, 3)
    assert by[(1, 1, "antilinear")].flags == fused_pairs.MATRIX_COMPLEX | fused_pairs.CONJ_U
