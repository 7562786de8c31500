"""Pins the convolution layer's oracle (CPU only).

* the depthwise kernel equals a general steerable kernel whose only nonzero
  readout rows are the diagonal copy blocks ``(n, n)`` -- linear ``A``,
  antilinear ``B``, real ``C`` -- (the reference's own check,
  tests/nn/test_depthwise.py:87-100): ``oracle.modules.depthwise_layer_messages``
  against ``oracle.modules.readout_messages``, which is pinned to the factored
  order and to the compiled reference (test_oracle_factored.py);
* the same messages against ``oracle.eager.depthwise_messages`` (pinned to the
  compiled reference's ``conv_forward``) on the readouts as the fused op
  receives them: the layout of ``(rc, cc)`` derived twice, independently;
* at ``r = 0`` the depthwise kernel is the per-copy intertwiner ``C(0)`` /
  ``A(0)`` (reference nn/depthwise.py:17-19).
"""

import pytest
import torch

import problems
from gm_attention_amd.nn.convolution import SO2Convolution
from gm_attention_amd.nn.depthwise import SO2DepthwiseKernel, stacked_coefficients
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import eager, modules

FIELDS = [{0: 3, 1: 2, 2: 2}, {1: 3}, {0: 4, 2: 1}]


def _depthwise(field, seed=0, **kw):
    torch.manual_seed(seed)
    k = SO2DepthwiseKernel(SO2FieldType(field), cutoff=problems.discretization(10, 20).coverage_radius,
                           dtype=torch.float64, **kw)
    with torch.no_grad():  # nonzero biases, so the bias rows are exercised too
        for p in k.parameters():
            p.add_(0.3 * torch.randn_like(p))
    return k


def _as_general(dw: SO2DepthwiseKernel) -> SO2SteerableKernel:
    ft = dw.field_type
    gen = SO2SteerableKernel(ft, ft, cutoff=dw.cutoff, n_radial_basis=dw.radial_basis.n_basis,
                             radial_hidden_features=[16], dtype=torch.float64)
    gen.radial_trunk.load_state_dict(dw.radial_trunk.state_dict())
    ranges, _ = modules.layout(ft, ft)
    start = {(n, m, r): s for n, m, r, s, _p in ranges}
    with torch.no_grad():
        if gen.complex_head is not None:
            gen.complex_head.weight.zero_()
            gen.complex_head.bias.zero_()
        if gen.real_head is not None:
            gen.real_head.weight.zero_()
            gen.real_head.bias.zero_()
        a0 = ft.multiplicity(0) if 0 in ft else 0
        for a in range(a0):  # real block rows (b, a): the diagonal
            gen.real_head.weight[a * a0 + a] = dw.real_head.weight[a]
            gen.real_head.bias[a * a0 + a] = dw.real_head.bias[a]
        coff = 0
        for n in ft.frequencies:
            if n == 0:
                continue
            an = ft.multiplicity(n)
            for role, src in (("linear", coff), ("antilinear", coff + 2 * an)):
                s = start[(n, n, role)]
                for a in range(an):
                    for r in range(2):  # rows (b, a, re/im) of the (n, n) block
                        gen.complex_head.weight[s + 2 * (a * an + a) + r] = dw.complex_head.weight[src + 2 * a + r]
                        gen.complex_head.bias[s + 2 * (a * an + a) + r] = dw.complex_head.bias[src + 2 * a + r]
            coff += 4 * an
    return gen


@pytest.mark.parametrize("field", FIELDS)
def test_depthwise_is_the_diagonal_general_kernel(field):
    dw = _depthwise(field)
    gen = _as_general(dw)
    edges = problems.discretization(10, 20).edge_geometry
    x = SO2FeatureField.from_flat(dw.field_type, problems.normal((edges.row_ptr.shape[0] - 1,
                                                                   dw.field_type.dimension), 1)).coefficients
    got = modules.depthwise_layer_messages(dw, x, edges)
    want = modules.readout_messages(gen, x, edges.source_index, edges.distances, edges.angular_phases,
                                    edges.transport_phases)
    for f in got:
        torch.testing.assert_close(got[f], want[f], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("field", FIELDS)
def test_layer_messages_match_the_op_boundary_oracle(field):
    dw = _depthwise(field, seed=3)
    edges = problems.discretization(10, 20).edge_geometry
    p, _ = problems.depthwise_layout(field)
    flat = problems.normal((edges.row_ptr.shape[0] - 1, dw.field_type.dimension), 2)
    x = SO2FeatureField.from_flat(dw.field_type, flat).coefficients
    rc, cc = stacked_coefficients([dw], edges)
    E = edges.n_edges
    tr = torch.view_as_real(edges.transport_phases.contiguous())
    an = torch.view_as_real(edges.angular_phases.contiguous())
    rho = edges.distances / dw.cutoff
    op = eager.depthwise_messages(flat, rc if rc is not None else flat.new_zeros(1, E, 0),
                                  cc if cc is not None else flat.new_zeros(1, E, 0), tr, an, rho, p.rows,
                                  edges.source_index)
    layer = modules.flat(modules.depthwise_layer_messages(dw, x, edges))
    torch.testing.assert_close(op.detach(), layer.detach(), rtol=1e-12, atol=1e-12)


def test_depthwise_at_the_origin_is_the_per_copy_intertwiner():
    dw = _depthwise({0: 3, 1: 2, 2: 2}, seed=5)
    edges = problems.discretization(10, 20).edge_geometry
    self_loops = (edges.source_index == edges.target_index).nonzero().squeeze(1)
    sub = edges.select(self_loops, n_nodes=edges.row_ptr.shape[0] - 1)
    assert float(sub.distances.max()) < 1e-15  # atan2 of a cross product at rounding level
    x = SO2FeatureField.from_flat(dw.field_type, problems.normal((sub.row_ptr.shape[0] - 1,
                                                                   dw.field_type.dimension), 4)).coefficients
    msgs = modules.depthwise_layer_messages(dw, x, sub)
    h = modules._trunk(dw, torch.zeros(1, dtype=torch.float64))
    c = (h @ dw.real_head.weight.T + dw.real_head.bias)[0]
    cc = (h @ dw.complex_head.weight.T + dw.complex_head.bias)[0]
    xs = x[0].index_select(0, sub.source_index)
    torch.testing.assert_close(msgs[0], c * xs, rtol=1e-12, atol=1e-12)
    coff = 0
    for n in (1, 2):
        A = torch.view_as_complex(cc[coff:coff + 8].reshape(2, 2, 2)[0].contiguous())
        z = torch.view_as_complex(x[n].index_select(0, sub.source_index).contiguous())  # transport at r = 0: identity
        torch.testing.assert_close(torch.view_as_complex(msgs[n].contiguous()), A * z, rtol=1e-12, atol=1e-12)
        coff += 4 * 2


def test_layer_rejects_mismatched_types_and_bad_arguments():
    a, b = SO2FieldType({0: 2, 1: 1}), SO2FieldType({0: 1})
    with pytest.raises(ValueError):
        SO2Convolution(a, b, cutoff=0.3, depthwise=True)
    with pytest.raises(ValueError):
        SO2Convolution(a, a, cutoff=0.3, window="box")
    with pytest.raises(ValueError):
        SO2Convolution(a, a, cutoff=0.3, eps=0.0)
    with pytest.raises(ValueError):
        SO2Convolution(a, a, cutoff=0.3, self_interaction="affine")


def test_stacked_coefficients_of_several_kernels_stack_each_kernels_readouts():
    """Three kernels of one field on one edge set: the stacked readouts are
    each kernel's own (its trunk and heads), kernel by kernel, and equal the
    oracle's trunk and heads (``modules._trunk`` and the heads' weights)."""
    field = {0: 3, 1: 2, 2: 2}
    kernels = [_depthwise(field, seed=11 + i) for i in range(3)]
    edges = problems.discretization(10, 20).edge_geometry
    rc, cc = stacked_coefficients(kernels, edges)
    assert rc.shape == (3, edges.n_edges, 3) and cc.shape == (3, edges.n_edges, 4 * 2 + 4 * 2)
    for i, k in enumerate(kernels):
        alone = stacked_coefficients([k], edges)
        torch.testing.assert_close(rc[i], alone[0][0], rtol=0, atol=0)
        torch.testing.assert_close(cc[i], alone[1][0], rtol=0, atol=0)
        hidden = modules._trunk(k, edges.distances)
        torch.testing.assert_close(rc[i], hidden @ k.real_head.weight.T + k.real_head.bias, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(cc[i], hidden @ k.complex_head.weight.T + k.complex_head.bias, rtol=1e-12,
                                   atol=1e-12)
