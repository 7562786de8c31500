"""Pins the oracle's layer-level pieces against something independent of the
product:

* ``modules.softmax_weights`` (the softmax inside ``mhsa_forward``, the oracle
  of every layer test) equals the reference's own compiled softmax
  (``oracle/_ref``, attention.h) fed the window tables this test derives from
  the reference's window definitions (convolution.py:47-91: the hard window's
  slack, the quartic ``relu(1 - (d/c)^2)^2``), hard and quartic, with the
  float32 slack admitting an edge just past the cutoff;
* ``modules.gaussian_basis`` (the radial basis of ``modules._trunk``) takes
  its closed-form values: ``phi_k(mu_k) = 1``, ``exp(-1/2)`` one width away,
  ``exp(-2)`` two widths away, at the distances that put ``s = (r/c)^2`` on
  the centres; and the product's basis module equals it;
* ``modules.linear`` equals the dense real intertwiner built from the
  weights (reference tests/support/intertwiners.py:212: the complex weight
  ``M + iN`` of frequency n acting on each ``(re, im)`` pair as
  ``[[M, -N], [N, M]]``), on non-square maps with frequencies the other side
  lacks, plus a hand-computed answer; and the dense matrix commutes with
  every rotation (an intertwiner);
* ``modules.head_type`` / ``modules.score_scale`` (the per-head type and
  score scale ``mhsa_forward`` derives itself) take hand-computed values at
  C1's and C2's fields (20 reals a head, 1/sqrt(20)) and on a field whose
  head width differs from D / H, and the product's heads carry the same."""

import math

import pytest
import torch

import problems
from gm_attention_amd.nn.kernels import GaussianRadialBasis
from gm_attention_amd.nn.linear import SO2Linear
from gm_attention_amd.representations.field_type import SO2FieldType
from oracle import modules, ref

D64 = torch.float64


# ---------------------------------------------------------------- softmax_weights


def _window(d, cutoff, kind, tol):
    if kind == "hard":
        return (d <= cutoff + tol).to(d.dtype)
    return torch.relu(1.0 - (d / cutoff) ** 2) ** 2


def _dict_field(flat, field):
    """The flat layout's frequency blocks: 0 first, then (copies, 2) pairs."""
    out, col = {}, 0
    for f in sorted(field):
        m = field[f]
        w = m if f == 0 else 2 * m
        out[f] = flat[:, col:col + w] if f == 0 else flat[:, col:col + w].reshape(-1, m, 2)
        col += w
    return out


@pytest.mark.parametrize("window", ["hard", "quartic"])
@pytest.mark.parametrize("field,heads", [({0: 8, 1: 8, 2: 8}, 4), ({0: 6, 1: 4, 2: 2}, 2), ({0: 4, 2: 2}, 1)])
def test_softmax_weights_match_the_compiled_reference(field, heads, window):
    if not ref.available():
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    disc = problems.discretization(12, 24)
    edges = disc.edge_geometry
    cutoff = disc.coverage_radius
    _, desc, scale = problems.attention_layout(field, heads)
    D = sum(m if f == 0 else 2 * m for f, m in field.items())
    q = problems.normal((edges.row_ptr.shape[0] - 1, D), 1)
    k = problems.normal((edges.row_ptr.shape[0] - 1, D), 2)
    got = modules.softmax_weights(_dict_field(q, field), _dict_field(k, field), edges, cutoff, window, heads, scale)
    d = edges.distances
    win = _window(d, cutoff, window, 1e-10)
    tiny = torch.finfo(D64).tiny
    bias = torch.log(win.clamp_min(tiny)) + torch.log(edges.tangent_quadrature_weights.clamp_min(tiny))
    transport = torch.view_as_real(edges.transport_phases.contiguous()).contiguous()
    want = ref.softmax_forward(q, k, transport, bias.contiguous(), (win > 0).to(torch.uint8), desc, edges.row_ptr,
                               edges.source_index, heads, scale)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-14)
    sums = torch.segment_reduce(got, "sum", offsets=edges.row_ptr, axis=0)
    torch.testing.assert_close(sums, torch.ones_like(sums), rtol=0, atol=1e-12)


def test_softmax_weights_admit_the_float32_slack_like_the_compiled_reference():
    """A hard window in float32 admits d <= c + 1e-5: with the cutoff set just
    below some edges' distances, those edges are in only under the slack, in
    the oracle (tolerance=1e-5) and in the reference fed the same table."""
    if not ref.available():
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    disc = problems.discretization(12, 24)
    edges = disc.edge_geometry
    d = edges.distances
    cutoff = float(d.max()) - 5e-6  # the farthest edges sit 5e-6 past the cutoff
    slack = d > cutoff
    assert int(slack.sum()) > 0
    field, heads = {0: 4, 1: 4, 2: 4}, 2
    _, desc, scale = problems.attention_layout(field, heads)
    q = problems.normal((edges.row_ptr.shape[0] - 1, 20), 3)
    k = problems.normal((edges.row_ptr.shape[0] - 1, 20), 4)
    got = modules.softmax_weights(_dict_field(q, field), _dict_field(k, field), edges, cutoff, "hard", heads, scale,
                                  tolerance=1e-5)
    assert bool((got[slack] > 0).all())
    strict = modules.softmax_weights(_dict_field(q, field), _dict_field(k, field), edges, cutoff, "hard", heads,
                                     scale, tolerance=1e-10)
    assert bool((strict[slack] == 0).all())
    win = _window(d, cutoff, "hard", 1e-5)
    tiny = torch.finfo(D64).tiny
    bias = torch.log(win.clamp_min(tiny)) + torch.log(edges.tangent_quadrature_weights.clamp_min(tiny))
    transport = torch.view_as_real(edges.transport_phases.contiguous()).contiguous()
    want = ref.softmax_forward(q, k, transport, bias.contiguous(), (win > 0).to(torch.uint8), desc, edges.row_ptr,
                               edges.source_index, heads, scale)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-14)


# ---------------------------------------------------------------- the radial basis


@pytest.mark.parametrize("n_basis", [2, 4, 8])
def test_gaussian_basis_takes_its_closed_form_values(n_basis):
    cutoff = 0.7
    width = 1.0 / (n_basis - 1)
    for k in range(n_basis):
        mu = k * width
        r = torch.tensor([math.sqrt(mu) * cutoff], dtype=D64)  # s = (r/c)^2 = mu_k
        phi = modules.gaussian_basis(r, n_basis, cutoff)[0]
        assert abs(float(phi[k]) - 1.0) < 1e-14
        for j in range(n_basis):
            steps = abs(j - k)
            assert abs(float(phi[j]) - math.exp(-0.5 * steps * steps)) < 1e-13, (k, j)


def test_gaussian_basis_with_one_function_is_exp_of_minus_half_s_squared():
    r = torch.linspace(0.0, 1.3, 9, dtype=D64)
    s = (r / 1.3) ** 2
    torch.testing.assert_close(modules.gaussian_basis(r, 1, 1.3)[:, 0], torch.exp(-0.5 * s * s), rtol=1e-15, atol=0)


@pytest.mark.parametrize("n_basis", [1, 4, 8])
def test_the_products_radial_basis_equals_the_oracles(n_basis):
    r = torch.linspace(0.0, 0.9, 57, dtype=D64)
    basis = GaussianRadialBasis(n_basis, 0.9, dtype=D64)
    torch.testing.assert_close(basis(r), modules.gaussian_basis(r, n_basis, 0.9), rtol=1e-14, atol=1e-15)


# ---------------------------------------------------------------- SO2Linear


def dense_intertwiner(lin, fin: SO2FieldType, fout: SO2FieldType) -> torch.Tensor:
    """The real (D_out, D_in) matrix of the layer, block by block from its weights."""
    def offsets(ft):
        out, col = {}, 0
        for f in ft.frequencies:
            out[f] = col
            col += ft.multiplicity(f) * (1 if f == 0 else 2)
        return out

    oi, oo = offsets(fin), offsets(fout)
    dense = torch.zeros(fout.dimension, fin.dimension, dtype=D64)
    for f in fout.frequencies:
        if f not in fin.frequencies or str(f) not in lin.weight:
            continue
        w = lin.weight[str(f)].detach()
        b, a = fout.multiplicity(f), fin.multiplicity(f)
        for i in range(b):
            for j in range(a):
                if f == 0:
                    dense[oo[0] + i, oi[0] + j] = w[i, j]
                else:
                    M, N = float(w[i, j, 0]), float(w[i, j, 1])
                    r, c = oo[f] + 2 * i, oi[f] + 2 * j
                    dense[r:r + 2, c:c + 2] = torch.tensor([[M, -N], [N, M]], dtype=D64)
    return dense


def _rotation(ft: SO2FieldType, theta: float) -> torch.Tensor:
    blocks = []
    for f in ft.frequencies:
        for _ in range(ft.multiplicity(f)):
            if f == 0:
                blocks.append(torch.ones(1, 1, dtype=D64))
            else:
                c, s = math.cos(f * theta), math.sin(f * theta)
                blocks.append(torch.tensor([[c, -s], [s, c]], dtype=D64))
    return torch.block_diag(*blocks)


@pytest.mark.parametrize("fin,fout", [({0: 3, 1: 2}, {0: 5, 1: 4}), ({0: 2, 1: 3, 2: 1}, {1: 2, 2: 4, 3: 1}),
                                      ({1: 2, 2: 3}, {0: 2, 1: 1, 2: 2})])
def test_linear_is_the_dense_intertwiner(fin, fout):
    fi, fo = SO2FieldType(fin), SO2FieldType(fout)
    torch.manual_seed(5)
    lin = SO2Linear(fi, fo, dtype=D64)
    with torch.no_grad():
        if lin.bias is not None:
            lin.bias.normal_()
    x = problems.normal((11, fi.dimension), 9)
    got = modules.flat(modules.linear(lin, _dict_field(x, fin), fo))
    dense = dense_intertwiner(lin, fi, fo)
    bias = torch.zeros(fo.dimension, dtype=D64)
    if lin.bias is not None and 0 in fout:
        bias[:fout[0]] = lin.bias.detach()
    torch.testing.assert_close(got, x @ dense.T + bias, rtol=1e-13, atol=1e-13)
    for theta in (0.3, 1.9, -2.4):  # the dense matrix intertwines the rotations
        torch.testing.assert_close(dense @ _rotation(fi, theta), _rotation(fo, theta) @ dense, rtol=0, atol=1e-13)


def test_linear_known_answer():
    """{0:1, 1:1} -> {0:1, 1:1}: w_0 = 2, bias 0.5, w_1 = 1 + 2i on x = (3 | 3 + 4i):
    y_0 = 2 * 3 + 0.5 = 6.5, y_1 = (1 + 2i)(3 + 4i) = -5 + 10i."""
    ft = SO2FieldType({0: 1, 1: 1})
    lin = SO2Linear(ft, ft, dtype=D64)
    with torch.no_grad():
        lin.weight["0"].copy_(torch.tensor([[2.0]], dtype=D64))
        lin.weight["1"].copy_(torch.tensor([[[1.0, 2.0]]], dtype=D64))
        lin.bias.copy_(torch.tensor([0.5], dtype=D64))
    x = {0: torch.tensor([[3.0]], dtype=D64), 1: torch.tensor([[[3.0, 4.0]]], dtype=D64)}
    y = modules.linear(lin, x, ft)
    assert float(y[0][0, 0].detach()) == 6.5
    assert y[1][0, 0].detach().tolist() == [-5.0, 10.0]


# ---------------------------------------------------------------- head type and score scale


@pytest.mark.parametrize("mult, heads, dim, want_types", [
    ({0: 16, 1: 16, 2: 16}, 4, 20, {0: 4, 1: 4, 2: 4}),   # C1: 16 + 2*16 + 2*16 = 80 reals, 4 heads
    ({0: 32, 1: 32, 2: 32}, 8, 20, {0: 4, 1: 4, 2: 4}),   # C2 / NS: 160 reals, 8 heads
    ({0: 8, 2: 4}, 4, 4, {0: 2, 2: 1}),                    # 16 reals, 4 heads: D / H = 4 by luck of 2 + 2*1
    ({0: 6, 1: 3}, 3, 4, {0: 2, 1: 1}),                    # 12 reals, 3 heads
    ({0: 4, 1: 8}, 4, 5, {0: 1, 1: 2}),                    # 20 reals, 4 heads: D / H = 5
    ({1: 4, 2: 2}, 2, 6, {1: 2, 2: 1}),                    # no scalar channel
])
def test_head_type_and_score_scale_known_answers(mult, heads, dim, want_types):
    attn = modules.head_type(mult, heads)
    assert attn.multiplicities == want_types
    assert attn.dimension == dim
    assert modules.score_scale(attn) == pytest.approx(1.0 / math.sqrt(dim), rel=1e-15)
    # the product (reference attention.py:217, :551-556) carries the same type and scale
    from gm_attention_amd.nn.attention import SO2MHSA

    mhsa = SO2MHSA(SO2FieldType(mult), heads, cutoff=0.3, batched=True, dtype=D64)
    for head in mhsa.heads:
        assert {f: head.field_type_attn.multiplicity(f) for f in head.field_type_attn.frequencies} == want_types
        assert head._score_scale == pytest.approx(modules.score_scale(attn), rel=1e-15)


def test_score_scale_numbers():
    """The scales as literal numbers, so a dimension counted per copy instead
    of per real (12 for C2, not 20) or the whole width (160) cannot hide."""
    c2 = modules.head_type({0: 32, 1: 32, 2: 32}, 8)
    assert modules.score_scale(c2) == pytest.approx(0.22360679774997896, rel=1e-15)
    assert modules.score_scale(modules.head_type({0: 16, 1: 16, 2: 16}, 4)) == pytest.approx(0.22360679774997896)
    with pytest.raises(ValueError):
        modules.head_type({0: 6, 1: 4}, 4)
