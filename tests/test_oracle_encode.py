"""Bipartite neighbourhoods, the grid hierarchy, the encoder oracle and the
wide-kernel tiling plan, on the CPU:

* the host bipartite CSR equals the all-pairs float64 brute force
  (oracle.sphere.brute_force_edges with a separate source set), and an
  uncovered target raises (reference edge_geometry.py:920-928);
* between a grid and itself the bipartite geometry is the same-grid geometry
  (edge list and every table): the concatenation of edge_geometry.py:930-961
  is pinned by the same-grid builder;
* the tiled hierarchy is the block-diagonal union of the samples' transfers;
* oracle.modules.encode_forward on a grid and itself is the pinned
  convolution oracle (SO2Convolution without self-interaction or
  normalisation, same kernel), and it is gauge equivariant under independent
  random rotations of the fine and coarse frames;
* the output tiles of a wide kernel cover every output column once, each within
  the fused op's bounds, and reproduce the full plan's mix columns."""

import math

import numpy as np
import pytest
import torch

import problems
from gm_attention_amd.discretization import edge_geometry as eg
from gm_attention_amd.discretization.frames import build_tangent_frames, rotate_tangent_frames
from gm_attention_amd.discretization.grid import build_equiangular_grid
from gm_attention_amd.discretization.hierarchy import build_grid_hierarchy
from gm_attention_amd.nn import fused_factored
from gm_attention_amd.nn.blocks import EquiEncode
from gm_attention_amd.nn.convolution import SO2Convolution
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.representations.field_type import SO2FieldType
from oracle import modules, sphere

D64 = torch.float64


def bipartite(fine, coarse, cutoff, frames=(None, None)):
    ff = build_tangent_frames(fine.nodes) if frames[0] is None else frames[0]
    cf = build_tangent_frames(coarse.nodes) if frames[1] is None else frames[1]
    return eg.compute_bipartite_edge_geometry(fine.nodes, ff, fine.quadrature_weights, coarse.nodes, cf,
                                              cutoff=cutoff, max_frequency=4, source_exact_nodes=fine.exact_nodes,
                                              target_exact_nodes=coarse.exact_nodes)


@pytest.mark.parametrize("fine,coarse,rows", [((17, 34), (9, 18), 1.5), ((16, 32), (8, 16), 2.0), ((9, 18), (5, 10), 1.0)])
def test_bipartite_csr_is_the_brute_force(fine, coarse, rows):
    f, c = build_equiangular_grid(*fine), build_equiangular_grid(*coarse)
    cutoff = rows * math.pi / (coarse[0] - 1)
    e = bipartite(f, c, cutoff)
    want = sphere.brute_force_edges(c.exact_nodes.numpy(), cutoff, sources=f.exact_nodes.numpy())
    assert np.array_equal(e.edge_index.numpy(), want)
    assert np.array_equal(e.row_ptr.numpy(), np.concatenate([[0], np.cumsum(np.bincount(want[0], minlength=c.n_nodes))]))


def test_uncovered_targets_raise():
    f, c = build_equiangular_grid(5, 8), build_equiangular_grid(9, 18)
    with pytest.raises(ValueError, match="no source within"):
        bipartite(f, c, 0.05)


def test_bipartite_on_one_grid_is_the_same_grid_geometry():
    g = build_equiangular_grid(12, 24)
    cutoff = 3.0 * math.pi / 11
    frames = build_tangent_frames(g.nodes)
    a = bipartite(g, g, cutoff, (frames, frames))
    b = eg.compute_edge_geometry(g, frames, cutoff)
    assert torch.equal(a.edge_index, b.edge_index) and torch.equal(a.row_ptr, b.row_ptr)
    for name in ("log_coordinates", "distances", "transport_angles", "tangent_quadrature_weights", "transport_phases"):
        torch.testing.assert_close(getattr(a, name), getattr(b, name), rtol=0, atol=1e-13)
    far = b.distances > 1e-9
    torch.testing.assert_close(a.angular_phases[far], b.angular_phases[far], rtol=0, atol=1e-13)


def hierarchy():
    grids = [build_equiangular_grid(17, 34), build_equiangular_grid(9, 18), build_equiangular_grid(5, 10)]
    return build_grid_hierarchy(grids, ["equiangular"] * 3, [(17, 34), (9, 18), (5, 10)],
                                restrict_cutoffs=[1.5 * math.pi / 8, 1.5 * math.pi / 4],
                                interpolate_cutoffs=[1.5 * math.pi / 8, 1.5 * math.pi / 4],
                                local_cutoffs=[None, [3 * math.pi / 8], [3 * math.pi / 4]])


def test_tiled_hierarchy_is_the_block_diagonal_union():
    h = hierarchy()
    t = h.tile(3)
    assert t.depth == 2 and t.levels[1].n_nodes == 3 * h.levels[1].n_nodes
    for k, (one, many) in enumerate(zip(h.down_edges, t.down_edges)):
        n_src, n_tgt = h.levels[k].n_nodes, h.levels[k + 1].n_nodes
        for b in range(3):
            rows = slice(int(many.row_ptr[b * n_tgt]), int(many.row_ptr[(b + 1) * n_tgt]))
            assert torch.equal(many.edge_index[0, rows] - b * n_tgt, one.edge_index[0])
            assert torch.equal(many.edge_index[1, rows] - b * n_src, one.edge_index[1])
    assert h.levels[0].discretization is None and h.levels[1].discretization is not None


def test_encode_oracle_on_one_grid_is_the_convolution_oracle():
    g = build_equiangular_grid(8, 16)
    cutoff = 3.0 * math.pi / 7
    frames = build_tangent_frames(g.nodes)
    edges = bipartite(g, g, cutoff, (frames, frames))
    torch.manual_seed(0)
    fin, fout = SO2FieldType({0: 3, 1: 2, 2: 1}), SO2FieldType({0: 2, 1: 3})
    enc = EquiEncode(fin, fout, cutoff=cutoff, window="quartic", n_radial_basis=4, dtype=D64)
    conv = SO2Convolution(fin, fout, cutoff=cutoff, window="quartic", n_radial_basis=4, dtype=D64)
    conv.kernel.load_state_dict(enc.integral.kernel.state_dict())
    x = {f: problems.normal((g.n_nodes, m) if f == 0 else (g.n_nodes, m, 2), 3 + f) for f, m in fin.items()}
    got = modules.encode_forward(enc.integral, x, edges)
    want = modules.conv_forward(conv, x, edges)
    for f in want:
        torch.testing.assert_close(got[f], want[f], rtol=1e-12, atol=1e-12)


def rotate(x, theta):
    return {f: t if f == 0 else torch.view_as_real(torch.view_as_complex(t.contiguous()) * torch.polar(
        torch.ones_like(theta), f * theta).unsqueeze(-1)) for f, t in x.items()}


def test_encode_oracle_is_gauge_equivariant():
    fine, coarse = build_equiangular_grid(12, 24), build_equiangular_grid(7, 14)
    cutoff = 1.5 * math.pi / 6
    ff, cf = build_tangent_frames(fine.nodes), build_tangent_frames(coarse.nodes)
    gen = torch.Generator().manual_seed(4)
    tf = torch.rand(fine.n_nodes, dtype=D64, generator=gen) * 2 * math.pi
    tc = torch.rand(coarse.n_nodes, dtype=D64, generator=gen) * 2 * math.pi
    base = bipartite(fine, coarse, cutoff, (ff, cf))
    turned = bipartite(fine, coarse, cutoff, (rotate_tangent_frames(ff, tf), rotate_tangent_frames(cf, tc)))
    torch.manual_seed(0)
    fin, fout = SO2FieldType({0: 2, 1: 2, 2: 2}), SO2FieldType({0: 3, 1: 2, 2: 2})
    enc = EquiEncode(fin, fout, cutoff=cutoff, n_radial_basis=4, dtype=D64)
    x = {f: problems.normal((fine.n_nodes, m) if f == 0 else (fine.n_nodes, m, 2), 9 + f) for f, m in fin.items()}
    y = modules.encode_forward(enc.integral, x, base)
    y_turned = modules.encode_forward(enc.integral, rotate(x, -tf), turned)
    want = rotate(y, -tc)
    for f in y:
        torch.testing.assert_close(y_turned[f], want[f], rtol=1e-9, atol=1e-9)
    assert max(float((y[f] - want[f]).detach().abs().max()) for f in (1, 2)) > 1e-3


@pytest.mark.parametrize("fin,fout", [({0: 8, 1: 8, 2: 8}, {0: 40, 1: 40, 2: 40}), ({0: 4}, {0: 64, 1: 64, 2: 64}),
                                      ({0: 64, 1: 64, 2: 64}, {0: 128, 1: 128, 2: 128})])
def test_wide_kernel_tiles_partition_the_output(fin, fout):
    kernel = SO2SteerableKernel(SO2FieldType(fin), SO2FieldType(fout), cutoff=0.3, n_radial_basis=4, dtype=D64)
    p = fused_factored.plan(kernel)
    tl = fused_factored.tiles(kernel)
    assert tl, "the kernel must tile"
    cols = [c for t in tl for c in t.out_cols]
    assert sorted(cols) == list(range(p.d_out))
    zc = sorted(c for t in tl for c in t.zc_cols)
    zr = sorted(set(c for t in tl for c in t.zr_cols))
    assert zc == list(range(p.wc)) and zr == list(range(p.wr))
    for t in tl:
        assert t.d_out <= fused_factored.MAX_OUT and t.max_bm <= fused_factored.MAX_BM
        assert 2 * len(t.zc_cols) + len(t.zr_cols) <= fused_factored.MAX_C
        assert t.d_out == len(t.out_cols)
        assert sum(r[0] == 0 for r in t.rows) <= 1
        for r in t.rows:  # every block of a piece writes the piece's whole output range
            width = r[2] * (1 if (r[0] == 0 or r[7]) else 2)
            assert r[6] + width <= t.d_out
    small = SO2SteerableKernel(SO2FieldType({0: 4, 1: 4}), SO2FieldType({0: 4, 1: 4}), cutoff=0.3, n_radial_basis=4)
    assert fused_factored.tiles(small) is None
