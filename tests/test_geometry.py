"""The host-side discretization that feeds every op (grid, CSR neighbourhoods,
per-edge geometry), pinned on the CPU:

* the CSR is bit-exact against an all-pairs float64 brute force
  (oracle.sphere.brute_force_edges: the membership rule of the reference's
  edge_geometry.py:381-387 decided with no tree, as its
  tests/discretization/test_neighborhoods.py:41-73 checks it), ordered
  target-major, source-minor, with row_ptr the cumulative degree;
* the Clenshaw-Curtis weights equal the moment solve (exact on every
  Chebyshev polynomial below n) and the sphere's weights integrate 1 and z^2
  exactly (the reference's tests/discretization/test_quadrature.py:89-145);
* the equiangular nodes equal their closed form;
* the per-edge geometry meets its closed forms: |log map| = geodesic
  distance, unit-modulus phases that are the powers of the order-1 phase,
  self-loops at distance 0 (to rounding) with no transport
  (tests/discretization/test_edge_geometry.py:56-515 in the reference)."""

import math

import numpy as np
import pytest
import torch

from gm_attention_amd.discretization.edge_geometry import build_row_ptr, compute_edge_geometry
from gm_attention_amd.discretization.frames import build_tangent_frames
from gm_attention_amd.discretization.grid import build_equiangular_grid, clenshaw_curtis
from oracle import sphere


def geometry(nlat, nlon, rows=3.0):
    grid = build_equiangular_grid(nlat, nlon)
    cutoff = rows * math.pi / (nlat - 1)
    return grid, cutoff, compute_edge_geometry(grid, build_tangent_frames(grid.nodes), cutoff)


@pytest.mark.parametrize("nlat,nlon,rows", [(8, 16, 3.0), (16, 32, 3.0), (32, 64, 3.0), (17, 20, 2.5)])
def test_csr_is_bit_exact_against_the_brute_force(nlat, nlon, rows):
    grid, cutoff, edges = geometry(nlat, nlon, rows)
    want = sphere.brute_force_edges(grid.exact_nodes.numpy(), cutoff)
    assert np.array_equal(edges.edge_index.numpy(), want)
    degrees = np.bincount(want[0], minlength=grid.n_nodes)
    assert np.array_equal(edges.row_ptr.numpy(), np.concatenate([[0], np.cumsum(degrees)]))
    assert torch.equal(build_row_ptr(edges.edge_index[0], grid.n_nodes), edges.row_ptr)
    # every node is its own neighbour, and neighbourhoods are symmetric
    pairs = set(map(tuple, want.T.tolist()))
    assert all((i, i) in pairs for i in range(grid.n_nodes))
    assert all((j, i) in pairs for i, j in pairs)


def test_the_32x64_edge_count_matches_the_survey_figure():
    _, _, edges = geometry(32, 64)
    assert edges.n_edges == 172_288


@pytest.mark.parametrize("n", [2, 3, 8, 17, 64, 257])
def test_clenshaw_curtis_weights_are_the_moment_solve(n):
    x, w = clenshaw_curtis(n)
    xo, wo = sphere.clenshaw_curtis_by_moments(n)
    np.testing.assert_allclose(x.numpy(), xo, rtol=0, atol=1e-14)
    np.testing.assert_allclose(w.numpy(), wo, rtol=0, atol=1e-13)


@pytest.mark.parametrize("nlat,nlon", [(8, 16), (33, 64), (128, 256)])
def test_sphere_weights_integrate_constants_and_z_squared(nlat, nlon):
    grid = build_equiangular_grid(nlat, nlon)
    w = grid.quadrature_weights
    z = grid.nodes[:, 2]
    assert float(w.sum()) == pytest.approx(4 * math.pi, rel=1e-13)
    assert float((w * z * z).sum()) == pytest.approx(4 * math.pi / 3, rel=1e-13)
    assert abs(float((w * z).sum())) < 1e-13


def test_equiangular_nodes_match_the_closed_form():
    grid = build_equiangular_grid(33, 64)
    np.testing.assert_allclose(grid.exact_nodes.numpy(), sphere.equiangular_nodes(33, 64), rtol=0, atol=1e-15)


def test_edge_geometry_closed_forms():
    grid, cutoff, edges = geometry(16, 32)
    d = edges.distances
    np.testing.assert_allclose(edges.log_coordinates.norm(dim=1).numpy(), d.numpy(), rtol=1e-12, atol=1e-14)
    t, s = edges.edge_index
    want = sphere.geodesic(grid.exact_nodes[t].numpy(), grid.exact_nodes[s].numpy())
    np.testing.assert_allclose(d.numpy(), want, rtol=0, atol=1e-13)
    for table, angle in ((edges.angular_phases, edges.polar_angles), (edges.transport_phases, edges.transport_angles)):
        np.testing.assert_allclose(table.abs().numpy(), 1.0, rtol=0, atol=1e-14)
        first = torch.polar(torch.ones_like(angle), angle)
        for k in range(table.shape[1]):
            np.testing.assert_allclose(table[:, k].numpy(), (first ** k).numpy(), rtol=0, atol=1e-13)
    loops = t == s
    assert int(loops.sum()) == grid.n_nodes
    assert float(d[loops].abs().max()) < 1e-15
    assert float(edges.log_coordinates[loops].abs().max()) < 1e-15
    assert float(edges.transport_angles[loops].abs().max()) < 1e-15


def test_gpu_builder_routing_and_errors_on_the_host():
    """Grids on the CPU keep the host builder; the GPU builder refuses the legacy
    rule and host tensors with a message instead of computing anything."""
    from gm_attention_amd import _native
    from gm_attention_amd.discretization import hip_builder

    grid = build_equiangular_grid(4, 6)
    assert not hip_builder.applies(grid)
    nodes = grid.exact_nodes
    with pytest.raises(RuntimeError, match="GPU only"):
        _native.radius_edges(nodes, nodes, 0.5)

    class NoLattice:
        exact_nodes = None

    with pytest.raises(ValueError, match="float64 lattice"):
        hip_builder._lattice(NoLattice(), torch.device("cpu"))


def test_target_chunks_partition_the_edges_into_whole_neighbourhoods():
    """EdgeGeometry.chunks: consecutive target ranges, every edge in exactly
    one chunk, each chunk's CSR the parent's rows for its targets (empty
    elsewhere), its tables views of the parent's, and its span recorded."""
    import torch

    import problems

    edges = problems.discretization(10, 20).edge_geometry
    ptr = edges.row_ptr
    seen = 0
    for chunk in edges.chunks(7):
        parent, e0, e1 = chunk.span()
        assert parent is edges and e0 == seen and e1 > e0
        assert torch.equal(chunk.edge_index, edges.edge_index[:, e0:e1])
        assert chunk.distances.data_ptr() == edges.distances[e0:].data_ptr()  # a view, not a copy
        assert torch.equal(chunk.row_ptr, (ptr - e0).clamp(0, e1 - e0))
        targets = chunk.target_index.unique()
        assert int(targets.max() - targets.min()) < 7
        # whole neighbourhoods: each target's edges all here
        assert int(chunk.row_ptr[-1]) == e1 - e0
        for t in targets.tolist():
            assert int(ptr[t + 1] - ptr[t]) == int(chunk.row_ptr[t + 1] - chunk.row_ptr[t])
        seen = e1
    assert seen == edges.n_edges
    with pytest.raises(ValueError, match="chunk_size must be at least 1"):
        next(edges.chunks(0))


def test_grid_hierarchy_reports_every_problem_with_its_arguments():
    from gm_attention_amd.discretization.grid import build_equiangular_grid
    from gm_attention_amd.discretization.hierarchy import build_grid_hierarchy

    grids = [build_equiangular_grid(9, 18), build_equiangular_grid(9, 18)]
    with pytest.raises(ValueError) as info:
        build_grid_hierarchy(grids, ["equiangular"], [(9, 18), (9, 18)], restrict_cutoffs=[0.5, 0.5],
                             interpolate_cutoffs=[0.5], local_cutoffs=[None, []])
    message = str(info.value)
    assert "grid_kinds has 1 entries for 2 levels" in message
    assert "restrict_cutoffs has 2 entries for 1 hops" in message
    assert "is not coarser than level 0" in message
    assert "local_cutoffs[1] is an empty list" in message
    with pytest.raises(ValueError, match="at least two levels"):
        build_grid_hierarchy(grids[:1], ["equiangular"], [(9, 18)], restrict_cutoffs=[], interpolate_cutoffs=[],
                             local_cutoffs=[None])
