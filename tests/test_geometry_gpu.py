"""The GPU neighbourhood / CSR / edge-geometry builder (discretization.hip_builder,
gm_radius_* and gm_edge_tables_f64):

* the edge list and row_ptr are bit-exact against the all-pairs float64 brute
  force (oracle.sphere.brute_force_edges, the reference's membership rule of
  edge_geometry.py:381-387 with no tree, as its
  tests/discretization/test_neighborhoods.py:41-73 checks it), including
  radii that keep only coincident nodes and radii near pi, grids whose size is
  no multiple of the 64-node boxes, and a bipartite (coarse targets, fine
  sources) neighbourhood;
* at 64x128 .. 256x512 it equals the host builder (KD-tree candidates plus the
  exact filter, itself pinned against the brute force in test_geometry.py);
* the per-edge tables agree with the host's float64 arithmetic to 1e-11 and
  meet their closed forms: |log map| = distance, unit phases that are powers of
  the order-1 phase, w_j d / sin d quadrature, equal distances and inverse
  transports on reverse edges, no transport on self-loops;
* SphericalDiscretization on the GPU serves the same radius subsets as on the CPU.
"""

import math
import time

import numpy as np
import pytest
import torch

from gm_attention_amd import _native
from gm_attention_amd.discretization import edge_geometry as eg
from gm_attention_amd.discretization import hip_builder
from gm_attention_amd.discretization.discretization import SphericalDiscretization
from gm_attention_amd.discretization.frames import build_tangent_frames
from gm_attention_amd.discretization.grid import build_equiangular_grid
from oracle import sphere

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def gpu_builder_on(monkeypatch):
    """These tests check the GPU builder itself, whatever GM_GPU_GEOMETRY says."""
    monkeypatch.setattr(hip_builder, "ENABLED", True)


def gpu_edges(nlat, nlon, radius, cuda):
    grid = build_equiangular_grid(nlat, nlon, device=cuda)
    assert hip_builder.applies(grid)
    return grid, eg.compute_edge_geometry(grid, build_tangent_frames(grid.nodes), radius)


def host_edges(nlat, nlon, radius):
    grid = build_equiangular_grid(nlat, nlon)
    return grid, eg.compute_edge_geometry(grid, build_tangent_frames(grid.nodes), radius)


BRUTE = [(8, 16, 3.0 * math.pi / 7), (16, 32, 3.0 * math.pi / 15), (32, 64, 3.0 * math.pi / 31),
         (17, 20, 2.5 * math.pi / 16), (9, 7, 1.0), (6, 10, 2.95), (12, 24, 1e-6), (3, 5, 0.5)]


@pytest.mark.parametrize("nlat,nlon,radius", BRUTE)
def test_csr_is_bit_exact_against_the_brute_force(nlat, nlon, radius, cuda):
    print(f"csr {nlat}x{nlon} r={radius}", flush=True)
    grid, edges = gpu_edges(nlat, nlon, radius, cuda)
    want = sphere.brute_force_edges(grid.exact_nodes.numpy(), radius)
    assert np.array_equal(edges.edge_index.cpu().numpy(), want)
    degrees = np.bincount(want[0], minlength=grid.n_nodes)
    assert np.array_equal(edges.row_ptr.cpu().numpy(), np.concatenate([[0], np.cumsum(degrees)]))
    assert edges.edge_index.device.type == "cuda" and edges.edge_index.dtype == torch.int64


@pytest.mark.parametrize("nlat,nlon", [(64, 128), (128, 256)])
def test_equals_the_host_builder(nlat, nlon, cuda):
    radius = 3.0 * math.pi / (nlat - 1)
    print(f"host vs gpu {nlat}x{nlon}", flush=True)
    _, got = gpu_edges(nlat, nlon, radius, cuda)
    _, want = host_edges(nlat, nlon, radius)
    assert torch.equal(got.edge_index.cpu(), want.edge_index)
    assert torch.equal(got.row_ptr.cpu(), want.row_ptr)
    far = want.distances > 1e-9  # the polar angle of coincident nodes is rounding noise on either side
    for name in ("log_coordinates", "distances", "tangent_quadrature_weights"):
        torch.testing.assert_close(getattr(got, name).cpu(), getattr(want, name), rtol=0, atol=1e-11, msg=name)
    for name in ("angular_phases", "transport_phases"):
        g, w = getattr(got, name).cpu(), getattr(want, name)
        rows = far if name == "angular_phases" else torch.ones_like(far)
        torch.testing.assert_close(g[rows], w[rows], rtol=0, atol=1e-11, msg=name)
    wrapped = torch.remainder(got.transport_angles.cpu() - want.transport_angles + math.pi, 2 * math.pi) - math.pi
    assert float(wrapped.abs().max()) < 1e-11


def test_256x512_edge_list_equals_the_host_builder(cuda):
    """The north-star grid (15.7 M edges per sample): the same integers as the host's
    KD-tree candidates filtered by the exact rule."""
    nlat, nlon = 256, 512
    radius = 3.0 * math.pi / (nlat - 1)
    grid = build_equiangular_grid(nlat, nlon, device=cuda)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    edge_index, row_ptr = hip_builder.radius_edges(hip_builder._lattice(grid, cuda), radius)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    exact = grid.exact_nodes
    candidates = eg.radius_edges(exact, radius, exact=True)
    want = candidates[:, eg.geodesic_distances(exact, candidates) <= radius + eg.EXACT_SLACK]
    t2 = time.perf_counter()
    print(f"256x512: {want.shape[1]} edges; gpu {1e3 * (t1 - t0):.1f} ms, host {1e3 * (t2 - t1):.0f} ms", flush=True)
    assert want.shape[1] == 15_740_928
    assert torch.equal(edge_index.cpu(), want)
    assert torch.equal(row_ptr.cpu(), eg.build_row_ptr(want[0], grid.n_nodes))


def test_bipartite_neighbourhood_is_bit_exact(cuda):
    """Coarse targets, fine sources (the shape of a grid-hierarchy hop)."""
    coarse = build_equiangular_grid(9, 18).exact_nodes
    fine = build_equiangular_grid(17, 36).exact_nodes
    radius = 2.0 * math.pi / 8
    edge_index, row_ptr = _native.radius_edges(coarse.to(cuda), fine.to(cuda), radius + eg.EXACT_SLACK)
    want = sphere.brute_force_edges(coarse.numpy(), radius, sources=fine.numpy())
    assert np.array_equal(edge_index.cpu().numpy(), want)
    assert np.array_equal(row_ptr.cpu().numpy(),
                          np.concatenate([[0], np.cumsum(np.bincount(want[0], minlength=coarse.shape[0]))]))
    # the reverse hop: fine targets, coarse sources
    edge_index, _ = _native.radius_edges(fine.to(cuda), coarse.to(cuda), radius + eg.EXACT_SLACK)
    assert np.array_equal(edge_index.cpu().numpy(), sphere.brute_force_edges(fine.numpy(), radius,
                                                                             sources=coarse.numpy()))


def test_tables_meet_their_closed_forms(cuda):
    nlat, nlon = 24, 48
    radius = 3.0 * math.pi / (nlat - 1)
    grid, e = gpu_edges(nlat, nlon, radius, cuda)
    t, s = e.edge_index
    d = e.distances
    assert e.distances.dtype == torch.float64 and e.angular_phases.dtype == torch.complex128
    torch.testing.assert_close(torch.linalg.vector_norm(e.log_coordinates, dim=1), d, rtol=0, atol=1e-13)
    far = d > 1e-9
    for table in (e.angular_phases, e.transport_phases):
        torch.testing.assert_close(table.abs(), torch.ones_like(table.abs()), rtol=0, atol=1e-14)
        powers = table[:, 1:2] ** torch.arange(table.shape[1], device=cuda)
        torch.testing.assert_close(table, powers, rtol=0, atol=1e-12)
    polar = torch.atan2(e.log_coordinates[:, 1], e.log_coordinates[:, 0])
    torch.testing.assert_close(e.polar_angles[far], polar[far], rtol=0, atol=1e-15)
    inv = torch.where(d > 0, d / torch.sin(d), torch.ones_like(d))
    torch.testing.assert_close(e.tangent_quadrature_weights, grid.quadrature_weights[s] * inv, rtol=1e-14, atol=0)
    # reverse edges: the same distance (bit for bit) and the inverse transport
    n = grid.n_nodes
    key = t * n + s
    rkey = s * n + t
    order = torch.argsort(key)
    rev = order[torch.searchsorted(key[order], rkey)]
    assert torch.equal(key[rev], rkey)
    assert torch.equal(d[rev], d)
    torch.testing.assert_close(e.transport_phases[rev, 1], e.transport_phases[:, 1].conj(), rtol=0, atol=1e-12)
    # self-loops: no transport; coincident nodes (self-loops, the poles' repeated
    # points, whose frames may differ): a vanishing log map
    loops = t == s
    assert int(loops.sum()) == n
    assert float(e.transport_angles[loops].abs().max()) < 1e-15
    assert float(e.log_coordinates[~far].abs().max()) < 1e-15


def test_float32_grid_casts_the_float64_tables(cuda):
    nlat, nlon = 16, 32
    radius = 3.0 * math.pi / 15
    grid = build_equiangular_grid(nlat, nlon, dtype=torch.float32, device=cuda)
    e32 = eg.compute_edge_geometry(grid, build_tangent_frames(grid.nodes), radius)
    _, e64 = gpu_edges(nlat, nlon, radius, cuda)
    assert torch.equal(e32.edge_index, e64.edge_index)
    assert e32.distances.dtype == torch.float32 and e32.angular_phases.dtype == torch.complex64
    torch.testing.assert_close(e32.distances, e64.distances.float(), rtol=1e-6, atol=1e-7)


def test_discretization_radius_subsets_match_the_host(cuda):
    nlat, nlon = 32, 64
    radius = 3.0 * math.pi / (nlat - 1)
    host = SphericalDiscretization.from_grid(build_equiangular_grid(nlat, nlon), radius)
    dev = SphericalDiscretization.from_grid(build_equiangular_grid(nlat, nlon, device=cuda), radius)
    assert dev.edge_geometry.edge_index.device.type == "cuda"
    for r in (radius, 2.0 * math.pi / (nlat - 1), 1.0 * math.pi / (nlat - 1), 0.5 * math.pi / (nlat - 1)):
        a, b = host.edges_within(r), dev.edges_within(r)
        assert torch.equal(a.edge_index, b.edge_index.cpu()), r
        assert torch.equal(a.row_ptr, b.row_ptr.cpu()), r


def test_out_of_range_indices_yield_nan_rows(cuda):
    nodes = build_equiangular_grid(5, 8).exact_nodes.to(cuda)
    frames = build_tangent_frames(nodes)
    quad = torch.ones(nodes.shape[0], dtype=torch.float64, device=cuda)
    edge_index = torch.tensor([[0, 1, 40, -1], [1, 0, 2, 3]], dtype=torch.int64, device=cuda)
    t = _native.edge_tables(nodes, frames, nodes, frames, quad, edge_index, 4)
    bad = torch.tensor([False, False, True, True], device=cuda)
    for name, x in t.items():
        rows = x.reshape(4, -1)
        assert bool(torch.isnan(rows[bad]).all()), name
        assert bool(torch.isfinite(rows[~bad]).all()), name
    d = _native.geodesic_distances(nodes, nodes, edge_index)
    assert bool(torch.isnan(d[bad]).all()) and bool(torch.isfinite(d[~bad]).all())


def test_nodes_off_the_unit_sphere_are_refused(cuda):
    nodes = build_equiangular_grid(5, 8).exact_nodes.to(cuda)
    with pytest.raises(RuntimeError, match="unit vectors"):
        _native.radius_edges(nodes * (1 + 1e-9), nodes, 0.5)
