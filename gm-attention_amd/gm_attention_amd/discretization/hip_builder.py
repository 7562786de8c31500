"""Neighbourhoods, CSR and per-edge geometry built on the GPU.

Restates the reference's ``compute_edge_geometry`` (discretization/
edge_geometry.py:320-396) for a grid whose nodes live on a HIP device:

* membership ``atan2(|p x q|, <p, q>) <= r + EXACT_SLACK`` from the float64
  lattice (:381-387, :492-503), decided for every candidate pair by
  ``gm_radius_*`` (64-node bounding boxes in place of the KD-tree ball query
  of :465-474, which only ever narrows the candidates), rows target-major and
  source-minor (:701-704) and ``row_ptr`` the cumulative degree (:622-653):
  the same integers as the host builder;
* the per-edge tables of ``edge_geometry_from_index`` (:506-619) in one
  float64 pass (``gm_edge_tables_f64``), cast to the grid's dtype.

``compute_edge_geometry`` (edge_geometry.py) routes here when the grid's nodes
are on the GPU; ``GM_GPU_GEOMETRY=0`` keeps the host builder (KD-tree on the
CPU, torch arithmetic on the nodes' device).  The legacy cutoff rule decides
membership in the nodes' own dtype with a KD-tree radius that differs from the
exact rule's, so it has no GPU builder here.
"""

from __future__ import annotations

import os

import torch
from torch import Tensor

from gm_attention_amd import _native
from gm_attention_amd.representations.so2 import complex_dtype

#: ``GM_GPU_GEOMETRY=0`` keeps the host builder for grids on the GPU.
ENABLED = os.environ.get("GM_GPU_GEOMETRY", "1") != "0"


def applies(grid) -> bool:
    return ENABLED and grid.nodes.device.type == "cuda"


def _lattice(grid, device: torch.device) -> Tensor:
    from gm_attention_amd.discretization.edge_geometry import CUTOFF_RULE

    if CUTOFF_RULE == "legacy" or grid.exact_nodes is None:
        raise ValueError("the GPU geometry builder decides membership on the float64 lattice (the whole-shell rule); "
                         "set GM_GPU_GEOMETRY=0 to build under GM_CUTOFF_RULE=legacy")
    return grid.exact_nodes.to(device=device, dtype=torch.float64).contiguous()


def radius_edges(exact: Tensor, coverage_radius: float) -> tuple[Tensor, Tensor]:
    """``(edge_index (2, E), row_ptr)`` of the pairs within ``coverage_radius + EXACT_SLACK``."""
    from gm_attention_amd.discretization.edge_geometry import EXACT_SLACK

    return _native.radius_edges(exact, exact, float(coverage_radius) + EXACT_SLACK)


def compute_edge_geometry(grid, frames: Tensor, coverage_radius: float, *, max_frequency: int):
    """The EdgeGeometry of ``grid`` (nodes on a HIP device) at ``coverage_radius``."""
    from gm_attention_amd.discretization.edge_geometry import EdgeGeometry

    device, dtype = grid.nodes.device, grid.nodes.dtype
    edge_index, row_ptr = radius_edges(_lattice(grid, device), coverage_radius)
    nodes = grid.nodes.to(torch.float64).contiguous()
    frames64 = frames.to(device=device, dtype=torch.float64).contiguous()
    quadrature = grid.quadrature_weights.to(device=device, dtype=torch.float64).contiguous()
    t = _native.edge_tables(nodes, frames64, nodes, frames64, quadrature, edge_index, max_frequency)
    cdtype = complex_dtype(dtype)

    def real(x: Tensor) -> Tensor:
        return x if dtype == torch.float64 else x.to(dtype)

    def phases(x: Tensor) -> Tensor:
        return torch.view_as_complex(x).to(cdtype)

    return EdgeGeometry(edge_index, row_ptr, real(t["log_coordinates"]), real(t["distances"]), real(t["polar_angles"]),
                        real(t["transport_angles"]), real(t["tangent_quadrature_weights"]),
                        phases(t["angular_phases"]), phases(t["transport_phases"]))


def exact_distances(grid, edge_index: Tensor) -> Tensor:
    """Float64 lattice distances of the edges (the radius subsets' membership), on the edges' device."""
    exact = _lattice(grid, edge_index.device)
    return _native.geodesic_distances(exact, exact, edge_index)


def compute_bipartite_edge_geometry(source_nodes: Tensor, source_frames: Tensor, source_quadrature: Tensor,
                                    target_nodes: Tensor, target_frames: Tensor, *, cutoff: float,
                                    max_frequency: int, source_exact_nodes: Tensor,
                                    target_exact_nodes: Tensor):
    """The bipartite EdgeGeometry (target <- source, own numbering on each side)
    of edge_geometry.compute_bipartite_edge_geometry, from the two float64
    lattices on the targets' device."""
    from gm_attention_amd.discretization.edge_geometry import EXACT_SLACK, EdgeGeometry, _check_covered

    device, dtype = target_nodes.device, target_nodes.dtype
    src64 = source_exact_nodes.to(device=device, dtype=torch.float64).contiguous()
    tgt64 = target_exact_nodes.to(device=device, dtype=torch.float64).contiguous()
    edge_index, row_ptr = _native.radius_edges(tgt64, src64, float(cutoff) + EXACT_SLACK)
    _check_covered(edge_index, target_nodes.shape[0], cutoff)
    f64 = dict(device=device, dtype=torch.float64)
    t = _native.edge_tables(target_nodes.to(**f64).contiguous(), target_frames.to(**f64).contiguous(),
                            source_nodes.to(**f64).contiguous(), source_frames.to(**f64).contiguous(),
                            source_quadrature.to(**f64).contiguous(), edge_index, max_frequency)
    cdtype = complex_dtype(dtype)

    def real(x: Tensor) -> Tensor:
        return x if dtype == torch.float64 else x.to(dtype)

    return EdgeGeometry(edge_index, row_ptr, real(t["log_coordinates"]), real(t["distances"]), real(t["polar_angles"]),
                        real(t["transport_angles"]), real(t["tangent_quadrature_weights"]),
                        torch.view_as_complex(t["angular_phases"]).to(cdtype),
                        torch.view_as_complex(t["transport_phases"]).to(cdtype))
