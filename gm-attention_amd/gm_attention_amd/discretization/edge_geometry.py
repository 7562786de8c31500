"""Directed edges ``i <- j`` within a geodesic radius, in CSR order, and their
geometry: log map in the target frame, Levi-Civita transport angle, tangent
quadrature weight, phase tables.

Restates ``discretization/edge_geometry.py`` of the reference:

* ``EdgeGeometry`` (:25-317): the per-edge tables, ``select``, ``tile``, ``to``;
* ``compute_edge_geometry`` (:320-396): a KD-tree ball query at the chord
  ``2 sin((r + EXACT_SLACK) / 2)`` (:465-474) over the float64 lattice, then
  membership ``d <= r + EXACT_SLACK`` from float64 geodesic distances
  ``atan2(|p x q|, <p, q>)`` (:381-387, :492-503), edges lexsorted target-major,
  source-minor (:701-704);
* ``edge_geometry_from_index`` (:506-619): ``log_p(q) = r/sin(r) (q - cos(r) p)``
  in the target frame, the transport ``R = I + K + K^2 / (1 + <q, p>)``
  (:718-771), ``gamma = atan2`` of ``E_i^T R E_j`` (:574-585), quadrature
  ``w_j r / sin r`` (:588-591), ``phi = atan2`` of the log coordinates;
* ``within_cutoff`` / ``cutoff_tolerance`` / ``GM_CUTOFF_RULE`` (:403-462);
* ``compute_bipartite_edge_geometry`` (:830-961) and its KD-tree search
  (:964-998): edges between two grids, each side in its own numbering.

A grid whose nodes are on the GPU is built by ``hip_builder`` (the same edge
list from the same float64 rule, tables in one HIP pass).

The per-edge arithmetic runs in slices of edges to bound host memory at
256x512 (elementwise per edge, so the values do not depend on the slicing).
"""

from __future__ import annotations

import math
import os
from dataclasses import dataclass

import numpy as np
import torch
from scipy.spatial import cKDTree
from torch import Tensor

from gm_attention_amd.representations.so2 import complex_dtype, phase_powers

DEFAULT_MAX_FREQUENCY = 4
EXACT_SLACK = 1e-10
CUTOFF_RULES = ("whole-shell", "legacy")
CUTOFF_RULE: str = os.environ.get("GM_CUTOFF_RULE", "whole-shell")
if CUTOFF_RULE not in CUTOFF_RULES:
    raise ValueError(f"GM_CUTOFF_RULE must be one of {CUTOFF_RULES}, got {CUTOFF_RULE!r}.")
_SLICE = 1 << 21  # edges per slice of the per-edge arithmetic


def cutoff_tolerance(dtype: torch.dtype) -> float:
    return 1e-10 if dtype == torch.float64 else 1e-5


def within_cutoff(distances: Tensor, cutoff: float) -> Tensor:
    if CUTOFF_RULE == "legacy":
        return distances <= float(cutoff)
    return distances <= float(cutoff) + cutoff_tolerance(distances.dtype)


def _query_chord_radius(cutoff: float, dtype: torch.dtype, *, exact: bool = False) -> float:
    if CUTOFF_RULE == "legacy":
        return 2.0 * math.sin(cutoff / 2.0) * (1.0 + 1e-12)
    slack = EXACT_SLACK if exact else cutoff_tolerance(dtype)
    return 2.0 * math.sin((cutoff + slack) / 2.0)


@dataclass(frozen=True)
class EdgeGeometry:
    edge_index: Tensor  # (2, n_edges): target, source
    row_ptr: Tensor  # (n_targets + 1,)
    log_coordinates: Tensor  # (n_edges, 2)
    distances: Tensor  # (n_edges,)
    polar_angles: Tensor  # (n_edges,)
    transport_angles: Tensor  # (n_edges,)
    tangent_quadrature_weights: Tensor  # (n_edges,)
    angular_phases: Tensor  # (n_edges, K + 1) complex
    transport_phases: Tensor  # (n_edges, K + 1) complex

    @property
    def n_edges(self) -> int:
        return int(self.edge_index.shape[1])

    @property
    def target_index(self) -> Tensor:
        return self.edge_index[0]

    @property
    def source_index(self) -> Tensor:
        return self.edge_index[1]

    @property
    def max_frequency(self) -> int:
        return int(self.angular_phases.shape[-1]) - 1

    def _harmonic(self, table: Tensor, order: int) -> Tensor:
        if abs(order) > self.max_frequency:
            raise ValueError(f"Harmonic order {order} is not tabulated (up to {self.max_frequency}).")
        column = table[:, abs(order)]
        return column.conj() if order < 0 else column

    def angular_harmonic(self, order: int) -> Tensor:
        return self._harmonic(self.angular_phases, order)

    def transport_harmonic(self, order: int) -> Tensor:
        return self._harmonic(self.transport_phases, order)

    def select(self, selection: Tensor, *, n_nodes: int | None = None) -> EdgeGeometry:
        edge_index = self.edge_index[:, selection].contiguous()
        n = self.row_ptr.shape[0] - 1 if n_nodes is None else n_nodes
        return EdgeGeometry(
            edge_index, build_row_ptr(edge_index[0], n), self.log_coordinates[selection].contiguous(),
            self.distances[selection].contiguous(), self.polar_angles[selection].contiguous(),
            self.transport_angles[selection].contiguous(), self.tangent_quadrature_weights[selection].contiguous(),
            self.angular_phases[selection].contiguous(), self.transport_phases[selection].contiguous(),
        )

    def tile(self, count: int, *, n_sources: int) -> EdgeGeometry:
        """The disjoint union of ``count`` copies (reference :216-252)."""
        if count == 1:
            return self
        n_targets = int(self.row_ptr.shape[0]) - 1
        offsets = torch.arange(count, device=self.edge_index.device, dtype=torch.long).unsqueeze(1)
        targets = (self.edge_index[0].unsqueeze(0) + offsets * n_targets).reshape(-1)
        sources = (self.edge_index[1].unsqueeze(0) + offsets * int(n_sources)).reshape(-1)
        row_ptr = torch.cat([self.row_ptr[:1], (self.row_ptr[1:].unsqueeze(0) + offsets * self.n_edges).reshape(-1)])

        def rep(t: Tensor) -> Tensor:
            return t.repeat(count, *([1] * (t.ndim - 1)))

        return EdgeGeometry(torch.stack([targets, sources]), row_ptr, rep(self.log_coordinates), rep(self.distances),
                            rep(self.polar_angles), rep(self.transport_angles), rep(self.tangent_quadrature_weights),
                            rep(self.angular_phases), rep(self.transport_phases))

    # ---- target-range chunks (the decomposition of forward_chunked)

    def host_row_ptr(self) -> np.ndarray:
        """``row_ptr`` on the host, read from the device once per edge set."""
        held = self.__dict__.get("_host_row_ptr")
        if held is None:
            held = self.row_ptr.detach().to("cpu").numpy()
            self.__dict__["_host_row_ptr"] = held
        return held

    def target_range(self, e0: int, e1: int) -> EdgeGeometry:
        """The edges ``[e0, e1)`` -- whole neighbourhoods of consecutive targets --
        as an edge set over the same nodes: every per-edge table a view of this
        one's, the rows of the other targets empty.  The result records
        ``(self, e0, e1)`` (:meth:`span`), so tables built for this edge set can
        be sliced for it instead of rebuilt."""
        part = slice(e0, e1)
        chunk = EdgeGeometry(self.edge_index[:, part], (self.row_ptr - e0).clamp(0, e1 - e0),
                             self.log_coordinates[part], self.distances[part], self.polar_angles[part],
                             self.transport_angles[part], self.tangent_quadrature_weights[part],
                             self.angular_phases[part], self.transport_phases[part])
        chunk.__dict__["_span"] = (self, int(e0), int(e1))
        return chunk

    def span(self) -> tuple[EdgeGeometry, int, int] | None:
        """``(parent, e0, e1)`` for an edge set made by :meth:`target_range`, else ``None``."""
        return self.__dict__.get("_span")

    def chunks(self, chunk_size: int):
        """Consecutive ranges of at most ``chunk_size`` targets with their whole
        neighbourhoods, as :meth:`target_range` edge sets; ranges without edges
        are skipped.  The bounds come from one host copy of ``row_ptr``."""
        if chunk_size < 1:
            raise ValueError(f"chunk_size must be at least 1, got {chunk_size}.")
        ptr = self.host_row_ptr()
        n = ptr.shape[0] - 1
        for first in range(0, n, chunk_size):
            e0, e1 = int(ptr[first]), int(ptr[min(n, first + chunk_size)])
            if e1 > e0:
                yield self.target_range(e0, e1)

    def to(self, device=None, dtype=None) -> EdgeGeometry:
        real = self.distances.dtype if dtype is None else dtype
        cplx = complex_dtype(real)
        return EdgeGeometry(
            self.edge_index.to(device), self.row_ptr.to(device), self.log_coordinates.to(device, real),
            self.distances.to(device, real), self.polar_angles.to(device, real), self.transport_angles.to(device, real),
            self.tangent_quadrature_weights.to(device, real), self.angular_phases.to(device, cplx),
            self.transport_phases.to(device, cplx),
        )


def build_row_ptr(target_index: Tensor, n_nodes: int) -> Tensor:
    """CSR offsets of target-sorted edges: bincount + cumsum (reference :622-653)."""
    if target_index.numel() > 1 and not bool(torch.all(target_index[1:] >= target_index[:-1])):
        raise ValueError("target_index must be sorted in non-decreasing order to build CSR row pointers.")
    counts = torch.bincount(target_index, minlength=n_nodes)
    row_ptr = torch.zeros(n_nodes + 1, dtype=torch.long, device=target_index.device)
    torch.cumsum(counts, dim=0, out=row_ptr[1:])
    return row_ptr


def geodesic_distances(nodes: Tensor, edge_index: Tensor) -> Tensor:
    """``atan2(|p x q|, <p, q>)`` per edge (reference :492-503)."""
    out = torch.empty(edge_index.shape[1], dtype=nodes.dtype, device=nodes.device)
    for lo in range(0, edge_index.shape[1], _SLICE):
        hi = min(lo + _SLICE, edge_index.shape[1])
        p, q = nodes[edge_index[0, lo:hi]], nodes[edge_index[1, lo:hi]]
        dot = torch.sum(p * q, dim=-1).clamp(min=-1.0, max=1.0)
        out[lo:hi] = torch.atan2(torch.linalg.vector_norm(torch.linalg.cross(p, q, dim=-1), dim=-1), dot)
    return out


def radius_edges(nodes: Tensor, coverage_radius: float, *, exact: bool = False, workers: int = -1) -> Tensor:
    """Candidate pairs from a KD-tree ball query (float64 CPU, ``workers``
    threads, -1 for every core), lexsorted target-major, source-minor
    (reference :656-715)."""
    cpu = nodes.detach().to("cpu", torch.float64).numpy()
    tree = cKDTree(cpu)
    lists = tree.query_ball_point(cpu, r=_query_chord_radius(coverage_radius, nodes.dtype, exact=exact),
                                  workers=workers)
    counts = np.fromiter((len(x) for x in lists), dtype=np.int64, count=len(lists))
    targets = np.repeat(np.arange(cpu.shape[0], dtype=np.int64), counts)
    sources = np.concatenate([np.asarray(x, dtype=np.int64) for x in lists]) if len(lists) else np.zeros(0, np.int64)
    order = np.lexsort((sources, targets))
    return torch.as_tensor(np.stack([targets[order], sources[order]]), dtype=torch.long)


def _transport_rotations(source_nodes: Tensor, target_nodes: Tensor, dot: Tensor) -> Tensor:
    """``R = I + K + K^2 / (1 + <q, p>)`` with K the cross-product matrix of q x p."""
    cross = torch.linalg.cross(source_nodes, target_nodes, dim=-1)
    n = source_nodes.shape[0]
    skew = torch.zeros(n, 3, 3, dtype=source_nodes.dtype, device=source_nodes.device)
    x, y, z = cross[:, 0], cross[:, 1], cross[:, 2]
    skew[:, 0, 1], skew[:, 0, 2] = -z, y
    skew[:, 1, 0], skew[:, 1, 2] = z, -x
    skew[:, 2, 0], skew[:, 2, 1] = -y, x
    identity = torch.eye(3, dtype=source_nodes.dtype, device=source_nodes.device).expand(n, -1, -1)
    return identity + skew + torch.bmm(skew, skew) / (1.0 + dot).reshape(-1, 1, 1)


def edge_geometry_from_index(nodes: Tensor, frames: Tensor, spherical_quadrature_weights: Tensor, edge_index: Tensor,
                             n_target_nodes: int, max_frequency: int) -> EdgeGeometry:
    n_edges = edge_index.shape[1]
    dtype, device = nodes.dtype, nodes.device
    log_coordinates = torch.empty(n_edges, 2, dtype=dtype, device=device)
    distances = torch.empty(n_edges, dtype=dtype, device=device)
    transport_angles = torch.empty(n_edges, dtype=dtype, device=device)
    quadrature = torch.empty(n_edges, dtype=dtype, device=device)
    for lo in range(0, n_edges, _SLICE):
        hi = min(lo + _SLICE, n_edges)
        t_idx, s_idx = edge_index[0, lo:hi], edge_index[1, lo:hi]
        p, q = nodes[t_idx], nodes[s_idx]
        dot = torch.sum(p * q, dim=-1).clamp(min=-1.0, max=1.0)
        d = torch.atan2(torch.linalg.vector_norm(torch.linalg.cross(p, q, dim=-1), dim=-1), dot)
        inv_density = torch.reciprocal(torch.sinc(d / math.pi))  # r / sin r, one at r = 0
        ambient = inv_density.unsqueeze(-1) * (q - dot.unsqueeze(-1) * p)
        ft, fs = frames[t_idx], frames[s_idx]
        log_coordinates[lo:hi] = torch.bmm(ft.transpose(1, 2), ambient.unsqueeze(-1)).squeeze(-1)
        rotation = _transport_rotations(q, p, dot)
        coordinate_transport = torch.bmm(ft.transpose(1, 2), torch.bmm(rotation, fs))
        transport_angles[lo:hi] = torch.atan2(coordinate_transport[:, 1, 0], coordinate_transport[:, 0, 0])
        quadrature[lo:hi] = spherical_quadrature_weights[s_idx] * inv_density
        distances[lo:hi] = d
    polar_angles = torch.atan2(log_coordinates[:, 1], log_coordinates[:, 0])
    return EdgeGeometry(
        edge_index.contiguous(), build_row_ptr(edge_index[0], n_target_nodes), log_coordinates.contiguous(),
        distances, polar_angles.contiguous(), transport_angles, quadrature,
        phase_powers(polar_angles, max_frequency).contiguous(), phase_powers(transport_angles, max_frequency).contiguous(),
    )


def compute_edge_geometry(grid, frames: Tensor, coverage_radius: float, *,
                          max_frequency: int = DEFAULT_MAX_FREQUENCY) -> EdgeGeometry:
    coverage_radius = float(coverage_radius)
    if not (0.0 < coverage_radius < math.pi):
        raise ValueError(f"coverage_radius must lie in (0, pi), got {coverage_radius}.")
    from gm_attention_amd.discretization import hip_builder

    if hip_builder.applies(grid):
        return hip_builder.compute_edge_geometry(grid, frames, coverage_radius, max_frequency=max_frequency)
    nodes = grid.nodes.contiguous()
    exact = None if CUTOFF_RULE == "legacy" else grid.exact_nodes
    edge_index = radius_edges(nodes if exact is None else exact, coverage_radius, exact=exact is not None)
    if exact is not None:
        keep = geodesic_distances(exact, edge_index) <= coverage_radius + EXACT_SLACK
    else:
        keep = geodesic_distances(nodes.detach().cpu(), edge_index) <= coverage_radius + cutoff_tolerance(nodes.dtype)
    edge_index = edge_index[:, keep].to(nodes.device)
    return edge_geometry_from_index(nodes, frames, grid.quadrature_weights.contiguous(), edge_index, nodes.shape[0],
                                    max_frequency)


def bipartite_radius_edges(source_nodes: Tensor, target_nodes: Tensor, cutoff: float, *, exact: bool = False,
                           workers: int = -1) -> Tensor:
    """Candidate ``target <- source`` pairs between two grids from a KD-tree over
    the sources (float64 CPU), lexsorted target-major, source-minor (reference
    :964-998)."""
    src = source_nodes.detach().to("cpu", torch.float64).numpy()
    tgt = target_nodes.detach().to("cpu", torch.float64).numpy()
    lists = cKDTree(src).query_ball_point(tgt, r=_query_chord_radius(cutoff, source_nodes.dtype, exact=exact),
                                          workers=workers)
    counts = np.fromiter((len(x) for x in lists), dtype=np.int64, count=len(lists))
    targets = np.repeat(np.arange(tgt.shape[0], dtype=np.int64), counts)
    sources = np.concatenate([np.asarray(x, dtype=np.int64) for x in lists]) if counts.sum() else np.zeros(0, np.int64)
    order = np.lexsort((sources, targets))
    return torch.as_tensor(np.stack([targets[order], sources[order]]), dtype=torch.long)


def _check_covered(edge_index: Tensor, n_target: int, cutoff: float) -> None:
    covered = torch.zeros(n_target, dtype=torch.bool, device=edge_index.device)
    covered[edge_index[0]] = True
    if not bool(covered.all()):
        missing = int((~covered).sum())
        raise ValueError(f"{missing} of {n_target} target nodes have no source within cutoff={cutoff}. Widen the "
                         "cutoff: an uncovered target aggregates to zero, which is indistinguishable from a genuine "
                         "zero downstream.")


def compute_bipartite_edge_geometry(source_nodes: Tensor, source_frames: Tensor,
                                    source_spherical_quadrature_weights: Tensor, target_nodes: Tensor,
                                    target_frames: Tensor, *, cutoff: float, max_frequency: int,
                                    source_exact_nodes: Tensor | None = None,
                                    target_exact_nodes: Tensor | None = None) -> EdgeGeometry:
    """Edges ``target i <- source j`` between two grids (reference :830-961):
    each side in its own numbering, ``row_ptr`` over the targets, quadrature
    from the sources, log coordinates and transport in the targets' frames.
    Membership from the float64 lattices with ``EXACT_SLACK`` when both are
    given (else from the working nodes with the dtype's slack); every target
    must have a source.  The tables are ``edge_geometry_from_index`` on the
    concatenation (targets first), the source indices rewritten back.  Nodes on
    the GPU take the GPU builder (same integers, tables in one HIP pass)."""
    if cutoff <= 0.0:
        raise ValueError(f"cutoff must be positive, got {cutoff}.")
    n_target = target_nodes.shape[0]
    exact = CUTOFF_RULE != "legacy" and source_exact_nodes is not None and target_exact_nodes is not None
    from gm_attention_amd.discretization import hip_builder

    if exact and hip_builder.ENABLED and target_nodes.device.type == "cuda":
        return hip_builder.compute_bipartite_edge_geometry(
            source_nodes, source_frames, source_spherical_quadrature_weights, target_nodes, target_frames,
            cutoff=cutoff, max_frequency=max_frequency, source_exact_nodes=source_exact_nodes,
            target_exact_nodes=target_exact_nodes)
    src_search, tgt_search = (source_exact_nodes, target_exact_nodes) if exact else (source_nodes, target_nodes)
    edge_index = bipartite_radius_edges(src_search, tgt_search, cutoff, exact=exact)
    if CUTOFF_RULE != "legacy":
        both = torch.cat([tgt_search.detach().cpu(), src_search.detach().cpu()], dim=0)
        shifted = torch.stack([edge_index[0], edge_index[1] + n_target])
        d = geodesic_distances(both.to(torch.float64) if exact else both, shifted)
        keep = d <= cutoff + EXACT_SLACK if exact else within_cutoff(d, cutoff)
        edge_index = edge_index[:, keep]
    edge_index = edge_index.to(source_nodes.device)
    _check_covered(edge_index, n_target, cutoff)
    nodes = torch.cat([target_nodes, source_nodes], dim=0)
    frames = torch.cat([target_frames, source_frames], dim=0)
    weights = torch.cat([source_spherical_quadrature_weights.new_zeros(n_target), source_spherical_quadrature_weights])
    combined = edge_geometry_from_index(nodes, frames, weights, torch.stack([edge_index[0], edge_index[1] + n_target]),
                                        n_target, max_frequency)
    return EdgeGeometry(torch.stack([combined.edge_index[0], combined.edge_index[1] - n_target]).contiguous(),
                        *(getattr(combined, f) for f in ("row_ptr", "log_coordinates", "distances", "polar_angles",
                                                        "transport_angles", "tangent_quadrature_weights",
                                                        "angular_phases", "transport_phases")))
