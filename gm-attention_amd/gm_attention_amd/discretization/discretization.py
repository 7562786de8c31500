"""A grid with frames and its coverage edges, serving radius subsets.

Restates ``discretization/discretization.py`` of the reference: ``from_grid``
(:119-168), ``edges_within`` (membership from the float64 lattice distances
with ``EXACT_SLACK``, cached per radius; :447-481), ``prepare_windows``
(:483-493), ``tile`` (the batch as a
disjoint union; :495-517) and ``to`` (:519-560).
"""

from __future__ import annotations

import math

import torch
from torch import Tensor

from gm_attention_amd.discretization import hip_builder
from gm_attention_amd.discretization.edge_geometry import (
    DEFAULT_MAX_FREQUENCY,
    EXACT_SLACK,
    CUTOFF_RULE,
    EdgeGeometry,
    compute_edge_geometry,
    geodesic_distances,
    within_cutoff,
)
from gm_attention_amd.discretization.frames import build_tangent_frames
from gm_attention_amd.discretization.grid import SphericalGrid


class SphericalDiscretization:
    def __init__(self, grid: SphericalGrid, frames: Tensor, edge_geometry: EdgeGeometry, coverage_radius: float,
                 exact_distances: Tensor | None = None) -> None:
        self.grid = grid
        self.frames = frames.contiguous()
        self.edge_geometry = edge_geometry
        self.coverage_radius = float(coverage_radius)
        self._exact_distances = None if exact_distances is None else exact_distances.detach().to("cpu", torch.float64)
        self._radius_cache: dict[float, EdgeGeometry] = {self._key(coverage_radius): edge_geometry}

    @staticmethod
    def _key(radius: float) -> float:
        return round(float(radius), 12)

    @classmethod
    def from_grid(cls, grid: SphericalGrid, coverage_radius: float, *, frames: Tensor | None = None,
                  max_frequency: int = DEFAULT_MAX_FREQUENCY) -> SphericalDiscretization:
        if frames is None:
            frames = build_tangent_frames(grid.nodes)
        edges = compute_edge_geometry(grid, frames, coverage_radius, max_frequency=max_frequency)
        exact = None if CUTOFF_RULE == "legacy" else grid.exact_nodes
        if exact is not None and hip_builder.applies(grid):
            distances = hip_builder.exact_distances(grid, edges.edge_index)
        else:
            distances = None if exact is None else geodesic_distances(exact, edges.edge_index.cpu())
        return cls(grid, frames, edges, coverage_radius, distances)

    @property
    def n_nodes(self) -> int:
        return self.grid.n_nodes

    @property
    def n_edges(self) -> int:
        return self.edge_geometry.n_edges

    def edges_within(self, radius: float) -> EdgeGeometry:
        radius = float(radius)
        if not (0.0 < radius < math.pi):
            raise ValueError(f"radius must lie in (0, pi), got {radius}.")
        if radius > self.coverage_radius + 1e-12:
            raise ValueError(f"Requested radius {radius:.12g} exceeds the discretization coverage radius "
                             f"{self.coverage_radius:.12g}.")
        key = self._key(radius)
        if key not in self._radius_cache:
            if self._exact_distances is not None:
                mask = (self._exact_distances <= radius + EXACT_SLACK).to(self.edge_geometry.distances.device)
            else:
                mask = within_cutoff(self.edge_geometry.distances, radius)
            self._radius_cache[key] = self.edge_geometry.select(mask)
        return self._radius_cache[key]

    def prepare_windows(self, support_radii) -> None:
        """Materialise the edge subset of every support radius (reference :483-493)."""
        for radius in support_radii:
            self.edges_within(radius)

    def tile(self, count: int) -> SphericalDiscretization:
        if count == 1:
            return self
        union = SphericalDiscretization(
            self.grid.tile(count), self.frames.repeat(count, 1, 1),
            self.edge_geometry.tile(count, n_sources=self.n_nodes), self.coverage_radius,
            None if self._exact_distances is None else self._exact_distances.repeat(count),
        )
        coverage = self._key(self.coverage_radius)
        for key, edges in self._radius_cache.items():
            if key != coverage:
                union._radius_cache[key] = edges.tile(count, n_sources=self.n_nodes)
        return union

    def to(self, device=None, dtype=None) -> SphericalDiscretization:
        moved = SphericalDiscretization(self.grid.to(device, dtype), self.frames.to(device=device, dtype=dtype),
                                        self.edge_geometry.to(device, dtype), self.coverage_radius,
                                        self._exact_distances)
        coverage = self._key(self.coverage_radius)
        for key, edges in self._radius_cache.items():
            if key != coverage:
                moved._radius_cache[key] = edges.to(device, dtype)
        return moved
