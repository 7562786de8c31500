"""Grid chains for hierarchical models: levels and the bipartite transfers between them.

Restates the reference's ``discretization/grids/equiangular.py:37-253``:
``TensorGridLevel`` (a grid, its frames and, when operators run on it, its
same-grid discretization), ``TensorGridHierarchy`` (levels finest first,
``down_edges[k]`` restricting level k onto k + 1, ``up_edges[k]``
interpolating level k + 1 onto level 0, optional ``lateral_edges[k]`` from
k + 2 onto k + 1; ``tile`` and ``to``) and ``build_grid_hierarchy``.  Every
transfer is a radius-based bipartite edge set
(``edge_geometry.compute_bipartite_edge_geometry``): on the GPU when the
grids' nodes are there, with the same integers as the host's KD-tree search.
"""

from __future__ import annotations

import itertools
from collections.abc import Sequence
from dataclasses import dataclass

from torch import Tensor

from gm_attention_amd.discretization.discretization import SphericalDiscretization
from gm_attention_amd.discretization.edge_geometry import (
    DEFAULT_MAX_FREQUENCY,
    EdgeGeometry,
    compute_bipartite_edge_geometry,
)
from gm_attention_amd.discretization.frames import build_tangent_frames
from gm_attention_amd.discretization.grid import SphericalGrid


@dataclass(frozen=True)
class TensorGridLevel:
    shape: tuple[int, ...]
    grid_kind: str
    grid: SphericalGrid
    frames: Tensor
    discretization: SphericalDiscretization | None

    @property
    def n_nodes(self) -> int:
        return self.grid.n_nodes

    def describe(self) -> str:
        if self.grid_kind == "icosphere":
            return f"icosphere L{self.shape[0]}"
        return f"{self.shape[0]}x{self.shape[1]} {self.grid_kind}"


@dataclass(frozen=True)
class TensorGridHierarchy:
    levels: tuple[TensorGridLevel, ...]
    down_edges: tuple[EdgeGeometry, ...]
    up_edges: tuple[EdgeGeometry, ...]
    lateral_edges: tuple[EdgeGeometry, ...] = ()

    @property
    def depth(self) -> int:
        return len(self.down_edges)

    @property
    def finest(self) -> TensorGridLevel:
        return self.levels[0]

    def tile(self, count: int) -> TensorGridHierarchy:
        """The hierarchy of ``count`` samples as one disjoint graph: node
        ``b * n + i`` of a level is node ``i`` of sample ``b``."""
        count = int(count)
        if count == 1:
            return self
        levels = tuple(
            TensorGridLevel(level.shape, level.grid_kind, level.grid.tile(count), level.frames.repeat(count, 1, 1),
                            None if level.discretization is None else level.discretization.tile(count))
            for level in self.levels)
        return TensorGridHierarchy(
            levels,
            tuple(e.tile(count, n_sources=self.levels[k].n_nodes) for k, e in enumerate(self.down_edges)),
            tuple(e.tile(count, n_sources=self.levels[k + 1].n_nodes) for k, e in enumerate(self.up_edges)),
            tuple(e.tile(count, n_sources=self.levels[k + 2].n_nodes) for k, e in enumerate(self.lateral_edges)))

    def to(self, device) -> TensorGridHierarchy:
        return TensorGridHierarchy(
            tuple(TensorGridLevel(level.shape, level.grid_kind, level.grid.to(device=device),
                                  level.frames.to(device=device),
                                  None if level.discretization is None else level.discretization.to(device=device))
                  for level in self.levels),
            tuple(e.to(device) for e in self.down_edges), tuple(e.to(device) for e in self.up_edges),
            tuple(e.to(device) for e in self.lateral_edges))


def _transfer(source: TensorGridLevel, target: TensorGridLevel, cutoff: float, max_frequency: int) -> EdgeGeometry:
    return compute_bipartite_edge_geometry(
        source.grid.nodes, source.frames, source.grid.quadrature_weights, target.grid.nodes, target.frames,
        cutoff=float(cutoff), max_frequency=max_frequency, source_exact_nodes=source.grid.exact_nodes,
        target_exact_nodes=target.grid.exact_nodes)


def build_grid_hierarchy(grids: Sequence[SphericalGrid], grid_kinds: Sequence[str], shapes: Sequence[tuple[int, ...]],
                         *, restrict_cutoffs: Sequence[float], interpolate_cutoffs: Sequence[float],
                         local_cutoffs: Sequence[Sequence[float] | None], frames: Sequence[Tensor | None] | None = None,
                         max_frequency: int = DEFAULT_MAX_FREQUENCY,
                         lateral_cutoffs: Sequence[float] | None = None) -> TensorGridHierarchy:
    """The hierarchy over prebuilt grids, finest first (reference equiangular.py:145-253)."""
    n_levels = len(grids)
    if n_levels < 2:
        raise ValueError(f"a hierarchy needs at least two levels, got {n_levels}.")
    if len(grid_kinds) != n_levels or len(local_cutoffs) != n_levels or len(shapes) != n_levels:
        raise ValueError("grid_kinds, shapes and local_cutoffs need one entry per level "
                         f"({n_levels}), got {len(grid_kinds)}, {len(shapes)} and {len(local_cutoffs)}.")
    n_hops = n_levels - 1
    if len(restrict_cutoffs) != n_hops or len(interpolate_cutoffs) != n_hops:
        raise ValueError(f"restrict_cutoffs and interpolate_cutoffs need one entry per hop ({n_hops}), got "
                         f"{len(restrict_cutoffs)} and {len(interpolate_cutoffs)}.")
    for fine, coarse in itertools.pairwise(grids):
        if coarse.n_nodes >= fine.n_nodes:
            raise ValueError(f"levels must be strictly coarser than their predecessor, got {fine.n_nodes} -> "
                             f"{coarse.n_nodes} nodes.")
    if frames is not None and len(frames) != n_levels:
        raise ValueError(f"frames needs one entry per level ({n_levels}), got {len(frames)}.")
    levels = []
    for index, (grid, kind, shape) in enumerate(zip(grids, grid_kinds, shapes, strict=True)):
        override = frames[index] if frames is not None else None
        level_frames = override if override is not None else build_tangent_frames(grid.nodes)
        radii = local_cutoffs[index]
        disc = None
        if radii is not None:
            if not radii:
                raise ValueError(f"local_cutoffs[{index}] is empty; pass None for no operator.")
            disc = SphericalDiscretization.from_grid(grid, max(radii), frames=level_frames,
                                                     max_frequency=max_frequency)
            disc.prepare_windows(radii)
        levels.append(TensorGridLevel(tuple(shape), kind, grid, level_frames, disc))
    down = tuple(_transfer(levels[h], levels[h + 1], restrict_cutoffs[h], max_frequency) for h in range(n_hops))
    up = tuple(_transfer(levels[h + 1], levels[0], interpolate_cutoffs[h], max_frequency) for h in range(n_hops))
    lateral: tuple[EdgeGeometry, ...] = ()
    if lateral_cutoffs is not None:
        if len(lateral_cutoffs) != n_hops - 1:
            raise ValueError(f"lateral_cutoffs needs one entry per hop after the first ({n_hops - 1}), got "
                             f"{len(lateral_cutoffs)}.")
        lateral = tuple(_transfer(levels[h + 2], levels[h + 1], c, max_frequency) for h, c in enumerate(lateral_cutoffs))
    return TensorGridHierarchy(tuple(levels), down, up, lateral)
