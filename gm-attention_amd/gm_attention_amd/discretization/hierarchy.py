"""Grid chains for hierarchical models: levels and the bipartite transfers between them.

Stands for the reference's ``discretization/grids/equiangular.py:37-253``
(``TensorGridLevel``, ``TensorGridHierarchy`` with ``tile`` / ``to``,
``build_grid_hierarchy``): the same classes, fields and builder signature, so
the encoder blocks and a model's step function use them unchanged.  Levels
are finest first; ``down_edges[k]`` restricts level k onto level k + 1,
``up_edges[k]`` interpolates level k + 1 back onto level 0 and the optional
``lateral_edges[k]`` interpolates level k + 2 onto level k + 1.

Here every transfer is described as a hop ``(source level, target level,
cutoff)`` and built by one radius search
(``edge_geometry.compute_bipartite_edge_geometry``: on the GPU when the grids'
nodes are there, with the host KD-tree search's integers); ``tile`` and ``to``
map one structural transform over every level and every transfer.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
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
    """One grid of the chain: its shape label, kind, nodes, tangent frames and,
    when operators run on it, its same-grid discretization (else ``None``)."""

    shape: tuple[int, ...]
    grid_kind: str
    grid: SphericalGrid
    frames: Tensor
    discretization: SphericalDiscretization | None

    @property
    def n_nodes(self) -> int:
        return self.grid.n_nodes

    def describe(self) -> str:
        """A label for logs: ``L<k> icosphere`` levels by subdivision, tensor grids by ``nlat x nlon``."""
        label = "x".join(str(s) for s in self.shape)
        return f"icosphere L{label}" if self.grid_kind == "icosphere" else f"{label} {self.grid_kind}"

    def _mapped(self, grid: Callable, frames: Callable, disc: Callable) -> TensorGridLevel:
        return TensorGridLevel(self.shape, self.grid_kind, grid(self.grid), frames(self.frames),
                               None if self.discretization is None else disc(self.discretization))


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

    def _sources(self) -> dict[str, list[int]]:
        """The source level of every transfer, per transfer family."""
        return {"down": list(range(self.depth)), "up": [k + 1 for k in range(self.depth)],
                "lateral": [k + 2 for k in range(len(self.lateral_edges))]}

    def _mapped(self, level_fn: Callable[[TensorGridLevel], TensorGridLevel],
                edge_fn: Callable[[EdgeGeometry, int], EdgeGeometry]) -> TensorGridHierarchy:
        src = self._sources()
        return TensorGridHierarchy(
            tuple(level_fn(level) for level in self.levels),
            tuple(edge_fn(e, s) for e, s in zip(self.down_edges, src["down"], strict=True)),
            tuple(edge_fn(e, s) for e, s in zip(self.up_edges, src["up"], strict=True)),
            tuple(edge_fn(e, s) for e, s in zip(self.lateral_edges, src["lateral"], strict=True)))

    def tile(self, count: int) -> TensorGridHierarchy:
        """``count`` samples as one disjoint graph: node ``b * n + i`` of a
        level is node ``i`` of sample ``b``, every transfer within its sample;
        ``count == 1`` is the hierarchy itself."""
        count = int(count)
        if count == 1:
            return self
        return self._mapped(
            lambda level: level._mapped(lambda g: g.tile(count), lambda f: f.repeat(count, 1, 1),
                                        lambda d: d.tile(count)),
            lambda e, source: e.tile(count, n_sources=self.levels[source].n_nodes))

    def to(self, device=None, dtype=None) -> TensorGridHierarchy:
        """Every level and transfer on ``device``, the real tables in ``dtype``
        (unchanged when None); neighbourhood membership stays the float64
        construction's."""
        return self._mapped(
            lambda level: level._mapped(lambda g: g.to(device, dtype), lambda f: f.to(device=device, dtype=dtype),
                                        lambda d: d.to(device, dtype)),
            lambda e, _source: e.to(device, dtype))


def _hop(levels: Sequence[TensorGridLevel], source: int, target: int, cutoff: float,
         max_frequency: int) -> EdgeGeometry:
    """Edges from every node of level ``source`` within ``cutoff`` of a node of level ``target``."""
    s, t = levels[source], levels[target]
    return compute_bipartite_edge_geometry(
        s.grid.nodes, s.frames, s.grid.quadrature_weights, t.grid.nodes, t.frames, cutoff=float(cutoff),
        max_frequency=max_frequency, source_exact_nodes=s.grid.exact_nodes, target_exact_nodes=t.grid.exact_nodes)


def _problems(grids, grid_kinds, shapes, restrict_cutoffs, interpolate_cutoffs, local_cutoffs, frames,
              lateral_cutoffs) -> list[str]:
    """Everything wrong with a hierarchy's arguments (empty when it can be built)."""
    n = len(grids)
    if n < 2:
        return [f"a hierarchy has at least two levels ({n} grids given)"]
    found = []
    per_level = {"grid_kinds": grid_kinds, "shapes": shapes, "local_cutoffs": local_cutoffs}
    if frames is not None:
        per_level["frames"] = frames
    found += [f"{name} has {len(seq)} entries for {n} levels" for name, seq in per_level.items() if len(seq) != n]
    per_hop = {"restrict_cutoffs": restrict_cutoffs, "interpolate_cutoffs": interpolate_cutoffs}
    found += [f"{name} has {len(seq)} entries for {n - 1} hops" for name, seq in per_hop.items() if len(seq) != n - 1]
    if lateral_cutoffs is not None and len(lateral_cutoffs) != n - 2:
        found.append(f"lateral_cutoffs has {len(lateral_cutoffs)} entries for the {n - 2} hops after the first")
    found += [f"level {k + 1} ({grids[k + 1].n_nodes} nodes) is not coarser than level {k} ({grids[k].n_nodes})"
              for k in range(n - 1) if grids[k + 1].n_nodes >= grids[k].n_nodes]
    found += [f"local_cutoffs[{k}] is an empty list (None means no operator on that level)"
              for k, radii in enumerate(local_cutoffs) if radii is not None and len(radii) == 0]
    return found


def build_grid_hierarchy(grids: Sequence[SphericalGrid], grid_kinds: Sequence[str], shapes: Sequence[tuple[int, ...]],
                         *, restrict_cutoffs: Sequence[float], interpolate_cutoffs: Sequence[float],
                         local_cutoffs: Sequence[Sequence[float] | None], frames: Sequence[Tensor | None] | None = None,
                         max_frequency: int = DEFAULT_MAX_FREQUENCY,
                         lateral_cutoffs: Sequence[float] | None = None) -> TensorGridHierarchy:
    """The hierarchy over prebuilt grids, finest first (reference equiangular.py:145-253): each level's
    frames (given or built), its discretization prepared for its local radii when it has any, and the
    restriction, interpolation and (optional) lateral transfers."""
    problems = _problems(grids, grid_kinds, shapes, restrict_cutoffs, interpolate_cutoffs, local_cutoffs, frames,
                         lateral_cutoffs)
    if problems:
        raise ValueError("cannot build the grid hierarchy: " + "; ".join(problems) + ".")
    levels = []
    for k, grid in enumerate(grids):
        given = frames[k] if frames is not None else None
        level_frames = build_tangent_frames(grid.nodes) if given is None else given
        radii = local_cutoffs[k]
        disc = None
        if radii is not None:
            disc = SphericalDiscretization.from_grid(grid, max(radii), frames=level_frames, max_frequency=max_frequency)
            disc.prepare_windows(radii)
        levels.append(TensorGridLevel(tuple(shapes[k]), grid_kinds[k], grid, level_frames, disc))
    hops = len(grids) - 1
    down = tuple(_hop(levels, k, k + 1, restrict_cutoffs[k], max_frequency) for k in range(hops))
    up = tuple(_hop(levels, k + 1, 0, interpolate_cutoffs[k], max_frequency) for k in range(hops))
    lateral = tuple(_hop(levels, k + 2, k + 1, c, max_frequency) for k, c in enumerate(lateral_cutoffs or ()))
    return TensorGridHierarchy(tuple(levels), down, up, lateral)
