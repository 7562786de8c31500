"""Synthetic op inputs on real equiangular geometry, shared by the tests.

The geometry comes from the package's host-side discretization (the same
tables the layers feed the ops); the fields are seeded N(0, 1).
"""

from __future__ import annotations

import functools
import math
import os
from dataclasses import dataclass

import torch
from torch import Tensor

from gm_attention_amd.discretization.discretization import SphericalDiscretization
from gm_attention_amd.discretization.grid import build_equiangular_grid
from gm_attention_amd.nn.fused_attention import evaluate_aggregation_window, plan_of
from gm_attention_amd.representations.field_type import SO2FieldType


@functools.cache
def discretization(nlat: int, nlon: int, rows: float = 3.0) -> SphericalDiscretization:
    grid = build_equiangular_grid(nlat, nlon)
    return SphericalDiscretization.from_grid(grid, rows * math.pi / (nlat - 1))


@dataclass
class Tables:
    transport: Tensor
    angular: Tensor
    rho: Tensor
    weights: Tensor
    bias: Tensor
    inside: Tensor
    row_ptr: Tensor
    source: Tensor
    n_nodes: int


def tables(nlat: int, nlon: int, batch: int = 1, window: str = "hard", dtype=torch.float64, rows: float = 3.0,
           max_order: int = 4) -> Tables:
    disc = discretization(nlat, nlon, rows)
    edges = disc.edge_geometry.tile(batch, n_sources=disc.n_nodes) if batch > 1 else disc.edge_geometry
    cutoff = disc.coverage_radius
    d = edges.distances.to(dtype)
    quad = edges.tangent_quadrature_weights.to(dtype)
    win = evaluate_aggregation_window(d, cutoff, window)
    tiny = torch.finfo(dtype).tiny
    return Tables(
        torch.view_as_real(edges.transport_phases[:, : max_order + 1].contiguous()).to(dtype).contiguous(),
        torch.view_as_real(edges.angular_phases[:, : max_order + 1].contiguous()).to(dtype).contiguous(),
        (d / cutoff).contiguous(), (win * quad).contiguous(),
        (torch.log(win.clamp_min(tiny)) + torch.log(quad.clamp_min(tiny))).contiguous(),
        (win > 0).to(torch.uint8).contiguous(), edges.row_ptr.contiguous(), edges.source_index.contiguous(),
        int(edges.row_ptr.shape[0] - 1),
    )


def attention_layout(field: dict[int, int], heads: int):
    full = SO2FieldType(field)
    per_head = SO2FieldType({n: m // heads for n, m in field.items()})
    p = plan_of(per_head, full, heads)
    return p, torch.tensor([list(r) for r in p.rows], dtype=torch.int64), 1.0 / math.sqrt(per_head.dimension)


def depthwise_layout(field: dict[int, int]):
    ft = SO2FieldType(field)
    p = plan_of(ft, ft, 1)
    return p, torch.tensor([list(r) for r in p.rows], dtype=torch.int64)


def normal(shape, seed: int, dtype=torch.float64) -> Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64).to(dtype)


def report_strict(got: Tensor, want: Tensor, name: str) -> None:
    """With GM_STRICT_REPORT naming a file, append the test's id, ``name`` and
    max |got - want| / (1e-5 |want| + 1e-6) -- the north star's elementwise
    bound with an unscaled absolute term -- to it (a measurement for the
    tests that hold a scaled absolute term; no assertion)."""
    path = os.environ.get("GM_STRICT_REPORT")
    if not path or want.numel() == 0:
        return
    ratio = float(((got.double().cpu() - want.double().cpu()).abs() / (1e-5 * want.double().cpu().abs() + 1e-6)).max())
    peak = float(want.abs().max())
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    with open(path, "a") as f:
        f.write(f"{test}\t{name}\t{ratio:.4f}\t{peak:.3e}\n")
