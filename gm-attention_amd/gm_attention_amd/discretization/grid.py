"""Quadrature grids on the unit sphere and the equiangular (Clenshaw-Curtis)
tensor-product grid.

``SphericalGrid`` restates ``discretization/grid.py:10-269`` (nodes,
quadrature weights, the float64 ``exact_nodes`` lattice membership is decided
from, ``tile``, ``to``).  ``build_equiangular_grid`` restates
``grids/torch_harmonics.py:41-145`` for ``grid="equiangular"``: the
colatitude rule comes from torch-harmonics 0.8.0 (``clenshaw_curtiss_weights``,
absent here), so :func:`clenshaw_curtis` computes the same nodes and weights
from the classical closed form (Waldvogel, BIT 46 (2006) 195-202;
Trefethen, SIAM Rev. 50 (2008) 67-87):

    x_k = cos(theta_k), theta_k = k pi / N, N = n - 1,
    w_k = (c_k / N) [1 - sum_{j=1}^{floor(N/2)} b_j cos(2 j theta_k) / (4 j^2 - 1)],
    c_0 = c_N = 1, c_k = 2 otherwise; b_{N/2} = 1, b_j = 2 otherwise.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor


def clenshaw_curtis(n: int) -> tuple[Tensor, Tensor]:
    """Clenshaw-Curtis nodes (ascending ``cos theta`` on [-1, 1]) and weights, float64."""
    if n < 2:
        raise ValueError(f"The 'equiangular' rule requires n_latitude >= 2, got {n}.")
    nodes = torch.cos(torch.linspace(math.pi, 0.0, n, dtype=torch.float64))
    N = n - 1
    theta = torch.arange(n, dtype=torch.float64) * (math.pi / N)
    total = torch.ones(n, dtype=torch.float64)
    for j in range(1, N // 2 + 1):
        b = 1.0 if 2 * j == N else 2.0
        total = total - (b / (4.0 * j * j - 1.0)) * torch.cos(2.0 * j * theta)
    c = torch.full((n,), 2.0, dtype=torch.float64)
    c[0] = 1.0
    c[-1] = 1.0
    weights = c * total / N
    # theta_k runs from 0 (x = 1) while the nodes ascend from x = -1; the rule is symmetric.
    return nodes, torch.flip(weights, dims=(0,))


class SphericalGrid:
    """Nodes ``(n, 3)``, quadrature weights ``(n,)``, and the float64 lattice."""

    __slots__ = ("exact_nodes", "nodes", "quadrature_weights")

    def __init__(self, nodes: Tensor, quadrature_weights: Tensor, exact_nodes: Tensor | None = None) -> None:
        if nodes.ndim != 2 or nodes.shape[1] != 3:
            raise ValueError(f"nodes must have shape (n_nodes, 3), got {tuple(nodes.shape)}.")
        if quadrature_weights.shape != (nodes.shape[0],):
            raise ValueError("quadrature_weights must have shape (n_nodes,).")
        self.nodes = nodes
        self.quadrature_weights = quadrature_weights
        self.exact_nodes = None if exact_nodes is None else exact_nodes.detach().to("cpu", torch.float64).contiguous()

    @property
    def n_nodes(self) -> int:
        return int(self.nodes.shape[0])

    def tile(self, count: int) -> SphericalGrid:
        if count == 1:
            return self
        return SphericalGrid(self.nodes.repeat(count, 1), self.quadrature_weights.repeat(count),
                             None if self.exact_nodes is None else self.exact_nodes.repeat(count, 1))

    def to(self, device=None, dtype=None) -> SphericalGrid:
        return SphericalGrid(self.nodes.to(device=device, dtype=dtype),
                             self.quadrature_weights.to(device=device, dtype=dtype), self.exact_nodes)


def build_equiangular_grid(n_latitude: int, n_longitude: int, *, dtype: torch.dtype = torch.float64,
                           device: torch.device | str | None = None) -> SphericalGrid:
    """The equiangular grid of ``build_torch_harmonics_grid("equiangular", ...)``:
    ascending colatitude (poles included), longitudes ``2 pi k / n_longitude``,
    weights ``w_lat * 2 pi / n_longitude``."""
    if n_longitude < 1:
        raise ValueError(f"n_longitude must be positive, got {n_longitude}.")
    cos_theta, latitude_weights = clenshaw_curtis(n_latitude)
    colatitude = torch.flip(torch.arccos(cos_theta), dims=(0,))
    latitude_weights = torch.flip(latitude_weights, dims=(0,))
    longitude = torch.linspace(0.0, 2.0 * math.pi, n_longitude + 1, dtype=torch.float64)[:-1]
    theta = colatitude.repeat_interleave(n_longitude)
    phi = longitude.repeat(n_latitude)
    sin_theta = torch.sin(theta)
    nodes = torch.stack([sin_theta * torch.cos(phi), sin_theta * torch.sin(phi), torch.cos(theta)], dim=-1)
    weights = latitude_weights.repeat_interleave(n_longitude) * (2.0 * math.pi / n_longitude)
    return SphericalGrid(nodes.to(dtype=dtype, device=device).contiguous(),
                         weights.to(dtype=dtype, device=device).contiguous(), exact_nodes=nodes)
