"""Brute-force neighbourhoods and quadrature checks in numpy float64.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

from __future__ import annotations

import math

import numpy as np


def geodesic(p: np.ndarray, q: np.ndarray) -> np.ndarray:
    """``atan2(|p x q|, <p, q>)`` (reference discretization/edge_geometry.py:492-503)."""
    dot = np.clip(np.sum(p * q, axis=-1), -1.0, 1.0)
    return np.arctan2(np.linalg.norm(np.cross(p, q), axis=-1), dot)


def brute_force_edges(nodes: np.ndarray, radius: float, slack: float = 1e-10,
                      sources: np.ndarray | None = None) -> np.ndarray:
    """All pairs ``(i, j)`` with ``d(p_i, q_j) <= radius + slack`` from float64
    coordinates, ordered target-major, source-minor: the membership rule of
    edge_geometry.py:381-387 decided with no tree (as the reference's
    tests/discretization/test_neighborhoods.py:41-73 checks it).  ``sources``
    (default: the targets themselves) gives a bipartite neighbourhood."""
    n = nodes.shape[0]
    src = nodes if sources is None else sources
    targets, sources_out = [], []
    for lo in range(0, n, 256):
        hi = min(n, lo + 256)
        d = geodesic(nodes[lo:hi, None, :], src[None, :, :])
        t, s = np.nonzero(d <= radius + slack)
        targets.append(t + lo)
        sources_out.append(s)
    t = np.concatenate(targets)
    s = np.concatenate(sources_out)
    order = np.lexsort((s, t))
    return np.stack([t[order], s[order]])


def clenshaw_curtis_by_moments(n: int) -> tuple[np.ndarray, np.ndarray]:
    """Nodes ``cos(k pi / (n - 1))`` (ascending) and the weights that integrate
    every Chebyshev polynomial T_k, k < n, exactly: the solve of
    ``sum_j T_k(x_j) w_j = int_{-1}^{1} T_k = 2 / (1 - k^2)`` (even k), 0 (odd k)."""
    theta = np.pi - np.arange(n) * np.pi / (n - 1)
    x = np.cos(theta)
    k = np.arange(n)[:, None]
    V = np.cos(k * theta[None, :])
    m = np.zeros(n)
    even = np.arange(0, n, 2, dtype=np.float64)
    m[0::2] = 2.0 / (1.0 - even**2)
    return x, np.linalg.solve(V, m)


def equiangular_nodes(nlat: int, nlon: int) -> np.ndarray:
    """Equiangular nodes (poles included) from colatitude ``k pi / (nlat - 1)``
    and longitude ``2 pi l / nlon``: the grid of grids/torch_harmonics.py:98-132,
    computed without the arccos(cos) round trip."""
    theta = np.arange(nlat) * math.pi / (nlat - 1)
    phi = np.arange(nlon) * 2.0 * math.pi / nlon
    t = np.repeat(theta, nlon)
    p = np.tile(phi, nlat)
    return np.stack([np.sin(t) * np.cos(p), np.sin(t) * np.sin(p), np.cos(t)], axis=-1)
