"""Tangent frames on the unit sphere.

``build_tangent_frames`` restates ``discretization/frames.py:136-226``: e_1 is
the normalised tangent projection of the coordinate axis least aligned with
p (``argmin |p_k|``, first index on ties), e_2 = p x e_1 renormalised.
``rotate_tangent_frames`` restates ``frames.py:7-90``: ``E' = E r(theta)``.
"""

from __future__ import annotations

import torch
from torch import Tensor


def planar_rotation_matrices(angles: Tensor) -> Tensor:
    c, s = torch.cos(angles), torch.sin(angles)
    return torch.stack((torch.stack((c, -s), dim=-1), torch.stack((s, c), dim=-1)), dim=-2)


def build_tangent_frames(nodes: Tensor) -> Tensor:
    """Oriented orthonormal frames ``(n_nodes, 3, 2)`` with e_1 x e_2 = p."""
    axes = torch.eye(3, dtype=nodes.dtype, device=nodes.device)[torch.argmin(torch.abs(nodes), dim=-1)]
    first = axes - torch.sum(axes * nodes, dim=-1, keepdim=True) * nodes
    first = first / torch.linalg.vector_norm(first, dim=-1, keepdim=True)
    second = torch.linalg.cross(nodes, first, dim=-1)
    second = second / torch.linalg.vector_norm(second, dim=-1, keepdim=True)
    return torch.stack((first, second), dim=-1).contiguous()


def rotate_tangent_frames(frames: Tensor, angles: Tensor) -> Tensor:
    """``E r(theta)`` per node: a change of gauge by ``theta``."""
    return torch.matmul(frames, planar_rotation_matrices(angles.to(frames.dtype))).contiguous()
