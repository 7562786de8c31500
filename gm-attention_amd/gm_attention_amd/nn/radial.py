"""Every head's radial trunk in one HIP pass.

The reference evaluates each value kernel's trunk on its own, with torch ops
(``nn/kernels.py:605-607`` ``_trunk_hidden``: ``_GaussianRadialBasis`` at
:191-231, then ``apply_radial_trunk``'s ``Linear`` + ``SiLU`` at :108-117).
Here the Gaussian basis of ``(r / cutoff)^2`` is formed once per edge and
every head's ``SiLU(W b + c)`` follows in registers (``gm_radial_trunk_*``);
the weights' and biases' gradients are reduced over the edges in a fixed
order.  Serves trunks of one ``Linear(B, 16)`` + ``SiLU`` (the reference's
default ``radial_hidden_features=(16,)``) in float32 on the GPU.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor, nn

from gm_attention_amd import _native


def eligible(kernels: list[Any], dtype: torch.dtype, device: torch.device) -> bool:
    if dtype != torch.float32 or device.type != "cuda" or not kernels:
        return False
    first = kernels[0]
    for k in kernels:
        layers = list(k.radial_trunk)
        if len(layers) != 2 or not isinstance(layers[0], nn.Linear) or not isinstance(layers[1], nn.SiLU):
            return False
        lin = layers[0]
        if lin.out_features != 16 or lin.in_features not in (4, 6, 8) or lin.weight.dtype != torch.float32:
            return False
        if (lin.bias is None) != (list(first.radial_trunk)[0].bias is None):
            return False
        if k.radial_basis.cutoff != first.radial_basis.cutoff or k.radial_basis.n_basis != first.radial_basis.n_basis:
            return False
    return True


class RadialTrunk(torch.autograd.Function):
    """``h (H, E, 16)`` from ``rho = d / cutoff`` and the heads' stacked trunk
    parameters, in rho's dtype or ``dtype`` (bfloat16 features, float32
    arithmetic; the gradient ``dh`` then comes in bfloat16 too)."""

    @staticmethod
    def forward(ctx: Any, rho: Tensor, weight: Tensor, bias: Tensor | None, centers: Tensor, width: float,
                dtype: torch.dtype | None = None) -> Tensor:
        with torch.profiler.record_function("gm::kernel/radial"):
            h = _native.radial_trunk_forward(rho, weight.contiguous(), None if bias is None else bias.contiguous(),
                                             centers, width, dtype)
        ctx.save_for_backward(rho, weight, bias if bias is not None else torch.empty(0, device=rho.device), centers)
        ctx.has_bias = bias is not None
        ctx.width = width
        return h

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, dh: Tensor) -> tuple:
        rho, weight, bias, centers = ctx.saved_tensors
        with torch.profiler.record_function("gm::kernel/radial_backward"):
            dw, db = _native.radial_trunk_backward(dh.contiguous(), rho, weight.contiguous(),
                                                   bias.contiguous() if ctx.has_bias else None, centers, ctx.width)
        return None, dw, db if ctx.has_bias else None, None, None, None


def stacked_trunk(kernels: list[Any]) -> tuple[Tensor, Tensor | None, Any]:
    """The heads' trunk parameters stacked, ``(W (H, 16, B), b (H, 16) or None)``, and the shared basis."""
    weight = torch.stack([list(k.radial_trunk)[0].weight for k in kernels])
    biases = [list(k.radial_trunk)[0].bias for k in kernels]
    return weight, None if biases[0] is None else torch.stack(biases), kernels[0].radial_basis


#: heads one trunk launch evaluates (the kernel keeps every head's weights in registers)
HEADS_PER_LAUNCH = 8


def trunk_hidden_heads(kernels: list[Any], rho: Tensor, dtype: torch.dtype | None = None) -> Tensor:
    """The stacked heads' trunk features ``(H, E, 16)`` on ``rho = d / cutoff``,
    at most ``HEADS_PER_LAUNCH`` heads a launch, in rho's dtype or ``dtype``
    (bfloat16: float32 arithmetic, the features rounded as stored)."""
    rb = kernels[0].radial_basis
    rho = rho.contiguous()
    parts = []
    for h0 in range(0, len(kernels), HEADS_PER_LAUNCH):
        chunk = kernels[h0:h0 + HEADS_PER_LAUNCH]
        weight = torch.stack([list(k.radial_trunk)[0].weight for k in chunk])
        biases = [list(k.radial_trunk)[0].bias for k in chunk]
        bias = None if biases[0] is None else torch.stack(biases)
        parts.append(RadialTrunk.apply(rho, weight, bias, rb.centers.contiguous(), float(rb.width), dtype))
    return parts[0] if len(parts) == 1 else torch.cat(parts, dim=0)
