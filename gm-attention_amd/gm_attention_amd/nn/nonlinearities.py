"""``SO2ScalarGatedNonlinearity``: SiLU on the scalars, a learned gate per copy above.

Restates the reference's ``nn/nonlinearities.py:51-166``: ``y_0 = SiLU(x_0)``
and, per nonzero frequency n, ``y_n,a = act(A_n x_0 + b_n)_a x_n,a`` on both
coordinates of copy a, with ``act = SiLU`` or ``2 sigmoid``; the gates read the
raw (not activated) scalars.  One ``nn.Linear`` per nonzero frequency, as in
the reference, so state dicts move unchanged.

On the GPU every frequency's gate Linear is one library GEMM over the stacked
weights (``(sum a_n, a_0)``), and the activation and gating are one HIP pass
(``gm_gate_*``) for float32, float64 and bfloat16 rows (bfloat16: float
arithmetic, the GEMM in bfloat16 with float accumulation).  CPU tensors take
the reference's torch arithmetic.
"""

from __future__ import annotations

from typing import Literal

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from gm_attention_amd import _native
from gm_attention_amd.nn.linear import FlatLinear
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType


class GateOp(torch.autograd.Function):
    """``y (N, D)`` from the rows ``h`` and the gates' pre-activations ``pre (N, G)``."""

    @staticmethod
    def forward(ctx, h: Tensor, pre: Tensor, layout, double_sigmoid: bool) -> Tensor:
        with torch.profiler.record_function("gm::pointwise/gate"):
            y = _native.gate_forward(h, pre, layout, double_sigmoid)
        ctx.save_for_backward(h, pre)
        ctx.layout = layout
        ctx.double_sigmoid = double_sigmoid
        return y

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, gy: Tensor):
        h, pre = ctx.saved_tensors
        with torch.profiler.record_function("gm::pointwise/gate_backward"):
            dh, dpre = _native.gate_backward(gy.contiguous(), h, pre, ctx.layout, ctx.double_sigmoid)
        return dh, dpre, None, None


class SO2ScalarGatedNonlinearity(nn.Module):
    def __init__(self, field_type: SO2FieldType, *, gate: Literal["silu", "double_sigmoid"] = "silu",
                 eps: float = 1e-6, dtype=None, device=None) -> None:
        super().__init__()
        if not isinstance(field_type, SO2FieldType):
            raise TypeError(f"field_type must be an SO2FieldType, got {type(field_type).__name__}.")
        if not (eps > 0.0):
            raise ValueError(f"eps must be positive, got {eps}.")
        if gate not in ("silu", "double_sigmoid"):
            raise ValueError(f"gate must be 'silu' or 'double_sigmoid', got {gate!r}.")
        if 0 not in field_type:
            raise ValueError("SO2ScalarGatedNonlinearity requires frequency-0 channels to condition its gates on, "
                             f"but got {field_type!r}.")
        self.field_type = field_type
        self.gate = gate
        self.eps = float(eps)
        a0 = field_type.multiplicity(0)
        self.gates = nn.ModuleDict({
            str(f): nn.Linear(a0, field_type.multiplicity(f), dtype=dtype, device=device)
            for f in field_type.frequencies if f != 0
        })

    def _layout(self):
        layout = self.__dict__.get("_pw_layout")
        if layout is None:
            layout = _native.PointwiseLayout(self.field_type)
            self.__dict__["_pw_layout"] = layout
        return layout

    def _activate(self, pre: Tensor) -> Tensor:
        return 2.0 * torch.sigmoid(pre) if self.gate == "double_sigmoid" else F.silu(pre)

    def uses_hip(self, flat: Tensor) -> bool:
        return flat.device.type == "cuda" and flat.dtype in (torch.float32, torch.float64, torch.bfloat16) \
            and self.field_type.dimension <= 1024

    def pre_activations(self, scalars: Tensor) -> Tensor:
        """Every frequency's gate pre-activations ``(N, sum a_n)``, frequency-major:
        one product with the stacked gate weights (``(a_0, sum a_n)``)."""
        order = [str(f) for f in self.field_type.frequencies if f != 0]
        weight = torch.cat([self.gates[k].weight for k in order]).t()
        biases = [self.gates[k].bias for k in order]
        return FlatLinear.apply(scalars, weight, None if biases[0] is None else torch.cat(biases))

    def forward_flat(self, flat: Tensor) -> Tensor:
        """The nonlinearity on flat rows ``(N, D)``."""
        if not self.uses_hip(flat):
            return self._eager(SO2FeatureField.from_flat(self.field_type, flat))._rows()
        flat = flat.contiguous()
        layout = self._layout()
        if layout.G == 0:
            pre = flat.new_empty(flat.shape[0], 0)
        else:
            pre = self.pre_activations(flat[:, : layout.a0])
        return GateOp.apply(flat, pre.contiguous(), layout, self.gate == "double_sigmoid")

    def forward(self, x: SO2FeatureField) -> SO2FeatureField:
        if x.field_type != self.field_type:
            raise ValueError(f"Expected a field of type {self.field_type!r}, got {x.field_type!r}.")
        flat = x._rows()
        if not self.uses_hip(flat):
            return self._eager(x)
        batch = flat.shape[:-1]
        out = self.forward_flat(flat.reshape(-1, flat.shape[-1]))
        return SO2FeatureField.from_flat(self.field_type, out.reshape(*batch, -1))

    def _eager(self, x: SO2FeatureField) -> SO2FeatureField:
        """The reference's torch arithmetic (nonlinearities.py:140-166)."""
        scalars = x[0]
        out = {0: F.silu(scalars)}
        for f in self.field_type.frequencies:
            if f != 0:
                out[f] = x[f] * self._activate(self.gates[str(f)](scalars)).unsqueeze(-1)
        return SO2FeatureField(self.field_type, out)

    def extra_repr(self) -> str:
        return f"field_type={self.field_type!r}, gate={self.gate!r}"
