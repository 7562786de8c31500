"""``SO2LayerNorm`` and ``SO2Dropout``: the transformer block's normalization and dropout.

Restates the reference's ``nn/normalization.py``: the merged equivariant layer
normalization (:22-190; one denominator pooled over the present frequencies'
mean-square magnitudes, only frequency 0 centred, a gain per copy and a bias on
frequency 0) and irrep-wise dropout (:193-278; one Bernoulli draw per copy,
shared by both coordinates of a nonzero-frequency copy).

On the GPU the normalization runs as one HIP pass over the flat rows
(``gm_layer_norm_*``: a wavefront per node, parameter gradients reduced in a
fixed order) for float32, float64 and bfloat16 rows; bfloat16 rows keep
float32 parameters and arithmetic.  CPU tensors take the reference's torch
arithmetic.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

from gm_attention_amd import _native
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

MAX_WIDTH = 1024  # flat width the HIP pass serves


class LayerNormOp(torch.autograd.Function):
    """``y (N, D)`` from rows ``x`` and the per-coordinate gains (and frequency-0 bias)."""

    @staticmethod
    def forward(ctx, x: Tensor, gamma: Tensor, beta: Tensor | None, layout, eps: float) -> Tensor:
        with torch.profiler.record_function("gm::pointwise/layer_norm"):
            y, mean, inv_d = _native.layer_norm_forward(x, gamma, beta, layout, eps)
        ctx.save_for_backward(x, gamma, mean, inv_d)
        ctx.layout = layout
        ctx.has_beta = beta is not None
        return y

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, gy: Tensor):
        x, gamma, mean, inv_d = ctx.saved_tensors
        with torch.profiler.record_function("gm::pointwise/layer_norm_backward"):
            dx, dparams = _native.layer_norm_backward(gy.contiguous(), x, gamma, mean, inv_d, ctx.layout)
        D = ctx.layout.D
        return dx, dparams[:D], dparams[D:] if ctx.has_beta else None, None, None


class SO2LayerNorm(nn.Module):
    def __init__(self, field_type: SO2FieldType, *, eps: float = 1e-5, bias: bool = True, dtype=None,
                 device=None) -> None:
        super().__init__()
        if not isinstance(field_type, SO2FieldType):
            raise TypeError(f"field_type must be an SO2FieldType, got {type(field_type).__name__}.")
        if not (eps > 0.0):
            raise ValueError(f"eps must be positive, got {eps}.")
        self.field_type = field_type
        self.eps = float(eps)
        self.gamma = nn.ParameterDict({
            str(f): nn.Parameter(torch.empty(m, dtype=dtype, device=device)) for f, m in field_type.items()
        })
        self.has_bias = bias and 0 in field_type
        if self.has_bias:
            self.beta = nn.Parameter(torch.empty(field_type.multiplicity(0), dtype=dtype, device=device))
        else:
            self.register_parameter("beta", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        for p in self.gamma.values():
            nn.init.ones_(p)
        if self.has_bias:
            nn.init.zeros_(self.beta)

    def _layout(self):
        layout = self.__dict__.get("_pw_layout")
        if layout is None:
            layout = _native.PointwiseLayout(self.field_type)
            self.__dict__["_pw_layout"] = layout
        return layout

    def gamma_flat(self, dtype: torch.dtype) -> Tensor:
        """The gains per flat coordinate (a copy's gain for both of its coordinates)."""
        parts = [self.gamma[str(f)] if f == 0 else self.gamma[str(f)].repeat_interleave(2)
                 for f in self.field_type.frequencies]
        return torch.cat(parts).to(dtype)

    def uses_hip(self, flat: Tensor) -> bool:
        return flat.device.type == "cuda" and flat.dtype in (torch.float32, torch.float64, torch.bfloat16) \
            and self.field_type.dimension <= MAX_WIDTH

    def forward_flat(self, flat: Tensor) -> Tensor:
        """The normalization of flat rows ``(N, D)``."""
        if not self.uses_hip(flat):
            return self._eager(SO2FeatureField.from_flat(self.field_type, flat))._rows()
        pd = _native.param_dtype(flat.dtype)
        beta = self.beta.to(pd) if self.has_bias else None
        return LayerNormOp.apply(flat.contiguous(), self.gamma_flat(pd), beta, self._layout(), self.eps)

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
        """The reference's torch arithmetic (normalization.py:150-190)."""
        stats = []
        centred0 = None
        if 0 in self.field_type:
            centred0 = x[0] - x[0].mean(dim=-1, keepdim=True)
            stats.append(centred0.pow(2).mean(dim=-1))
        for f in self.field_type.frequencies:
            if f != 0:
                stats.append(0.5 * x[f].pow(2).sum(dim=-1).mean(dim=-1))
        d = torch.sqrt(torch.stack(stats, dim=-1).mean(dim=-1) + self.eps)
        out = {}
        for f in self.field_type.frequencies:
            if f == 0:
                out[0] = self.gamma["0"] * (centred0 / d.unsqueeze(-1))
                if self.has_bias:
                    out[0] = out[0] + self.beta
            else:
                out[f] = self.gamma[str(f)].unsqueeze(-1) * (x[f] / d.unsqueeze(-1).unsqueeze(-1))
        return SO2FeatureField(self.field_type, out)

    def extra_repr(self) -> str:
        return f"field_type={self.field_type!r}, eps={self.eps:.3g}, bias={self.has_bias}"


class SO2Dropout(nn.Module):
    def __init__(self, field_type: SO2FieldType, p: float = 0.5) -> None:
        super().__init__()
        if not isinstance(field_type, SO2FieldType):
            raise TypeError(f"field_type must be an SO2FieldType, got {type(field_type).__name__}.")
        if not (0.0 <= p < 1.0):
            raise ValueError(f"p must satisfy 0 <= p < 1, got {p}.")
        self.field_type = field_type
        self.p = float(p)

    def active(self) -> bool:
        return self.training and self.p > 0.0

    def forward(self, x: SO2FeatureField) -> SO2FeatureField:
        if x.field_type != self.field_type:
            raise ValueError(f"Expected a field of type {self.field_type!r}, got {x.field_type!r}.")
        if not self.active():
            return x
        keep = 1.0 - self.p
        out = {}
        for f in self.field_type.frequencies:
            xn = x[f]
            shape = xn.shape if f == 0 else xn.shape[:-1]
            scale = torch.bernoulli(torch.full(shape, keep, dtype=xn.dtype, device=xn.device)) / keep
            out[f] = xn * scale if f == 0 else xn * scale.unsqueeze(-1)
        return SO2FeatureField(self.field_type, out)

    def forward_flat(self, flat: Tensor) -> Tensor:
        if not self.active():
            return flat
        return self(SO2FeatureField.from_flat(self.field_type, flat))._rows()

    def extra_repr(self) -> str:
        return f"field_type={self.field_type!r}, p={self.p:.3g}"
