"""``SO2Linear``: the frequency-block-diagonal intertwiner.

Restates the reference's ``nn/linear.py``: per common frequency a real
``(b_0, a_0)`` matrix at 0 and a complex ``(b_n, a_n)`` matrix (stored
``(b_n, a_n, 2)``) above, a bias on the frequency-0 outputs, and the
``nn.Linear``-style uniform initialisation with the block's real fan-in
(:22-128).  The forward (:130-190) is one matrix product per frequency; the
complex product is written as one real product on the interleaved pairs,
``[re, im] @ [[Wr^T, Wi^T], [-Wi^T, Wr^T]]``, so each frequency is a single
library GEMM on MFMA.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor, nn

from gm_attention_amd.representations import so2
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType


def complex_as_real(weight: Tensor) -> Tensor:
    """``(b, a, 2)`` complex weights as the real ``(2a, 2b)`` right factor acting
    on interleaved ``(a, 2)`` pairs: ``out = x_flat @ M`` with ``x_flat`` ``(..., 2a)``."""
    wr, wi = weight[..., 0].T, weight[..., 1].T  # (a, b)
    from_real = torch.stack([wr, wi], dim=-1)  # (a, b, 2): re_in -> (re_out, im_out)
    from_imag = torch.stack([-wi, wr], dim=-1)  # im_in -> (re_out, im_out)
    a, b = wr.shape
    return torch.stack([from_real, from_imag], dim=1).reshape(2 * a, 2 * b)


class SO2Linear(nn.Module):
    def __init__(self, field_type_in: SO2FieldType, field_type_out: SO2FieldType, *, bias: bool = True, dtype=None,
                 device=None) -> None:
        super().__init__()
        if not isinstance(field_type_in, SO2FieldType) or not isinstance(field_type_out, SO2FieldType):
            raise TypeError("field_type_in and field_type_out must be SO2FieldType instances.")
        self.field_type_in = field_type_in
        self.field_type_out = field_type_out
        self.common_frequencies = field_type_in.common_frequencies(field_type_out)
        self.weight = nn.ParameterDict()
        for f in self.common_frequencies:
            a, b = field_type_in.multiplicity(f), field_type_out.multiplicity(f)
            shape = (b, a) if f == 0 else (b, a, 2)
            self.weight[str(f)] = nn.Parameter(torch.empty(shape, dtype=dtype, device=device))
        self.has_bias = bias and 0 in field_type_out
        if self.has_bias:
            self.bias = nn.Parameter(torch.empty(field_type_out.multiplicity(0), dtype=dtype, device=device))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        for f in self.common_frequencies:
            bound = 1.0 / math.sqrt(self.field_type_in.multiplicity(f) * so2.irrep_dimension(f))
            nn.init.uniform_(self.weight[str(f)], -bound, bound)
        if self.has_bias:
            fan_in = self.field_type_in.multiplicity(0) if 0 in self.common_frequencies else 1
            bound = 1.0 / math.sqrt(fan_in)
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x: SO2FeatureField) -> SO2FeatureField:
        if x.field_type != self.field_type_in:
            raise ValueError(f"Expected a field of type {self.field_type_in!r}, got {x.field_type!r}.")
        return apply_linear(self.field_type_out, self.common_frequencies, dict(self.weight.items()), self.bias, x)


def apply_linear(field_type_out: SO2FieldType, common: tuple[int, ...], weights: dict[str, Tensor],
                 bias: Tensor | None, x: SO2FeatureField) -> SO2FeatureField:
    """The intertwiner with the given per-frequency weights (and bias) on ``x``."""
    outputs: dict[int, Tensor] = {}
    batch = tuple(x.batch_shape)
    for f in field_type_out.frequencies:
        b = field_type_out.multiplicity(f)
        if f not in common:
            outputs[f] = x[x.frequencies[0]].new_zeros(batch + ((b,) if f == 0 else (b, 2)))
            if f == 0 and bias is not None:
                outputs[f] = outputs[f] + bias
            continue
        w = weights[str(f)]
        if f == 0:
            out = x[0] @ w.T
            outputs[0] = out + bias if bias is not None else out
        else:
            flat = x[f].reshape(*batch, -1) @ complex_as_real(w).to(x.dtype)
            outputs[f] = flat.reshape(*batch, b, 2)
    return SO2FeatureField(field_type_out, outputs)
