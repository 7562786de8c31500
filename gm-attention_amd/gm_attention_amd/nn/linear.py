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


class RowsMatmul(torch.autograd.Function):
    """``x @ w`` for many rows and few columns (``x (M, a)``, ``w (a, b)``):
    the weight gradient ``x^T g`` sums blocks of rows through one batched
    product instead of a single long reduction, which the GEMM libraries
    run on a handful of workgroups.  The sum over blocks is in a fixed order."""

    BLOCK = 8192

    @staticmethod
    def forward(ctx, x: Tensor, w: Tensor) -> Tensor:
        ctx.save_for_backward(x, w)
        return x @ w

    @staticmethod
    def backward(ctx, g: Tensor):
        x, w = ctx.saved_tensors
        dx = g @ w.t() if ctx.needs_input_grad[0] else None
        dw = blocked_gram(x, g, RowsMatmul.BLOCK) if ctx.needs_input_grad[1] else None
        return dx, dw


def blocked_gram(x: Tensor, g: Tensor, block: int) -> Tensor:
    """``x^T g`` over the rows, summed as per-block partial products."""
    rows = x.shape[0]
    nb = rows // block
    if nb < 2:
        return x.t() @ g
    head = nb * block
    xs = x[:head].reshape(nb, block, x.shape[1]).transpose(1, 2)
    gs = g[:head].reshape(nb, block, g.shape[1]).contiguous()
    out = torch.bmm(xs, gs).sum(0)
    if head < rows:
        out = out + x[head:].t() @ g[head:]
    return out


def rows_matmul(x: Tensor, w: Tensor) -> Tensor:
    return RowsMatmul.apply(x, w) if x.dim() == 2 else x @ w


def complex_as_real(weight: Tensor) -> Tensor:
    """``(b, a, 2)`` complex weights as the real ``(2a, 2b)`` right factor acting
    on interleaved ``(a, 2)`` pairs: ``out = x_flat @ M`` with ``x_flat`` ``(..., 2a)``."""
    wr, wi = weight[..., 0].T, weight[..., 1].T  # (a, b)
    from_real = torch.stack([wr, wi], dim=-1)  # (a, b, 2): re_in -> (re_out, im_out)
    from_imag = torch.stack([-wi, wr], dim=-1)  # im_in -> (re_out, im_out)
    a, b = wr.shape
    return torch.stack([from_real, from_imag], dim=1).reshape(2 * a, 2 * b)


class FlatLinear(torch.autograd.Function):
    """``x @ M + bias`` on flat rows with ``M (D_in, D_out)`` the layer's
    block-diagonal matrix: one GEMM (bias in its epilogue) straight between
    the flat layouts.  ``M`` and the bias stay in the parameters' dtype and are
    rounded to the rows' dtype for the product (bfloat16 rows: a bfloat16 GEMM
    with float accumulation); their gradients come back in the parameters'
    dtype: the blocked ``x^T g`` and the bias's column sums."""

    @staticmethod
    def forward(ctx, x: Tensor, m: Tensor, bias_flat: Tensor | None) -> Tensor:
        ctx.save_for_backward(x, m)
        ctx.has_bias = bias_flat is not None
        mx = m.to(x.dtype)
        return torch.addmm(bias_flat.to(x.dtype), x, mx) if bias_flat is not None else x @ mx

    @staticmethod
    def backward(ctx, g: Tensor):
        x, m = ctx.saved_tensors
        g = g.contiguous()
        dx = g @ m.t().to(g.dtype) if ctx.needs_input_grad[0] else None
        dm = None
        if ctx.needs_input_grad[1]:
            dm = blocked_gram(x.to(m.dtype), g.to(m.dtype), RowsMatmul.BLOCK)
        db = g.sum(0, dtype=m.dtype) if ctx.has_bias else None
        return dx, dm, db


def block_matrix(lin: "SO2Linear") -> Tensor:
    """The layer as one ``(D_in, D_out)`` matrix acting on flat rows (zero off its frequency blocks)."""
    return weights_matrix(lin.field_type_in, lin.field_type_out, lin.common_frequencies, lin.weight)


def weights_matrix(fin: SO2FieldType, fout: SO2FieldType, common, weights) -> Tensor:
    """Per-frequency intertwiner weights (``(b, a)`` real at 0, ``(b, a, 2)``
    complex above) as one ``(D_in, D_out)`` matrix on flat rows."""
    sin, sout = fin.slices(), fout.slices()
    ref = next(iter(weights.values()))
    m = ref.new_zeros(fin.dimension, fout.dimension)
    for f in common:
        w = weights[str(f)]
        m[sin[f], sout[f]] = w.T if f == 0 else complex_as_real(w)
    return m


def flat_bias(bias: Tensor | None, fout: SO2FieldType) -> Tensor | None:
    """A frequency-0 bias spread over the flat columns (zero elsewhere)."""
    if bias is None:
        return None
    return torch.cat([bias, bias.new_zeros(fout.dimension - fout.multiplicity(0))])


def flat_forward(lin: "SO2Linear", flat: Tensor) -> Tensor:
    """``lin`` on flat rows ``(N, D_in)`` -> ``(N, D_out)``."""
    bias = flat_bias(lin.bias if lin.has_bias else None, lin.field_type_out)
    return FlatLinear.apply(flat, block_matrix(lin), bias)


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
            out = rows_matmul(x[0].reshape(-1, x[0].shape[-1]), w.T).reshape(*batch, b)
            outputs[0] = out + bias if bias is not None else out
        else:
            flat = rows_matmul(x[f].reshape(-1, 2 * x[f].shape[-2]), complex_as_real(w).to(x.dtype))
            outputs[f] = flat.reshape(*batch, b, 2)
    return SO2FeatureField(field_type_out, outputs)
