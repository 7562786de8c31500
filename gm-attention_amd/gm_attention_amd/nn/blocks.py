"""``SO2TransformerBlock``: the pre-norm transformer block of the reference.

Restates ``nn/blocks.py:97-356`` of the reference,

    x'  = x  + Drop(Mixer(LN(x), edges))
    x'' = x' + Drop(W_2 sigma(W_1 LN(x'))),

with the mixer ``SO2MHSA`` (or a type-preserving ``SO2Convolution`` under
``mixer="convolution"``), ``SO2LayerNorm``, the scalar-gated nonlinearity and
two ``SO2Linear`` layers widening to ``field_type.scaled(ffn_multiplier)`` and
back; the constructor, parameter names and ``forward`` / ``forward_chunked``
signatures are the reference's (:171-330).

The residual stream stays in the flat node layout between the operators: the
layer norms and the gate are single HIP passes over flat rows, each
``SO2Linear`` is one GEMM against its block-diagonal matrix, so no per-frequency
split or concatenation is materialised.  Rows may be bfloat16 while the
parameters are float32 (the C4 configuration's "bf16 activations with fp32
accumulation"): the norms and the gate read and write bfloat16 and compute in
float32, the feed-forward GEMMs run in bfloat16 with float accumulation, and
the mixer, whose kernels are float32, takes its input rounded up to float32 and
hands back float32 that the residual addition rounds to bfloat16.

``IcoEncode`` / ``EquiEncode`` (reference :359-505, :799-869) restrict a
field from a fine grid onto a coarse one over bipartite edges
(``discretization.hierarchy``): the steerable-kernel integral of
``SO2Convolution`` with fine sources and coarse targets, through the fused
factored aggregate (kernels wider than the op's bounds run as output tiles).
"""

from __future__ import annotations

from functools import partial
from typing import Literal

import torch
from torch import Tensor, nn

from gm_attention_amd.nn import fused_factored, kernels
from gm_attention_amd.nn.attention import SO2MHSA, batched_flat_serves, gather_to_edges, weighted_segment_sum
from gm_attention_amd.nn.convolution import SO2Convolution
from gm_attention_amd.nn.fused_attention import evaluate_aggregation_window
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.nn import ffn
from gm_attention_amd.nn.linear import SO2Linear, flat_forward
from gm_attention_amd.nn.nonlinearities import SO2ScalarGatedNonlinearity
from gm_attention_amd.nn.normalization import SO2Dropout, SO2LayerNorm
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

MixerKind = Literal["attention", "convolution"]
NonlinearityKind = Literal["scalar_gate", "scalar_gate_double_sigmoid"]

_FFN_MULTIPLIER_DEFAULT = 2

_NONLINEARITIES = {
    "scalar_gate": SO2ScalarGatedNonlinearity,
    "scalar_gate_double_sigmoid": partial(SO2ScalarGatedNonlinearity, gate="double_sigmoid"),
}


def build_nonlinearity(kind: NonlinearityKind, field_type: SO2FieldType, *, dtype=None, device=None) -> nn.Module:
    """The equivariant activation ``kind`` names (reference blocks.py:69-86)."""
    if kind not in _NONLINEARITIES:
        raise ValueError(f"nonlinearity must be one of {tuple(_NONLINEARITIES)}, got {kind!r}.")
    return _NONLINEARITIES[kind](field_type, dtype=dtype, device=device)


def _add_fields(a: SO2FeatureField, b: SO2FeatureField) -> SO2FeatureField:
    return SO2FeatureField(a.field_type, {f: a[f] + b[f] for f in a.field_type.frequencies})


class SO2TransformerBlock(nn.Module):
    def __init__(self, field_type: SO2FieldType, num_heads: int, *, ffn_multiplier: int = 2,
                 hidden_field_type: SO2FieldType | None = None, cutoff: float, window: str = "hard",
                 n_radial_basis: int = 8, radial_hidden_features=(16,), radial_basis: str = "gaussian",
                 dropout: float = 0.0, eps: float = 1e-5, bias: bool = True,
                 nonlinearity: NonlinearityKind = "scalar_gate_double_sigmoid", mixer: MixerKind = "attention",
                 attention_batched: bool = False, value_kind: str = "steerable", dtype=None, device=None) -> None:
        super().__init__()
        if not isinstance(field_type, SO2FieldType):
            raise TypeError(f"field_type must be an SO2FieldType, got {type(field_type).__name__}.")
        if hidden_field_type is not None and ffn_multiplier != _FFN_MULTIPLIER_DEFAULT:
            raise ValueError("Pass either ffn_multiplier or hidden_field_type, not both -- "
                             f"got ffn_multiplier={ffn_multiplier} and hidden_field_type={hidden_field_type!r}, "
                             "which would usually disagree.")
        if hidden_field_type is not None and not isinstance(hidden_field_type, SO2FieldType):
            raise TypeError(f"hidden_field_type must be an SO2FieldType, got {type(hidden_field_type).__name__}.")
        if nonlinearity not in _NONLINEARITIES:
            raise ValueError(f"nonlinearity must be one of {tuple(_NONLINEARITIES)}, got {nonlinearity!r}.")
        if mixer not in ("attention", "convolution"):
            raise ValueError(f"mixer must be 'attention' or 'convolution', got {mixer!r}.")
        self.nonlinearity = nonlinearity
        self.field_type = field_type
        self.hidden_field_type = hidden_field_type if hidden_field_type is not None else field_type.scaled(ffn_multiplier)
        self.mixer = mixer
        kw = dict(dtype=dtype, device=device)
        self.norm1 = SO2LayerNorm(field_type, eps=eps, bias=bias, **kw)
        self.attention: nn.Module
        if mixer == "attention":
            self.attention = SO2MHSA(field_type, num_heads, cutoff=cutoff, window=window,
                                      n_radial_basis=n_radial_basis, radial_hidden_features=radial_hidden_features,
                                      radial_basis=radial_basis, bias=bias, batched=attention_batched,
                                      value_kind=value_kind, **kw)
        else:
            self.attention = SO2Convolution(field_type, field_type, cutoff=cutoff, window=window,
                                            self_interaction="none", n_radial_basis=n_radial_basis,
                                            radial_hidden_features=radial_hidden_features,
                                            radial_basis=radial_basis, bias=bias, **kw)
        self.attention_dropout = SO2Dropout(field_type, p=dropout)
        self.norm2 = SO2LayerNorm(field_type, eps=eps, bias=bias, **kw)
        self.linear1 = SO2Linear(field_type, self.hidden_field_type, bias=bias, **kw)
        self.activation = build_nonlinearity(nonlinearity, self.hidden_field_type, **kw)
        self.linear2 = SO2Linear(self.hidden_field_type, field_type, bias=bias, **kw)
        self.mlp_dropout = SO2Dropout(field_type, p=dropout)

    def forward(self, x: SO2FeatureField, edges) -> SO2FeatureField:
        return self._run(x, edges, chunk_size=None)

    def forward_chunked(self, x: SO2FeatureField, edges, *, chunk_size: int) -> SO2FeatureField:
        return self._run(x, edges, chunk_size=chunk_size)

    def _mix(self, h: Tensor, edges, chunk_size: int | None) -> Tensor:
        """The mixer on flat rows: bfloat16 rows straight into the batched
        attention's fused path where it serves them (its scores and node mixes
        read them, its arithmetic is float32), else the rows in the mixer's
        parameter dtype; the result in float32 or that dtype."""
        if h.dtype == torch.bfloat16 and chunk_size is None and self.mixer == "attention":
            field = SO2FeatureField.from_flat(self.field_type, h)
            if batched_flat_serves(self.attention, field, edges):
                return self.attention(field, edges)._rows()
        pdtype = next(self.attention.parameters()).dtype
        field = SO2FeatureField.from_flat(self.field_type, h.to(pdtype))
        if chunk_size is None:
            out = self.attention(field, edges)
        else:
            out = self.attention.forward_chunked(field, edges, chunk_size=chunk_size)
        return out._rows()

    def _run(self, x: SO2FeatureField, edges, *, chunk_size: int | None) -> SO2FeatureField:
        if x.field_type != self.field_type:
            raise ValueError(f"Expected a field of type {self.field_type!r}, got {x.field_type!r}.")
        flat = x._rows()
        batch = flat.shape[:-1]
        rows = flat.reshape(-1, flat.shape[-1])
        return SO2FeatureField.from_flat(self.field_type, self.forward_flat(rows, edges, chunk_size).reshape(*batch, -1))

    def forward_flat(self, rows: Tensor, edges, chunk_size: int | None = None) -> Tensor:
        """The block on flat rows ``(N, D)``; returns ``(N, D)`` in the rows' dtype."""
        attended = self._mix(self.norm1.forward_flat(rows), edges, chunk_size)
        rows = rows + self.attention_dropout.forward_flat(attended).to(rows.dtype)
        if ffn.serves(self, rows):  # bfloat16 rows: the whole feed-forward as one fused pass per direction
            return ffn.forward(self, rows)
        hidden = flat_forward(self.linear1, self.norm2.forward_flat(rows))
        hidden = self.activation.forward_flat(hidden)
        hidden = flat_forward(self.linear2, hidden)
        return rows + self.mlp_dropout.forward_flat(hidden)

    def extra_repr(self) -> str:
        return (f"field_type={self.field_type!r}, hidden_field_type={self.hidden_field_type!r}, "
                f"nonlinearity={self.nonlinearity!r}")


class IcoEncode(nn.Module):
    """Fine -> coarse restriction over bipartite edges (reference blocks.py:359-505)."""

    def __init__(self, field_type_in: SO2FieldType, field_type_out: SO2FieldType, *, cutoff: float,
                 window: str = "hard", n_radial_basis: int = 8, radial_hidden_features=(16,),
                 radial_basis: str = "gaussian", bias: bool = True, dtype=None, device=None) -> None:
        super().__init__()
        if window not in ("hard", "quartic"):
            raise ValueError(f"window must be 'hard' or 'quartic', got {window!r}.")
        self.field_type_in = field_type_in
        self.field_type_out = field_type_out
        self.cutoff = float(cutoff)
        self.window = window
        self.kernel = SO2SteerableKernel(field_type_in, field_type_out, cutoff=cutoff, n_radial_basis=n_radial_basis,
                                         radial_hidden_features=radial_hidden_features, radial_basis=radial_basis,
                                         bias=bias, dtype=dtype, device=device)

    def forward(self, x: SO2FeatureField, edges) -> SO2FeatureField:
        """``y_i = sum_j c(v_ij) w_ij K(v_ij) rho(g_{i<-j}) x_j``, i a coarse target, j a fine source."""
        if x.field_type != self.field_type_in:
            raise ValueError(f"Expected a field of type {self.field_type_in!r}, got {x.field_type!r}.")
        weight = evaluate_aggregation_window(edges.distances, self.cutoff, self.window) * \
            edges.tangent_quadrature_weights
        if kernels.factored_enabled():
            enabled = fused_factored.enabled(self.kernel, x, edges)
            groups = (fused_factored.source_groups(edges.source_index,
                                                   fused_factored.group_key(edges, 0, int(edges.n_edges)),
                                                   owner=edges.edge_index)
                      if enabled else None)
            if enabled:  # float32 rows: the grouped kernels over shares of the output copies
                shares = fused_factored.forward_aggregated_shares(self.kernel, x, edges, weight, groups)
                if shares is not None:
                    return shares
            products = self.kernel.node_products(x)
            return self.kernel.forward_factored_aggregated(x, edges, weight, products, groups)
        messages = self.kernel(gather_to_edges(x, edges.source_index), edges)
        return SO2FeatureField(self.field_type_out,
                               weighted_segment_sum(weight, messages.coefficients, edges.row_ptr))

    def extra_repr(self) -> str:
        return (f"field_type_in={self.field_type_in!r}, field_type_out={self.field_type_out!r}, "
                f"cutoff={self.cutoff:.6g}, window={self.window!r}")


class EquiEncode(nn.Module):
    """Fine -> coarse restriction between two arbitrary grids (reference blocks.py:799-869)."""

    def __init__(self, field_type_in: SO2FieldType, field_type_out: SO2FieldType, *, cutoff: float,
                 mode: str = "learned_integral", window: str = "quartic", n_radial_basis: int = 8,
                 radial_hidden_features=(16,), radial_basis: str = "gaussian", bias: bool = True, dtype=None,
                 device=None) -> None:
        super().__init__()
        if mode != "learned_integral":
            raise ValueError(f"mode must be 'learned_integral', got {mode!r}.")
        self.field_type_in = field_type_in
        self.field_type_out = field_type_out
        self.mode = mode
        self.cutoff = float(cutoff)
        self.integral = IcoEncode(field_type_in, field_type_out, cutoff=cutoff, window=window,
                                  n_radial_basis=n_radial_basis, radial_hidden_features=radial_hidden_features,
                                  radial_basis=radial_basis, bias=bias, dtype=dtype, device=device)

    def forward(self, x: SO2FeatureField, down_edges) -> SO2FeatureField:
        return self.integral(x, down_edges)

    def extra_repr(self) -> str:
        return f"{self.field_type_in!r} -> {self.field_type_out!r}, mode={self.mode!r}, cutoff={self.cutoff:.6g}"
