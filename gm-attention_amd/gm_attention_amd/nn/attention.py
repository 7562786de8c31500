"""Gauge-equivariant neighbourhood attention on the sphere over the fused ops.

Restates the reference's ``nn/attention.py`` layers with their parameters,
signatures and call structure:

* ``SO2Attention`` (:97-476): intertwiner query and key maps, a steerable
  value kernel, ``s_ij = <q_i, rho(g_ij) k_j> / sqrt(dim rho_attn)``, the
  window-and-quadrature-weighted softmax per target, ``y_i = sum_j alpha_ij
  V(v_ij) rho(g_ij) x_j``, an optional pointwise self map; ``forward_chunked``
  over target ranges (:344-402);
* ``SO2MHSA`` (:477-650): the heads' split of the field type, head-major
  concatenation, the output intertwiner, and the batched pass
  ``_attend_batched`` (:858-909): the heads' stacked query and key maps
  (:653-669), the scores and softmax of every head in one fused op, the value
  kernels in the factored order with one shared source grouping
  (``_aggregated_factored``, :801-822).

Every score, softmax and value aggregation runs in the HIP ops
(``fused_attention.Softmax``, ``fused_factored.FactoredAggregate``; under
``GM_FACTORED_KERNEL=0`` the value kernels' per-edge readout runs in the fused
pair terms, ``fused_pairs``, and the weighted messages are summed per target);
the projections are per-frequency dense products.  A call an op's predicate
declines (CPU tensors, a ``GM_FUSED_*`` switch at ``"0"``) runs the same
numbers in torch (``eager_ops``), as the reference falls back to its eager path.
"""

from __future__ import annotations

import functools
import math
import os
from collections.abc import Sequence
from typing import cast

import torch
import torch.utils.checkpoint
from torch import Tensor, nn

from gm_attention_amd.discretization.discretization import SphericalDiscretization
from gm_attention_amd.nn import fused_attention, fused_factored, kernels, radial
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.nn.linear import FlatLinear, SO2Linear, apply_linear, block_matrix, flat_bias, weights_matrix
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

REMATERIALIZE_CHUNKS = os.environ.get("GM_CHUNK_REMATERIALIZE", "1") != "0"


def _resolve_edges(edges, cutoff: float):
    return edges.edges_within(cutoff) if isinstance(edges, SphericalDiscretization) else edges


def _validate_node_field(x: SO2FeatureField, field_type: SO2FieldType, edges) -> None:
    if x.field_type != field_type:
        raise ValueError(f"Expected a field of type {field_type!r}, got {x.field_type!r}.")
    n_nodes = edges.row_ptr.shape[0] - 1
    if tuple(x.batch_shape) != (n_nodes,):
        raise ValueError(f"x.batch_shape must equal (n_nodes,) = ({n_nodes},), inferred from edges.row_ptr, "
                         f"got {tuple(x.batch_shape)}.")


def gather_to_edges(x: SO2FeatureField, index: Tensor) -> SO2FeatureField:
    """Every frequency's rows at ``index`` (reference nn/_scatter.py:17-33)."""
    return SO2FeatureField(x.field_type, {f: x[f].index_select(0, index) for f in x.field_type.frequencies})


def weighted_segment_sum(weight: Tensor, messages: dict[int, Tensor], row_ptr: Tensor) -> dict[int, Tensor]:
    """``sum_e w_e m_e`` over each target's CSR segment, per frequency
    (reference nn/_scatter.py:36-58 on the weighted messages)."""
    return {f: torch.segment_reduce(weight.reshape(-1, *([1] * (m.ndim - 1))) * m, "sum", offsets=row_ptr, axis=0)
            for f, m in messages.items()}


def sum_partials(partials: list[dict[int, Tensor]]) -> dict[int, Tensor]:
    """Per frequency, the sum of the target ranges' outputs (each zero off its range)."""
    return {f: functools.reduce(torch.add, [p[f] for p in partials]) for f in partials[0]}


def _checkpointed(module: nn.Module, compute):
    if module.training and torch.is_grad_enabled() and REMATERIALIZE_CHUNKS:
        return torch.utils.checkpoint.checkpoint(compute, use_reentrant=False)
    return compute()


def _concatenate_heads(fields: Sequence[SO2FeatureField], field_type: SO2FieldType) -> SO2FeatureField:
    """Direct sum of equal-typed fields along each frequency's multiplicity axis (:456-474)."""
    return SO2FeatureField(field_type, {
        f: torch.cat([fld[f] for fld in fields], dim=-1 if f == 0 else -2) for f in field_type.frequencies})


class SO2Attention(nn.Module):
    def __init__(self, field_type_in: SO2FieldType, field_type_attn: SO2FieldType, field_type_out: SO2FieldType, *,
                 cutoff: float, window: str = "hard", self_interaction: str = "none", n_radial_basis: int = 8,
                 radial_hidden_features: Sequence[int] = (16,), radial_basis: str = "gaussian", bias: bool = True,
                 value_kind: str = "steerable", dtype=None, device=None) -> None:
        super().__init__()
        if window not in ("hard", "quartic"):
            raise ValueError(f"window must be 'hard' or 'quartic', got {window!r}.")
        if self_interaction not in ("none", "linear"):
            raise ValueError(f"self_interaction must be 'none' or 'linear', got {self_interaction!r}.")
        if value_kind != "steerable":
            raise ValueError(f"value_kind must be 'steerable', got {value_kind!r}.")
        self.value_kind = value_kind
        self.field_type_in = field_type_in
        self.field_type_attn = field_type_attn
        self.field_type_out = field_type_out
        self.cutoff = float(cutoff)
        self.window = window
        self.self_interaction = self_interaction
        self.query = SO2Linear(field_type_in, field_type_attn, bias=bias, dtype=dtype, device=device)
        self.key = SO2Linear(field_type_in, field_type_attn, bias=bias, dtype=dtype, device=device)
        self.value = SO2SteerableKernel(field_type_in, field_type_out, cutoff=cutoff, n_radial_basis=n_radial_basis,
                                        radial_hidden_features=radial_hidden_features, radial_basis=radial_basis,
                                        bias=bias, dtype=dtype, device=device)
        self.self_linear = (SO2Linear(field_type_in, field_type_out, bias=False, dtype=dtype, device=device)
                            if self_interaction == "linear" else None)
        self._score_scale = 1.0 / math.sqrt(field_type_attn.dimension)

    def forward(self, x: SO2FeatureField, edges) -> SO2FeatureField:
        edges = _resolve_edges(edges, self.cutoff)
        _validate_node_field(x, self.field_type_in, edges)
        with torch.profiler.record_function("gm::attention/attend"):
            attended = self._attend(x, edges)
        return self._finish(x, attended)

    def _attend(self, x: SO2FeatureField, edges, products=None, groups=None) -> dict[int, Tensor]:
        q, k = self.query(x), self.key(x)
        if fused_attention.softmax_head_enabled(self, x, edges):
            alpha = fused_attention.softmax_head(self, q._rows(), k._rows(), edges)
        else:  # the reference's eager weights (attention.py:263-268)
            alpha = fused_attention.softmax_eager(fused_attention.plan_head(self), q._rows(), k._rows(), edges,
                                                  self.cutoff, self.window, self._score_scale).reshape(-1)
        if not kernels.factored_enabled():  # the per-edge readout through the fused pair terms
            messages = self.value(gather_to_edges(x, edges.source_index), edges)
            return weighted_segment_sum(alpha, messages.coefficients, edges.row_ptr)
        return self.value.forward_factored_aggregated(x, edges, alpha, products, groups).coefficients

    def forward_chunked(self, x: SO2FeatureField, edges, *, chunk_size: int) -> SO2FeatureField:
        """:meth:`forward` over consecutive ranges of at most ``chunk_size``
        targets with their whole neighbourhoods (reference :344-402), the node
        mixes formed once for every range; under training each range is
        recomputed in the backward rather than kept."""
        edges = _resolve_edges(edges, self.cutoff)
        _validate_node_field(x, self.field_type_in, edges)
        products = self.value.node_products(x) if kernels.factored_enabled() else None
        partials = [_checkpointed(self, functools.partial(self._attend, x, chunk, products,
                                                          fused_factored.groups_for(chunk, chunk.source_index)))
                    for chunk in edges.chunks(chunk_size)]
        return self._finish(x, sum_partials(partials) if partials else self._attend(x, edges))

    def _finish(self, x: SO2FeatureField, outputs: dict[int, Tensor]) -> SO2FeatureField:
        attended = SO2FeatureField(self.field_type_out, outputs)
        if self.self_linear is None:
            return attended
        pointwise = self.self_linear(x)
        return SO2FeatureField(self.field_type_out, {f: attended[f] + pointwise[f] for f in self.field_type_out.frequencies})


class SO2MHSA(nn.Module):
    def __init__(self, field_type_in: SO2FieldType, num_heads: int, *, cutoff: float, window: str = "hard",
                 n_radial_basis: int = 8, radial_hidden_features: Sequence[int] = (16,), radial_basis: str = "gaussian",
                 bias: bool = True, batched: bool = False, value_kind: str = "steerable", dtype=None,
                 device=None) -> None:
        super().__init__()
        if num_heads < 1:
            raise ValueError(f"num_heads must be at least 1, got {num_heads}.")
        offending = {f: m for f, m in field_type_in.items() if m % num_heads != 0}
        if offending:
            raise ValueError(f"num_heads ({num_heads}) must divide the multiplicity of every present frequency; "
                             f"offending frequencies (as frequency: multiplicity): {offending}.")
        self.batched = bool(batched)
        self.value_kind = value_kind
        self.field_type_in = field_type_in
        self.num_heads = num_heads
        self.cutoff = float(cutoff)
        self.field_type_attn = SO2FieldType({f: m // num_heads for f, m in field_type_in.items()})
        self.heads = nn.ModuleList([
            SO2Attention(field_type_in, self.field_type_attn, self.field_type_attn, cutoff=cutoff, window=window,
                         n_radial_basis=n_radial_basis, radial_hidden_features=radial_hidden_features,
                         radial_basis=radial_basis, bias=bias, value_kind=value_kind, dtype=dtype, device=device)
            for _ in range(num_heads)])
        self.output_projection = SO2Linear(field_type_in, field_type_in, bias=bias, dtype=dtype, device=device)

    def forward(self, x: SO2FeatureField, edges) -> SO2FeatureField:
        edges = _resolve_edges(edges, self.cutoff)
        if self.batched:
            _validate_node_field(x, self.field_type_in, edges)
            rows = _attend_batched_flat(self, x, edges)
            if rows is not None:
                return SO2FeatureField.from_flat(self.field_type_in, rows)
            return self.output_projection(SO2FeatureField(self.field_type_in, _attend_batched(self, x, edges)))
        fused = _concatenate_heads([head(x, edges) for head in self.heads], self.field_type_in)
        return self.output_projection(fused)

    def forward_chunked(self, x: SO2FeatureField, edges, *, chunk_size: int) -> SO2FeatureField:
        edges = _resolve_edges(edges, self.cutoff)
        outs = [cast(SO2Attention, h).forward_chunked(x, edges, chunk_size=chunk_size) for h in self.heads]
        return self.output_projection(_concatenate_heads(outs, self.field_type_in))


def _stacked_projection(linears: Sequence[SO2Linear], x: SO2FeatureField) -> SO2FeatureField:
    """The heads' intertwiners as one map onto their direct sum, head-major (:653-669)."""
    weights = {str(f): torch.cat([lin.weight[str(f)] for lin in linears], dim=0) for f in x.field_type.frequencies}
    bias = torch.cat([lin.bias for lin in linears]) if linears[0].has_bias else None
    return apply_linear(x.field_type, x.field_type.frequencies, weights, bias, x)


def _stacked_flat(linears: Sequence[SO2Linear], field_type_out: SO2FieldType, rows: Tensor) -> Tensor:
    """``_stacked_projection`` on flat rows: the heads' stacked intertwiner as one
    ``(D_in, D_out)`` block matrix, one GEMM onto the direct sum's flat layout."""
    lin = linears[0]
    weights = {str(f): torch.cat([h.weight[str(f)] for h in linears], dim=0) for f in lin.common_frequencies}
    bias = torch.cat([h.bias for h in linears]) if lin.has_bias else None
    m = weights_matrix(lin.field_type_in, field_type_out, lin.common_frequencies, weights)
    return FlatLinear.apply(rows, m, flat_bias(bias, field_type_out))


def _heads_permutation(mhsa: SO2MHSA, device: torch.device) -> Tensor:
    """For column ``head * d + c`` of the heads' outputs ``(N, H, d)`` (each in the
    per-head flat layout), its column in the direct sum's flat layout."""
    key = ("_heads_permutation", str(device))
    perm = mhsa.__dict__.get(key)
    if perm is None:
        attn, full = mhsa.field_type_attn, mhsa.field_type_in
        sa, sf = attn.slices(), full.slices()
        cols = []
        for head in range(mhsa.num_heads):
            for f, a in attn.items():
                dim = 1 if f == 0 else 2
                for c in range(sa[f].stop - sa[f].start):
                    cols.append(sf[f].start + (head * a + c // dim) * dim + c % dim)
        perm = torch.tensor(cols, dtype=torch.long, device=device)
        mhsa.__dict__[key] = perm
    return perm


def batched_flat_serves(mhsa: SO2MHSA, x: SO2FeatureField, edges) -> bool:
    """Whether :func:`_attend_batched_flat` serves ``x`` (bfloat16 rows are
    served only there: the scores read them in place of float32 rows, the
    node mixes read them, everything after runs in float32)."""
    if not mhsa.batched or x._rows().ndim != 2:
        return False
    edges = _resolve_edges(edges, mhsa.cutoff)
    values = [cast(SO2SteerableKernel, head.value) for head in mhsa.heads]
    return (fused_attention.softmax_enabled(mhsa, x, edges) and kernels.factored_enabled()
            and fused_factored.enabled(values[0], x, edges))


def _attend_batched_flat(mhsa: SO2MHSA, x: SO2FeatureField, edges) -> Tensor | None:
    """The batched layer on flat rows when the fused softmax and the fused
    factored heads serve it (else None): the stacked query and key
    projections as one GEMM each, and the output projection reading the heads'
    ``(N, H, d)`` outputs directly through its block matrix with the rows put
    in the heads' column order -- no per-frequency splits or concatenations."""
    heads = [cast(SO2Attention, h) for h in mhsa.heads]
    values = [cast(SO2SteerableKernel, head.value) for head in heads]
    if (not fused_attention.softmax_enabled(mhsa, x, edges) or not kernels.factored_enabled()
            or not fused_factored.enabled(values[0], x, edges)):
        return None
    rows = x._rows()
    if rows.ndim != 2:
        return None
    with torch.profiler.record_function("gm::attention/attend"):
        queries = _stacked_flat([h.query for h in heads], mhsa.field_type_in, rows)
        keys = _stacked_flat([h.key for h in heads], mhsa.field_type_in, rows)
        alpha = fused_attention.softmax(mhsa, queries, keys, edges)  # (n_edges, n_heads)
        groups = fused_factored.groups_for(edges, edges.source_index)
        compute = torch.float32 if x.dtype == torch.bfloat16 else x.dtype
        if radial.eligible(values, compute, x.device):
            h, trunk = None, functools.partial(radial.trunk_hidden_heads, values)
        else:
            h, trunk = torch.stack([k._trunk_hidden(edges.distances) for k in values]), None
        out = fused_factored.forward_aggregated_heads(values, x, edges, alpha, h, groups, trunk)  # (N, H, d)
    proj = mhsa.output_projection
    m = block_matrix(proj).index_select(0, _heads_permutation(mhsa, rows.device))
    return FlatLinear.apply(out.reshape(out.shape[0], -1), m,
                            flat_bias(proj.bias if proj.has_bias else None, proj.field_type_out))


def _attend_batched(mhsa: SO2MHSA, x: SO2FeatureField, edges) -> dict[int, Tensor]:
    heads = [cast(SO2Attention, h) for h in mhsa.heads]
    with torch.profiler.record_function("gm::attention/attend"):
        queries = _stacked_projection([h.query for h in heads], x)
        keys = _stacked_projection([h.key for h in heads], x)
        if fused_attention.softmax_enabled(mhsa, x, edges):
            alpha = fused_attention.softmax(mhsa, queries._rows(), keys._rows(), edges)  # (n_edges, n_heads)
        else:  # the reference's eager weights (attention.py:880-886)
            alpha = fused_attention.softmax_eager(fused_attention.plan(mhsa), queries._rows(), keys._rows(), edges,
                                                  mhsa.cutoff, heads[0].window, heads[0]._score_scale)
        return _aggregated_factored(mhsa, x, edges, alpha)


def _aggregated_factored(mhsa: SO2MHSA, x: SO2FeatureField, edges, alpha: Tensor) -> dict[int, Tensor]:
    """Every head's value kernel, factored and aggregated under its attention
    weights, with one source grouping for all heads (:801-822).

    All heads go through one pass (``fused_factored.forward_aggregated_heads``):
    the trunk features of every head from one HIP trunk pass (or the heads'
    own trunks when that kernel does not serve them), every head's node
    mixes from one matrix product per input frequency, then the fused factored
    op per head on those mixes in place."""
    if not kernels.factored_enabled():  # per-edge readouts through the fused pair terms, head by head
        source = gather_to_edges(x, edges.source_index)
        fields = []
        for head, weights in zip(mhsa.heads, alpha.unbind(1), strict=True):
            messages = cast(SO2SteerableKernel, head.value)(source, edges)
            fields.append(SO2FeatureField(mhsa.field_type_attn,
                                          weighted_segment_sum(weights, messages.coefficients, edges.row_ptr)))
        return _concatenate_heads(fields, mhsa.field_type_in).coefficients
    groups = fused_factored.groups_for(edges, edges.source_index)
    values = [cast(SO2SteerableKernel, head.value) for head in mhsa.heads]
    if fused_factored.enabled(values[0], x, edges):
        if radial.eligible(values, x.dtype, x.device):
            h, trunk = None, functools.partial(radial.trunk_hidden_heads, values)
        else:
            h, trunk = torch.stack([k._trunk_hidden(edges.distances) for k in values]), None
        out = fused_factored.forward_aggregated_heads(values, x, edges, alpha, h, groups, trunk)  # (N, H, d_out)
        attn = mhsa.field_type_attn
        return _concatenate_heads([SO2FeatureField.from_flat(attn, o) for o in out.unbind(1)],
                                  mhsa.field_type_in).coefficients
    fields = []
    for head, weights in zip(mhsa.heads, alpha.unbind(1), strict=True):
        kernel = cast(SO2SteerableKernel, head.value)
        fields.append(kernel.forward_factored_aggregated(x, edges, weights.contiguous(), kernel.node_products(x),
                                                         groups))
    return _concatenate_heads(fields, mhsa.field_type_in).coefficients
