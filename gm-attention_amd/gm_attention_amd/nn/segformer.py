"""The gauge-equivariant SegFormer's encoder stages and fusion decoder: the C5
workload (restrictions onto coarser grids, attention + Mix-FFN blocks on each
level, per-point class logits back on the input grid).

Stands for the reference's ``experiments/stanford_2d3ds/model.py``:

* ``GmSegformerBlock`` (:163-237): pre-norm ``x + Drop(MHSA(LN x))`` then the
  Mix-FFN ``x + Drop(W_out sigma(DWConv(W_in LN x)))`` with a depthwise
  steerable convolution as the mix;
* ``GmSegformer`` (:240-899) restricted to the options the benchmark's
  encoder stage uses: per stage a learned restriction (``EquiEncode`` over the
  hierarchy's ``down_edges``) with its layer norm, the stage's blocks and a
  closing layer norm; per stage a steerable-convolution readout onto scalars;
  the ``"fusion"`` decoder (a linear map of the coarsest readout, then at each
  finer stage the carried channels interpolated over ``lateral_edges``,
  joined with that stage's readout and mapped back through a GELU), the
  final interpolation onto the input grid over ``up_edges[0]`` and the
  ``1x1`` intertwiner head.  The dataset-specific options of the reference
  (gravity and vertical conditioning, the stem, the MLP head) are not built;
* ``IcoLowPassRestriction`` (reference nn/blocks.py:508-600) as
  :class:`LowPassRestriction`: the fixed normalised window-and-quadrature
  average the decoder interpolates with (scalar channels: no transport).

Every operator is this package's: the attention, the convolutions and the
restrictions run on the HIP kernels.
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from dataclasses import dataclass

import torch
from torch import Tensor, nn

from gm_attention_amd.discretization.grid import build_equiangular_grid
from gm_attention_amd.discretization.hierarchy import TensorGridHierarchy, build_grid_hierarchy
from gm_attention_amd.nn.attention import SO2MHSA
from gm_attention_amd.nn.blocks import EquiEncode, build_nonlinearity
from gm_attention_amd.nn.convolution import SO2Convolution
from gm_attention_amd.nn.eager_ops import segment_sum
from gm_attention_amd.nn.fused_attention import evaluate_aggregation_window
from gm_attention_amd.nn.linear import SO2Linear
from gm_attention_amd.nn.normalization import SO2LayerNorm
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType


def _add(a: SO2FeatureField, b: SO2FeatureField) -> SO2FeatureField:
    return SO2FeatureField(a.field_type, {f: a[f] + b[f] for f in a.field_type.frequencies})


class SO2DropPath(nn.Module):
    """A residual branch dropped whole with probability ``p`` in training and
    rescaled by ``1 / (1 - p)`` when kept (reference nn/stochastic_depth.py:49);
    the identity at ``p = 0`` and in evaluation."""

    def __init__(self, p: float = 0.0) -> None:
        super().__init__()
        if not 0.0 <= p < 1.0:
            raise ValueError(f"p must satisfy 0 <= p < 1, got {p}.")
        self.p = float(p)

    def forward(self, x: SO2FeatureField) -> SO2FeatureField:
        if not self.training or self.p == 0.0:
            return x
        first = next(iter(x.coefficients.values()))
        scale = (torch.rand((), device=first.device) >= self.p).to(first.dtype) / (1.0 - self.p)
        return SO2FeatureField(x.field_type, {f: t * scale for f, t in x.coefficients.items()})


class GmSegformerBlock(nn.Module):
    """One attention + Mix-FFN pair of a stage (reference model.py:163-237)."""

    def __init__(self, field_type: SO2FieldType, num_heads: int, *, attention_cutoff: float, mix_cutoff: float,
                 window: str = "hard", nonlinearity: str = "scalar_gate_double_sigmoid", drop_path: float = 0.0,
                 n_radial_basis: int = 8, radial_hidden_features: Sequence[int] = (16,),
                 radial_basis: str = "gaussian", bias: bool = True, attention_batched: bool = True,
                 value_kind: str = "steerable", ffn_expansion: int = 1, eps: float = 1e-5,
                 normalized_mix: bool = False, dtype=None, device=None) -> None:
        super().__init__()
        if ffn_expansion < 1:
            raise ValueError(f"ffn_expansion must be at least 1, got {ffn_expansion}.")
        kw = dict(dtype=dtype, device=device)
        radial = dict(n_radial_basis=n_radial_basis, radial_hidden_features=radial_hidden_features,
                      radial_basis=radial_basis, bias=bias)
        self.field_type = field_type
        self.hidden_field_type = field_type.scaled(int(ffn_expansion))
        self.norm1 = SO2LayerNorm(field_type, eps=eps, bias=bias, **kw)
        self.attention = SO2MHSA(field_type, num_heads, cutoff=attention_cutoff, window=window,
                                 batched=attention_batched, value_kind=value_kind, **radial, **kw)
        self.drop_path1 = SO2DropPath(drop_path)
        self.norm2 = SO2LayerNorm(field_type, eps=eps, bias=bias, **kw)
        self.linear_in = SO2Linear(field_type, self.hidden_field_type, bias=bias, **kw)
        self.mix = SO2Convolution(self.hidden_field_type, self.hidden_field_type, cutoff=mix_cutoff, window=window,
                                  self_interaction="none", depthwise=True, normalize=normalized_mix, **radial, **kw)
        self.activation = build_nonlinearity(nonlinearity, self.hidden_field_type, **kw)
        self.linear_out = SO2Linear(self.hidden_field_type, field_type, bias=bias, **kw)
        self.drop_path2 = SO2DropPath(drop_path)

    def forward(self, x: SO2FeatureField, discretization) -> SO2FeatureField:
        x = _add(x, self.drop_path1(self.attention(self.norm1(x), discretization)))
        hidden = self.mix(self.linear_in(self.norm2(x)), discretization)
        return _add(x, self.drop_path2(self.linear_out(self.activation(hidden))))


def _transpose(edges, n_sources: int) -> tuple[Tensor, Tensor, Tensor]:
    """``(src_ptr, order, target[order])``: the edges grouped by source (stably),
    cached on the edge set."""
    key = ("_low_pass_transpose", n_sources)
    hit = edges.__dict__.get(key)
    if hit is None:
        source = edges.source_index
        order = torch.argsort(source, stable=True)
        src_ptr = torch.zeros(n_sources + 1, dtype=torch.int64, device=source.device)
        torch.cumsum(torch.bincount(source, minlength=n_sources), dim=0, out=src_ptr[1:])
        hit = (src_ptr, order.contiguous(), edges.target_index.index_select(0, order).contiguous())
        edges.__dict__[key] = hit
    return hit


class _LowPass(torch.autograd.Function):
    """``out_i = sum_e w_e x[source_e]`` over target i's edges with fixed
    weights, both directions on the HIP gather-aggregate kernel: the forward
    walks the targets' CSR, the backward the sources' (no atomics)."""

    @staticmethod
    def forward(ctx, x: Tensor, w: Tensor, edges, n_sources: int) -> Tensor:
        from gm_attention_amd import _native

        ctx.edges, ctx.n_sources = edges, n_sources
        ctx.save_for_backward(w)
        return _native.aggregate_gather(x.contiguous(), edges.source_index.contiguous(), w, edges.row_ptr.contiguous())

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad: Tensor):
        from gm_attention_amd import _native

        (w,) = ctx.saved_tensors
        src_ptr, order, target = _transpose(ctx.edges, ctx.n_sources)
        dx = _native.aggregate_gather(grad.contiguous(), target, w.index_select(0, order).contiguous(), src_ptr)
        return dx, None, None, None


class LowPassRestriction(nn.Module):
    """``(R f)_i = sum_j c(r_ij) q_ij f_j / max(sum_j c(r_ij) q_ij, eps)`` over
    bipartite edges (reference nn/blocks.py:508-600 ``IcoLowPassRestriction``),
    for scalar fields, where the transport acts trivially; no parameters.
    Float32 fields on the GPU take the HIP gather-aggregate kernels (the
    normalised weights formed once per call), others torch's segment sums."""

    def __init__(self, field_type: SO2FieldType, *, cutoff: float, window: str = "quartic", eps: float = 1e-12) -> None:
        super().__init__()
        if window not in ("hard", "quartic"):
            raise ValueError(f"window must be 'hard' or 'quartic', got {window!r}.")
        if set(field_type.frequencies) != {0}:
            raise ValueError(f"this restriction serves scalar fields, got {field_type!r}.")
        self.field_type = field_type
        self.cutoff = float(cutoff)
        self.window = window
        self.eps = float(eps)

    def forward(self, x: SO2FeatureField, edges) -> SO2FeatureField:
        if x.field_type != self.field_type:
            raise ValueError(f"Expected a field of type {self.field_type!r}, got {x.field_type!r}.")
        x0 = x[0]
        weight = (evaluate_aggregation_window(edges.distances, self.cutoff, self.window)
                  * edges.tangent_quadrature_weights).to(x0.dtype)
        mass = segment_sum(weight, edges.row_ptr).clamp_min(self.eps)
        if x0.is_cuda and x0.dtype == torch.float32 and x0.shape[1] <= 128:
            w = (weight / mass.index_select(0, edges.target_index)).contiguous()
            return SO2FeatureField(self.field_type, {0: _LowPass.apply(x0, w, edges, x0.shape[0])})
        summed = segment_sum(weight.unsqueeze(-1) * x0.index_select(0, edges.source_index), edges.row_ptr)
        return SO2FeatureField(self.field_type, {0: summed / mass.unsqueeze(-1)})


class GmSegformer(nn.Module):
    """Encoder stages and the fusion decoder (reference model.py:240-899, the
    benchmark's options; see the module docstring).  ``forward(x, hierarchy)``
    takes ``{0: in_channels}`` on the hierarchy's finest level, whose levels
    1.. carry the stages' discretizations (prepared for the attention, mix and
    readout radii) and whose ``lateral_edges`` / ``up_edges[0]`` carry the
    decoder's interpolations; out ``{0: num_classes}`` on the finest level."""

    def __init__(self, *, in_channels: int, num_classes: int, stage_field_types: Sequence[SO2FieldType],
                 heads: Sequence[int], depths: Sequence[int], merge_cutoffs: Sequence[float],
                 attention_cutoffs: Sequence[float], mix_cutoffs: Sequence[float],
                 interpolate_cutoffs: Sequence[float], readout_cutoffs: Sequence[float],
                 readout_channels: Sequence[int], window: str = "hard",
                 nonlinearity: str = "scalar_gate_double_sigmoid", drop_path_rate: float = 0.0,
                 attention_batched: bool = True, ffn_expansion: int = 1, normalized_mix: bool = False,
                 normalized_readout: bool = False, decoder_channels: int = 32, n_radial_basis: int = 8,
                 radial_hidden_features: Sequence[int] = (16,), bias: bool = True, eps: float = 1e-5, dtype=None,
                 device=None) -> None:
        super().__init__()
        stages = len(stage_field_types)
        per_stage = dict(heads=heads, depths=depths, merge_cutoffs=merge_cutoffs, attention_cutoffs=attention_cutoffs,
                         mix_cutoffs=mix_cutoffs, interpolate_cutoffs=interpolate_cutoffs,
                         readout_cutoffs=readout_cutoffs, readout_channels=readout_channels)
        wrong = [f"{k} ({len(v)})" for k, v in per_stage.items() if len(v) != stages]
        if stages < 1 or wrong:
            raise ValueError(f"one entry per stage ({stages}) needed: " + ", ".join(wrong))
        if not 0.0 <= drop_path_rate < 1.0:
            raise ValueError(f"drop_path_rate must satisfy 0 <= p < 1, got {drop_path_rate}.")
        kw = dict(dtype=dtype, device=device)
        radial = dict(n_radial_basis=n_radial_basis, radial_hidden_features=radial_hidden_features, bias=bias)
        self.input_field_type = SO2FieldType({0: int(in_channels)})
        self.output_field_type = SO2FieldType({0: int(num_classes)})
        self.stage_field_types = tuple(stage_field_types)
        rates = torch.linspace(0.0, drop_path_rate, sum(depths)).tolist()
        self.merges, self.merge_norms, self.stages, self.stage_norms = (nn.ModuleList() for _ in range(4))
        previous, block_index = self.input_field_type, 0
        for i, ft in enumerate(self.stage_field_types):
            self.merges.append(EquiEncode(previous, ft, cutoff=merge_cutoffs[i], window=window, **radial, **kw))
            self.merge_norms.append(SO2LayerNorm(ft, eps=eps, bias=bias, **kw))
            blocks = []
            for _ in range(depths[i]):
                blocks.append(GmSegformerBlock(ft, heads[i], attention_cutoff=attention_cutoffs[i],
                                               mix_cutoff=mix_cutoffs[i], window=window, nonlinearity=nonlinearity,
                                               drop_path=rates[block_index], attention_batched=attention_batched,
                                               ffn_expansion=ffn_expansion, eps=eps, normalized_mix=normalized_mix,
                                               **radial, **kw))
                block_index += 1
            self.stages.append(nn.ModuleList(blocks))
            self.stage_norms.append(SO2LayerNorm(ft, eps=eps, bias=bias, **kw))
            previous = ft
        self.readouts = nn.ModuleList(
            SO2Convolution(ft, SO2FieldType({0: int(c)}), cutoff=readout_cutoffs[i], window=window,
                           self_interaction="linear", normalize=normalized_readout, **radial, **kw)
            for i, (ft, c) in enumerate(zip(self.stage_field_types, readout_channels, strict=True)))
        width = int(decoder_channels)
        self.fused_field_type = SO2FieldType({0: width})
        self.fusion_in = nn.Linear(int(readout_channels[-1]), width, **kw)
        finer = list(range(stages - 2, -1, -1))  # the stages the decoder walks back through
        self.fusions = nn.ModuleList(nn.Linear(int(readout_channels[k]) + width, width, **kw) for k in finer)
        self.lateral_interpolations = nn.ModuleList(
            LowPassRestriction(self.fused_field_type, cutoff=interpolate_cutoffs[k + 1]) for k in finer)
        self.final_interpolation = LowPassRestriction(self.fused_field_type, cutoff=interpolate_cutoffs[0])
        self.head = SO2Linear(self.fused_field_type, self.output_field_type, bias=bias, **kw)

    @property
    def num_stages(self) -> int:
        return len(self.stage_field_types)

    def encode(self, x: SO2FeatureField, hierarchy) -> list[SO2FeatureField]:
        """Every stage's features on its own level, finest stage first (reference :728-764)."""
        if hierarchy.depth != self.num_stages:
            raise ValueError(f"the hierarchy has {hierarchy.depth} hops, the model {self.num_stages} stages.")
        features, feature = [], x
        for i in range(self.num_stages):
            level = hierarchy.levels[i + 1]
            if level.discretization is None:
                raise ValueError(f"hierarchy level {i + 1} has no same-grid discretization for the stage's blocks.")
            feature = self.merge_norms[i](self.merges[i](feature, hierarchy.down_edges[i]))
            for block in self.stages[i]:
                feature = block(feature, level.discretization)
            feature = self.stage_norms[i](feature)
            features.append(feature)
        return features

    def decode(self, features: Sequence[SO2FeatureField], hierarchy) -> SO2FeatureField:
        """Readouts, top-down fusion, the final interpolation and the head (reference :823-880)."""
        if len(hierarchy.lateral_edges) != self.num_stages - 1:
            raise ValueError(f"the fusion decoder needs {self.num_stages - 1} lateral edge sets, the hierarchy has "
                             f"{len(hierarchy.lateral_edges)}.")
        readouts = [self.readouts[i](f, hierarchy.levels[i + 1].discretization)[0] for i, f in enumerate(features)]
        gelu = nn.functional.gelu
        fused: Tensor = gelu(self.fusion_in(readouts[-1]))
        for j, k in enumerate(range(self.num_stages - 2, -1, -1)):
            up = self.lateral_interpolations[j](SO2FeatureField(self.fused_field_type, {0: fused}),
                                                hierarchy.lateral_edges[k])[0]
            fused = gelu(self.fusions[j](torch.cat([readouts[k], up], dim=-1)))
        fine = self.final_interpolation(SO2FeatureField(self.fused_field_type, {0: fused}), hierarchy.up_edges[0])
        return self.head(fine)

    def forward(self, x: SO2FeatureField, hierarchy) -> SO2FeatureField:
        if x.field_type != self.input_field_type:
            raise ValueError(f"Expected an input of type {self.input_field_type!r}, got {x.field_type!r}.")
        return self.decode(self.encode(x, hierarchy), hierarchy)


@dataclass(frozen=True)
class StageRadii:
    """One radius per stage for each cross-node operator (reference
    experiments/stanford_2d3ds/geometry.py:110-127 ``SegformerRadii``): the
    restriction onto the stage, its attention, its depthwise mix, the
    interpolation out of the stage and its readout convolution."""

    merge: tuple[float, ...]
    attention: tuple[float, ...]
    mix: tuple[float, ...]
    interpolate: tuple[float, ...]
    readout: tuple[float, ...]


def stage_radii(stage_shapes: Sequence[tuple[int, int]], *, merge_rows: float = 2.0, attention_rows: float = 3.0,
                mix_rows: float = 2.0, interpolate_rows: float = 1.5, readout_rows: float = 1.5) -> StageRadii:
    """Every radius as a multiple of its stage grid's row spacing ``pi / (nlat - 1)``
    (the equiangular grids carry rows at both poles)."""
    rows = dict(merge=merge_rows, attention=attention_rows, mix=mix_rows, interpolate=interpolate_rows,
                readout=readout_rows)
    bad = {k: v for k, v in rows.items() if not v > 0}
    if bad:
        raise ValueError(f"every radius must be positive, got {bad}.")
    spacing = [math.pi / (nlat - 1) for nlat, _ in stage_shapes]
    return StageRadii(**{k: tuple(v * h for h in spacing) for k, v in rows.items()})


def build_stage_hierarchy(img_size: tuple[int, int], stage_shapes: Sequence[tuple[int, int]], radii: StageRadii, *,
                          device=None) -> TensorGridHierarchy:
    """The equiangular chain ``img_size -> stage 1 -> ...`` with the transfers
    and same-grid neighbourhoods a :class:`GmSegformer` reads (reference
    geometry.py:169-232 ``build_segformer_hierarchy`` with ``lateral=True``):
    each stage level prepared for its attention, mix and readout radii, the
    restrictions at the merge radii, the interpolations back to the input
    grid and the top-down lateral transfers at the interpolation radii."""
    shapes = [tuple(img_size), *[tuple(s) for s in stage_shapes]]
    grids = [build_equiangular_grid(nlat, nlon, device=device) for nlat, nlon in shapes]
    local = [None] + [[a, m, r] for a, m, r in zip(radii.attention, radii.mix, radii.readout, strict=True)]
    return build_grid_hierarchy(grids, ["equiangular"] * len(shapes), shapes, restrict_cutoffs=list(radii.merge),
                                interpolate_cutoffs=list(radii.interpolate), local_cutoffs=local,
                                lateral_cutoffs=list(radii.interpolate[1:]))
