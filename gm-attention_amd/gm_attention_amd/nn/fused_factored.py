"""The factored steerable kernel as one fused op per direction (HIP).

The drop-in for the reference's ``gm_attention/nn/fused_factored.py``: the
switch ``GM_FUSED_FACTORED`` (read at import), the block plan and its int32
descriptors (:81-139), the packing of ``node_products`` into ``zc``/``zr``
(:145-180), the cached source grouping (:183-227), the eligibility predicate
(:230-244), the autograd Functions ``Factored`` (:247-270) and
``FactoredAggregate`` (:273-299) with the same signatures, and the per-call
``inputs`` / ``forward`` / ``forward_aggregated`` (:302-376).  The arithmetic
runs in ``libgmhip.so`` (``_native.factored()``).

Semantics kept exactly: one descriptor row per coefficient block
``(kind, z_offset, b_m, angular, transport, power, out_offset, take_real)``,
the blocks stably sorted by output offset and the complex blocks' mixes packed
in that order; angular and transport orders ``(m, 0)`` for ``0 -> m``,
``(n, -n)`` for ``n -> 0`` (real part), ``(m - n, n)`` linear,
``(m + n, -n)`` antilinear; power ``|m - n|`` linear, ``m + n`` antilinear.

This build defaults the switch to ``"1"``: the layers here implement only
the fused path, so ``"0"`` makes them raise rather than silently run torch.
"""

from __future__ import annotations

import os
import weakref
from collections import OrderedDict
from dataclasses import dataclass
from typing import Any

import torch
from torch import Tensor

from gm_attention_amd import _native
from gm_attention_amd.representations.field_type import SO2FeatureField

MAX_K, MAX_OUT, MAX_BM, MAX_C, DESC = 20, 128, 32, 320, 8
MODE = os.environ.get("GM_FUSED_FACTORED", "1")


def extension(cuda: bool = True) -> Any:
    """The native module: ``forward``, ``aggregate``, ``backward``, ``backward_aggregated``."""
    return _native.factored()


@dataclass(frozen=True)
class Block:
    block: tuple[int, int, str]
    kind: int
    z_offset: int
    b_m: int
    angular: int
    transport: int
    power: int
    out_offset: int
    take_real: int

    def row(self) -> list[int]:
        return [self.kind, self.z_offset, self.b_m, self.angular, self.transport, self.power, self.out_offset,
                self.take_real]


@dataclass(frozen=True)
class Plan:
    blocks: tuple[Block, ...]
    wc: int
    wr: int
    d_out: int
    max_bm: int


def _orders(n: int, m: int, role: str) -> tuple[int, int]:
    """The block's (angular, transport) harmonic orders."""
    if n == 0:
        return m, 0
    if m == 0:
        return n, -n
    if role == "linear":
        return m - n, n
    return m + n, -n


def plan(kernel: Any) -> Plan:
    """The kernel's blocks as descriptor rows, grouped by output frequency,
    the complex blocks' mixes packed in that order (cached on the kernel)."""
    cached = kernel.__dict__.get("_fused_factored_plan")
    if cached is not None:
        return cached
    out_type = kernel.field_type_out
    slices = out_type.slices()
    ordered = sorted(kernel._blocks(), key=lambda blk: slices[blk[1]].start)  # stable
    blocks: list[Block] = []
    wc = wr = 0
    for n, m, role in ordered:
        b_m = out_type.multiplicity(m)
        if role == "real":
            blocks.append(Block((n, m, role), 0, 0, b_m, 0, 0, 0, slices[0].start, 0))
            wr = b_m
            continue
        angular, transport = _orders(n, m, role)
        blocks.append(Block((n, m, role), 1, wc, b_m, angular, transport, int(kernel._pair_powers[(n, m, role)]),
                            slices[m].start, int(m == 0)))
        wc += b_m
    result = Plan(tuple(blocks), wc, wr, out_type.dimension, max((b.b_m for b in blocks), default=1))
    kernel.__dict__["_fused_factored_plan"] = result
    return result


def descriptors(kernel: Any, device: torch.device) -> Tensor:
    """The plan as an int32 ``(n_blocks, 8)`` tensor, cached per device."""
    cache = kernel.__dict__.setdefault("_fused_factored_descriptors", {})
    key = str(device)
    if key not in cache:
        cache[key] = torch.tensor([b.row() for b in plan(kernel).blocks], dtype=torch.int32, device=device)
    return cache[key]


PACKED = "_packed"


def pack(kernel: Any, products: dict) -> tuple[Tensor, Tensor]:
    """``node_products`` as ``zc (n_nodes, K, wc, 2)`` and ``zr (n_nodes, K, wr)``,
    remembered on the dict under :data:`PACKED`."""
    packed = products.get(PACKED)
    if packed is not None:
        return packed
    with torch.profiler.record_function("gm::kernel/pack"):
        p = plan(kernel)
        first = next(v for key, v in products.items() if key != PACKED)
        n_nodes, k = first.shape[0], first.shape[1]
        real_dtype = first.real.dtype if first.is_complex() else first.dtype
        complex_blocks = [b.block for b in p.blocks if b.kind == 1]
        if complex_blocks:
            zc = torch.view_as_real(torch.cat([products[b] for b in complex_blocks], dim=-1).contiguous()).contiguous()
        else:
            zc = torch.zeros(n_nodes, k, 0, 2, dtype=real_dtype, device=first.device)
        real = [b.block for b in p.blocks if b.kind == 0]
        zr = products[real[0]].contiguous() if real else torch.zeros(n_nodes, k, 0, dtype=real_dtype,
                                                                    device=first.device)
        packed = (zc, zr)
    products[PACKED] = packed
    return packed


_GROUPS: OrderedDict[tuple, tuple[Any, tuple[Tensor, Tensor, Tensor]]] = OrderedDict()
GROUP_CACHE_SIZE = 512


def source_groups(source_index: Tensor, key: tuple | None = None,
                  owner: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """``(order, group_ptr, group_source)``: the edges stably sorted by source,
    each source's half-open run in that order, and the sources; cached under
    ``key`` (tied to ``owner`` while it lives) when given."""
    if key is not None:
        hit = _GROUPS.get(key)
        if hit is not None:
            held, groups = hit
            same = (owner is None) if held is None else (held() is not None and held() is owner)
            if same and groups[0].device == source_index.device:
                _GROUPS.move_to_end(key)
                return groups
    order = torch.argsort(source_index, stable=True)
    group_source, counts = torch.unique_consecutive(source_index[order], return_counts=True)
    group_ptr = torch.zeros(group_source.shape[0] + 1, dtype=torch.long, device=source_index.device)
    group_ptr[1:] = torch.cumsum(counts, dim=0)
    result = (order.contiguous(), group_ptr.contiguous(), group_source.contiguous())
    if key is not None:
        _GROUPS[key] = (None if owner is None else weakref.ref(owner), result)
        while len(_GROUPS) > GROUP_CACHE_SIZE:
            _GROUPS.popitem(last=False)
    return result


def group_key(parent: Any, first: int, last: int) -> tuple:
    return (id(parent), parent.edge_index.data_ptr(), int(parent.n_edges), int(first), int(last))


def groups_for(edges: Any, source: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """The cached source grouping of ``edges`` (of its registered parent range for a chunk)."""
    from gm_attention_amd.nn import fused_attention

    registered = fused_attention.chunk_of(edges)
    parent, first, last = registered if registered is not None else (edges, 0, int(edges.n_edges))
    return source_groups(source, group_key(parent, first, last), owner=parent.edge_index)


def declined(kernel: Any, x: SO2FeatureField, edges: Any) -> str:
    """Why :func:`enabled` is False (empty string when it is True)."""
    if MODE == "0":
        return "GM_FUSED_FACTORED=0: this build implements the factored kernel only through the fused HIP op"
    if x.device.type != "cuda":
        return "the fused factored op runs on the GPU only (this build has no CPU driver)"
    if x.dtype not in (torch.float32, torch.float64):
        return f"the fused factored op takes float32 or float64, got {x.dtype}"
    p = plan(kernel)
    trunk = kernel.complex_head.in_features if kernel.complex_head is not None else kernel.real_head.in_features
    if trunk + 1 > MAX_K or p.d_out > MAX_OUT or p.max_bm > MAX_BM or 2 * p.wc + p.wr > MAX_C:
        return "the kernel's widths exceed the fused op's bounds (K <= 20, d_out <= 128, b_m <= 32, 2wc + wr <= 320)"
    if edges.n_edges == 0:
        return "no edges"
    return ""


def enabled(kernel: Any, x: SO2FeatureField, edges: Any) -> bool:
    """Whether :meth:`SO2SteerableKernel.forward_factored` takes the fused op (reference :230-244)."""
    return declined(kernel, x, edges) == ""


class Factored(torch.autograd.Function):
    """The rows ``(n_edges, d_out)`` as one differentiable op on ``(h, zc, zr)``."""

    @staticmethod
    def forward(ctx: Any, h: Tensor, zc: Tensor, zr: Tensor, angular: Tensor, transport: Tensor, rho: Tensor,
                desc: Tensor, source: Tensor, order: Tensor, group_ptr: Tensor, group_source: Tensor, d_out: int,
                max_bm: int) -> Tensor:
        ext = extension(cuda=h.is_cuda)
        with torch.profiler.record_function("gm::kernel/pairs"):
            out = ext.forward(h, zc, zr, angular, transport, rho, desc, source, order, group_ptr, group_source, d_out,
                              max_bm)
        ctx.save_for_backward(h, zc, zr, angular, transport, rho, desc, source, order, group_ptr, group_source)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_out: Tensor) -> tuple:
        h, zc, zr, angular, transport, rho, desc, source, order, group_ptr, group_source = ctx.saved_tensors
        ext = extension(cuda=h.is_cuda)
        with torch.profiler.record_function("gm::kernel/pairs_backward"):
            dh, dzc, dzr = ext.backward(grad_out.contiguous(), h, zc, zr, angular, transport, rho, desc, source, order,
                                        group_ptr, group_source)
        return dh, dzc, dzr, None, None, None, None, None, None, None, None, None, None


class FactoredAggregate(torch.autograd.Function):
    """Each target's weighted sum of the rows as one op on ``(h, zc, zr, weights)``."""

    @staticmethod
    def forward(ctx: Any, h: Tensor, zc: Tensor, zr: Tensor, weights: Tensor, angular: Tensor, transport: Tensor,
                rho: Tensor, desc: Tensor, source: Tensor, target: Tensor, row_ptr: Tensor, order: Tensor,
                group_ptr: Tensor, group_source: Tensor, d_out: int, max_bm: int) -> Tensor:
        ext = extension(cuda=h.is_cuda)
        with torch.profiler.record_function("gm::kernel/pairs"):
            rows = ext.forward(h, zc, zr, angular, transport, rho, desc, source, order, group_ptr, group_source, d_out,
                               max_bm)
        with torch.profiler.record_function("gm::kernel/aggregate"):
            out = ext.aggregate(rows, weights, row_ptr)
        ctx.save_for_backward(h, zc, zr, weights, rows, angular, transport, rho, desc, source, target, order,
                              group_ptr, group_source)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_out: Tensor) -> tuple:
        (h, zc, zr, weights, rows, angular, transport, rho, desc, source, target, order, group_ptr,
         group_source) = ctx.saved_tensors
        ext = extension(cuda=h.is_cuda)
        with torch.profiler.record_function("gm::kernel/pairs_backward"):
            dh, dzc, dzr, dweights = ext.backward_aggregated(grad_out.contiguous(), target, weights, rows, h, zc, zr,
                                                             angular, transport, rho, desc, source, order, group_ptr,
                                                             group_source)
        return (dh, dzc, dzr, dweights, None, None, None, None, None, None, None, None, None, None, None, None)


@dataclass(frozen=True)
class Inputs:
    h: Tensor
    zc: Tensor
    zr: Tensor
    angular: Tensor
    transport: Tensor
    rho: Tensor
    desc: Tensor
    source: Tensor
    plan: Plan


def inputs(kernel: Any, x: SO2FeatureField, edges: Any, products: dict | None) -> Inputs:
    """One call's op inputs, the phase tables checked against the blocks' orders (reference :314-335)."""
    if products is None:
        products = kernel.node_products(x)
    h = kernel._trunk_hidden(edges.distances)
    zc, zr = pack(kernel, products)
    rho = (edges.distances / kernel.radial_basis.cutoff).to(h.dtype).contiguous()
    angular = torch.view_as_real(edges.angular_phases.contiguous()).contiguous().to(h.dtype)
    transport = torch.view_as_real(edges.transport_phases.contiguous()).contiguous().to(h.dtype)
    p = plan(kernel)
    needed = max((max(abs(b.angular), abs(b.transport)) for b in p.blocks), default=0)
    if needed >= angular.shape[1] or needed >= transport.shape[1]:
        raise ValueError(f"the geometry's phase tables ({angular.shape[1]} orders) are narrower than the kernel's "
                         f"blocks need (order {needed})")
    return Inputs(h.contiguous(), zc, zr, angular, transport, rho, descriptors(kernel, h.device),
                  edges.source_index.contiguous(), p)


def forward(kernel: Any, x: SO2FeatureField, edges: Any, products: dict | None = None,
            groups: tuple[Tensor, Tensor, Tensor] | None = None) -> SO2FeatureField:
    """The messages on the edges, ``(n_edges,)`` of the kernel's output type."""
    i = inputs(kernel, x, edges, products)
    order, group_ptr, group_source = groups_for(edges, i.source) if groups is None else groups
    flat = Factored.apply(i.h, i.zc, i.zr, i.angular, i.transport, i.rho, i.desc, i.source, order, group_ptr,
                          group_source, i.plan.d_out, i.plan.max_bm)
    return SO2FeatureField.from_flat(kernel.field_type_out, flat)


def forward_aggregated(kernel: Any, x: SO2FeatureField, edges: Any, weights: Tensor, products: dict | None = None,
                       groups: tuple[Tensor, Tensor, Tensor] | None = None) -> SO2FeatureField:
    """Each target's weighted sum of its messages, ``(n_targets,)`` of the output type."""
    i = inputs(kernel, x, edges, products)
    order, group_ptr, group_source = groups_for(edges, i.source) if groups is None else groups
    flat = FactoredAggregate.apply(i.h, i.zc, i.zr, weights.to(i.h.dtype).contiguous(), i.angular, i.transport, i.rho,
                                   i.desc, i.source, edges.target_index.contiguous(), edges.row_ptr.contiguous(),
                                   order, group_ptr, group_source, i.plan.d_out, i.plan.max_bm)
    return SO2FeatureField.from_flat(kernel.field_type_out, flat)
