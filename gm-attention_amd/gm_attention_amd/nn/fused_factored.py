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
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

MAX_K, MAX_OUT, MAX_BM, MAX_C, DESC = 20, 128, 32, 320, 8
MAX_C_MFMA = 128  # packed columns the float32 MFMA kernels take (K <= 17)
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
    if x.dtype not in (torch.float32, torch.float64, torch.bfloat16):
        return f"the fused factored op takes float32, float64 or bfloat16 rows, got {x.dtype}"
    trunk = kernel.complex_head.in_features if kernel.complex_head is not None else kernel.real_head.in_features
    if trunk + 1 > MAX_K:
        return "the kernel's trunk exceeds the fused op's bound (K <= 20)"
    if x.dtype == torch.bfloat16:
        widest = max((m if f == 0 else 2 * m) for f, m in kernel.field_type_in.items())
        if head_split(kernel, trunk + 1) == 0 or widest > 64:
            return ("bfloat16 rows take the grouped kernels only (float32 arithmetic, node vectors at most 64 "
                    "reals); this kernel does not fit them")
    if tiles(kernel) == ():
        return "an output copy's blocks exceed the fused op's bounds even one copy at a time"
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


# ---------------------------------------------------------------- output tiles of wide kernels


@dataclass(frozen=True)
class Tile:
    """A slice of a wide kernel's plan that fits the fused op: its descriptor
    rows (offsets local to the tile), the full plan's complex and real mix
    columns it reads, and the full output columns it writes, in tile order."""

    rows: tuple[tuple[int, ...], ...]
    zc_cols: tuple[int, ...]
    zr_cols: tuple[int, ...]
    out_cols: tuple[int, ...]
    d_out: int
    max_bm: int


def _piece(p: Plan, m: int, c0: int, c1: int, base: tuple[int, int, int], start: int) -> tuple[list, list, list, list]:
    """Output copies [c0, c1) of frequency m: every block writing them, cut to those copies."""
    out0, zc0, zr0 = base
    rows, zc_cols, zr_cols = [], [], []
    width = (c1 - c0) * (1 if m == 0 else 2)
    for b in p.blocks:
        if b.block[1] != m:
            continue
        if b.kind == 0:
            rows.append([0, zr0 + len(zr_cols), c1 - c0, 0, 0, 0, out0, 0])
            zr_cols += range(c0, c1)
        else:
            rows.append([1, zc0 + len(zc_cols), c1 - c0, b.angular, b.transport, b.power, out0, b.take_real])
            zc_cols += range(b.z_offset + c0, b.z_offset + c1)
    out_cols = list(range(start + c0, start + c1)) if m == 0 else list(range(start + 2 * c0, start + 2 * c1))
    assert len(out_cols) == width
    return rows, zc_cols, zr_cols, out_cols


def tiles(kernel: Any) -> tuple[Tile, ...] | None:
    """``None`` when the kernel's plan fits the fused op as is; else the plan
    cut into output tiles (each output frequency's copies in chunks of at most
    ``MAX_BM``, halved until one chunk's blocks fit, chunks packed greedily
    into tiles within ``MAX_OUT``, ``MAX_C`` and one real block); ``()`` when even single
    copies do not fit.  Blocks are separable by output copy, so the tiles'
    outputs side by side are the kernel's output."""
    cached = kernel.__dict__.get("_fused_factored_tiles", False)
    if cached is not False:
        return cached
    p = plan(kernel)
    result: tuple[Tile, ...] | None = None
    if p.d_out > MAX_OUT or p.max_bm > MAX_BM or 2 * p.wc + p.wr > MAX_C:
        out_type = kernel.field_type_out
        slices = out_type.slices()
        # float32 tiles stay within the MFMA kernels' packed width
        width = MAX_C_MFMA if next(kernel.parameters()).dtype == torch.float32 else MAX_C

        def fits(rows, zc_cols, zr_cols, out_cols) -> bool:
            # the op takes one real block, covering the tile's real mixes
            return (len(out_cols) <= MAX_OUT and 2 * len(zc_cols) + len(zr_cols) <= width
                    and sum(r[0] == 0 for r in rows) <= 1 and len(rows) <= 64)

        built: list[Tile] = []
        current: tuple[list, list, list, list] = ([], [], [], [])
        ok = True
        for m in out_type.frequencies:
            copies = out_type.multiplicity(m)
            chunk = MAX_BM
            while chunk > 1 and not fits(*_piece(p, m, 0, min(chunk, copies), (0, 0, 0), slices[m].start)):
                chunk //= 2
            if not fits(*_piece(p, m, 0, min(chunk, copies), (0, 0, 0), slices[m].start)):
                ok = False
                break
            for c0 in range(0, copies, chunk):
                c1 = min(copies, c0 + chunk)
                base = (len(current[3]), len(current[1]), len(current[2]))
                piece = _piece(p, m, c0, c1, base, slices[m].start)
                grown = tuple(a + b for a, b in zip(current, piece))
                if current[3] and not fits(*grown):
                    built.append(_tile(current))
                    piece = _piece(p, m, c0, c1, (0, 0, 0), slices[m].start)
                    grown = piece
                current = grown
        if ok and current[3]:
            built.append(_tile(current))
        result = tuple(built) if ok else ()
    kernel.__dict__["_fused_factored_tiles"] = result
    return result


def _tile(parts: tuple[list, list, list, list]) -> Tile:
    rows, zc_cols, zr_cols, out_cols = parts
    return Tile(tuple(tuple(r) for r in rows), tuple(zc_cols), tuple(zr_cols), tuple(out_cols), len(out_cols),
                max(r[2] for r in rows))


def _tile_tensors(kernel: Any, t: Tile, index: int, device: torch.device) -> tuple[Tensor, Tensor, Tensor]:
    cache = kernel.__dict__.setdefault("_fused_factored_tile_tensors", {})
    key = (index, str(device))
    if key not in cache:
        cache[key] = (torch.tensor(t.rows, dtype=torch.int32, device=device),
                      torch.tensor(t.zc_cols, dtype=torch.int64, device=device),
                      torch.tensor(t.zr_cols, dtype=torch.int64, device=device))
    return cache[key]


def _untile(kernel: Any, parts: list[Tensor], device: torch.device) -> Tensor:
    """The tiles' outputs side by side, reordered to the full output columns."""
    cache = kernel.__dict__.setdefault("_fused_factored_untile", {})
    key = str(device)
    if key not in cache:
        cols = [c for t in tiles(kernel) for c in t.out_cols]
        inverse = torch.empty(len(cols), dtype=torch.int64)
        inverse[torch.tensor(cols)] = torch.arange(len(cols))
        cache[key] = inverse.to(device)
    return torch.cat(parts, dim=1).index_select(1, cache[key])


def _tiled(kernel: Any, i: "Inputs", launch) -> Tensor:
    parts = []
    for index, t in enumerate(tiles(kernel)):
        desc, _, _ = _tile_tensors(kernel, t, index, i.h.device)
        parts.append(launch(_take_columns(i.zc, t.zc_cols), _take_columns(i.zr, t.zr_cols), desc, t.d_out, t.max_bm))
    return _untile(kernel, parts, i.h.device)


def _ranges(cols: tuple[int, ...]) -> list[tuple[int, int]]:
    """Ascending columns as maximal contiguous ``[start, stop)`` ranges."""
    out: list[tuple[int, int]] = []
    for c in cols:
        if out and out[-1][1] == c:
            out[-1] = (out[-1][0], c + 1)
        else:
            out.append((c, c + 1))
    return out


def _take_columns(z: Tensor, cols: tuple[int, ...]) -> Tensor:
    """``z[:, :, cols]`` contiguous, copied range by range (a tile's columns are
    a few contiguous ranges: slice copies rather than an indexed gather)."""
    rs = _ranges(cols)
    if not rs:
        return z[:, :, :0].contiguous()
    if len(rs) == 1:
        return z[:, :, rs[0][0]:rs[0][1]].contiguous()
    return torch.cat([z[:, :, lo:hi] for lo, hi in rs], dim=2)


def _put_columns(dst: Tensor, cols: tuple[int, ...], src: Tensor) -> None:
    """``dst[:, :, cols] = src`` range by range."""
    at = 0
    for lo, hi in _ranges(cols):
        dst[:, :, lo:hi].copy_(src[:, :, at:at + hi - lo])
        at += hi - lo


class TiledAggregate(torch.autograd.Function):
    """A wide kernel's aggregate as one op over its output tiles: each tile's
    mixes gathered from the full ``zc``/``zr``, the fused forward and
    aggregate per tile, the outputs side by side in the full column order.
    The backward writes every tile's mix gradient straight into its columns of
    one ``dzc``/``dzr`` (the tiles partition the columns, so each is written
    once) and accumulates ``dh`` and ``dweights`` in place."""

    @staticmethod
    def forward(ctx: Any, h: Tensor, zc: Tensor, zr: Tensor, weights: Tensor, angular: Tensor, transport: Tensor,
                rho: Tensor, source: Tensor, target: Tensor, row_ptr: Tensor, order: Tensor, group_ptr: Tensor,
                group_source: Tensor, kernel: Any) -> Tensor:
        ext = extension(cuda=h.is_cuda)
        parts, saved = [], []
        with torch.profiler.record_function("gm::kernel/pairs_tiles"):
            for index, t in enumerate(tiles(kernel)):
                desc, _, _ = _tile_tensors(kernel, t, index, h.device)
                zc_t, zr_t = _take_columns(zc, t.zc_cols), _take_columns(zr, t.zr_cols)
                r = ext.forward(h, zc_t, zr_t, angular, transport, rho, desc, source, order, group_ptr, group_source,
                                t.d_out, t.max_bm)
                saved += [r, zc_t, zr_t]  # the tiles' mixes together hold what zc and zr hold
                parts.append(ext.aggregate(r, weights, row_ptr))
        ctx.save_for_backward(h, weights, angular, transport, rho, source, target, order, group_ptr, group_source,
                              *saved)
        ctx.kernel = kernel
        ctx.shapes = (zc.shape, zr.shape, zc.dtype)
        return _untile(kernel, parts, h.device)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_out: Tensor) -> tuple:
        h, weights, angular, transport, rho, source, target, order, group_ptr, group_source = ctx.saved_tensors[:10]
        per_tile = ctx.saved_tensors[10:]
        kernel = ctx.kernel
        ext = extension(cuda=h.is_cuda)
        grad_out = grad_out.contiguous()
        zc_shape, zr_shape, dtype = ctx.shapes
        dzc = torch.empty(zc_shape, dtype=dtype, device=h.device)
        dzr = torch.empty(zr_shape, dtype=dtype, device=h.device)
        dh = dweights = None
        offset = 0
        with torch.profiler.record_function("gm::kernel/pairs_tiles_backward"):
            for index, t in enumerate(tiles(kernel)):
                r, zc_t, zr_t = per_tile[3 * index:3 * index + 3]
                desc, _, _ = _tile_tensors(kernel, t, index, h.device)
                cols = _untile_columns(kernel, h.device)[offset:offset + t.d_out]
                offset += t.d_out
                g_t = grad_out.index_select(1, cols).contiguous()
                dh_t, dzc_t, dzr_t, dw_t = ext.backward_aggregated(g_t, target, weights, r, h, zc_t, zr_t, angular,
                                                                   transport, rho, desc, source, order, group_ptr,
                                                                   group_source)
                _put_columns(dzc, t.zc_cols, dzc_t)
                _put_columns(dzr, t.zr_cols, dzr_t)
                dh = dh_t if dh is None else dh.add_(dh_t)
                dweights = dw_t if dweights is None else dweights.add_(dw_t)
        return dh, dzc, dzr, dweights, None, None, None, None, None, None, None, None, None, None


def _untile_columns(kernel: Any, device: torch.device) -> Tensor:
    """The full output columns of the tiles' outputs side by side."""
    cache = kernel.__dict__.setdefault("_fused_factored_tile_columns", {})
    key = str(device)
    if key not in cache:
        cache[key] = torch.tensor([c for t in tiles(kernel) for c in t.out_cols], dtype=torch.int64, device=device)
    return cache[key]


def forward(kernel: Any, x: SO2FeatureField, edges: Any, products: dict | None = None,
            groups: tuple[Tensor, Tensor, Tensor] | None = None) -> SO2FeatureField:
    """The messages on the edges, ``(n_edges,)`` of the kernel's output type."""
    i = inputs(kernel, x, edges, products)
    order, group_ptr, group_source = groups_for(edges, i.source) if groups is None else groups

    def launch(zc, zr, desc, d_out, max_bm):
        return Factored.apply(i.h, zc, zr, i.angular, i.transport, i.rho, desc, i.source, order, group_ptr,
                              group_source, d_out, max_bm)

    if tiles(kernel) is None:
        flat = launch(i.zc, i.zr, i.desc, i.plan.d_out, i.plan.max_bm)
    else:
        flat = _tiled(kernel, i, launch)
    return SO2FeatureField.from_flat(kernel.field_type_out, flat)


def forward_aggregated(kernel: Any, x: SO2FeatureField, edges: Any, weights: Tensor, products: dict | None = None,
                       groups: tuple[Tensor, Tensor, Tensor] | None = None) -> SO2FeatureField:
    """Each target's weighted sum of its messages, ``(n_targets,)`` of the output type."""
    i = inputs(kernel, x, edges, products)
    order, group_ptr, group_source = groups_for(edges, i.source) if groups is None else groups
    w = weights.to(i.h.dtype).contiguous()
    target, row_ptr = edges.target_index.contiguous(), edges.row_ptr.contiguous()

    if tiles(kernel) is None:
        flat = FactoredAggregate.apply(i.h, i.zc, i.zr, w, i.angular, i.transport, i.rho, i.desc, i.source, target,
                                       row_ptr, order, group_ptr, group_source, i.plan.d_out, i.plan.max_bm)
    else:
        flat = TiledAggregate.apply(i.h, i.zc, i.zr, w, i.angular, i.transport, i.rho, i.source, target, row_ptr,
                                    order, group_ptr, group_source, kernel)
    return SO2FeatureField.from_flat(kernel.field_type_out, flat)


# ---------------------------------------------------------------- every head at once


@dataclass(frozen=True)
class HeadsPlan:
    """The heads' common plan with the complex blocks' mixes packed by input
    frequency (their columns in ``zc`` grouped by the node vector's frequency
    n, in descriptor order within a frequency), so one matrix product per
    input frequency yields every head's mixes where the op reads them.

    ``groups[n] = (blocks reading x_n in packed order, complex width, real width)``."""

    plan: Plan
    desc_rows: tuple[tuple[int, ...], ...]
    groups: tuple[tuple[int, tuple[Block, ...], int, int], ...]  # (n, blocks, 2 * complex columns, real columns)


def heads_plan(kernel: Any) -> HeadsPlan:
    cached = kernel.__dict__.get("_fused_heads_plan")
    if cached is not None:
        return cached
    base = plan(kernel)
    by_n: dict[int, list[Block]] = {}
    real: list[Block] = []
    for b in base.blocks:
        (real if b.kind == 0 else by_n.setdefault(b.block[0], [])).append(b)
    offset = 0
    zoff: dict[tuple[int, int, str], int] = {}
    groups = []
    for n in sorted(set(by_n) | ({0} if real else set())):
        blocks = by_n.get(n, [])
        for b in blocks:
            zoff[b.block] = offset
            offset += b.b_m
        width = 2 * sum(b.b_m for b in blocks)
        groups.append((n, tuple(blocks) + (tuple(real) if n == 0 else ()), width, base.wr if n == 0 else 0))
    rows = []
    for b in base.blocks:
        row = b.row()
        if b.kind == 1:
            row[1] = zoff[b.block]
        rows.append(tuple(row))
    result = HeadsPlan(base, tuple(rows), tuple(groups))
    kernel.__dict__["_fused_heads_plan"] = result
    return result


class SubHead:
    """The value kernel of one head restricted to an equal share of its output
    copies: copies ``[s b_m / split, (s + 1) b_m / split)`` of every output
    frequency, share ``s``.  A kernel's blocks are separable by output copy,
    so a head's rows are its shares' rows side by side (per frequency); the
    shares have the head's blocks, harmonic orders and powers, ``b_m / split``
    copies each.  Stands in for the kernel where only the plan is read."""

    def __init__(self, kernel: Any, split: int) -> None:
        out = kernel.field_type_out
        if any(m % split for m in out.multiplicities):
            raise ValueError(f"split {split} does not divide every multiplicity of {out!r}")
        self.kernel = kernel
        self.split = split
        self.field_type_in = kernel.field_type_in
        self.field_type_out = SO2FieldType({f: m // split for f, m in out.items()})
        self._pair_powers = kernel._pair_powers
        self.complex_head, self.real_head = kernel.complex_head, kernel.real_head
        self.radial_basis = kernel.radial_basis

    def _blocks(self) -> list[tuple[int, int, str]]:
        return self.kernel._blocks()


def sub_head(kernel: Any, split: int) -> Any:
    """``kernel`` itself for ``split == 1``, else its :class:`SubHead` (cached)."""
    if split == 1:
        return kernel
    key = ("_sub_head", split)
    sub = kernel.__dict__.get(key)
    if sub is None:
        sub = SubHead(kernel, split)
        kernel.__dict__[key] = sub
    return sub


def share_columns(kernel: Any, split: int, heads: int, device: torch.device) -> Tensor:
    """For column ``h d + c`` of the heads' rows ``(N, H, d)`` (each head in
    the per-head flat layout), its column in the shares' rows
    ``(N, H split, d / split)`` -- the gather that puts the shares' outputs
    back side by side."""
    key = ("_share_columns", split, heads, str(device))
    cols = kernel.__dict__.get(key)
    if cols is None:
        out = kernel.field_type_out
        part = SO2FieldType({f: m // split for f, m in out.items()})
        full_s, part_s = out.slices(), part.slices()
        d_part = part.dimension
        index = []
        for head in range(heads):
            for f, m in out.items():
                dim = 1 if f == 0 else 2
                per = m // split
                for c in range(full_s[f].stop - full_s[f].start):
                    copy, re = divmod(c, dim)
                    share, local = divmod(copy, per)
                    index.append((head * split + share) * d_part + part_s[f].start + local * dim + re)
        cols = torch.tensor(index, dtype=torch.int64, device=device)
        kernel.__dict__[key] = cols
    return cols


def _heads_mixing_from(kernels: list[Any], hp: HeadsPlan, params: list[list[Tensor | None]],
                       split: int = 1) -> list[Tensor]:
    """``heads_mixing`` from stand-in readout parameters (one list per head);
    with ``split > 1`` the columns run over the heads' shares (head-major)."""
    from gm_attention_amd.nn.node_products import mixing_matrix

    mats = []
    for n, blocks, _cw, _rw in hp.groups:
        per_share = []
        for k, pk in zip(kernels, params, strict=True):
            weights = {b.block: k._block_weights(b.block, pk) for b in blocks}  # (b_m, a_n, K) of the full head
            for share in range(split):
                pieces = []
                for b in blocks:
                    w = weights[b.block][share * b.b_m:(share + 1) * b.b_m]
                    if b.kind == 0:
                        m = mixing_matrix(w, "real")  # (a_0, K * b_0)
                        pieces.append(m.reshape(m.shape[0], w.shape[-1], -1))
                        continue
                    bn, bm, role = b.block
                    mode = "promote" if bn == 0 else ("conj" if (bm == 0 or role == "antilinear") else "plain")
                    m = mixing_matrix(w, mode)  # (w_n, K * b_m * 2)
                    pieces.append(m.reshape(m.shape[0], w.shape[-1], -1))
                per_share.append(torch.cat(pieces, dim=-1))  # (w_n, K, C_n)
        stacked = torch.stack(per_share, dim=1)  # (w_n, H split, K, C_n)
        mats.append(stacked.reshape(stacked.shape[0], -1))
    return mats


_MIXING_MAPS: OrderedDict = OrderedDict()


def _mixing_maps(kernels: list[Any], hp: HeadsPlan, split: int = 1) -> dict:
    """``{"maps": [(index, sign) per input frequency]}`` with ``M_n = sign *
    flat[index]``, ``flat`` the heads' readout parameters concatenated
    (``readout_parameters`` order, head by head): found once by running the
    construction on the parameters' positions (+1) as float64 values, which it
    only moves and negates.  :class:`_SignedGather` keeps its gradient plan in
    the same dictionary."""
    shapes = tuple(tuple(None if p is None else tuple(p.shape) for p in k.readout_parameters()) for k in kernels)
    key = (tuple(id(k) for k in kernels), shapes, split)
    hit = _MIXING_MAPS.get(key)
    if hit is not None:
        return hit
    device = kernels[0].complex_head.weight.device
    offset, ids = 1, []
    for k in kernels:
        per = []
        for p in k.readout_parameters():
            if p is None:
                per.append(None)
                continue
            per.append(torch.arange(offset, offset + p.numel(), dtype=torch.float64).reshape(p.shape))
            offset += p.numel()
        ids.append(per)
    maps = []
    for m in _heads_mixing_from(kernels, hp, ids, split):
        index = (m.abs().round().long() - 1).clamp_min(0)
        maps.append((index.to(device), torch.sign(m).to(device)))
    maps = dict(maps=maps)  # the gather's gradient plan joins it on the first backward
    _MIXING_MAPS[key] = maps
    while len(_MIXING_MAPS) > 16:
        _MIXING_MAPS.popitem(last=False)
    return maps


class _SignedGather(torch.autograd.Function):
    """``[flat[index] * sign for each map]`` with a gradient that sums each
    parameter's uses in a fixed order, prepared once per set of maps: the
    maps' positions sorted by the parameter they read (stable, so a
    parameter's uses keep their order), then per parameter its uses' values
    added in that order -- as up to kMaxUses padded columns (the heads' maps
    use a parameter at most twice), else one segment sum.  (Autograd's own
    gradient of the indexing sorts the indices on every call.)"""

    kMaxUses = 16

    @staticmethod
    def forward(ctx: Any, flat: Tensor, plan: dict, *maps: tuple) -> tuple:
        ctx.plan = plan
        ctx.shapes = [index.shape for index, _ in plan["maps"]]
        ctx.n = flat.numel()
        return tuple(flat.index_select(0, index.reshape(-1)).reshape(index.shape) * sign.to(flat.dtype)
                     for index, sign in plan["maps"])

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, *grads: Tensor) -> tuple:
        plan = ctx.plan
        if "order" not in plan:
            index = torch.cat([i.reshape(-1) for i, _ in plan["maps"]])
            plan["sign"] = torch.cat([s.reshape(-1) for _, s in plan["maps"]])
            plan["order"] = torch.argsort(index, stable=True)
            counts = torch.bincount(index, minlength=ctx.n)
            plan["offsets"] = torch.cat([counts.new_zeros(1), torch.cumsum(counts, 0)])
            uses = int(counts.max()) if counts.numel() else 0
            if uses <= _SignedGather.kMaxUses:
                # column j: each parameter's j-th use (its position), or the appended zero
                total = index.numel()
                srt = index.index_select(0, plan["order"])
                rank = torch.arange(total, device=index.device) - plan["offsets"].index_select(0, srt)
                cols = torch.full((max(uses, 1), ctx.n), total, dtype=torch.int64, device=index.device)
                cols[rank, srt] = plan["order"]
                plan["cols"] = cols
        g = torch.cat([(gi if gi is not None else torch.zeros(sh, dtype=plan["sign"].dtype, device=plan["sign"].device))
                       .reshape(-1) for gi, sh in zip(grads, ctx.shapes, strict=True)])
        vals = g * plan["sign"].to(g.dtype)
        if "cols" in plan:
            vals = torch.cat([vals, vals.new_zeros(1)])
            cols = plan["cols"]
            dflat = vals.index_select(0, cols[0])
            for j in range(1, cols.shape[0]):
                dflat = dflat + vals.index_select(0, cols[j])
        else:
            dflat = torch.segment_reduce(vals.index_select(0, plan["order"]), "sum", offsets=plan["offsets"], axis=0)
        return (dflat, None)


def heads_mixing(kernels: list[Any], hp: HeadsPlan, split: int = 1) -> list[Tensor]:
    """Per input frequency n, ``M_n`` of ``(reals of x_n, H * K * C_n)``: columns
    ``(head, t, [complex pairs in packed order | the real block's columns])``,
    so ``X_n M_n`` is every head's ``Z_t`` for the blocks reading x_n.  Every
    entry is one readout parameter, possibly negated, or zero: the matrices
    are one gather from the heads' concatenated parameters (a handful of
    kernels, differentiable) rather than a per-head, per-block build.  With
    ``split > 1``, ``hp`` is the shares' plan and the columns run over
    ``H * split`` shares."""
    plan = _mixing_maps(kernels, hp, split)
    flat = torch.cat([p.reshape(-1) for k in kernels for p in k.readout_parameters() if p is not None])
    return list(_SignedGather.apply(flat, plan))


def node_vectors(x: SO2FeatureField, hp: HeadsPlan) -> list[Tensor]:
    """The node field's reals each input frequency's product reads."""
    n_nodes = x.batch_shape[0]
    return [x[0] if n == 0 else x[n].reshape(n_nodes, -1) for n, *_ in hp.groups]


def heads_mixes(x: SO2FeatureField, hp: HeadsPlan, mats: list[Tensor]) -> list[Tensor]:
    """Every head's node mixes, one ``(N, H K C_n)`` array per input frequency:
    the MFMA node-mix kernels on the flat rows where they serve the call
    (:class:`node_products.NodeMixes`), else one matrix product per frequency."""
    from gm_attention_amd.nn.node_products import NodeMixes, mixes_eligible

    rows = x._rows()
    slices = x.field_type.slices()
    columns = tuple((slices[n].start, slices[n].stop - slices[n].start) for n, *_ in hp.groups)
    if mixes_eligible(rows, [w for _, w in columns], mats):
        return list(NodeMixes.apply(rows, columns, *[m.to(torch.float32) for m in mats]))
    vecs = node_vectors(x, hp)
    with torch.profiler.record_function("gm::kernel/node_products"):
        return [v @ m.to(v.dtype) for v, m in zip(vecs, mats, strict=True)]


class FactoredHeads(torch.autograd.Function):
    """Every head's factored value aggregation on the mixes ``X_n M_n``.

    Inputs: ``h (H, E, T)``, ``alpha (E, H)``, then one ``(N, H * K * C_n)`` mix
    array per input frequency; out ``(N, H, d_out)``.  The backward returns
    ``dh``, ``dalpha`` and the mix arrays' gradients (written in place by the
    HIP backward), so autograd carries them through the products to the
    node field and the heads' readout weights."""

    @staticmethod
    def forward(ctx: Any, h: Tensor, alpha: Tensor, meta: dict, *mixes: Tensor) -> Tensor:
        H, E = h.shape[0], h.shape[1]
        N = meta["n_nodes"]
        ext = extension()
        rows, outs = [], []
        for head in range(H):
            runs = _heads_runs(meta, mixes, head, None)
            with torch.profiler.record_function("gm::kernel/pairs"):
                r = _native.factored_forward_seg(h[head], runs, N, meta["angular"], meta["transport"], meta["rho"],
                                                 meta["desc"], meta["order"], meta["group_ptr"], meta["group_source"],
                                                 meta["K"], meta["wc"], meta["wr"], meta["d_out"], meta["max_bm"])
            with torch.profiler.record_function("gm::kernel/aggregate"):
                outs.append(ext.aggregate(r, alpha[:, head].contiguous(), meta["row_ptr"]))
            rows.append(r)
        ctx.meta = meta
        ctx.save_for_backward(h, alpha, *rows, *mixes)
        return torch.stack(outs, dim=1)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad: Tensor) -> tuple:
        meta = ctx.meta
        saved = ctx.saved_tensors
        h, alpha = saved[0], saved[1]
        H = h.shape[0]
        rows, mixes = saved[2:2 + H], saved[2 + H:]
        dmixes = [torch.zeros_like(m) for m in mixes]
        dh = torch.empty_like(h)
        dalpha = torch.empty_like(alpha)
        for head in range(H):
            runs = _heads_runs(meta, mixes, head, dmixes)
            with torch.profiler.record_function("gm::kernel/pairs_backward"):
                dw = _native.factored_backward_seg(grad[:, head].contiguous(), meta["target"],
                                                   alpha[:, head].contiguous(), rows[head], h[head], runs,
                                                   meta["n_nodes"], meta["angular"], meta["transport"], meta["rho"],
                                                   meta["desc"], meta["order"], meta["group_ptr"],
                                                   meta["group_source"], meta["K"], meta["wc"], meta["wr"], dh[head])
            dalpha[:, head] = dw
        return (dh, dalpha, None, *dmixes)


def _heads_runs(meta: dict, mixes: tuple[Tensor, ...], head: int, grads: list[Tensor] | None) -> _native.MixRuns:
    """Head ``head``'s mix runs in packed-column order: every input
    frequency's complex columns, then the real block's."""
    K, H = meta["K"], meta["heads"]
    complex_runs, real_runs = [], []
    for (n, _blocks, cw, rw), mix in zip(meta["groups"], mixes, strict=True):
        C = cw + rw
        base = head * K * C
        if cw:
            complex_runs.append((mix, base, H * K * C, C, cw))
        if rw:
            real_runs.append((mix, base + cw, H * K * C, C, rw))
    runs = complex_runs + real_runs
    views = [(m.view(-1)[off:], ns, ts, w) for m, off, ns, ts, w in runs]
    grad_views = None
    if grads is not None:
        by_id = {id(m): g for m, g in zip(mixes, grads, strict=True)}
        grad_views = [by_id[id(m)].view(-1)[off:] for m, off, *_ in runs]
    return _native.MixRuns(views, grad_views)


@dataclass
class GroupedStreams:
    """An edge set's per-edge streams in the order of its source grouping:
    ``perm`` (= the grouping's order), its inverse ``inv``, ``rho_g``, the
    phase rows ``phase_g (E, 8, 2)`` (angular orders ``0..pa-1`` then
    transport orders ``0..pt-1``) and ``target_g``."""

    perm: Tensor
    inv: Tensor
    rho_g: Tensor
    phase_g: Tensor
    target_g: Tensor
    pa: int
    pt: int
    zw_g: Tensor | None = None  # (E, 4): r e^{i phi}, e^{i gamma} (order-1 phases) in grouping order
    group_order: Tensor | None = None


_STREAMS: OrderedDict[tuple, tuple[Any, GroupedStreams]] = OrderedDict()


def grouped_streams(edges: Any, order: Tensor, cutoff: float, pa: int, pt: int, dtype: torch.dtype) -> GroupedStreams:
    """The grouped streams of ``edges`` under ``order``, cached while the edge set lives."""
    key = (id(edges.edge_index), edges.edge_index.data_ptr(), int(edges.n_edges), order.data_ptr(), float(cutoff), pa,
           pt, dtype)
    hit = _STREAMS.get(key)
    if hit is not None and hit[0]() is edges.edge_index:
        return hit[1]
    with torch.profiler.record_function("gm::kernel/group_streams"):
        perm = order
        inv = torch.empty_like(perm)
        inv[perm] = torch.arange(perm.shape[0], device=perm.device)
        rho_g = (edges.distances.index_select(0, perm) / cutoff).to(dtype).contiguous()
        ang = torch.view_as_real(edges.angular_phases[:, :pa].index_select(0, perm))
        tra = torch.view_as_real(edges.transport_phases[:, :pt].index_select(0, perm))
        phase_g = torch.zeros(perm.shape[0], 8, 2, dtype=dtype, device=perm.device)
        phase_g[:, :pa] = ang.to(dtype)
        phase_g[:, pa:pa + pt] = tra.to(dtype)
        # r e^{i phi} and e^{i gamma}: every block factor is a product of their powers
        r64 = edges.distances.index_select(0, perm).double() / cutoff
        a1 = edges.angular_phases[:, 1].index_select(0, perm).to(torch.complex128) * r64
        t1 = edges.transport_phases[:, 1].index_select(0, perm).to(torch.complex128)
        zw_g = torch.stack([a1.real, a1.imag, t1.real, t1.imag], dim=1).to(dtype).contiguous()
        streams = GroupedStreams(perm, inv, rho_g, phase_g.contiguous(),
                                 edges.target_index.index_select(0, perm).contiguous(), pa, pt, zw_g)
    for stale in [k for k, (ref, _) in _STREAMS.items() if ref() is None]:
        del _STREAMS[stale]
    _STREAMS[key] = (weakref.ref(edges.edge_index), streams)
    while len(_STREAMS) > 8:
        _STREAMS.popitem(last=False)
    return streams


def grouped_eligible(hp: HeadsPlan, h_dtype: torch.dtype, K: int) -> tuple[bool, int, int]:
    """Whether the heads take the grouped kernels (fp32, K = 17, <= 128 packed
    columns, phase orders within one 8-pair row); with (pa, pt)."""
    p = hp.plan
    pa = max((abs(b.angular) for b in p.blocks), default=0) + 1
    pt = max((abs(b.transport) for b in p.blocks), default=0) + 1
    ok = (h_dtype == torch.float32 and K == 17 and 2 * p.wc + p.wr <= 128 and pa + pt <= 8
          and os.environ.get("GM_FACTORED_GROUPED", "1") != "0")
    return ok, pa, pt


class FactoredHeadsGrouped(torch.autograd.Function):
    """:class:`FactoredHeads` over the grouped streams: ``h_g (H, E, 16)`` in
    the grouping's order, ``alpha (E, H)`` in edge order, the mix arrays;
    out ``(N, H split, d_out)``; gradients ``dh_g``, ``dalpha`` and the mixes'.
    With ``meta["split"] > 1`` the launches run over the heads' shares (share
    ``v`` of head ``v // split``), which read their head's trunk features and
    attention weights."""

    @staticmethod
    def forward(ctx: Any, h_g: Tensor, alpha: Tensor, meta: dict, *mixes: Tensor) -> Tensor:
        E, split = h_g.shape[1], meta["split"]
        st: GroupedStreams = meta["streams"]
        shares = meta["heads"]
        rows = torch.empty(shares, E, meta["d_out"], dtype=h_g.dtype, device=h_g.device)
        for v in range(shares):
            runs = _heads_runs(meta, mixes, v, None)
            with torch.profiler.record_function("gm::kernel/pairs"):
                _native.factored_forward_grouped(h_g[v // split], runs, meta["n_nodes"], st.phase_g, st.rho_g,
                                                 st.zw_g, st.pa, st.pt, meta["desc"], meta["group_ptr"],
                                                 meta["group_source"], meta["group_order"], meta["K"], meta["wc"],
                                                 meta["wr"], meta["d_out"], out=rows[v])
        with torch.profiler.record_function("gm::kernel/aggregate"):
            out = _native.aggregate_heads(rows, st.inv, alpha, meta["row_ptr"], split)
        ctx.meta = meta
        ctx.save_for_backward(h_g, alpha, rows, *mixes)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad: Tensor) -> tuple:
        meta = ctx.meta
        st: GroupedStreams = meta["streams"]
        h_g, alpha, rows, *mixes = ctx.saved_tensors
        split, shares = meta["split"], meta["heads"]
        # every source node has a group (and so every mix row is written) unless some node has no edge out
        fill = torch.zeros_like if meta["group_source"].shape[0] < meta["n_nodes"] else torch.empty_like
        dmixes = [fill(m) for m in mixes]
        dh_g = torch.empty_like(h_g)
        alpha_gt = _native.gather_transpose(alpha, st.perm)  # (H, E) in the grouping's order
        dalpha_gt = torch.empty_like(alpha_gt)
        grad = grad.contiguous()
        for v in range(shares):
            head, share = divmod(v, split)
            runs = _heads_runs(meta, mixes, v, dmixes)
            # a head's shares read the same trunk features and weights: the later shares add their gradients
            with torch.profiler.record_function("gm::kernel/pairs_backward"):
                _native.factored_backward_grouped(
                    grad[:, v], st.target_g, alpha_gt[head], rows[v], h_g[head], runs,
                    meta["n_nodes"], st.phase_g, st.rho_g, st.zw_g, st.pa, st.pt, meta["desc"], meta["group_ptr"],
                    meta["group_source"], meta["group_order"], meta["K"], meta["wc"], meta["wr"],
                    dh_g[head], dweights=dalpha_gt[head], accumulate=share > 0)
        dalpha = _native.scatter_transpose(dalpha_gt, st.perm)
        return (dh_g, dalpha, None, *dmixes)


class FactoredHeadsTrunk(torch.autograd.Function):
    """:class:`FactoredHeadsGrouped` with each head's radial trunk evaluated
    inside the lane-owned kernels from ``rho_g`` (no ``h (H, E, 16)`` tensor):
    in ``trunk_w (H, 16, B)``, ``trunk_b (H, 16)`` or None, ``alpha (E, H)``
    and the mix arrays; out ``(N, H, d_out)``; gradients for the trunk's
    parameters (the trunk kernel's backward on the ``dh`` the factored
    backward writes), ``alpha`` and the mixes."""

    @staticmethod
    def forward(ctx: Any, trunk_w: Tensor, trunk_b: Tensor | None, alpha: Tensor, meta: dict,
                *mixes: Tensor) -> Tensor:
        st: GroupedStreams = meta["streams"]
        H, E = trunk_w.shape[0], st.rho_g.shape[0]
        trunks = [_native.FusedTrunk(trunk_w[hh].contiguous(), None if trunk_b is None else trunk_b[hh].contiguous(),
                                     meta["centers"], meta["width"]) for hh in range(H)]
        rows = torch.empty(H, E, meta["d_out"], dtype=alpha.dtype, device=alpha.device)
        for head in range(H):
            runs = _heads_runs(meta, mixes, head, None)
            with torch.profiler.record_function("gm::kernel/pairs"):
                _native.factored_forward_grouped(None, runs, meta["n_nodes"], st.phase_g, st.rho_g, st.zw_g, st.pa,
                                                 st.pt, meta["desc"], meta["group_ptr"], meta["group_source"],
                                                 meta["group_order"], meta["K"], meta["wc"], meta["wr"],
                                                 meta["d_out"], out=rows[head], trunk=trunks[head])
        with torch.profiler.record_function("gm::kernel/aggregate"):
            out = _native.aggregate_heads(rows, st.inv, alpha, meta["row_ptr"])
        ctx.meta = meta
        ctx.trunks = trunks
        ctx.has_bias = trunk_b is not None
        ctx.save_for_backward(trunk_w, trunk_b if trunk_b is not None else alpha.new_empty(0), alpha, rows, *mixes)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad: Tensor) -> tuple:
        meta = ctx.meta
        st: GroupedStreams = meta["streams"]
        trunk_w, trunk_b, alpha, rows, *mixes = ctx.saved_tensors
        H, E = trunk_w.shape[0], st.rho_g.shape[0]
        fill = torch.zeros_like if meta["group_source"].shape[0] < meta["n_nodes"] else torch.empty_like
        dmixes = [fill(m) for m in mixes]
        dh_g = torch.empty(H, E, 16, dtype=alpha.dtype, device=alpha.device)
        alpha_gt = _native.gather_transpose(alpha, st.perm)
        dalpha_gt = torch.empty_like(alpha_gt)
        grad = grad.contiguous()
        for head in range(H):
            runs = _heads_runs(meta, mixes, head, dmixes)
            with torch.profiler.record_function("gm::kernel/pairs_backward"):
                _native.factored_backward_grouped(
                    grad[:, head], st.target_g, alpha_gt[head], rows[head], None, runs, meta["n_nodes"],
                    st.phase_g, st.rho_g, st.zw_g, st.pa, st.pt, meta["desc"], meta["group_ptr"],
                    meta["group_source"], meta["group_order"], meta["K"], meta["wc"], meta["wr"], dh_g[head],
                    dweights=dalpha_gt[head], trunk=ctx.trunks[head])
        dalpha = _native.scatter_transpose(dalpha_gt, st.perm)
        with torch.profiler.record_function("gm::kernel/radial_backward"):
            dw, db = _native.radial_trunk_backward(dh_g, st.rho_g, trunk_w.contiguous(),
                                                   trunk_b.contiguous() if ctx.has_bias else None,
                                                   meta["centers_t"], meta["width"])
        return (dw, db if ctx.has_bias else None, dalpha, None, *dmixes)


#: ``GM_FACTORED_TRUNK=1`` evaluates each head's radial trunk inside the lane-owned
#: kernels instead of a pass of its own: no ``h (H, E, 16)`` or ``dh`` tensor (64 GB at
#: 256x512, B = 4, 8 heads), at the cost of time -- the lane kernels are issue-bound, so
#: the recomputation costs more than the round trip it saves (168 vs 155 ms a step there).
FUSED_TRUNK = os.environ.get("GM_FACTORED_TRUNK", "0") == "1"

#: For bfloat16 node rows (a bfloat16 block), the grouped kernels keep their
#: per-edge streams -- the trunk features, the value rows and the features'
#: gradients -- in bfloat16, with float32 arithmetic, as the reference's block
#: keeps them in the rows' dtype (``blocks.py:326-349``); ``GM_BF16_STREAMS=0``
#: keeps them float32.  Plans with compiled-in lane slots only.
BF16_STREAMS = os.environ.get("GM_BF16_STREAMS", "1") != "0"


def _lanes_apply(kernel: Any, hp: HeadsPlan, pa: int, pt: int) -> bool:
    """Whether the grouped kernels take the lane-owned form for this plan."""
    key = ("_lanes_apply", pa, pt, os.environ.get("GM_FACTORED_LANES", "1"))
    hit = kernel.__dict__.get(key)
    if hit is None:
        p = hp.plan
        n_slots, _, _ = _native.lane_tables(torch.tensor([list(r) for r in hp.desc_rows], dtype=torch.int32), p.wc,
                                            p.wr, p.d_out, pa, pt)
        hit = n_slots > 0
        kernel.__dict__[key] = hit
    return hit


def _lanes_fixed(kernel: Any, hp: HeadsPlan, pa: int, pt: int) -> bool:
    """Whether the grouped kernels take compiled-in lane slots for this plan
    (the kernels that also take bfloat16 streams)."""
    key = ("_lanes_fixed", pa, pt, os.environ.get("GM_FACTORED_LANES", "1"), os.environ.get("GM_FACTORED_STATIC", "1"))
    hit = kernel.__dict__.get(key)
    if hit is None:
        p = hp.plan
        hit = _native.lanes_fixed(torch.tensor([list(r) for r in hp.desc_rows], dtype=torch.int32), p.wc, p.wr,
                                  p.d_out, pa, pt)
        kernel.__dict__[key] = hit
    return hit


def head_split(kernel: Any, K: int) -> int:
    """Into how many shares of output copies each head's value kernel is cut
    for the grouped kernels: 1 when its plan fits them as is, else the
    smallest power of two (at most 64) dividing every output multiplicity
    whose shares fit (packed mix width ``2 wc + wr <= 128``); 0 when none does.
    A restriction onto 128 copies of frequencies 0..2 runs as 32 shares of
    four copies each, the attention heads' shape."""
    key = ("_head_split", K, os.environ.get("GM_FACTORED_GROUPED", "1"))
    hit = kernel.__dict__.get(key)
    if hit is None:
        hit = 0
        for split in (1, 2, 4, 8, 16, 32, 64):
            if any(m % split for m in kernel.field_type_out.multiplicities):
                break
            ok, _, _ = grouped_eligible(heads_plan(sub_head(kernel, split)), torch.float32, K)
            if ok:
                hit = split
                break
        kernel.__dict__[key] = hit
    return hit


def forward_aggregated_heads(kernels: list[Any], x: SO2FeatureField, edges: Any, alpha: Tensor, h: Tensor | None,
                             groups: tuple[Tensor, Tensor, Tensor], trunk=None) -> Tensor:
    """Every head's ``forward_factored_aggregated`` at once: ``(N, H, d_out)``.

    ``h`` is every head's trunk features in edge order; alternatively
    ``trunk(rho, dtype)`` computes them from ``rho = d / cutoff`` in whatever
    order it is given (in ``dtype``, None for rho's), which lets the grouped
    kernels have them in the grouping's order directly.  Heads too wide for
    the grouped kernels run there as shares of their output copies
    (:func:`head_split`).  Bfloat16 node rows keep the per-edge streams in
    bfloat16 (:data:`BF16_STREAMS`)."""
    K = (h.shape[2] if h is not None else kernels[0].complex_head.in_features) + 1
    # bfloat16 rows: the node mixes read them as they are, everything after runs in float32
    dtype = h.dtype if h is not None else (torch.float32 if x.dtype == torch.bfloat16 else x.dtype)
    split = head_split(kernels[0], K) if dtype == torch.float32 else 0
    hp = heads_plan(sub_head(kernels[0], max(split, 1)))
    ok, pa, pt = grouped_eligible(hp, dtype, K)
    if ok and split:
        p = hp.plan
        unit = sub_head(kernels[0], split)
        mixes = heads_mixes(x, hp, heads_mixing(kernels, hp, split))
        order, group_ptr, group_source = groups
        st = grouped_streams(edges, order, kernels[0].radial_basis.cutoff, pa, pt, dtype)
        fused = (FUSED_TRUNK and split == 1 and len(kernels) <= 8 and trunk is not None
                 and _lanes_apply(kernels[0], hp, pa, pt))
        b16 = (BF16_STREAMS and not fused and trunk is not None and x.dtype == torch.bfloat16
               and _lanes_fixed(kernels[0], hp, pa, pt))
        h_g = None if fused else (trunk(st.rho_g, torch.bfloat16 if b16 else None) if trunk is not None
                                  else h.index_select(1, st.perm))
        if st.group_order is None and os.environ.get("GM_FACTORED_LPT", "0") == "1":
            # the groups largest first: the long pole groups start early instead of trailing the launch
            st.group_order = torch.argsort(group_ptr[1:] - group_ptr[:-1], descending=True, stable=True).contiguous()
        meta = dict(n_nodes=x.batch_shape[0], heads=len(kernels) * split, split=split, K=K, wc=p.wc, wr=p.wr,
                    d_out=p.d_out, groups=hp.groups, desc=_heads_desc(unit, hp, x.device), group_ptr=group_ptr,
                    group_source=group_source, row_ptr=edges.row_ptr.contiguous(), streams=st,
                    group_order=st.group_order if os.environ.get("GM_FACTORED_LPT", "0") == "1" else None)
        if fused:
            from gm_attention_amd.nn import radial

            w, b, rb = radial.stacked_trunk(kernels)
            centers = kernels[0].__dict__.get("_centers_host")
            if centers is None:  # the basis centres are a fixed buffer: one host copy per kernel
                centers = [float(c) for c in rb.centers.detach().cpu().tolist()]
                kernels[0].__dict__["_centers_host"] = centers
            meta.update(centers=centers, centers_t=rb.centers.contiguous(), width=float(rb.width))
            return FactoredHeadsTrunk.apply(w, b, alpha.to(dtype).contiguous(), meta, *mixes)
        out = FactoredHeadsGrouped.apply(h_g.contiguous(), alpha.to(dtype).contiguous(), meta, *mixes)
        if split == 1:
            return out
        n = out.shape[0]
        cols = share_columns(kernels[0], split, len(kernels), out.device)
        return out.reshape(n, -1).index_select(1, cols).reshape(n, len(kernels), -1)
    if h is None:
        h = trunk((edges.distances / kernels[0].radial_basis.cutoff).to(dtype).contiguous())
    return _forward_aggregated_heads_seg(kernels, x, edges, alpha, h, groups)


def forward_aggregated_shares(kernel: Any, x: SO2FeatureField, edges: Any, weights: Tensor,
                              groups: tuple[Tensor, Tensor, Tensor] | None = None) -> SO2FeatureField | None:
    """One kernel's weighted aggregate on the grouped kernels, as a single head
    cut into shares of its output copies (:func:`head_split`) with the edge
    weights as the head's ``alpha``; ``None`` where they do not serve it (rows
    other than float32, or no share fits).  A kernel wider than the MFMA
    kernels' 128 packed columns -- a readout onto 32 scalars from 64 or 128
    copies of frequencies 0..2 has 160 -- then still runs on matrix cores."""
    from gm_attention_amd.nn import radial

    head = kernel.complex_head if kernel.complex_head is not None else kernel.real_head
    if x.dtype != torch.float32 or head_split(kernel, head.in_features + 1) == 0:
        return None
    if groups is None:
        groups = groups_for(edges, edges.source_index)
    values = [kernel]
    if radial.eligible(values, x.dtype, x.device):
        h, trunk = None, lambda rho, dtype=None: radial.trunk_hidden_heads(values, rho, dtype)
    else:
        h, trunk = kernel._trunk_hidden(edges.distances).unsqueeze(0), None
    out = forward_aggregated_heads(values, x, edges, weights.unsqueeze(1), h, groups, trunk)
    return SO2FeatureField.from_flat(kernel.field_type_out, out.reshape(out.shape[0], -1))


def _heads_desc(kernel: Any, hp: HeadsPlan, device: torch.device) -> Tensor:
    key = ("_fused_heads_desc", str(device))
    desc = kernel.__dict__.get(key)
    if desc is None:
        desc = torch.tensor([list(r) for r in hp.desc_rows], dtype=torch.int32, device=device)
        kernel.__dict__[key] = desc
    return desc


def _forward_aggregated_heads_seg(kernels: list[Any], x: SO2FeatureField, edges: Any, alpha: Tensor, h: Tensor,
                                  groups: tuple[Tensor, Tensor, Tensor]) -> Tensor:
    """Every head's ``forward_factored_aggregated`` at once: ``(N, H, d_out)``."""
    hp = heads_plan(kernels[0])
    p = hp.plan
    mixes = heads_mixes(x, hp, heads_mixing(kernels, hp))
    order, group_ptr, group_source = groups
    angular = torch.view_as_real(edges.angular_phases.contiguous()).contiguous().to(h.dtype)
    transport = torch.view_as_real(edges.transport_phases.contiguous()).contiguous().to(h.dtype)
    needed = max((max(abs(b.angular), abs(b.transport)) for b in p.blocks), default=0)
    if needed >= angular.shape[1]:
        raise ValueError(f"the geometry's phase tables ({angular.shape[1]} orders) are narrower than the kernel's "
                         f"blocks need (order {needed})")
    desc = _heads_desc(kernels[0], hp, h.device)
    meta = dict(n_nodes=x.batch_shape[0], heads=len(kernels), K=h.shape[2] + 1, wc=p.wc, wr=p.wr, d_out=p.d_out,
                max_bm=p.max_bm, groups=hp.groups, angular=angular, transport=transport,
                rho=(edges.distances / kernels[0].radial_basis.cutoff).to(h.dtype).contiguous(), desc=desc,
                order=order, group_ptr=group_ptr, group_source=group_source,
                target=edges.target_index.contiguous(), row_ptr=edges.row_ptr.contiguous())
    return FactoredHeads.apply(h, alpha.to(h.dtype).contiguous(), meta, *mixes)
