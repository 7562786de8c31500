"""The depthwise convolution with its radial heads evaluated inside the fused walk.

The reference evaluates a depthwise layer's radial trunk and readout heads
per edge with torch products (``stacked_coefficients``, nn/depthwise.py:206-238)
and hands the coefficient rows ``rc (E, a_0)`` and ``cc (E, sum 4 a_n)`` to its
fused walk (nn/convolution.py:432-441, fused_attention.py:329-368).  Here the
walk evaluates them from ``rho = d / cutoff`` in registers
(``gm_conv_radial_*``): the Gaussian basis and the trunk per lane, the
readout on MFMA from the packed readout matrix ``R`` (rows in the walk's tile
order, the bias as column 16), so no per-edge coefficient tensor exists in
either direction.  The backward returns ``dR`` (re-scattered to the heads'
weights and biases by the packing's autograd), the trunk's ``dW1``, ``db1``
and ``dv``; parameter gradients are reduced in a fixed order.

Serves float32 depthwise kernels with a ``Linear(B, 16) + SiLU`` trunk
(``B`` in 4, 6, 8) and frequencies up to 2, every multiplicity a multiple of
4.  One walk takes at most 32 scalar copies and 64 copies of frequencies 1
and 2 together; a wider field runs as equal groups of copies, one walk each
(``channel_groups``).  Other kernels take the reference's split
(``stacked_coefficients`` + ``fused_attention.Depthwise``).
"""

from __future__ import annotations

import os
from typing import Any

import torch
from torch import Tensor, nn

from gm_attention_amd import _native
from gm_attention_amd.nn import fused_attention

#: ``GM_DEPTHWISE_RADIAL=0`` keeps the reference's split (coefficients by torch products, then the walk).
ENABLED = os.environ.get("GM_DEPTHWISE_RADIAL", "1") != "0"

NS, NC = _native.RADIAL_TILES_SCALAR, _native.RADIAL_TILES_COMPLEX
NT = NS + NC


def channel_groups(ft: Any) -> tuple[tuple[tuple[int, int, int], ...], ...] | None:
    """``None`` when one walk takes the whole field; else the field cut into
    ``G`` equal groups of copies (each frequency's copies in G contiguous
    ranges, a multiple of 4 each) that each fit one walk, as ``(n, start,
    stop)`` per frequency; ``()`` when no such cut exists.  A depthwise
    kernel maps every copy to itself from one radial trunk, so the groups'
    outputs side by side are the layer's."""
    a0 = ft.multiplicity(0) if 0 in ft else 0
    complex_copies = sum(ft.multiplicity(n) for n in ft.frequencies if n != 0)
    if a0 <= 16 * NS and complex_copies <= 4 * NC:
        return None
    g = max(-(-a0 // (16 * NS)), -(-complex_copies // (4 * NC)))
    if any(m % (4 * g) for m in ft.multiplicities):
        return ()
    return tuple(tuple((n, k * m // g, (k + 1) * m // g) for n, m in ft.items()) for k in range(g))


def eligible(kernel: Any, x: Any, edges: Any) -> bool:
    if not ENABLED or x.dtype != torch.float32 or x.device.type != "cuda":
        return False
    layers = list(kernel.radial_trunk)
    if len(layers) != 2 or not isinstance(layers[0], nn.Linear) or not isinstance(layers[1], nn.SiLU):
        return False
    if layers[0].out_features != 16 or layers[0].in_features not in (4, 6, 8):
        return False
    ft = kernel.field_type
    if any(n > 2 for n in ft.frequencies) or any(m % 4 for m in ft.multiplicities):
        return False
    if channel_groups(ft) == ():
        return False
    return edges.max_frequency >= 4 and edges.n_edges > 0


class Packing:
    """Where every row of the packed readout comes from, the complex tiles and,
    for a group of copies (``(n, start, stop)`` per frequency; None: every
    copy), the node field's columns the group reads, in the walk's layout."""

    def __init__(self, kernel: Any, device: torch.device, group: tuple[tuple[int, int, int], ...] | None = None):
        ft = kernel.field_type
        ranges = {n: (0, m) for n, m in ft.items()} if group is None else {n: (c0, c1) for n, c0, c1 in group}
        full_a0 = ft.multiplicity(0) if 0 in ft else 0
        wc = sum(4 * ft.multiplicity(n) for n in ft.frequencies if n != 0)
        zero = full_a0 + wc  # index of the zero row in cat(real rows, complex rows, zero)
        rowmap = [zero] * (NT * 16)
        s0, s1 = ranges.get(0, (0, 0))
        a0 = s1 - s0
        for a in range(a0):
            rowmap[a] = s0 + a
        slices = ft.slices()
        columns = list(range(slices[0].start + s0, slices[0].start + s1)) if 0 in ft else []
        tile_n, tile_col = [], []
        copies = []  # (n, copy, coefficient offset, column in the walk's layout) of every complex copy in tile order
        coff = 0
        for n in ft.frequencies:
            if n == 0:
                continue
            an = ft.multiplicity(n)
            c0, c1 = ranges[n]
            for cidx in range(c0, c1):
                copies.append((n, cidx, coff, len(columns)))
                columns += [slices[n].start + 2 * cidx, slices[n].start + 2 * cidx + 1]
            coff += 4 * an
        for u, (n, cidx, off, col) in enumerate(copies):
            m, q = divmod(u, 4)
            an = ft.multiplicity(n)
            base = 16 * (NS + m) + 4 * q
            for r, src in enumerate((off + 2 * cidx, off + 2 * cidx + 1, off + 2 * an + 2 * cidx,
                                     off + 2 * an + 2 * cidx + 1)):
                rowmap[base + r] = full_a0 + src
            if q == 0:
                tile_n.append(n)
                tile_col.append(col)
        self.columns = None if group is None else torch.tensor(columns, dtype=torch.int64, device=device)
        self.a0 = a0
        self.ns = (a0 + 15) // 16
        self.rowmap = torch.tensor(rowmap, dtype=torch.int64, device=device)
        self.tiles = torch.tensor([tile_n, tile_col], dtype=torch.int32).reshape(2, len(tile_n)).contiguous()
        # the A operands' gathers: rf[m, s, l] = R[16 m + l % 16, 4 (l // 16) + s], rb[m, r, l] = R[16 m + 4 (l // 16) + r, l % 16]
        lanes = torch.arange(64)
        m = torch.arange(NT).view(NT, 1, 1)
        s = torch.arange(4).view(1, 4, 1)
        qq = (lanes // 16).view(1, 1, 64)
        self.rf_rows = (16 * m + (lanes % 16).view(1, 1, 64)).expand(NT, 4, 64).reshape(-1).to(device)
        self.rf_cols = (4 * qq + s).expand(NT, 4, 64).reshape(-1).to(device)
        r = torch.arange(4).view(1, 4, 1)
        self.rb_rows = (16 * m + 4 * qq + r).expand(NT, 4, 64).reshape(-1).to(device)
        self.rb_cols = (lanes % 16).view(1, 1, 64).expand(NT, 4, 64).reshape(-1).to(device)
        # dR's lane layout back to rows: raw[m * 256 + (16 q + k) * 4 + r] = dR[16 m + 4 q + r, k]
        rows = torch.arange(NT * 16).view(-1, 1)
        tile, within = rows // 16, rows % 16
        kk = torch.arange(16).view(1, -1)
        self.dr_index = (tile * 256 + (16 * (within // 4) + kk) * 4 + within % 4).reshape(-1).to(device)
        rb = kernel.radial_basis
        self.centers = [float(c) for c in rb.centers.detach().cpu().tolist()]
        self.width = float(rb.width)


def packing(kernel: Any, device: torch.device, group: tuple | None = None) -> Packing:
    key = ("_radial_packing", str(device), group)
    p = kernel.__dict__.get(key)
    if p is None:
        p = Packing(kernel, device, group)
        kernel.__dict__[key] = p
    return p


def packed_readout(kernel: Any, p: Packing) -> Tensor:
    """``R (NT * 16, 17)``: the heads' rows (weights, then bias) in tile order, zero rows padding."""
    parts = []
    for head in (kernel.real_head, kernel.complex_head):
        if head is None:
            continue
        bias = head.bias if head.bias is not None else head.weight.new_zeros(head.out_features)
        parts.append(torch.cat([head.weight, bias.unsqueeze(1)], dim=1))
    table = torch.cat(parts + [parts[0].new_zeros(1, 17)], dim=0)
    return table.index_select(0, p.rowmap)


class ConvRadial(torch.autograd.Function):
    """``out (N, D)`` from ``v``, the packed readout ``R`` and the trunk's ``(W1, b1)``."""

    @staticmethod
    def forward(ctx: Any, v: Tensor, R: Tensor, w1: Tensor, b1: Tensor | None, meta: dict) -> Tensor:
        p: Packing = meta["packing"]
        rf = R[p.rf_rows, p.rf_cols].contiguous()
        rbias = R[:, 16].contiguous()
        g = meta["geometry"]
        with torch.profiler.record_function("gm::conv/radial_fused"):
            out = _native.conv_radial_forward(v, rf, rbias, w1.contiguous(), None if b1 is None else b1.contiguous(),
                                              meta["centers"], meta["width"], g.transport, g.angular, g.rho,
                                              meta["weights"], g.row_ptr, g.source, p.a0, p.ns, p.tiles)
        ctx.save_for_backward(v, R, w1, b1 if b1 is not None else torch.empty(0, device=v.device), rf, rbias)
        ctx.meta = meta
        ctx.has_b1 = b1 is not None
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad: Tensor) -> tuple:
        v, R, w1, b1, rf, rbias = ctx.saved_tensors
        meta = ctx.meta
        p: Packing = meta["packing"]
        g = meta["geometry"]
        rb = R[p.rb_rows, p.rb_cols].contiguous()
        with torch.profiler.record_function("gm::conv/radial_fused_backward"):
            dv, flat = _native.conv_radial_backward(grad.contiguous(), v, rf, rbias, rb, w1.contiguous(),
                                                    b1.contiguous() if ctx.has_b1 else None, meta["centers"],
                                                    meta["width"], g.transport, g.angular, g.rho, meta["weights"],
                                                    g.source, g.row_ptr, p.a0, p.ns, p.tiles)
        n_dr = NT * 256
        dR = torch.cat([flat[:n_dr].index_select(0, p.dr_index).view(NT * 16, 16),
                        flat[n_dr:n_dr + NT * 16].view(NT * 16, 1)], dim=1)
        trunk = flat[n_dr + NT * 16:]
        nb = w1.shape[1]
        dw1 = trunk[:16 * 8].view(16, 8)[:, :nb].contiguous()
        db1 = trunk[16 * 8:16 * 8 + 16].contiguous() if ctx.has_b1 else None
        return dv, dR, dw1, db1, None


def _ungroup(kernel: Any, groups: tuple, device: torch.device) -> Tensor:
    """For every column of the flat layout, its position in the groups' outputs side by side."""
    key = ("_radial_ungroup", str(device))
    inv = kernel.__dict__.get(key)
    if inv is None:
        cols = torch.cat([packing(kernel, device, g).columns for g in groups]).cpu()
        inv = torch.empty_like(cols)
        inv[cols] = torch.arange(cols.shape[0])
        inv = inv.to(device)
        kernel.__dict__[key] = inv
    return inv


def forward(conv: Any, v: Tensor, edges: Any) -> Tensor:
    """The depthwise layer's aggregation ``(N, D)`` on the flat node field
    ``v``: one walk, or one walk per group of copies for fields wider than a
    walk takes (each group reading its columns of ``v``, sharing the trunk)."""
    kernel = conv.kernel
    g = fused_attention.geometry(edges, conv.cutoff, conv.window, v.dtype)
    trunk = list(kernel.radial_trunk)[0]
    weights = g.aggregation_weights(bool(conv.normalize), float(conv.eps))
    groups = channel_groups(kernel.field_type)
    v = v.contiguous()
    outs = []
    for group in (None,) if groups is None else groups:
        p = packing(kernel, v.device, group)
        meta = dict(packing=p, geometry=g, weights=weights, centers=p.centers, width=p.width)
        vg = v if group is None else v.index_select(1, p.columns)
        outs.append(ConvRadial.apply(vg, packed_readout(kernel, p), trunk.weight, trunk.bias, meta))
    if groups is None:
        return outs[0]
    return torch.cat(outs, dim=1).index_select(1, _ungroup(kernel, groups, v.device))
