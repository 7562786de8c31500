"""The fused ops' contracts in plain torch: what a layer runs when the fused
path declines a call.

The reference's layers fall back to their eager torch path whenever a fused
op's predicate declines (CPU tensors, a ``GM_FUSED_*`` switch at ``"0"``,
shapes beyond the kernels' bounds: reference nn/attention.py:880-886,
nn/kernels.py:671-672 / 724-725 / 762-763, nn/convolution.py:297-308).  This
module is this build's eager path: each function evaluates the same numbers as
its HIP op from the same plans and descriptor rows the kernels consume
(``fused_attention.Plan``, ``fused_factored.Plan``, ``fused_pairs.plan``),
with autograd for the gradients, on any device and in any float dtype.

``calls`` counts the evaluations, so a test of the HIP path can assert that
none of its work fell back here.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor

#: evaluations taken by this module since import (per function name)
calls: dict[str, int] = {}


def _count(name: str) -> None:
    calls[name] = calls.get(name, 0) + 1


def _targets(row_ptr: Tensor) -> Tensor:
    return torch.repeat_interleave(torch.arange(row_ptr.shape[0] - 1, device=row_ptr.device),
                                   row_ptr[1:] - row_ptr[:-1])


def _phase(table: Tensor, order: int) -> Tensor:
    """``e^{i order angle}`` per edge from a complex ``(E, K + 1)`` harmonic table."""
    column = table[:, abs(order)]
    return column.conj() if order < 0 else column


def segment_sum(values: Tensor, row_ptr: Tensor) -> Tensor:
    """Per target, the sum of its CSR segment of ``values`` (first axis)."""
    out = values.new_zeros((row_ptr.shape[0] - 1, *values.shape[1:]))
    return out.index_add_(0, _targets(row_ptr), values)


# ---------------------------------------------------------------- scores and softmax


def softmax(q: Tensor, k: Tensor, transport: Tensor, bias: Tensor, inside: Tensor, rows, row_ptr: Tensor,
            source: Tensor, heads: int, scale: float) -> Tensor:
    """``Softmax.apply``'s numbers (reference fused/attention.h:145-165, 295-316):
    ``alpha (E, H)``, the softmax over each target's edges with ``inside`` of
    ``scale sum_n Re<q_i,n,h, tau_n k_j,n,h> + bias``.  ``q``, ``k`` are flat
    ``(N, D)`` rows laid out by ``rows`` (the plan's ``(n, a_n, offset, -, dim)``
    per frequency, heads' copies head-major); ``transport`` is ``(E, orders, 2)``."""
    _count("softmax")
    target = _targets(row_ptr)
    E = source.shape[0]
    score = q.new_zeros(E, heads)
    for n, a, off, _coff, dim in rows:
        width = heads * a * dim
        qe = q[:, off:off + width].index_select(0, target).reshape(E, heads, a, dim)
        ke = k[:, off:off + width].index_select(0, source).reshape(E, heads, a, dim)
        if n:
            c, s = transport[:, n, 0].reshape(E, 1, 1), transport[:, n, 1].reshape(E, 1, 1)
            k0, k1 = ke[..., 0], ke[..., 1]
            ke = torch.stack((c * k0 - s * k1, c * k1 + s * k0), dim=-1)
        score = score + (qe * ke).sum(dim=(2, 3))
    logits = (scale * score + bias.unsqueeze(-1)).masked_fill(~inside.bool().unsqueeze(-1), float("-inf"))
    peak = torch.segment_reduce(logits.detach(), "max", offsets=row_ptr, axis=0)
    peak = torch.where(torch.isfinite(peak), peak, torch.zeros_like(peak))
    u = torch.exp(logits - peak.index_select(0, target))
    return u / segment_sum(u, row_ptr).clamp_min(torch.finfo(u.dtype).tiny).index_select(0, target)


# ---------------------------------------------------------------- factored value kernels


def factored_rows(kernel: Any, x, edges, products: dict | None = None) -> Tensor:
    """The factored op's per-edge rows ``(E, d_out)`` (reference
    fused/factored.h:158-250): for every descriptor block, the block's factor
    ``e^{i a phi} e^{i s gamma} (r/c)^p`` times ``sum_t h~_t Z_t(source)``,
    its real part onto the scalars, accumulated at the block's output
    columns.  ``Z`` are the kernel's node products (the real block's real)."""
    from gm_attention_amd.nn import fused_factored

    _count("factored")
    p = fused_factored.plan(kernel)
    if products is None:
        products = kernel.node_products(x)
    source = edges.source_index
    hidden = kernel._trunk_hidden(edges.distances)
    h = torch.cat([torch.ones_like(hidden[:, :1]), hidden], dim=1)  # (E, K): the bias rides on t = 0
    rho = edges.distances / kernel.radial_basis.cutoff
    E = source.shape[0]
    rows = hidden.new_zeros(E, p.d_out)
    for b in p.blocks:
        z = products[b.block].index_select(0, source)  # (E, K, b_m)
        combined = torch.einsum("et,etb->eb", h.to(z.dtype), z)
        if b.kind == 0:
            rows[:, b.out_offset:b.out_offset + b.b_m] += combined
            continue
        factor = _phase(edges.angular_phases, b.angular) * _phase(edges.transport_phases, b.transport)
        factor = factor * rho.pow(b.power).to(factor.dtype) if b.power else factor
        term = factor.unsqueeze(-1) * combined
        if b.take_real:
            rows[:, b.out_offset:b.out_offset + b.b_m] += term.real
        else:
            rows[:, b.out_offset:b.out_offset + 2 * b.b_m] += torch.view_as_real(term).reshape(E, 2 * b.b_m)
    return rows


# ---------------------------------------------------------------- per-edge readout (pair terms)


def readout(kernel: Any, x, edges) -> dict[int, Tensor]:
    """The pair terms' per-edge messages (reference fused/pairs.h:1-22): for each
    term of ``fused_pairs.plan``, the block ``M(e) = W h(e) + b`` (complex when
    the flags say so) applied to the (conjugated, phase-rotated) transported
    input, times the radial power, the post phase or the real part; ``x`` is
    edge-shaped (the source field gathered to the edges)."""
    from gm_attention_amd.nn import fused_pairs

    _count("readout")
    hidden = kernel._trunk_hidden(edges.distances)
    rho = edges.distances / kernel.radial_basis.cutoff
    E = hidden.shape[0]
    cplx = torch.complex64 if hidden.dtype == torch.float32 else torch.complex128
    out = {m: hidden.new_zeros(E, kernel.field_type_out.multiplicity(m), dtype=hidden.dtype if m == 0 else cplx)
           for m in kernel.field_type_out.frequencies}
    for t in fused_pairs.plan(kernel):
        head = kernel.real_head if t.real_head else kernel.complex_head
        coeff = hidden @ head.weight[t.rows].T
        if head.bias is not None:
            coeff = coeff + head.bias[t.rows]
        if t.flags & fused_pairs.MATRIX_COMPLEX:
            block = torch.view_as_complex(coeff.reshape(E, t.b, t.a, 2).contiguous())
        else:
            block = coeff.reshape(E, t.b, t.a)
        if t.n == 0:
            u = x[0].to(block.dtype)
        else:
            u = _phase(edges.transport_phases, t.n).unsqueeze(-1) * torch.view_as_complex(x[t.n].contiguous())
            if t.flags & fused_pairs.CONJ_U:
                u = u.conj()
        if t.pre_order is not None:
            u = _phase(edges.angular_phases, t.pre_order).unsqueeze(-1) * u
        y = torch.matmul(block, u.unsqueeze(-1)).squeeze(-1)
        if t.power:
            y = y * rho.pow(t.power).unsqueeze(-1).to(y.dtype)
        if t.post_order is not None:
            y = _phase(edges.angular_phases, t.post_order).unsqueeze(-1) * y
        out[t.m] = out[t.m] + (y.real if t.flags & fused_pairs.OUT_REAL and y.is_complex() else y)
    return {m: v if m == 0 else torch.view_as_real(v) for m, v in out.items()}


# ---------------------------------------------------------------- depthwise kernel


def depthwise_messages(kernel: Any, x, edges) -> dict[int, Tensor]:
    """``SO2DepthwiseKernel.forward`` (reference nn/depthwise.py:147-193) on an
    edge-shaped field: ``C x_0`` on the scalars and, per copy of frequency n,
    ``A z + (r/c)^{2n} e^{2 i n phi} B conj(z)`` with ``z`` the transported copy;
    the coefficients are the kernel's readouts laid out ``(2, a_n, 2)`` per
    frequency (``A | B``, copy, re/im)."""
    from gm_attention_amd.nn.depthwise import stacked_coefficients

    _count("depthwise")
    rc, cc = stacked_coefficients([kernel], edges)
    ft = kernel.field_type
    rho = edges.distances / kernel.cutoff
    E = edges.distances.shape[0]
    out: dict[int, Tensor] = {}
    if rc is not None:
        out[0] = rc[0] * x[0]
    start = 0
    for n in ft.frequencies:
        if n == 0:
            continue
        a = ft.multiplicity(n)
        block = torch.view_as_complex(cc[0, :, start:start + 4 * a].reshape(E, 2, a, 2).contiguous())
        start += 4 * a
        z = _phase(edges.transport_phases, n).unsqueeze(-1) * torch.view_as_complex(x[n].contiguous())
        w = (rho.pow(2 * n).to(z.dtype) * _phase(edges.angular_phases, 2 * n)).unsqueeze(-1)
        out[n] = torch.view_as_real(block[:, 0] * z + w * block[:, 1] * z.conj())
    return out
