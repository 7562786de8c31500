"""The reference's eager (pure-PyTorch) path, restated in float64 at the
fused ops' boundary.  TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Every function takes the same tensors as the corresponding fused op and
recomputes its result the way the reference's eager code does: gather to
edges, transport, per-edge arithmetic, segment reductions.  Gradients come
from autograd on the returned tensor, which is what the reference's eager
path differentiates.
"""

from __future__ import annotations

import torch
from torch import Tensor


def targets_of(row_ptr: Tensor) -> Tensor:
    n = row_ptr.shape[0] - 1
    return torch.repeat_interleave(torch.arange(n, device=row_ptr.device), row_ptr[1:] - row_ptr[:-1])


def _phase(table: Tensor, order: int) -> Tensor:
    """``exp(i order x)`` from an ``(E, K + 1, 2)`` real table; a negative order is
    the conjugate (reference EdgeGeometry._harmonic, edge_geometry.py:135-157)."""
    col = torch.complex(table[:, abs(order), 0], table[:, abs(order), 1])
    return col.conj() if order < 0 else col


def _pairs(block: Tensor) -> Tensor:
    return torch.view_as_complex(block.reshape(*block.shape[:-1], -1, 2).clone())


def softmax_op(q: Tensor, k: Tensor, transport: Tensor, bias: Tensor, inside: Tensor, rows, row_ptr: Tensor,
               source: Tensor, heads: int, scale: float) -> Tensor:
    """alpha (E, H): ``_softmax_weights`` of nn/attention.py:825-855 with the
    window and quadrature terms given as ``bias = log c + log w`` and the
    support as ``inside`` (their construction: fused_attention.py:234-247).

    * query gathered by target, key by source, the key transported by
      ``exp(i n gamma)`` per frequency (kernels.py:156-189);
    * per head, the scores summed over frequencies and copies, times ``scale``;
    * ``masked_fill(-inf)`` outside the window, a detached per-target max,
      ``exp``, a per-target sum, the division (attention.py:839-855).
    """
    E = source.shape[0]
    target = targets_of(row_ptr)
    qe, ke = q.index_select(0, target), k.index_select(0, source)
    score = torch.zeros(E, heads, dtype=q.dtype)
    for n, a, off, _coff, dim in rows:
        width = heads * a * dim
        qb, kb = qe[:, off:off + width], ke[:, off:off + width]
        if n != 0:
            tk = _phase(transport, n).unsqueeze(-1) * _pairs(kb)
            kb = torch.view_as_real(tk).reshape(E, width)
        score = score + (qb * kb).reshape(E, heads, -1).sum(-1)
    score = score * scale
    log_weight = (score + bias.unsqueeze(-1)).masked_fill(~inside.bool().unsqueeze(-1), float("-inf"))
    node_max = torch.segment_reduce(log_weight, "max", offsets=row_ptr, axis=0).detach()
    u = torch.exp(log_weight - node_max.index_select(0, target))
    norm = torch.segment_reduce(u, "sum", offsets=row_ptr, axis=0)
    return u / norm.index_select(0, target)


def depthwise_messages(v: Tensor, rc: Tensor, cc: Tensor, transport: Tensor, angular: Tensor, rho: Tensor, rows,
                       source: Tensor) -> Tensor:
    """Per-edge messages (E, D) of SO2DepthwiseKernel.forward (depthwise.py:147-193)
    from the readouts as the fused op receives them: rc (E, a_0), and per
    frequency n >= 1 the (2, a_n, 2) block of cc at its coefficient offset --
    A = C[:, 0], B = C[:, 1] -- with m = A z + (r/c)^{2n} e^{2 i n phi} B conj(z),
    z = exp(i n gamma) v_j; the radial power by repeated multiplication."""
    E = source.shape[0]
    ve = v.index_select(0, source)
    out = []
    for n, a, off, coff, dim in rows:
        if n == 0:
            out.append(rc.reshape(E, -1)[:, :a] * ve[:, off:off + a])
            continue
        z = _phase(transport, n).unsqueeze(-1) * _pairs(ve[:, off:off + 2 * a])
        block = cc.reshape(E, -1)[:, coff:coff + 4 * a].reshape(E, 2, a, 2)
        A = torch.view_as_complex(block[:, 0].contiguous())
        B = torch.view_as_complex(block[:, 1].contiguous())
        scale = torch.ones_like(rho)
        for _ in range(2 * n):
            scale = scale * rho
        w = (scale * _phase(angular, 2 * n)).unsqueeze(-1)
        out.append(torch.view_as_real(A * z + w * B * z.conj()).reshape(E, 2 * a))
    return torch.cat(out, dim=-1)


def conv_op(v: Tensor, rc: Tensor, cc: Tensor, transport: Tensor, angular: Tensor, rho: Tensor, weights: Tensor,
            rows, row_ptr: Tensor, source: Tensor) -> Tensor:
    """The depthwise convolution's aggregation: the weighted segment sum of the
    messages (convolution.py:310-355 with the fused path's given weights)."""
    m = depthwise_messages(v, rc, cc, transport, angular, rho, rows, source)
    return torch.segment_reduce(weights.unsqueeze(-1) * m, "sum", offsets=row_ptr, axis=0)


# ---------------------------------------------------------------- factored steerable kernel


def _block_factor(angular: Tensor, transport: Tensor, rho: Tensor, ang: int, tr: int, power: int) -> Tensor:
    """``e^{i ang phi} e^{i tr gamma} (r / c)^power`` per edge: the factor of one
    phase-carrying block (kernels.py:615-643), the radial power by repeated
    multiplication as ``_radial_powers`` tabulates it (kernels.py:734-750)."""
    factor = torch.ones(rho.shape[0], dtype=torch.complex128 if rho.dtype == torch.float64 else torch.complex64)
    if ang != 0:
        factor = factor * _phase(angular, ang)
    if tr != 0:
        factor = factor * _phase(transport, tr)
    scale = torch.ones_like(rho)
    for _ in range(power):
        scale = scale * rho
    return factor * scale


def factored_rows(h: Tensor, zc: Tensor, zr: Tensor, angular: Tensor, transport: Tensor, rho: Tensor, blocks,
                  source: Tensor, d_out: int) -> Tensor:
    """The messages ``(E, d_out)`` of ``SO2SteerableKernel.forward_factored``'s
    eager branch (kernels.py:645-697) from the fused op's inputs: per output
    frequency, every block's ``sum_t h~_t Z_t(j)`` (``h~ = (1, h)``; ``Z`` from
    the packed ``zc (N, K, wc, 2)`` / ``zr (N, K, wr)`` of fused_factored.pack,
    fused_factored.py:156-180) times the block's factor, the real part taken
    for the rows onto frequency 0.  ``blocks`` are the descriptor rows
    ``(kind, z_offset, b_m, angular, transport, power, out_offset, take_real)``
    of fused_factored.plan (fused_factored.py:101-139)."""
    E = h.shape[0]
    ht = torch.cat([torch.ones(E, 1, dtype=h.dtype), h], dim=1)  # (E, K)
    zcc = torch.view_as_complex(zc.contiguous()) if zc.shape[2] > 0 else None  # (N, K, wc)
    groups: dict[int, list] = {}
    for row in blocks:
        groups.setdefault(int(row[6]), []).append(row)
    out = torch.zeros(E, d_out, dtype=h.dtype)
    pieces = []
    for offset, rows in sorted(groups.items()):
        scalar = rows[0][0] == 0 or rows[0][7] == 1
        b_m = rows[0][2]
        acc = torch.zeros(E, b_m, dtype=h.dtype if scalar else (zcc.dtype if zcc is not None else h.dtype))
        for kind, zoff, bm, ang, tr, power, _ooff, take_real in rows:
            if kind == 0:
                mixed = zr.index_select(0, source)[:, :, zoff:zoff + bm]  # (E, K, b)
                acc = acc + (ht.unsqueeze(-1) * mixed).sum(dim=1)
                continue
            mixed = zcc.index_select(0, source)[:, :, zoff:zoff + bm]  # (E, K, b) complex
            combined = (ht.unsqueeze(-1) * mixed).sum(dim=1)
            term = _block_factor(angular, transport, rho, ang, tr, power).unsqueeze(-1) * combined
            acc = acc + (term.real if take_real else term)
        flat = acc if scalar else torch.view_as_real(acc).reshape(E, 2 * b_m)
        pieces.append((offset, flat))
    cols = []
    for offset, flat in pieces:
        cols.append(flat)
    result = torch.cat(cols, dim=1) if cols else out
    if result.shape[1] != d_out:
        raise ValueError("the blocks' output groups must tile the flat output row")
    return result


def factored_aggregate(rows: Tensor, weights: Tensor, row_ptr: Tensor) -> Tensor:
    """``out_i = sum_{e -> i} w_e rows_e`` (kernels.py:715-725 with
    _scatter.py:36-58's segment sum)."""
    return torch.segment_reduce(weights.unsqueeze(-1) * rows, "sum", offsets=row_ptr, axis=0)


def pair_term(hidden: Tensor, weight: Tensor, bias: Tensor | None, u: Tensor, pre: Tensor | None, post: Tensor | None,
              scale: Tensor | None, a: int, b: int, flags: int) -> Tensor:
    """One fused pair term's contribution (E, b) (reference nn/fused/pairs.h:1-22
    and forward_edge :286-309): M(e) = W h(e) + bias as a (b, a) block, complex
    from (re, im) row pairs under MATRIX_COMPLEX (1); uu = pre * u~ with u~ =
    conj(u) under CONJ_U (4) or a real u promoted under U_REAL (2); q = M uu;
    Re(q) * scale under OUT_REAL (8), else post * scale * q."""
    E = hidden.shape[0]
    m = hidden @ weight.T + (bias if bias is not None else 0.0)
    if flags & 1:
        M = torch.complex(m[:, 0::2], m[:, 1::2]).reshape(E, b, a)
    else:
        M = m.reshape(E, b, a).to(torch.complex128 if hidden.dtype == torch.float64 else torch.complex64)
    uu = u.to(M.dtype) if flags & 2 else (u.conj() if flags & 4 else u)
    if pre is not None:
        uu = pre.unsqueeze(-1) * uu
    q = (M * uu.unsqueeze(-2)).sum(-1)
    s = scale if scale is not None else torch.ones(E, dtype=hidden.dtype)
    if flags & 8:
        return q.real * s.unsqueeze(-1)
    p = (post if post is not None else torch.ones(E, dtype=M.dtype)) * s
    return p.unsqueeze(-1) * q
