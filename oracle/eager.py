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
