"""The factored kernel's node-side channel mixing, ``Z_t(j) = W_t v_j``, as
real matrix products.

The reference forms it as one complex ``einsum("ja,bat->jtb")`` per node
vector (``nn/kernels.py:575-603``).  Here every node vector's blocks become
one real matrix ``M`` of ``(width of the vector's reals, K * sum b_m * 2)``
that encodes the complex product and the conjugation of the input, so the
mixing is one dense real product ``X_n M`` over the node field's frequency-n
columns (``x_0`` or the ``(a_n, 2)`` pairs of ``x_n``).  ``M`` is built from
the kernel's parameters by differentiable torch ops, so the parameters'
gradients follow from autograd on the product.
"""

from __future__ import annotations

import torch
from torch import Tensor

from gm_attention_amd.representations import so2
from gm_attention_amd.representations.field_type import SO2FeatureField


def mixing_matrix(weights: Tensor, kind: str) -> Tensor:
    """The real ``M`` with ``X M = (re, im)`` of ``sum_a v_a W[b, a, t]`` laid out
    ``(t, b, re/im)``: ``weights`` is ``(sum b, a, K)``, complex (real for the
    real block); ``kind`` is ``"real"``, ``"plain"`` (``v = x_0`` or ``x_n``) or
    ``"conj"`` (``v = conj(x_n)``), and ``promote`` marks a real ``x_0`` read by
    complex blocks."""
    b, a, k = weights.shape
    if kind == "real":
        return weights.permute(1, 2, 0).reshape(a, k * b)  # (a, t, b)
    wr, wi = weights.real.permute(1, 2, 0), weights.imag.permute(1, 2, 0)  # (a, t, b)
    if kind == "promote":  # real x_0 times complex W
        return torch.stack([wr, wi], dim=-1).reshape(a, k * b * 2)
    sign = -1.0 if kind == "conj" else 1.0  # d/d(imag part): (-Wi, Wr) for v, (Wi, -Wr) for conj(v)
    # row 2a is the input's real part, row 2a + 1 its imaginary part
    from_real = torch.stack([wr, wi], dim=-1)  # (a, t, b, 2)
    from_imag = torch.stack([-sign * wi, sign * wr], dim=-1)
    return torch.stack([from_real, from_imag], dim=1).reshape(2 * a, k * b * 2)


def node_products(kernel, x: SO2FeatureField) -> dict[tuple[int, int, str], Tensor]:
    """``(n_nodes, K, b_m)`` per block, complex except the real block: one real
    product per node-vector group, all of them in one :class:`NodeMixes` call
    where the MFMA kernels serve it."""
    products: dict[tuple[int, int, str], Tensor] = {}
    n_nodes = x.batch_shape[0]
    groups = []
    for (n, kind), blocks in kernel.node_vector_groups():
        weights = torch.cat([kernel._block_weights(b) for b in blocks], dim=0)  # (sum b, a_n, K)
        mode = "real" if kind == "real" else ("promote" if n == 0 else kind)
        groups.append((n, kind, blocks, weights.shape[-1], mixing_matrix(weights, mode)))
    rows = x._rows()
    slices = x.field_type.slices()
    columns = tuple((slices[n].start, slices[n].stop - slices[n].start) for n, *_ in groups)
    mats = [g[4] for g in groups]
    with torch.profiler.record_function("gm::kernel/node_products"):
        if mixes_eligible(rows, [w for _, w in columns], mats):
            flats = NodeMixes.apply(rows, columns, *[m.to(torch.float32) for m in mats])
        else:
            flats = [(x[0] if n == 0 else x[n].reshape(n_nodes, -1)) @ m.to(x.dtype)
                     for (n, *_), m in zip(groups, mats, strict=True)]
    for (n, kind, blocks, k, _), flat in zip(groups, flats, strict=True):
        widths = [kernel.field_type_out.multiplicity(m) for _, m, _ in blocks]
        mixed = flat.reshape(n_nodes, k, -1) if kind == "real" else so2.as_complex(flat.reshape(n_nodes, k, -1, 2))
        for block, piece in zip(blocks, torch.split(mixed, widths, dim=-1), strict=True):
            products[block] = piece
    return products


class NodeMixes(torch.autograd.Function):
    """Every head's node mixes ``X_n M_n`` for each input frequency n on the
    HIP MFMA kernels (``gm_node_mix_*``), read straight from the flat node rows.

    ``rows`` is the flat node field ``(N, D)`` (float32, GPU), ``columns`` the
    ``(offset, width)`` of the reals each product reads in it (products may
    read the same columns), then one mixing matrix ``(width, C_n)`` per
    product; out one ``(N, C_n)`` mix array per product.  The backward writes
    the input gradients into one ``(N, D)`` gradient (adding where products
    share columns) and sums each matrix's gradient over the nodes in a fixed
    order (deterministic)."""

    @staticmethod
    def forward(ctx, rows: Tensor, columns: tuple[tuple[int, int], ...], *mats: Tensor) -> tuple[Tensor, ...]:
        from gm_attention_amd import _native

        mats = tuple(m.contiguous() for m in mats)
        with torch.profiler.record_function("gm::kernel/node_products"):
            outs = tuple(_native.node_mix_forward(rows[:, off:off + w], m) for (off, w), m in zip(columns, mats,
                                                                                                  strict=True))
        ctx.columns = columns
        ctx.save_for_backward(rows, *mats)
        return outs

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, *dmixes: Tensor) -> tuple:
        from gm_attention_amd import _native

        rows, *mats = ctx.saved_tensors
        columns = ctx.columns
        dx = None
        with torch.profiler.record_function("gm::kernel/node_products_backward"):
            if ctx.needs_input_grad[0]:
                # each column range is written by its first product and added to by any later one reading it
                ranges = sorted(columns)
                disjoint = all(a[0] + a[1] <= b[0] for a, b in zip(ranges, ranges[1:]))
                covered = (disjoint and sum(w for _, w in columns) == rows.shape[1]
                           and all(d is not None for d in dmixes))
                # the input gradient in float32 (bfloat16 rows: autograd rounds it into their dtype)
                dx = (torch.empty if covered else torch.zeros)(rows.shape, dtype=torch.float32, device=rows.device)
                written: list[tuple[int, int]] = []
                for (off, w), m, d in zip(columns, mats, dmixes, strict=True):
                    if d is None:
                        continue
                    if any(off < o + ww and o < off + w for o, ww in written):
                        part = torch.empty(rows.shape[0], w, dtype=torch.float32, device=rows.device)
                        _native.node_mix_backward_input(d.contiguous(), m, part)
                        dx[:, off:off + w] += part
                    else:
                        _native.node_mix_backward_input(d.contiguous(), m, dx[:, off:off + w])
                    written.append((off, w))
            dmats = []
            for i, ((off, w), m, d) in enumerate(zip(columns, mats, dmixes, strict=True)):
                if not ctx.needs_input_grad[2 + i]:
                    dmats.append(None)
                elif d is None:
                    dmats.append(torch.zeros_like(m))
                else:
                    dmats.append(_native.node_mix_backward_weight(rows[:, off:off + w], d.contiguous()))
        return (dx, None, *dmats)


def mixes_eligible(rows: Tensor, widths: list[int], mats: list[Tensor]) -> bool:
    """Whether :class:`NodeMixes` serves these products: float32 flat rows on
    the GPU with node vectors at most 128 reals wide, or bfloat16 rows with
    vectors at most 64 wide (float32 mixes either way); mix widths a multiple of 4."""
    widest = 128 if rows.dtype == torch.float32 else (64 if rows.dtype == torch.bfloat16 else 0)
    return (rows.device.type == "cuda" and rows.dim() == 2 and all(1 <= w <= widest for w in widths)
            and all(m.shape[1] % 4 == 0 for m in mats))
