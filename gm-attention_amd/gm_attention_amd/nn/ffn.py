"""The transformer block's feed-forward as one fused HIP pass per direction.

Replaces, for bfloat16 rows, the sequence of ``SO2TransformerBlock.forward``
after the mixer (reference ``nn/blocks.py:326-349``): ``norm2`` (the merged
equivariant layer norm, ``nn/normalization.py:117-178``), ``linear1``
(``nn/linear.py:130-190``), the scalar gate (``nn/nonlinearities.py:140-166``),
``linear2`` and the residual sum, with the dropout inactive.  The forward is
one kernel on the bf16 matrix cores (``gm_ffn_forward_bf16``): no hidden
activation reaches memory.  The backward kernel (``gm_ffn_backward_bf16``)
recomputes the forward from the saved statistics and returns ``dx`` with the
factors of the parameter gradients, whose products (``x^T g`` over the nodes)
run on the node-mix weight-gradient kernels in a fixed order (the factors in
bfloat16, widened exactly, the products float32-accurate).

Served: frequencies 0, 1, 2 with 32 copies each, the hidden field 64 or 128
copies of each (``ffn_multiplier`` 2 or 4), CUDA bfloat16 rows, the split
products on (their weight-gradient kernels read the bfloat16 factors);
``GM_FUSED_FFN=0`` keeps the separate passes.
"""

from __future__ import annotations

import os
from typing import Any

import torch
from torch import Tensor

from gm_attention_amd import _native
from gm_attention_amd.nn.linear import complex_as_real
from gm_attention_amd.nn.nonlinearities import SO2ScalarGatedNonlinearity
from gm_attention_amd.nn.normalization import SO2LayerNorm

ENABLED = os.environ.get("GM_FUSED_FFN", "1") != "0" and os.environ.get("GM_SPLIT_PRODUCTS", "1") != "0"
A_SERVED, B_SERVED = (32,), (64, 128)


def _uniform(field_type: Any, copies: tuple[int, ...]) -> int | None:
    """The common multiplicity when the field is frequencies 0, 1, 2 with equal copies among ``copies``."""
    items = dict(field_type.items())
    if sorted(items) != [0, 1, 2] or len(set(items.values())) != 1:
        return None
    m = items[0]
    return m if m in copies else None


def serves(block: Any, rows: Tensor) -> bool:
    """Whether the fused feed-forward runs ``block``'s feed-forward on ``rows``."""
    if not (ENABLED and rows.is_cuda and rows.dtype == torch.bfloat16 and rows.dim() == 2):
        return False
    if block.mlp_dropout.active() or not isinstance(block.norm2, SO2LayerNorm):
        return False
    act = block.activation
    if not isinstance(act, SO2ScalarGatedNonlinearity):
        return False
    return _uniform(block.field_type, A_SERVED) is not None and _uniform(block.hidden_field_type, B_SERVED) is not None


def _real_block(lin: Any, f: int) -> Tensor:
    """Frequency f's block of the layer's flat matrix (``D_in,f x D_out,f``)."""
    w = lin.weight[str(f)]
    return w.t() if f == 0 else complex_as_real(w)


class FusedFFN(torch.autograd.Function):
    """``x + linear2(act(linear1(norm(x))))`` on bfloat16 rows ``x (N, 5A)``.

    Inputs after ``x``: the norm's ``gamma`` (per flat coordinate) and ``beta``,
    the first layer's three frequency blocks and bias, the gates' stacked
    weights and biases, the second layer's blocks and bias (float32; None for
    absent biases), then the static ``meta``.  Gradients for all of them."""

    @staticmethod
    def forward(ctx: Any, x: Tensor, gamma: Tensor, beta: Tensor | None, m1_0: Tensor, m1_1: Tensor, m1_2: Tensor,
                b1: Tensor | None, wg: Tensor, bg: Tensor | None, m2_0: Tensor, m2_1: Tensor, m2_2: Tensor,
                b2: Tensor | None, meta: dict) -> Tensor:
        bf = torch.bfloat16
        m1 = (m1_0, m1_1, m1_2)
        m2 = (m2_0, m2_1, m2_2)
        w1t = [m.t().contiguous().to(bf) for m in m1]
        w2t = [m.t().contiguous().to(bf) for m in m2]
        wgb = wg.contiguous().to(bf)
        vec = [None if t is None else t.detach().float().contiguous() for t in (gamma, beta, b1, bg, b2)]
        with torch.profiler.record_function("gm::pointwise/ffn"):
            out, mean, inv_d = _native.ffn_forward(x.contiguous(), meta["A"], meta["B"], meta["eps"], meta["dsig"],
                                                   vec[0], vec[1], w1t, vec[2], wgb, vec[3], w2t, vec[4])
        ctx.meta = meta
        ctx.has = tuple(t is not None for t in (beta, b1, bg, b2))
        ctx.w1t, ctx.w2t, ctx.wg = w1t, w2t, wgb
        ctx.w1n = [m.contiguous().to(bf) for m in m1]
        ctx.w2n = [m.contiguous().to(bf) for m in m2]
        ctx.wgt = wg.t().contiguous().to(bf)
        ctx.vec = vec
        ctx.save_for_backward(x, mean, inv_d)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, dz: Tensor) -> tuple:
        x, mean, inv_d = ctx.saved_tensors
        meta = ctx.meta
        A, B = meta["A"], meta["B"]
        gamma, beta, b1, bg, _ = ctx.vec
        dz = dz.to(torch.bfloat16).contiguous()
        with torch.profiler.record_function("gm::pointwise/ffn_backward"):
            r = _native.ffn_backward(dz, x, A, B, meta["eps"], meta["dsig"], gamma, beta, ctx.w1t, ctx.w1n, b1,
                                     ctx.wg, ctx.wgt, bg, ctx.w2t, ctx.w2n, mean, inv_d)
        # the parameter gradients: x^T g products over the nodes, a frequency block at a time
        cols = ((0, A), (A, 3 * A), (3 * A, 5 * A))
        dm1 = [_native.node_mix_backward_weight(r["xhat"][:, a:b], r["dhidden"][f]) for f, (a, b) in enumerate(cols)]
        dm2 = [_native.node_mix_backward_weight(dz[:, a:b], r["outs"][f]).t() for f, (a, b) in enumerate(cols)]
        dwg = _native.node_mix_backward_weight(r["hidden0"], r["dpre"]).t()
        has_beta, has_b1, has_bg, has_b2 = ctx.has
        dgamma = r["dgb"][: 5 * A]
        dbeta = r["dgb"][5 * A:] if has_beta else None
        db1 = r["dhidden"][0].float().sum(0) if has_b1 else None
        dbg = r["dpre"].float().sum(0) if has_bg else None
        db2 = dz[:, :A].float().sum(0) if has_b2 else None
        return (r["dx"], dgamma, dbeta, dm1[0], dm1[1], dm1[2], db1, dwg, dbg, dm2[0], dm2[1], dm2[2], db2, None)


def forward(block: Any, rows: Tensor) -> Tensor:
    """``rows + linear2(act(linear1(norm2(rows))))`` through :class:`FusedFFN`
    (the caller has checked :func:`serves`)."""
    norm, act, l1, l2 = block.norm2, block.activation, block.linear1, block.linear2
    A = _uniform(block.field_type, A_SERVED)
    B = _uniform(block.hidden_field_type, B_SERVED)
    order = ("1", "2")
    wg = torch.cat([act.gates[k].weight for k in order])
    gate_bias = [act.gates[k].bias for k in order]
    bg = None if any(b is None for b in gate_bias) else torch.cat(gate_bias)
    meta = dict(A=A, B=B, eps=float(norm.eps), dsig=act.gate == "double_sigmoid")
    return FusedFFN.apply(rows, norm.gamma_flat(torch.float32), norm.beta if norm.has_bias else None,
                          _real_block(l1, 0), _real_block(l1, 1), _real_block(l1, 2), l1.bias if l1.has_bias else None,
                          wg, bg, _real_block(l2, 0), _real_block(l2, 1), _real_block(l2, 2),
                          l2.bias if l2.has_bias else None, meta)
