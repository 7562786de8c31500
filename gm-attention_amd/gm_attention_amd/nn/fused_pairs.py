"""The steerable kernel's per-edge readout as fused pair terms on the HIP path.

Restates the reference's ``nn/fused_pairs.py``: each ``(n, m, role)`` term of
``SO2SteerableKernel._forward_general`` (reference nn/kernels.py:752-915) is
one launch (``gm_pairs_forward``) that forms its ``b_m x a_n`` coefficient
block in registers from the trunk output and the readout rows, applies the
phases and the radial power, and accumulates into the output; the backward is
one launch per term giving the input and trunk gradients and that term's rows
of the coefficient gradient, then one blocked product for the readout
weights' gradient.  Same names, plan and switch as the reference:

* ``MODE = GM_FUSED_PAIRS`` (:39-40): ``"0"`` off, ``"1"`` device tensors,
  ``"cpu"`` accepted (a CPU tensor then raises: this build has no CPU driver);
* ``Term`` / ``plan`` (:96-123), ``enabled`` (:126-149), ``_FusedPairs``
  (:156-238), ``forward_general`` (:249-295).

Every block side and trunk width in ``1..16`` runs the same kernels (the sides
are loop bounds, not compile-time sizes), so ``SUPPORTED`` covers ``1..16``.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any

import torch
from torch import Tensor

from gm_attention_amd import _native
from gm_attention_amd.representations.field_type import SO2FeatureField

MATRIX_COMPLEX, U_REAL, CONJ_U, OUT_REAL = (_native.PAIRS_MATRIX_COMPLEX, _native.PAIRS_U_REAL, _native.PAIRS_CONJ_U,
                                            _native.PAIRS_OUT_REAL)
MAX_MULT = _native.PAIRS_MAX_MULT
MAX_TRUNK = _native.PAIRS_MAX_TRUNK
SUPPORTED = tuple(range(1, MAX_MULT + 1))

#: ``"0"`` off, ``"1"`` on for device tensors, ``"cpu"`` on everywhere (reference :39-40).
MODE = os.environ.get("GM_FUSED_PAIRS", "1")

#: Rows per block of the readout weights' gradient (a sum over every edge).
WEIGHT_GRAD_BLOCK = 16384


def extension(size: tuple[int, int, int] | None = None) -> Any:
    """The pair-term entry points (one build serves every block size)."""
    return _native.pairs()


@dataclass(frozen=True)
class Term:
    n: int
    m: int
    role: str
    flags: int
    a: int
    b: int
    real_head: bool  # rows of the real head (the (0, 0) block) or the complex head
    rows: slice
    pre_order: int | None
    post_order: int | None
    power: int | None


def plan(kernel: Any) -> list[Term]:
    """The terms of the per-edge readout's pair loop, in its order (reference :96-123)."""
    cached = kernel.__dict__.get("_fused_plan")
    if cached is not None:
        return cached
    terms: list[Term] = []
    for m in kernel.field_type_out.frequencies:
        b = kernel.field_type_out.multiplicity(m)
        for n in kernel.field_type_in.frequencies:
            a = kernel.field_type_in.multiplicity(n)
            if n == 0 and m == 0:
                terms.append(Term(n, m, "real", U_REAL | OUT_REAL, a, b, True, slice(0, a * b), None, None, None))
            elif n == 0:
                terms.append(Term(n, m, "linear", MATRIX_COMPLEX | U_REAL, a, b, False,
                                  kernel._pair_ranges[(n, m, "linear")], None, m, kernel._pair_powers[(n, m, "linear")]))
            elif m == 0:
                # Re[A conj(e^{-i n phi} z)] = Re[A (e^{i n phi} conj z)]
                terms.append(Term(n, m, "linear", MATRIX_COMPLEX | CONJ_U | OUT_REAL, a, b, False,
                                  kernel._pair_ranges[(n, m, "linear")], n, None,
                                  kernel._pair_powers[(n, m, "linear")]))
            else:
                terms.append(Term(n, m, "linear", MATRIX_COMPLEX, a, b, False, kernel._pair_ranges[(n, m, "linear")],
                                  m - n, None, kernel._pair_powers[(n, m, "linear")]))
                terms.append(Term(n, m, "antilinear", MATRIX_COMPLEX | CONJ_U, a, b, False,
                                  kernel._pair_ranges[(n, m, "antilinear")], m + n, None,
                                  kernel._pair_powers[(n, m, "antilinear")]))
    kernel.__dict__["_fused_plan"] = terms
    return terms


def enabled(kernel: Any, x: SO2FeatureField, edges: Any) -> bool:
    """Whether this call takes the fused terms (reference :126-149): the mode
    allows the device, float32/64, every block and the trunk within 16, and
    every phase order tabulated on ``edges``."""
    if MODE == "0":
        return False
    if MODE != "cpu" and x.device.type != "cuda":
        return False
    if x.dtype not in (torch.float32, torch.float64):
        return False
    head = kernel.complex_head if kernel.complex_head is not None else kernel.real_head
    if not 1 <= head.in_features <= MAX_TRUNK:
        return False
    for term in plan(kernel):
        if not (1 <= term.a <= MAX_MULT and 1 <= term.b <= MAX_MULT):
            return False
        for order in (term.pre_order, term.post_order):
            if order is not None and abs(order) > edges.max_frequency:
                return False
    return True


def _rows_product(gk: Tensor, operand: Tensor, block: int) -> Tensor:
    """``gk @ operand`` for ``gk (width, E)`` and ``operand (E, c)``: the sum over
    the edges as per-block partial products (one batched product, summed in a
    fixed order) instead of one long reduction on a few workgroups."""
    width, E = gk.shape
    nb = E // block
    if nb < 2:
        return gk @ operand
    head = nb * block
    parts = torch.bmm(gk[:, :head].reshape(width, nb, block).permute(1, 0, 2),
                      operand[:head].reshape(nb, block, operand.shape[1]))
    out = parts.sum(0)
    if head < E:
        out = out + gk[:, head:] @ operand[head:]
    return out


def _rows(term: Term, cw: Tensor | None, cb: Tensor | None, rw: Tensor | None,
          rb: Tensor | None) -> tuple[Tensor, Tensor | None]:
    weight, bias = (rw, rb) if term.real_head else (cw, cb)
    assert weight is not None
    return weight[term.rows].contiguous(), None if bias is None else bias[term.rows].contiguous()


def _empty(like: Tensor) -> Tensor:
    return like.new_empty(0)


class _FusedPairs(torch.autograd.Function):
    """All terms of one kernel call (reference :156-238)."""

    @staticmethod
    def forward(ctx: Any, hidden: Tensor, complex_weight: Tensor | None, complex_bias: Tensor | None,
                real_weight: Tensor | None, real_bias: Tensor | None, meta: dict, phases: tuple[Tensor, ...],
                scales: tuple[Tensor, ...], *vectors: Tensor) -> tuple[Tensor, ...]:
        terms: list[Term] = meta["terms"]
        n_edges = hidden.shape[0]
        cdtype = torch.complex64 if hidden.dtype == torch.float32 else torch.complex128
        outputs = [torch.zeros(n_edges, meta["out_multiplicity"][m], dtype=hidden.dtype if m == 0 else cdtype,
                               device=hidden.device) for m in meta["out_frequencies"]]
        ext = extension()
        for term, (pre, post, scale) in zip(terms, meta["tables"], strict=True):
            weight, bias = _rows(term, complex_weight, complex_bias, real_weight, real_bias)
            with torch.profiler.record_function("gm::kernel/pairs"):
                ext.forward(hidden, weight, bias if bias is not None else _empty(hidden),
                            vectors[meta["in_index"][term.n]],
                            phases[pre] if pre is not None else _empty(hidden),
                            phases[post] if post is not None else _empty(hidden),
                            scales[scale] if scale is not None else _empty(hidden),
                            outputs[meta["out_index"][term.m]], term.a, term.b, term.flags)
        ctx.save_for_backward(hidden, complex_weight, complex_bias, real_weight, real_bias, *phases, *scales, *vectors)
        ctx.meta = meta
        ctx.counts = (len(phases), len(scales))
        return tuple(outputs)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, *grad_outputs: Tensor | None) -> tuple:
        meta = ctx.meta
        n_phases, n_scales = ctx.counts
        saved = ctx.saved_tensors
        hidden, complex_weight, complex_bias, real_weight, real_bias = saved[:5]
        phases = saved[5:5 + n_phases]
        scales = saved[5 + n_phases:5 + n_phases + n_scales]
        vectors = saved[5 + n_phases + n_scales:]
        terms: list[Term] = meta["terms"]
        n_edges = hidden.shape[0]
        cdtype = torch.complex64 if hidden.dtype == torch.float32 else torch.complex128
        grads_out = [(g if g is not None else torch.zeros(n_edges, meta["out_multiplicity"][m],
                                                          dtype=hidden.dtype if m == 0 else cdtype,
                                                          device=hidden.device)).contiguous()
                     for g, m in zip(grad_outputs, meta["out_frequencies"], strict=True)]
        grad_hidden = torch.zeros_like(hidden)
        grad_vectors = [torch.zeros_like(v) for v in vectors]
        # coefficient gradients coefficient-major (width, n_edges): a term's rows are one contiguous slab
        grad_complex = hidden.new_empty(complex_weight.shape[0], n_edges) if complex_weight is not None else None
        grad_real = hidden.new_empty(real_weight.shape[0], n_edges) if real_weight is not None else None
        ext = extension()
        for term, (pre, post, scale) in zip(terms, meta["tables"], strict=True):
            weight, bias = _rows(term, complex_weight, complex_bias, real_weight, real_bias)
            grad_k = grad_real if term.real_head else grad_complex
            assert grad_k is not None
            with torch.profiler.record_function("gm::kernel/pairs_backward"):
                ext.backward(hidden, weight, bias if bias is not None else _empty(hidden),
                             vectors[meta["in_index"][term.n]],
                             phases[pre] if pre is not None else _empty(hidden),
                             phases[post] if post is not None else _empty(hidden),
                             scales[scale] if scale is not None else _empty(hidden),
                             grads_out[meta["out_index"][term.m]], grad_vectors[meta["in_index"][term.n]],
                             grad_hidden, grad_k[term.rows], term.a, term.b, term.flags)
        # the bias gradient is the coefficient gradient summed over the edges: a column of
        # ones beside the trunk output folds it into the weight product
        with_bias = complex_bias is not None or real_bias is not None
        operand = torch.cat((hidden, hidden.new_ones(n_edges, 1)), dim=1) if with_bias else hidden

        def head_gradients(grad_k: Tensor | None, bias: Tensor | None) -> tuple[Tensor | None, Tensor | None]:
            if grad_k is None:
                return None, None
            grad = _rows_product(grad_k, operand, WEIGHT_GRAD_BLOCK)  # (width, trunk [+ 1])
            if not with_bias:
                return grad.contiguous(), None
            return grad[:, :-1].contiguous(), (grad[:, -1].contiguous() if bias is not None else None)

        grad_cw, grad_cb = head_gradients(grad_complex, complex_bias)
        grad_rw, grad_rb = head_gradients(grad_real, real_bias)
        return (grad_hidden, grad_cw, grad_cb, grad_rw, grad_rb, None, None, None, *grad_vectors)


def _radial_powers(kernel: Any, distances: Tensor, top: int) -> Tensor:
    """``(r / cutoff)^p`` for ``p = 0..top`` by repeated products (reference kernels.py:734-750)."""
    normalized = distances / kernel.radial_basis.cutoff
    table = [torch.ones_like(normalized)]
    for _ in range(top):
        table.append(table[-1] * normalized)
    return torch.stack(table, dim=-1)


def forward_general(kernel: Any, x: SO2FeatureField, edges: Any) -> SO2FeatureField:
    """The kernel's per-edge messages on the edge-shaped field ``x`` through the
    fused terms (reference :249-295): trunk, transport, phase tables, radial
    powers, then every term."""
    terms = plan(kernel)
    with torch.profiler.record_function("gm::kernel/radial"):
        hidden = kernel._trunk_hidden(edges.distances).contiguous()
    in_frequencies = list(kernel.field_type_in.frequencies)
    out_frequencies = list(kernel.field_type_out.frequencies)
    vectors = []
    for n in in_frequencies:
        if n == 0:
            vectors.append(x[0].contiguous())
        else:  # transported: e^{i n gamma} z
            z = torch.view_as_complex(x[n].contiguous())
            vectors.append((edges.transport_harmonic(n).unsqueeze(-1) * z).contiguous())
    orders = sorted({o for t in terms for o in (t.pre_order, t.post_order) if o is not None})
    phases = tuple(edges.angular_harmonic(o).contiguous() for o in orders)
    powers = sorted({t.power for t in terms if t.power is not None})
    table = _radial_powers(kernel, edges.distances, max(powers)) if powers else None
    scales = tuple(table[:, p].contiguous() for p in powers) if table is not None else ()
    order_index = {o: i for i, o in enumerate(orders)}
    power_index = {p: i for i, p in enumerate(powers)}
    meta = {
        "terms": terms,
        "tables": [(order_index[t.pre_order] if t.pre_order is not None else None,
                    order_index[t.post_order] if t.post_order is not None else None,
                    power_index[t.power] if t.power is not None else None) for t in terms],
        "in_index": {n: i for i, n in enumerate(in_frequencies)},
        "out_index": {m: i for i, m in enumerate(out_frequencies)},
        "out_frequencies": out_frequencies,
        "out_multiplicity": {m: kernel.field_type_out.multiplicity(m) for m in out_frequencies},
    }
    ch, rh = kernel.complex_head, kernel.real_head
    outputs = _FusedPairs.apply(hidden, ch.weight if ch is not None else None, ch.bias if ch is not None else None,
                                rh.weight if rh is not None else None, rh.bias if rh is not None else None, meta,
                                phases, scales, *vectors)
    return SO2FeatureField(kernel.field_type_out,
                           {m: (out if m == 0 else torch.view_as_real(out))
                            for m, out in zip(out_frequencies, outputs, strict=True)})


__all__ = ["MODE", "Term", "enabled", "extension", "forward_general", "plan"]
