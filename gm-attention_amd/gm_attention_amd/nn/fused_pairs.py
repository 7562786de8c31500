"""The steerable kernel's per-edge readout as fused pair terms on the HIP path.

The drop-in for the reference's ``nn/fused_pairs.py`` under the same switch
(``GM_FUSED_PAIRS``, :39-40) and names (``Term``, ``plan``, ``enabled``,
``_FusedPairs``, ``forward_general``; reference :51-295): the per-edge readout
of ``SO2SteerableKernel._forward_general`` (reference nn/kernels.py:752-915)
as one HIP launch per ``(n, m, role)`` term (``gm_pairs_forward``), each
forming its ``b_m x a_n`` coefficient block in registers from the trunk
output and the readout rows.

Design of this module:

* a term's flags and phase orders follow from three facts about its block
  (is the input scalar, is the output scalar, is it the antilinear half),
  tabulated in :data:`_RULES`; :func:`plan` lists the kernel's blocks in the
  readout's pair order and applies the table;
* :func:`forward_general` turns the plan into a *schedule* for this call --
  one entry per launch with the positions of its input, output, phase and
  radial-power tensors resolved -- so the autograd Function only replays it;
* the backward replays the schedule for the input and trunk gradients and
  forms each term's readout-weight gradient right after its launch, from the
  term's own ``(width, E)`` coefficient gradient: weight rows by a product
  with the trunk output summed over edge blocks in a fixed order, bias rows
  by a row sum.

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
from gm_attention_amd.nn.linear import blocked_gram
from gm_attention_amd.representations.field_type import SO2FeatureField

MATRIX_COMPLEX, U_REAL, CONJ_U, OUT_REAL = (_native.PAIRS_MATRIX_COMPLEX, _native.PAIRS_U_REAL, _native.PAIRS_CONJ_U,
                                            _native.PAIRS_OUT_REAL)
MAX_MULT = _native.PAIRS_MAX_MULT
MAX_TRUNK = _native.PAIRS_MAX_TRUNK
SUPPORTED = tuple(range(1, MAX_MULT + 1))

#: ``"0"`` off, ``"1"`` on for device tensors, ``"cpu"`` on everywhere (reference :39-40): device tensors
#: take the HIP terms, CPU tensors the eager readout (this build has no CPU driver).
MODE = os.environ.get("GM_FUSED_PAIRS", "1")

#: Edges per block of a readout weight gradient's fixed-order sum.
WEIGHT_GRAD_BLOCK = 16384


def extension(size: tuple[int, int, int] | None = None) -> Any:
    """The pair-term entry points (one build serves every block size)."""
    return _native.pairs()


@dataclass(frozen=True)
class Term:
    """One launch of the readout: block ``(n -> m, role)`` of ``a`` input and
    ``b`` output copies, its kernel flags, which readout head and rows hold
    its coefficients, the angular phase orders applied before (``pre``) or
    after (``post``) the block and its radial power (``None``: not applied)."""

    n: int
    m: int
    role: str
    flags: int
    a: int
    b: int
    real_head: bool
    rows: slice
    pre_order: int | None
    post_order: int | None
    power: int | None


# (input scalar, output scalar, antilinear) -> flags and the phase orders as functions of (n, m).
# The scalar-to-scalar block is the real head's; a scalar output takes the real part of
# A (e^{i n phi} conj z); a scalar input gets e^{i m phi} after the block; the rest rotate the
# (conjugated, for the antilinear half) transported input by e^{i (m -+ n) phi} first.
_RULES: dict[tuple[bool, bool, bool], tuple[int, Any, Any]] = {
    (True, True, False): (U_REAL | OUT_REAL, None, None),
    (True, False, False): (MATRIX_COMPLEX | U_REAL, None, lambda n, m: m),
    (False, True, False): (MATRIX_COMPLEX | CONJ_U | OUT_REAL, lambda n, m: n, None),
    (False, False, False): (MATRIX_COMPLEX, lambda n, m: m - n, None),
    (False, False, True): (MATRIX_COMPLEX | CONJ_U, lambda n, m: m + n, None),
}


def _term(kernel: Any, n: int, m: int, role: str) -> Term:
    fin, fout = kernel.field_type_in, kernel.field_type_out
    a, b = fin.multiplicity(n), fout.multiplicity(m)
    flags, pre, post = _RULES[(n == 0, m == 0, role == "antilinear")]
    if n == 0 and m == 0:
        return Term(0, 0, "real", flags, a, b, True, slice(0, a * b), None, None, None)
    return Term(n, m, role, flags, a, b, False, kernel._pair_ranges[(n, m, role)],
                pre(n, m) if pre is not None else None, post(n, m) if post is not None else None,
                kernel._pair_powers[(n, m, role)])


def plan(kernel: Any) -> list[Term]:
    """The readout's terms in its pair order (reference :96-123): output
    frequencies outer, input frequencies inner, the linear half of a block
    before its antilinear half (present when both frequencies are nonzero)."""
    cached = kernel.__dict__.get("_fused_plan")
    if cached is None:
        cached = [_term(kernel, n, m, role)
                  for m in kernel.field_type_out.frequencies
                  for n in kernel.field_type_in.frequencies
                  for role in (("real",) if n == m == 0 else ("linear", "antilinear") if n and m else ("linear",))]
        kernel.__dict__["_fused_plan"] = cached
    return cached


def enabled(kernel: Any, x: SO2FeatureField, edges: Any) -> bool:
    """Whether this call takes the fused terms (reference :126-149): the switch
    admits the tensors' device, the dtype is float32/64, the trunk and every
    block side are within 16, and every phase order is tabulated on ``edges``."""
    if MODE == "0" or x.device.type != "cuda" or x.dtype not in (torch.float32, torch.float64):
        return False
    head = kernel.complex_head if kernel.complex_head is not None else kernel.real_head
    if head.in_features > MAX_TRUNK:
        return False
    terms = plan(kernel)
    sides_fit = all(t.a in SUPPORTED and t.b in SUPPORTED for t in terms)
    orders = [abs(o) for t in terms for o in (t.pre_order, t.post_order) if o is not None]
    return sides_fit and max(orders, default=0) <= edges.max_frequency


@dataclass(frozen=True)
class _Launch:
    """One scheduled term: the term, then the positions of its input vector,
    output, pre/post phase tables and radial power among the call's tensors."""

    term: Term
    u: int
    out: int
    pre: int | None
    post: int | None
    scale: int | None


@dataclass(frozen=True)
class _Call:
    """What one kernel call launches: the schedule and the outputs it writes
    (frequency, copies, real or complex)."""

    launches: tuple[_Launch, ...]
    outputs: tuple[tuple[int, int, bool], ...]


def _empty(like: Tensor) -> Tensor:
    return like.new_empty(0)


def _pick(tables: tuple[Tensor, ...], index: int | None, like: Tensor) -> Tensor:
    return tables[index] if index is not None else _empty(like)


def _coefficients(term: Term, heads: tuple[Tensor | None, ...]) -> tuple[Tensor, Tensor]:
    """The term's readout rows and bias rows (an empty tensor for no bias)."""
    cw, cb, rw, rb = heads
    weight, bias = (rw, rb) if term.real_head else (cw, cb)
    assert weight is not None
    rows = weight[term.rows].contiguous()
    return rows, bias[term.rows].contiguous() if bias is not None else _empty(rows)


class _FusedPairs(torch.autograd.Function):
    """Every term of one kernel call (reference :156-238).  Inputs: the trunk
    output ``hidden (E, T)``, the heads' weights and biases, the call
    (:class:`_Call`), the angular phase tables, the radial power tables, then
    one per-edge input vector per input frequency; out one per-edge message
    per output frequency."""

    @staticmethod
    def forward(ctx: Any, hidden: Tensor, complex_weight: Tensor | None, complex_bias: Tensor | None,
                real_weight: Tensor | None, real_bias: Tensor | None, call: _Call, phases: tuple[Tensor, ...],
                scales: tuple[Tensor, ...], *vectors: Tensor) -> tuple[Tensor, ...]:
        ext = extension()
        E = hidden.shape[0]
        cplx = torch.complex64 if hidden.dtype == torch.float32 else torch.complex128
        outs = tuple(torch.zeros(E, b, dtype=hidden.dtype if real else cplx, device=hidden.device)
                     for _m, b, real in call.outputs)
        heads = (complex_weight, complex_bias, real_weight, real_bias)
        for step in call.launches:
            t = step.term
            weight, bias = _coefficients(t, heads)
            with torch.profiler.record_function("gm::kernel/pairs"):
                ext.forward(hidden, weight, bias, vectors[step.u], _pick(phases, step.pre, hidden),
                            _pick(phases, step.post, hidden), _pick(scales, step.scale, hidden), outs[step.out],
                            t.a, t.b, t.flags)
        ctx.call = call
        ctx.sizes = (len(phases), len(scales))
        ctx.save_for_backward(hidden, complex_weight, complex_bias, real_weight, real_bias, *phases, *scales, *vectors)
        return outs

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, *grad_outs: Tensor | None) -> tuple:
        call: _Call = ctx.call
        n_phases, n_scales = ctx.sizes
        hidden, cw, cb, rw, rb, *rest = ctx.saved_tensors
        phases, scales, vectors = (tuple(rest[:n_phases]), tuple(rest[n_phases:n_phases + n_scales]),
                                   tuple(rest[n_phases + n_scales:]))
        ext = extension()
        E = hidden.shape[0]
        cplx = torch.complex64 if hidden.dtype == torch.float32 else torch.complex128
        grads = [(g if g is not None else torch.zeros(E, b, dtype=hidden.dtype if real else cplx,
                                                      device=hidden.device)).contiguous()
                 for g, (_m, b, real) in zip(grad_outs, call.outputs, strict=True)]
        d_hidden = torch.zeros_like(hidden)
        d_vectors = [torch.zeros_like(v) for v in vectors]
        heads = (cw, cb, rw, rb)
        # each readout head's gradient, row block by row block as the terms come
        d_head = {True: (torch.zeros_like(rw) if rw is not None else None,
                         torch.zeros_like(rb) if rb is not None else None),
                  False: (torch.zeros_like(cw) if cw is not None else None,
                          torch.zeros_like(cb) if cb is not None else None)}
        for step in call.launches:
            t = step.term
            weight, bias = _coefficients(t, heads)
            d_coeff = hidden.new_empty(weight.shape[0], E)  # this term's coefficient gradient, row-major by edge
            with torch.profiler.record_function("gm::kernel/pairs_backward"):
                ext.backward(hidden, weight, bias, vectors[step.u], _pick(phases, step.pre, hidden),
                             _pick(phases, step.post, hidden), _pick(scales, step.scale, hidden), grads[step.out],
                             d_vectors[step.u], d_hidden, d_coeff, t.a, t.b, t.flags)
            dw, db = d_head[t.real_head]
            dw[t.rows] += blocked_gram(d_coeff.t(), hidden, WEIGHT_GRAD_BLOCK)
            if db is not None:
                db[t.rows] += d_coeff.sum(dim=1)
        return (d_hidden, d_head[False][0], d_head[False][1], d_head[True][0], d_head[True][1], None, None, None,
                *d_vectors)


def _radial_powers(distances: Tensor, cutoff: float, powers: list[int]) -> tuple[Tensor, ...]:
    """``(r / cutoff)^p`` for each listed ``p``, as repeated products (reference kernels.py:734-750)."""
    rho = distances / cutoff
    table, current = {}, torch.ones_like(rho)
    for p in range(max(powers, default=-1) + 1):
        if p:
            current = current * rho
        table[p] = current
    return tuple(table[p].contiguous() for p in powers)


def forward_general(kernel: Any, x: SO2FeatureField, edges: Any) -> SO2FeatureField:
    """The kernel's per-edge messages on the edge-shaped field ``x`` through the
    fused terms (reference :249-295)."""
    terms = plan(kernel)
    fin, fout = list(kernel.field_type_in.frequencies), list(kernel.field_type_out.frequencies)
    with torch.profiler.record_function("gm::kernel/radial"):
        hidden = kernel._trunk_hidden(edges.distances).contiguous()
    # the input vectors: scalars as they are, higher frequencies transported (e^{i n gamma} z)
    vectors = [x[0].contiguous() if n == 0 else
               (edges.transport_harmonic(n).unsqueeze(-1) * torch.view_as_complex(x[n].contiguous())).contiguous()
               for n in fin]
    orders = sorted({o for t in terms for o in (t.pre_order, t.post_order) if o is not None})
    powers = sorted({t.power for t in terms if t.power is not None})
    phases = tuple(edges.angular_harmonic(o).contiguous() for o in orders)
    scales = _radial_powers(edges.distances, kernel.radial_basis.cutoff, powers)
    launches = tuple(_Launch(t, fin.index(t.n), fout.index(t.m),
                             orders.index(t.pre_order) if t.pre_order is not None else None,
                             orders.index(t.post_order) if t.post_order is not None else None,
                             powers.index(t.power) if t.power is not None else None) for t in terms)
    call = _Call(launches, tuple((m, kernel.field_type_out.multiplicity(m), m == 0) for m in fout))
    ch, rh = kernel.complex_head, kernel.real_head
    outs = _FusedPairs.apply(hidden, None if ch is None else ch.weight, None if ch is None else ch.bias,
                             None if rh is None else rh.weight, None if rh is None else rh.bias, call, phases, scales,
                             *vectors)
    return SO2FeatureField(kernel.field_type_out, {m: out if m == 0 else torch.view_as_real(out)
                                                   for m, out in zip(fout, outs, strict=True)})


__all__ = ["MODE", "Term", "enabled", "extension", "forward_general", "plan"]
