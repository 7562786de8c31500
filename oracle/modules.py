"""Eager restatements of the reference's steerable-kernel evaluation, from a
kernel's parameters.  TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

* :func:`readout_messages` -- ``SO2SteerableKernel._forward_general``
  (reference nn/kernels.py:752-915): per edge, the radial trunk's readout of
  every block's coefficient matrix, applied to the transported source field
  under the block's harmonic and radial power.  The coefficient layout is
  derived here from the field types (kernels.py:336-397), independently of
  the product's bookkeeping.
* :func:`node_products` -- the complex ``einsum("ja,bat->jtb")`` of
  kernels.py:575-603 over ``_block_weights`` (kernels.py:506-536).
* :func:`factored_messages` -- the eager factored branch (kernels.py:645-697):
  the node products gathered to the edges, combined with ``h~ = (1, h)`` and
  each block's factor.

The readout and the factored branch are the same function regrouped by
associativity (the reference's own check: tests/nn/test_fused_factored.py:
126-208), so each pins the other.

The transformer block's pieces (:func:`layer_norm`, :func:`gated`,
:func:`block_forward`) restate nn/normalization.py, nn/nonlinearities.py and
nn/blocks.py of the reference; tests/test_oracle_block.py pins them (torch's
LayerNorm and RMSNorm on one-frequency fields, the pooled denominator, the
identity gate, gauge equivariance).
"""

from __future__ import annotations

import math

import torch
from torch import Tensor


def _phase(table: Tensor, order: int) -> Tensor:
    col = table[:, abs(order)]
    return col.conj() if order < 0 else col


def gaussian_basis(distances: Tensor, n_basis: int, cutoff: float) -> Tensor:
    """``_GaussianRadialBasis`` (reference kernels.py:191-231), from its
    definition: ``phi_k(s) = exp(-(s - mu_k)^2 / (2 sigma^2))`` of
    ``s = (r / cutoff)^2``, centres ``mu_k = k / (n - 1)`` evenly over
    ``[0, 1]`` (one centre at 0 when ``n = 1``), ``sigma`` the spacing
    ``1 / (n - 1)`` (1 when ``n = 1``)."""
    spacing = 1.0 / (n_basis - 1) if n_basis > 1 else 1.0
    centres = torch.tensor([k / (n_basis - 1) for k in range(n_basis)] if n_basis > 1 else [0.0],
                           dtype=distances.dtype)
    s = (distances / cutoff) * (distances / cutoff)
    return torch.exp(-0.5 * ((s.unsqueeze(-1) - centres) / spacing) ** 2)


def _trunk(kernel, distances: Tensor) -> Tensor:
    """The Gaussian basis of ``(r / cutoff)^2`` then the ``Linear``/``SiLU`` trunk (kernels.py:191-231, 108-117).
    Only the basis size and cutoff are read from the module; the basis itself is :func:`gaussian_basis`."""
    rb = kernel.radial_basis
    hidden = gaussian_basis(distances, rb.n_basis, rb.cutoff)
    for layer in kernel.radial_trunk:
        if isinstance(layer, torch.nn.Linear):
            hidden = hidden @ layer.weight.T + (layer.bias if layer.bias is not None else 0.0)
        else:
            hidden = torch.nn.functional.silu(hidden)
    return hidden


def _apply(matrix: Tensor, v: Tensor) -> Tensor:
    """Per edge, ``(E, b, a) @ (E, a) -> (E, b)``."""
    return torch.matmul(matrix, v.unsqueeze(-1)).squeeze(-1)


def layout(fin, fout) -> tuple[list[tuple[int, int, str, int, int]], int]:
    """The complex head's ranges ``(n, m, role, start, power)`` in readout
    order and the real head's width: every pair ``(n, m)`` but ``(0, 0)`` a
    linear range of ``2 b_m a_n`` reals, ``n, m >= 1`` an antilinear one after it."""
    ranges, offset, real = [], 0, 0
    for n in fin.frequencies:
        for m in fout.frequencies:
            a, b = fin.multiplicity(n), fout.multiplicity(m)
            if n == 0 and m == 0:
                real = a * b
                continue
            ranges.append((n, m, "linear", offset, abs(m - n)))
            offset += 2 * a * b
            if n >= 1 and m >= 1:
                ranges.append((n, m, "antilinear", offset, m + n))
                offset += 2 * a * b
    return ranges, real


def readout_messages(kernel, x: dict[int, Tensor], source: Tensor, distances: Tensor, angular: Tensor,
                     transport: Tensor) -> dict[int, Tensor]:
    """Per-edge messages of the kernel on the node field ``x`` (frequency ->
    ``(N, a_0)`` / ``(N, a_n, 2)``) gathered by ``source``; ``angular`` and
    ``transport`` are complex ``(E, K + 1)`` phase tables."""
    fin, fout = kernel.field_type_in, kernel.field_type_out
    E = source.shape[0]
    hidden = _trunk(kernel, distances)
    ranges, _ = layout(fin, fout)
    real = None
    if kernel.real_head is not None:
        real = hidden @ kernel.real_head.weight.T
        if kernel.real_head.bias is not None:
            real = real + kernel.real_head.bias
    rho = distances / kernel.radial_basis.cutoff
    xs = {}
    for n in fin.frequencies:
        v = x[n].index_select(0, source)
        if n == 0:
            xs[0] = v
        else:
            xs[n] = _phase(transport, n).unsqueeze(-1) * torch.view_as_complex(v.contiguous())  # transported

    def power(p: int) -> Tensor:
        s = torch.ones_like(rho)
        for _ in range(p):
            s = s * rho
        return s.unsqueeze(-1)

    def matrix(n: int, m: int, role: str) -> Tensor:
        # each block's rows of the complex head read out on their own (the same
        # numbers as slicing the whole readout, without an (E, width) gradient per slice)
        for nn, mm, rr, start, _p in ranges:
            if (nn, mm, rr) == (n, m, role):
                a, b = fin.multiplicity(n), fout.multiplicity(m)
                rows = slice(start, start + 2 * a * b)
                block = hidden @ kernel.complex_head.weight[rows].T
                if kernel.complex_head.bias is not None:
                    block = block + kernel.complex_head.bias[rows]
                return torch.view_as_complex(block.reshape(E, b, a, 2).contiguous())
        raise KeyError((n, m, role))

    out: dict[int, Tensor] = {}
    for m in fout.frequencies:
        b = fout.multiplicity(m)
        acc = torch.zeros(E, b, dtype=distances.dtype if m == 0 else angular.dtype)
        for n in fin.frequencies:
            a = fin.multiplicity(n)
            if n == 0 and m == 0:
                acc = acc + _apply(real.reshape(E, b, a), xs[0])
                continue
            lin = matrix(n, m, "linear")
            if n == 0:
                term = _phase(angular, m).unsqueeze(-1) * _apply(lin, xs[0].to(lin.dtype))
                acc = acc + term * power(abs(m - n))
            elif m == 0:
                rotated = _phase(angular, -n).unsqueeze(-1) * xs[n]
                acc = acc + _apply(lin, rotated.conj()).real * power(n)
            else:
                anti = matrix(n, m, "antilinear")
                lterm = _apply(lin, _phase(angular, m - n).unsqueeze(-1) * xs[n])
                aterm = _apply(anti, _phase(angular, m + n).unsqueeze(-1) * xs[n].conj())
                acc = acc + lterm * power(abs(m - n)) + aterm * power(m + n)
        out[m] = acc if m == 0 else torch.view_as_real(acc)
    return out


def block_weights(kernel, n: int, m: int, role: str) -> Tensor:
    """``(W_0 = bias, W_1..W_T)`` of one block, ``(b_m, a_n, T + 1)`` (kernels.py:506-536)."""
    fin, fout = kernel.field_type_in, kernel.field_type_out
    a, b = fin.multiplicity(n), fout.multiplicity(m)
    if role == "real":
        w = kernel.real_head.weight.reshape(b, a, -1)
        bias = kernel.real_head.bias.reshape(b, a) if kernel.real_head.bias is not None else w.new_zeros(b, a)
        return torch.cat([bias.unsqueeze(-1), w], dim=-1)
    ranges, _ = layout(fin, fout)
    start = next(s for nn, mm, rr, s, _p in ranges if (nn, mm, rr) == (n, m, role))
    rows = slice(start, start + 2 * a * b)
    w = torch.view_as_complex(kernel.complex_head.weight[rows].reshape(b, a, 2, -1).permute(0, 1, 3, 2).contiguous())
    if kernel.complex_head.bias is not None:
        bias = torch.view_as_complex(kernel.complex_head.bias[rows].reshape(b, a, 2).contiguous())
    else:
        bias = w.new_zeros(b, a)
    return torch.cat([bias.unsqueeze(-1), w], dim=-1)


def blocks_of(kernel) -> list[tuple[int, int, str]]:
    fin, fout = kernel.field_type_in, kernel.field_type_out
    ranges, real = layout(fin, fout)
    return ([(0, 0, "real")] if real else []) + [(n, m, r) for n, m, r, _s, _p in ranges]


def node_products(kernel, x: dict[int, Tensor]) -> dict[tuple[int, int, str], Tensor]:
    """``W_t v_j`` per block, ``(N, T + 1, b_m)``, by complex einsum (kernels.py:575-603)."""
    out = {}
    for n, m, role in blocks_of(kernel):
        w = block_weights(kernel, n, m, role)
        if role == "real":
            v = x[0]
        elif n == 0:
            v = x[0].to(w.dtype)
        else:
            v = torch.view_as_complex(x[n].contiguous())
            if m == 0 or role == "antilinear":
                v = v.conj()
        out[(n, m, role)] = torch.einsum("ja,bat->jtb", v, w.to(v.dtype))
    return out


def factored_messages(kernel, x: dict[int, Tensor], source: Tensor, distances: Tensor, angular: Tensor,
                      transport: Tensor) -> dict[int, Tensor]:
    """The eager factored branch (kernels.py:645-697)."""
    fout = kernel.field_type_out
    products = node_products(kernel, x)
    hidden = _trunk(kernel, distances)
    h = torch.cat([torch.ones(hidden.shape[0], 1, dtype=hidden.dtype), hidden], dim=-1)
    rho = distances / kernel.radial_basis.cutoff
    ranges, _ = layout(kernel.field_type_in, fout)
    powers = {(n, m, r): p for n, m, r, _s, p in ranges}
    out = {}
    for m in fout.frequencies:
        acc = None
        for block in blocks_of(kernel):
            n, mm, role = block
            if mm != m:
                continue
            gathered = products[block].index_select(0, source)
            combined = torch.matmul(h.to(gathered.dtype).unsqueeze(1), gathered).squeeze(1)
            if role == "real":
                term = combined
            else:
                if n == 0:
                    phase = _phase(angular, m)
                elif m == 0:
                    phase = _phase(angular, n) * _phase(transport, -n)
                elif role == "linear":
                    phase = _phase(angular, m - n) * _phase(transport, n)
                else:
                    phase = _phase(angular, m + n) * _phase(transport, -n)
                s = torch.ones_like(rho)
                for _ in range(powers[block]):
                    s = s * rho
                term = (phase * s).unsqueeze(-1) * combined
                term = term.real if m == 0 else term
            acc = term if acc is None else acc + term
        out[m] = acc if m == 0 else torch.view_as_real(acc)
    return out


# ---------------------------------------------------------------- attention layers


def linear(lin, x: dict[int, Tensor], fout) -> dict[int, Tensor]:
    """``SO2Linear.forward`` (reference nn/linear.py:130-190): real matmul at 0,
    complex matmul above, bias on frequency 0."""
    out = {}
    batch = next(iter(x.values())).shape[0]
    for f in fout.frequencies:
        b = fout.multiplicity(f)
        if str(f) not in lin.weight:
            z = torch.zeros(batch, b, dtype=torch.float64) if f == 0 else torch.zeros(batch, b, 2, dtype=torch.float64)
            out[f] = z + (lin.bias if (f == 0 and lin.bias is not None) else 0.0)
            continue
        w = lin.weight[str(f)]
        if f == 0:
            out[0] = x[0] @ w.T + (lin.bias if lin.bias is not None else 0.0)
        else:
            out[f] = torch.view_as_real(torch.view_as_complex(x[f].contiguous())
                                        @ torch.view_as_complex(w.contiguous()).T)
    return out


def flat(x: dict[int, Tensor]) -> Tensor:
    return torch.cat([x[f] if f == 0 else x[f].flatten(-2) for f in sorted(x)], dim=-1)


def softmax_weights(q: dict[int, Tensor], k: dict[int, Tensor], edges, cutoff: float, window: str, n_heads: int,
                    scale: float, tolerance: float | None = None) -> Tensor:
    """``_softmax_weights`` (reference attention.py:825-855) straight from the
    edges: gathered queries, gathered and transported keys, per-head scores,
    ``log c + log w`` with the tiny clamp, the window's support masked to
    ``-inf``, a detached per-target max, exp, per-target normalisation."""
    target, source = edges.target_index, edges.source_index
    E = source.shape[0]
    score = torch.zeros(E, n_heads, dtype=next(iter(q.values())).dtype)
    for f in sorted(q):
        qe, ke = q[f].index_select(0, target), k[f].index_select(0, source)
        if f != 0:
            ke = torch.view_as_real(edges.transport_phases[:, f].unsqueeze(-1) * torch.view_as_complex(ke.contiguous()))
        prod = (qe * ke).reshape(E, n_heads, -1)
        score = score + prod.sum(-1)
    score = score * scale
    d = edges.distances
    # the hard window's slack is the distances' dtype's (edge_geometry.py:403-428); a float64
    # oracle of a float32 run passes the float32 slack explicitly
    tol = tolerance if tolerance is not None else (1e-10 if d.dtype == torch.float64 else 1e-5)
    win = (d <= cutoff + tol).to(d.dtype) if window == "hard" else torch.relu(1.0 - (d / cutoff) ** 2) ** 2
    tiny = torch.finfo(score.dtype).tiny
    lw = score + (torch.log(win.clamp_min(tiny)) + torch.log(edges.tangent_quadrature_weights.clamp_min(tiny))).unsqueeze(-1)
    lw = lw.masked_fill(~(win > 0).unsqueeze(-1), float("-inf"))
    mx = torch.segment_reduce(lw, "max", offsets=edges.row_ptr, axis=0).detach()
    u = torch.exp(lw - mx.index_select(0, target))
    return u / torch.segment_reduce(u, "sum", offsets=edges.row_ptr, axis=0).index_select(0, target)


class HeadType:
    """The oracle's own per-head field type: ``{frequency: multiplicity}`` with
    the two accessors :func:`linear` reads.  Its dimension counts one real per
    frequency-0 copy and two (re, im) per copy above (reference
    representations/field_type.py: a frequency-n copy is a real 2-vector)."""

    def __init__(self, multiplicities: dict[int, int]):
        self.multiplicities = {int(f): int(m) for f, m in multiplicities.items() if m}
        self.frequencies = sorted(self.multiplicities)
        self.dimension = sum(m if f == 0 else 2 * m for f, m in self.multiplicities.items())

    def multiplicity(self, f: int) -> int:
        return self.multiplicities[f]


def head_type(multiplicities: dict[int, int], n_heads: int) -> HeadType:
    """Each head's type: every frequency's multiplicity divided by the head
    count (reference attention.py:551-556; the head count must divide each)."""
    for f, m in multiplicities.items():
        if m % n_heads:
            raise ValueError(f"{n_heads} heads do not divide frequency {f}'s {m} copies")
    return HeadType({f: m // n_heads for f, m in multiplicities.items()})


def score_scale(attn: HeadType) -> float:
    """``S(q, k) = <q, k> / sqrt(dim rho_attn)`` (reference attention.py:216-217)."""
    return 1.0 / math.sqrt(attn.dimension)


def mhsa_forward(mhsa, x: dict[int, Tensor], edges, tolerance: float | None = None,
                 messages: str = "readout") -> dict[int, Tensor]:
    """``SO2MHSA.forward`` (reference attention.py:582-608), head by head
    (the function the batched pass computes, attention.py:858-909): each
    head's query and key maps, its softmax, its value kernel's per-edge
    messages (``messages``: the per-edge readout, or the factored branch --
    the same function regrouped, cheaper for wide fields) weighted and summed
    per target; heads concatenated head-major; the output intertwiner."""
    evaluate = {"readout": readout_messages, "factored": factored_messages}[messages]
    fin = mhsa.field_type_in
    # the per-head type and score scale from the input type and head count alone,
    # never from the module under test
    attn = head_type({f: fin.multiplicity(f) for f in fin.frequencies}, len(mhsa.heads))
    outs = []
    for head in mhsa.heads:
        q = linear(head.query, x, attn)
        k = linear(head.key, x, attn)
        alpha = softmax_weights(q, k, edges, head.cutoff, head.window, 1, score_scale(attn), tolerance)[:, 0]
        msgs = evaluate(head.value, x, edges.source_index, edges.distances, edges.angular_phases,
                        edges.transport_phases)
        agg = {f: torch.segment_reduce(alpha.reshape(-1, *([1] * (m.ndim - 1))) * m, "sum", offsets=edges.row_ptr,
                                       axis=0) for f, m in msgs.items()}
        outs.append(agg)
    fused = {f: torch.cat([o[f] for o in outs], dim=-1 if f == 0 else -2) for f in fin.frequencies}
    return linear(mhsa.output_projection, fused, fin)


# ---------------------------------------------------------------- convolution layers


def depthwise_layer_messages(kernel, x: dict[int, Tensor], edges) -> dict[int, Tensor]:
    """``SO2DepthwiseKernel.forward`` on the gathered source field (reference
    nn/depthwise.py:147-193): the shared trunk, the real head ``C`` per scalar
    copy, the complex head per frequency ``n`` as ``(2, a_n, 2)`` = (A | B,
    copy, re/im); ``m = C x`` at 0, ``A z + (r/c)^{2n} e^{2 i n phi} B conj(z)``
    above, ``z`` the transported copy; the radial power by repeated products."""
    ft = kernel.field_type
    source = edges.source_index
    E = source.shape[0]
    hidden = _trunk(kernel, edges.distances)
    out: dict[int, Tensor] = {}
    if kernel.real_head is not None:
        c = hidden @ kernel.real_head.weight.T + (kernel.real_head.bias if kernel.real_head.bias is not None else 0.0)
        out[0] = c * x[0].index_select(0, source)
    if kernel.complex_head is not None:
        cc = hidden @ kernel.complex_head.weight.T
        if kernel.complex_head.bias is not None:
            cc = cc + kernel.complex_head.bias
        rho = edges.distances / kernel.radial_basis.cutoff
        start = 0
        for n in ft.frequencies:
            if n == 0:
                continue
            a = ft.multiplicity(n)
            block = cc[:, start:start + 4 * a].reshape(E, 2, a, 2)
            start += 4 * a
            A = torch.view_as_complex(block[:, 0].contiguous())
            B = torch.view_as_complex(block[:, 1].contiguous())
            z = edges.transport_phases[:, n].unsqueeze(-1) * torch.view_as_complex(
                x[n].index_select(0, source).contiguous())
            scale = torch.ones_like(rho)
            for _ in range(2 * n):
                scale = scale * rho
            w = (scale * edges.angular_phases[:, 2 * n]).unsqueeze(-1)
            out[n] = torch.view_as_real(A * z + w * B * z.conj())
    return out


def conv_forward(conv, x: dict[int, Tensor], edges, tolerance: float | None = None,
                 messages: str = "readout") -> dict[int, Tensor]:
    """``SO2Convolution.forward`` eagerly (reference nn/convolution.py:271-355):
    per-edge messages (the depthwise kernel's, or the general kernel's
    per-edge readout or factored branch), each weighted by the window times
    the quadrature weight, summed per target, divided by the window mass
    under ``normalize``, plus the self-intertwiner."""
    if conv.depthwise:
        msgs = depthwise_layer_messages(conv.kernel, x, edges)
    else:
        evaluate = {"readout": readout_messages, "factored": factored_messages}[messages]
        msgs = evaluate(conv.kernel, x, edges.source_index, edges.distances, edges.angular_phases,
                        edges.transport_phases)
    d = edges.distances
    tol = tolerance if tolerance is not None else (1e-10 if d.dtype == torch.float64 else 1e-5)
    win = (d <= conv.cutoff + tol).to(d.dtype) if conv.window == "hard" else torch.relu(1.0 - (d / conv.cutoff) ** 2) ** 2
    weight = win * edges.tangent_quadrature_weights
    out = {}
    for f, m in msgs.items():
        s = torch.segment_reduce(weight.reshape(-1, *([1] * (m.ndim - 1))) * m, "sum", offsets=edges.row_ptr, axis=0)
        if conv.normalize:
            mass = torch.segment_reduce(weight, "sum", offsets=edges.row_ptr, axis=0).clamp_min(conv.eps)
            s = s / mass.reshape(-1, *([1] * (s.ndim - 1)))
        out[f] = s
    if conv.self_linear is not None:
        pointwise = linear(conv.self_linear, x, conv.field_type_out)
        out = {f: out[f] + pointwise[f] for f in out}
    return out


# ---------------------------------------------------------------- transformer block


def layer_norm(norm, x: dict[int, Tensor]) -> dict[int, Tensor]:
    """``SO2LayerNorm.forward`` (reference nn/normalization.py:150-190): only
    frequency 0 centred; v_0 = mean (x_0 - mu)^2, v_n = mean_a |x_n,a|^2 / 2;
    one denominator sqrt(mean_n v_n + eps); a gain per copy, a bias on
    frequency 0."""
    stats = []
    out = {}
    if 0 in x:
        c0 = x[0] - x[0].mean(dim=-1, keepdim=True)
        stats.append((c0 * c0).mean(dim=-1))
    for f in sorted(x):
        if f != 0:
            stats.append((x[f] * x[f]).sum(dim=-1).mean(dim=-1) / 2)
    d = torch.sqrt(sum(stats) / len(stats) + norm.eps)
    for f in sorted(x):
        g = norm.gamma[str(f)]
        if f == 0:
            out[0] = g * c0 / d.unsqueeze(-1) + (norm.beta if norm.beta is not None else 0.0)
        else:
            out[f] = g.unsqueeze(-1) * x[f] / d.unsqueeze(-1).unsqueeze(-1)
    return out


def gated(act, x: dict[int, Tensor]) -> dict[int, Tensor]:
    """``SO2ScalarGatedNonlinearity.forward`` (reference
    nn/nonlinearities.py:140-166): SiLU on the scalars; each copy of frequency n
    times act(A_n x_0 + b_n), act = SiLU or 2 sigmoid, from the raw scalars."""
    s = x[0]
    out = {0: s * torch.sigmoid(s)}
    for f in sorted(x):
        if f == 0:
            continue
        lin = act.gates[str(f)]
        pre = s @ lin.weight.T + (lin.bias if lin.bias is not None else 0.0)
        g = 2 * torch.sigmoid(pre) if act.gate == "double_sigmoid" else pre * torch.sigmoid(pre)
        out[f] = x[f] * g.unsqueeze(-1)
    return out


def block_forward(block, x: dict[int, Tensor], edges, tolerance: float | None = None,
                  messages: str = "readout") -> dict[int, Tensor]:
    """``SO2TransformerBlock._run`` (reference nn/blocks.py:326-349) with
    dropout off: x + Mixer(LN1 x), then + W2 act(W1 LN2 x)."""
    normed = layer_norm(block.norm1, x)
    if block.mixer == "attention":
        mixed = mhsa_forward(block.attention, normed, edges, tolerance, messages)
    else:
        mixed = conv_forward(block.attention, normed, edges, tolerance)
    x = {f: x[f] + mixed[f] for f in x}
    hidden = linear(block.linear1, layer_norm(block.norm2, x), block.hidden_field_type)
    hidden = linear(block.linear2, gated(block.activation, hidden), block.field_type)
    return {f: x[f] + hidden[f] for f in x}


def encode_forward(enc, x: dict[int, Tensor], edges, tolerance: float | None = None,
                   messages: str = "readout") -> dict[int, Tensor]:
    """``IcoEncode.forward`` (reference nn/blocks.py:427-493) on bipartite edges:
    the per-edge readout of the kernel on the fine sources, times window times
    quadrature, summed per coarse target."""
    evaluate = {"readout": readout_messages, "factored": factored_messages}[messages]
    msgs = evaluate(enc.kernel, x, edges.source_index, edges.distances, edges.angular_phases, edges.transport_phases)
    d = edges.distances
    tol = tolerance if tolerance is not None else (1e-10 if d.dtype == torch.float64 else 1e-5)
    win = (d <= enc.cutoff + tol).to(d.dtype) if enc.window == "hard" else torch.relu(1.0 - (d / enc.cutoff) ** 2) ** 2
    weight = win * edges.tangent_quadrature_weights
    return {f: torch.segment_reduce(weight.reshape(-1, *([1] * (m.ndim - 1))) * m, "sum", offsets=edges.row_ptr,
                                    axis=0) for f, m in msgs.items()}


# ---------------------------------------------------------------- segmentation stage (C5)


def low_pass(restriction, x0: Tensor, edges) -> Tensor:
    """``IcoLowPassRestriction.forward`` (reference nn/blocks.py:508-600) on a
    scalar field: per target, sum_j c(r) q x_j / max(sum_j c(r) q, eps), c the
    quartic or hard window of the restriction's cutoff."""
    d = edges.distances
    if restriction.window == "hard":
        win = (d <= restriction.cutoff + (1e-10 if d.dtype == torch.float64 else 1e-5)).to(d.dtype)
    else:
        win = torch.relu(1.0 - (d / restriction.cutoff) ** 2) ** 2
    w = win * edges.tangent_quadrature_weights
    mass = torch.segment_reduce(w, "sum", offsets=edges.row_ptr, axis=0).clamp_min(restriction.eps)
    num = torch.segment_reduce(w.unsqueeze(-1) * x0.index_select(0, edges.source_index), "sum",
                               offsets=edges.row_ptr, axis=0)
    return num / mass.unsqueeze(-1)


def segformer_block_forward(block, x: dict[int, Tensor], disc, tolerance: float | None = None,
                            messages: str = "readout") -> dict[int, Tensor]:
    """``GmSegformerBlock.forward`` (reference experiments/stanford_2d3ds/
    model.py:225-237) without drop path: x + MHSA(LN1 x), then
    x + W_out act(DWConv(W_in LN2 x)); each operator on the level's edges
    within its own radius."""
    attn = block.attention
    mixed = mhsa_forward(attn, layer_norm(block.norm1, x), disc.edges_within(attn.cutoff), tolerance, messages)
    x = {f: x[f] + mixed[f] for f in x}
    hidden = linear(block.linear_in, layer_norm(block.norm2, x), block.hidden_field_type)
    hidden = conv_forward(block.mix, hidden, disc.edges_within(block.mix.cutoff), tolerance)
    hidden = linear(block.linear_out, gated(block.activation, hidden), block.field_type)
    return {f: x[f] + hidden[f] for f in x}


def segformer_forward(model, x0: Tensor, hierarchy, tolerance: float | None = None,
                      messages: str = "readout") -> Tensor:
    """``GmSegformer.forward`` (reference model.py:728-764 ``encode``, :823-880
    ``decode``) for the benchmark's options: per stage the learned restriction
    and its norm, the blocks, the stage norm; per stage a convolution readout
    onto scalars; the fusion decoder (GELU(Linear) of the coarsest readout,
    then per finer stage the carried channels low-passed over the lateral
    edges, joined with the readout, GELU(Linear)); the low pass onto the input
    grid over up_edges[0]; the head intertwiner.  ``x0`` is the input's
    scalars; returns the logits ``(n_input, classes)``."""
    feature = {0: x0}
    features = []
    for i in range(len(model.stages)):
        disc = hierarchy.levels[i + 1].discretization
        feature = encode_forward(model.merges[i].integral, feature, hierarchy.down_edges[i], tolerance, messages)
        feature = layer_norm(model.merge_norms[i], feature)
        for block in model.stages[i]:
            feature = segformer_block_forward(block, feature, disc, tolerance, messages)
        feature = layer_norm(model.stage_norms[i], feature)
        features.append(feature)
    readouts = []
    for i, f in enumerate(features):
        conv = model.readouts[i]
        disc = hierarchy.levels[i + 1].discretization
        readouts.append(conv_forward(conv, f, disc.edges_within(conv.cutoff), tolerance, messages)[0])
    gelu = torch.nn.functional.gelu
    fused = gelu(readouts[-1] @ model.fusion_in.weight.T + model.fusion_in.bias)
    for j, k in enumerate(range(len(features) - 2, -1, -1)):
        up = low_pass(model.lateral_interpolations[j], fused, hierarchy.lateral_edges[k])
        lin = model.fusions[j]
        fused = gelu(torch.cat([readouts[k], up], dim=-1) @ lin.weight.T + lin.bias)
    fine = low_pass(model.final_interpolation, fused, hierarchy.up_edges[0])
    return linear(model.head, {0: fine}, model.output_field_type)[0]
