"""The scores-and-softmax op and the depthwise convolution as HIP kernels.

The drop-in for the reference's ``gm_attention/nn/fused_attention.py``: the
same switch (``GM_FUSED_ATTENTION``, read at import: ``"0"`` off, ``"1"`` on for
device tensors, ``"cpu"`` accepted for compatibility), the same ``Plan`` /
``descriptors`` layout (:74-123), the same per-edge ``Geometry`` constants and
cache (:126-255), the same eligibility predicates (:258-326) and the same
autograd Functions ``Softmax`` (:371-397) and ``Depthwise`` (:329-353), so the
attention and convolution layers call it unchanged.  The arithmetic runs in
``libgmhip.so`` (``_native.attention()``); there is no CPU driver, so a CPU
tensor reaching an op is an error rather than a silent fallback.

Differences from the reference, all implementation limits rather than
semantics: no neighbourhood-size bound (the reference declines when
``max_degree * heads > 8192``, which excludes the 256x512 grid); the key and
value gradients are gathered per source node instead of added atomically,
so they are deterministic; the geometry keeps a copy of the transport table
narrowed to the orders a layer reads.
"""

from __future__ import annotations

import os
import weakref
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Any

import torch
from torch import Tensor

from gm_attention_amd import _native

MAX_H, MAX_F, MAX_D, DESC = 8, 8, 512, 5
#: ``"0"`` off, ``"1"`` on for device tensors, ``"cpu"`` accepted (no CPU driver in this build).
#: The default is ``"1"``: this build's layers run only through the fused ops (``"0"`` makes them raise).
MODE = os.environ.get("GM_FUSED_ATTENTION", "1")


def extension(cuda: bool = True) -> Any:
    """The native module: ``softmax_forward/backward``, ``conv_forward/backward``."""
    return _native.attention()


@dataclass(frozen=True)
class Plan:
    """One descriptor row per frequency ``(n, a_n, flat offset, coefficient offset, dim)``."""

    rows: tuple[tuple[int, int, int, int, int], ...]
    heads: int
    width: int
    a_0: int
    complex_width: int
    max_order: int


def plan(mhsa: Any) -> Plan:
    return _plan(mhsa, mhsa.field_type_attn, mhsa.field_type_in, mhsa.num_heads)


def plan_depthwise(conv: Any) -> Plan:
    return _plan(conv, conv.kernel.field_type, conv.kernel.field_type, 1)


def plan_head(head: Any) -> Plan:
    return _plan(head, head.field_type_attn, head.field_type_attn, 1)


def _plan(owner: Any, attn: Any, full: Any, heads: int) -> Plan:
    cached = owner.__dict__.get("_fused_attention_plan")
    if cached is not None:
        return cached
    result = plan_of(attn, full, heads)
    owner.__dict__["_fused_attention_plan"] = result
    return result


def plan_of(attn: Any, full: Any, heads: int) -> Plan:
    """The plan of a per-head type ``attn`` inside ``full`` (reference :98-114)."""
    slices = full.slices()
    rows: list[tuple[int, int, int, int, int]] = []
    coff = 0
    for n, a_n in attn.items():
        if n == 0:
            rows.append((0, a_n, slices[0].start, 0, 1))
        else:
            rows.append((n, a_n, slices[n].start, coff, 2))
            coff += 4 * a_n
    return Plan(tuple(rows), heads, full.dimension, attn.multiplicity(0) if 0 in attn else 0, coff,
                max((2 * n for n, _ in attn.items()), default=0))


def descriptors(owner: Any, p: Plan, device: torch.device) -> Tensor:
    key = ("_fused_attention_desc", str(device))
    cached = owner.__dict__.get(key)
    if cached is None:
        cached = torch.tensor([list(row) for row in p.rows], dtype=torch.int64, device=device)
        owner.__dict__[key] = cached
    return cached


def evaluate_aggregation_window(distances: Tensor, radius: float, kind: str) -> Tensor:
    """``hard``: 1[d <= r + tol]; ``quartic``: relu(1 - (d/r)^2)^2 (reference convolution.py:47-91)."""
    from gm_attention_amd.discretization.edge_geometry import within_cutoff

    if kind == "hard":
        return within_cutoff(distances, radius).to(distances.dtype)
    if kind == "quartic":
        return torch.relu(1.0 - (distances / radius) ** 2) ** 2
    raise ValueError(f"window must be 'hard' or 'quartic', got {kind!r}.")


@dataclass
class Geometry:
    transport: Tensor  # (n_edges, orders, 2)
    angular: Tensor  # (n_edges, orders, 2)
    rho: Tensor
    weights: Tensor
    bias: Tensor
    inside: Tensor  # uint8
    row_ptr: Tensor
    source: Tensor
    max_degree: int
    normalized: dict[float, Tensor] = field(default_factory=dict)
    base: Geometry | None = None
    span: tuple[int, int] | None = None
    chunk_degrees: dict[tuple[int, int], int] = field(default_factory=dict)
    narrowed: dict[int, Tensor] = field(default_factory=dict)

    def aggregation_weights(self, normalize: bool, eps: float) -> Tensor:
        """``c(r) w``, divided by each target's window mass (clamped at ``eps``) when ``normalize``."""
        if self.base is not None and self.span is not None:
            return self.base.aggregation_weights(normalize, eps)[self.span[0]:self.span[1]]
        if not normalize:
            return self.weights
        cached = self.normalized.get(eps)
        if cached is None:
            mass = torch.segment_reduce(self.weights, "sum", offsets=self.row_ptr, axis=0).clamp_min(eps)
            target = torch.repeat_interleave(torch.arange(mass.shape[0], device=mass.device),
                                             self.row_ptr[1:] - self.row_ptr[:-1])
            cached = (self.weights / mass.index_select(0, target)).contiguous()
            self.normalized[eps] = cached
        return cached

    def transport_to(self, order: int) -> Tensor:
        """The transport table narrowed to orders ``0..order`` (contiguous, cached):
        the softmax reads only the heads' own frequencies."""
        if order + 1 >= self.transport.shape[1]:
            return self.transport
        if self.base is not None and self.span is not None:
            return self.base.transport_to(order)[self.span[0]:self.span[1]]
        cached = self.narrowed.get(order)
        if cached is None:
            cached = self.transport[:, : order + 1].contiguous()
            self.narrowed[order] = cached
        return cached


_GEOMETRIES: OrderedDict[tuple, tuple[Any, Geometry]] = OrderedDict()
_GEOMETRY_CACHE = 64
_CHUNKS: dict[int, tuple[Any, Any, int, int]] = {}


def register_chunk(chunk: Any, parent: Any, first: int, last: int) -> None:
    _purge()
    _CHUNKS[id(chunk.row_ptr)] = (weakref.ref(chunk.row_ptr), parent, int(first), int(last))


def chunk_of(edges: Any) -> tuple[Any, int, int] | None:
    registered = _CHUNKS.get(id(edges.row_ptr))
    if registered is None or registered[0]() is not edges.row_ptr:
        return None
    return registered[1], registered[2], registered[3]


def _purge() -> None:
    for key in [k for k, (held, _) in _GEOMETRIES.items() if held() is None]:
        del _GEOMETRIES[key]
    for key in [k for k, (held, _, _, _) in _CHUNKS.items() if held() is None]:
        del _CHUNKS[key]


def geometry(edges: Any, cutoff: float, window: str, dtype: torch.dtype) -> Geometry:
    """The per-edge constants of ``edges`` (reference :203-255), cached while the edge set lives."""
    _purge()
    registered = _CHUNKS.get(id(edges.row_ptr))
    if registered is not None and registered[0]() is edges.row_ptr:
        _, parent, first, last = registered
        base = geometry(parent, cutoff, window, dtype)
        degree = base.chunk_degrees.get((first, last))
        if degree is None:
            rp = edges.row_ptr
            degree = int((rp[1:] - rp[:-1]).max()) if rp.numel() > 1 else 0
            base.chunk_degrees[(first, last)] = degree
        return Geometry(base.transport[first:last], base.angular[first:last], base.rho[first:last],
                        base.weights[first:last], base.bias[first:last], base.inside[first:last],
                        edges.row_ptr.contiguous(), edges.source_index.contiguous(), degree, base=base,
                        span=(first, last))
    key = (id(edges.row_ptr), float(cutoff), window, dtype, str(edges.row_ptr.device))
    held = _GEOMETRIES.get(key)
    if held is not None and held[0]() is edges.row_ptr:
        _GEOMETRIES.move_to_end(key)
        return held[1]
    tiny = torch.finfo(dtype).tiny
    distances = edges.distances.to(dtype)
    quadrature = edges.tangent_quadrature_weights.to(dtype)
    window_values = evaluate_aggregation_window(distances, cutoff, window)
    bias = torch.log(window_values.clamp_min(tiny)) + torch.log(quadrature.clamp_min(tiny))
    row_ptr = edges.row_ptr.contiguous()
    max_degree = int((row_ptr[1:] - row_ptr[:-1]).max()) if row_ptr.numel() > 1 else 0
    result = Geometry(
        torch.view_as_real(edges.transport_phases.contiguous()).to(dtype).contiguous(),
        torch.view_as_real(edges.angular_phases.contiguous()).to(dtype).contiguous(),
        (distances / cutoff).contiguous(), (window_values * quadrature).contiguous(), bias.contiguous(),
        (window_values > 0.0).to(torch.uint8).contiguous(), row_ptr, edges.source_index.contiguous(), max_degree,
    )
    _GEOMETRIES[key] = (weakref.ref(edges.row_ptr), result)
    while len(_GEOMETRIES) > _GEOMETRY_CACHE:
        _GEOMETRIES.popitem(last=False)
    return result


def _device_ok(x: Any) -> bool:
    if MODE == "0":
        return False
    if MODE != "cpu" and x.device.type != "cuda":
        return False
    return x.dtype in (torch.float32, torch.float64)


def softmax_enabled(mhsa: Any, x: Any, edges: Any) -> bool:
    """Whether the batched attention takes the fused scores-and-softmax op."""
    if not _device_ok(x) or mhsa.num_heads > MAX_H:
        return False
    p = plan(mhsa)
    if len(p.rows) > MAX_F or p.width > MAX_D or max((n for n, *_ in p.rows), default=0) > edges.max_frequency:
        return False
    return edges.n_edges > 0


def softmax_head_enabled(head: Any, x: Any, edges: Any) -> bool:
    if not _device_ok(x):
        return False
    p = plan_head(head)
    if len(p.rows) > MAX_F or p.width > MAX_D or max((n for n, *_ in p.rows), default=0) > edges.max_frequency:
        return False
    return edges.n_edges > 0


def enabled_depthwise(conv: Any, x: Any, edges: Any) -> bool:
    if not _device_ok(x):
        return False
    p = plan_depthwise(conv)
    if len(p.rows) > MAX_F or p.width > MAX_D or p.max_order > edges.max_frequency:
        return False
    return edges.n_edges > 0


class Depthwise(torch.autograd.Function):
    """The depthwise convolution as one differentiable op on ``v`` and the
    per-edge coefficients ``(rc, cc)`` (reference :329-353)."""

    @staticmethod
    def forward(ctx: Any, v: Tensor, rc: Tensor, cc: Tensor, transport: Tensor, angular: Tensor, rho: Tensor,
                weights: Tensor, desc: Tensor, row_ptr: Tensor, source: Tensor, a_0: int, complex_width: int) -> Tensor:
        ext = extension(cuda=v.is_cuda)
        with torch.profiler.record_function("gm::conv/fused"):
            out = ext.conv_forward(v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, a_0, complex_width)
        ctx.save_for_backward(v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source)
        ctx.ints = (a_0, complex_width)
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_out: Tensor) -> tuple:
        v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source = ctx.saved_tensors
        a_0, complex_width = ctx.ints
        ext = extension(cuda=v.is_cuda)
        with torch.profiler.record_function("gm::conv/fused_backward"):
            dv, drc, dcc = ext.conv_backward(grad_out.contiguous(), v, rc, cc, transport, angular, rho, weights, desc,
                                             row_ptr, source, a_0, complex_width)
        return dv, drc, dcc, None, None, None, None, None, None, None, None, None


def forward_depthwise(conv: Any, v: Tensor, real_coefficients: Tensor | None, complex_coefficients: Tensor | None,
                      edges: Any) -> Tensor:
    """The depthwise convolution over ``edges`` on the flat node field (reference :356-368)."""
    p = plan_depthwise(conv)
    g = geometry(edges, conv.cutoff, conv.window, v.dtype)
    empty = v.new_zeros(0)
    rc = empty if real_coefficients is None else real_coefficients.contiguous()
    cc = empty if complex_coefficients is None else complex_coefficients.contiguous()
    weights = g.aggregation_weights(bool(conv.normalize), float(conv.eps))
    return Depthwise.apply(v.contiguous(), rc, cc, g.transport, g.angular, g.rho, weights,
                           descriptors(conv, p, v.device), g.row_ptr, g.source, p.a_0, p.complex_width)


class Softmax(torch.autograd.Function):
    """The heads' scores and neighbourhood softmax as one differentiable op on
    ``(q, k)``: ``alpha (n_edges, H)`` out; ``dq``, ``dk`` back (reference :371-397)."""

    @staticmethod
    def forward(ctx: Any, q: Tensor, k: Tensor, transport: Tensor, bias: Tensor, inside: Tensor, desc: Tensor,
                row_ptr: Tensor, source: Tensor, heads: int, scale: float, max_degree: int) -> Tensor:
        ext = extension(cuda=q.is_cuda)
        with torch.profiler.record_function("gm::attention/fused_softmax"):
            alpha = ext.softmax_forward(q, k, transport, bias, inside, desc, row_ptr, source, heads, scale, max_degree)
        ctx.save_for_backward(q, k, transport, bias, inside, desc, row_ptr, source, alpha)
        ctx.ints = (heads, scale, max_degree)
        return alpha

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx: Any, grad_alpha: Tensor) -> tuple:
        q, k, transport, bias, inside, desc, row_ptr, source, alpha = ctx.saved_tensors
        heads, scale, max_degree = ctx.ints
        ext = extension(cuda=q.is_cuda)
        with torch.profiler.record_function("gm::attention/fused_softmax_backward"):
            dq, dk = ext.softmax_backward(grad_alpha.contiguous(), q, k, transport, bias, inside, desc, row_ptr,
                                          source, alpha, heads, scale, max_degree)
        return dq, dk, None, None, None, None, None, None, None, None, None


def softmax(mhsa: Any, q: Tensor, k: Tensor, edges: Any) -> Tensor:
    """The heads' attention weights ``(n_edges, n_heads)`` (reference :400-410)."""
    p = plan(mhsa)
    g = geometry(edges, mhsa.cutoff, mhsa.heads[0].window, q.dtype)
    scale = float(mhsa.heads[0]._score_scale)
    top = max((n for n, *_ in p.rows), default=0)
    return Softmax.apply(q.contiguous(), k.contiguous(), g.transport_to(top), g.bias, g.inside,
                         descriptors(mhsa, p, q.device), g.row_ptr, g.source, p.heads, scale, max(g.max_degree, 1))


def softmax_head(head: Any, q: Tensor, k: Tensor, edges: Any) -> Tensor:
    """One head's attention weights ``(n_edges,)`` (reference :413-422)."""
    p = plan_head(head)
    g = geometry(edges, head.cutoff, head.window, q.dtype)
    scale = float(head._score_scale)
    top = max((n for n, *_ in p.rows), default=0)
    alpha = Softmax.apply(q.contiguous(), k.contiguous(), g.transport_to(top), g.bias, g.inside,
                          descriptors(head, p, q.device), g.row_ptr, g.source, 1, scale, max(g.max_degree, 1))
    return alpha.reshape(-1)
