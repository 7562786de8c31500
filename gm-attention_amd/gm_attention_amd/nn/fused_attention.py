"""The scores-and-softmax op and the depthwise convolution as HIP kernels.

The drop-in for the reference's ``gm_attention/nn/fused_attention.py``: the
same switch (``GM_FUSED_ATTENTION``, read at import: ``"0"`` off, ``"1"`` on for
device tensors, ``"cpu"`` on everywhere), the same ``Plan`` /
``descriptors`` layout (:74-123), the same per-edge ``Geometry`` constants
(:126-255), the same eligibility predicates (:258-326) and the same
autograd Functions ``Softmax`` (:371-397) and ``Depthwise`` (:329-353), so the
attention and convolution layers call it unchanged.  The arithmetic runs in
``libgmhip.so`` (``_native.attention()``); there is no CPU driver, so under
every switch value the predicates send CPU tensors to the eager path (the
reference's ``"cpu"`` runs its CPU driver of the same function there,
attention_cpu.cpp:256-261), and a CPU tensor reaching an op itself is an error.

Differences from the reference, all implementation limits rather than
semantics: no neighbourhood-size bound (the reference declines when
``max_degree * heads > 8192``, which excludes the 256x512 grid); the key and
value gradients are gathered per source node instead of added atomically,
so they are deterministic; a call the predicates decline runs the same
numbers in torch (``eager_ops``) as the reference runs its eager path; the
geometry keeps a copy of the transport table
narrowed to the orders a layer reads; the per-edge tables live on the edge
set they describe (built once, dropped with it) instead of a process-wide
cache.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch
from torch import Tensor

from gm_attention_amd import _native

MAX_H, MAX_F, MAX_D, DESC = 16, 8, 1024, 5
#: ``"0"`` off, ``"1"`` on for device tensors, ``"cpu"`` on everywhere: device tensors take the HIP
#: ops and CPU tensors the eager path, this build having no CPU driver (reference :43-60).  The default is ``"1"`` (the reference's is ``"0"``): this build exists
#: to run the HIP path; a declined call runs ``eager_ops`` as the reference runs its eager layers.
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
    """The per-edge constants the fused ops read for one edge set, cutoff,
    window and dtype (the constants of reference :126-164): the transport and
    angular phase tables as ``(E, orders, 2)`` real pairs, ``rho = d / cutoff``,
    the aggregation weights ``c(d) w``, the softmax bias ``log c + log w``
    (each clamped at the dtype's tiny), the window support ``inside``, the CSR
    and the largest neighbourhood.  Derived tables (the weights divided by
    each target's window mass, the transport narrowed to a layer's orders)
    are memoised in ``derived``; a chunk's geometry (``parent``, ``edges``)
    takes them as views of its parent's."""

    transport: Tensor
    angular: Tensor
    rho: Tensor
    weights: Tensor
    bias: Tensor
    inside: Tensor
    row_ptr: Tensor
    source: Tensor
    max_degree: int
    derived: dict = field(default_factory=dict)
    parent: Geometry | None = None
    edges: tuple[int, int] | None = None

    def _derive(self, key: tuple, make) -> Tensor:
        if self.parent is not None and self.edges is not None:
            e0, e1 = self.edges
            return self.parent._derive(key, make)[e0:e1]
        held = self.derived.get(key)
        if held is None:
            held = make()
            self.derived[key] = held
        return held

    def aggregation_weights(self, normalize: bool, eps: float) -> Tensor:
        """``c(d) w``; under ``normalize`` divided by each target's window mass
        clamped at ``eps`` (a chunk holds whole neighbourhoods: its parent's masses)."""
        if not normalize:
            return self.weights

        def normalized() -> Tensor:
            counts = self.row_ptr[1:] - self.row_ptr[:-1]
            mass = torch.segment_reduce(self.weights, "sum", offsets=self.row_ptr, axis=0).clamp_min(eps)
            return (self.weights / torch.repeat_interleave(mass, counts)).contiguous()

        return self._derive(("normalized", float(eps)), normalized)

    def transport_to(self, order: int) -> Tensor:
        """The transport table narrowed to orders ``0..order`` (contiguous): the
        softmax reads only the heads' own frequencies."""
        if order + 1 >= self.transport.shape[1]:
            return self.transport
        return self._derive(("transport", int(order)), lambda: self.transport[:, : order + 1].contiguous())

    def host_row_ptr(self) -> np.ndarray:
        """The CSR offsets on the host (read once)."""
        held = self.derived.get("host_row_ptr")
        if held is None:
            held = self.row_ptr.detach().to("cpu").numpy()
            self.derived["host_row_ptr"] = held
        return held


def _tables(edges: Any, cutoff: float, window: str, dtype: torch.dtype) -> Geometry:
    tiny = torch.finfo(dtype).tiny
    d = edges.distances.to(dtype)
    quad = edges.tangent_quadrature_weights.to(dtype)
    win = evaluate_aggregation_window(d, cutoff, window)
    row_ptr = edges.row_ptr.contiguous()
    g = Geometry(torch.view_as_real(edges.transport_phases.contiguous()).to(dtype).contiguous(),
                 torch.view_as_real(edges.angular_phases.contiguous()).to(dtype).contiguous(),
                 (d / cutoff).contiguous(), (win * quad).contiguous(),
                 (torch.log(win.clamp_min(tiny)) + torch.log(quad.clamp_min(tiny))).contiguous(),
                 (win > 0.0).to(torch.uint8).contiguous(), row_ptr, edges.source_index.contiguous(), 0)
    degrees = np.diff(g.host_row_ptr())
    g.max_degree = int(degrees.max()) if degrees.size else 0
    return g


def _chunk_tables(parent: Geometry, edges: Any, e0: int, e1: int) -> Geometry:
    """Views of ``parent``'s tables over its edges ``[e0, e1)`` (whole neighbourhoods of the
    targets ``first .. last - 1``), with the chunk's own CSR and largest neighbourhood."""
    ptr = parent.host_row_ptr()
    first, last = int(np.searchsorted(ptr, e0, side="right")) - 1, int(np.searchsorted(ptr, e1, side="left"))
    degrees = np.diff(ptr[max(first, 0):last + 1])
    part = slice(e0, e1)
    return Geometry(parent.transport[part], parent.angular[part], parent.rho[part], parent.weights[part],
                    parent.bias[part], parent.inside[part], edges.row_ptr.contiguous(),
                    edges.source_index.contiguous(), int(degrees.max()) if degrees.size else 0, parent=parent,
                    edges=(e0, e1))


def register_chunk(chunk: Any, parent: Any, first: int, last: int) -> None:
    """Record that ``chunk`` is ``parent``'s edges ``first .. last`` in order
    (reference :176-187), so its tables are views of the parent's; edge sets
    made by ``EdgeGeometry.target_range`` carry this already."""
    chunk.__dict__["_span"] = (parent, int(first), int(last))


def chunk_of(edges: Any) -> tuple[Any, int, int] | None:
    """``(parent, first, last)`` of a chunk edge set, else ``None``."""
    return edges.__dict__.get("_span")


def geometry(edges: Any, cutoff: float, window: str, dtype: torch.dtype) -> Geometry:
    """The per-edge constants of ``edges`` (reference :203-255), built once and
    kept on the edge set itself (so for as long as it lives); a chunk's are
    views of its parent's."""
    store = edges.__dict__.setdefault("_fused_geometry", {})
    key = (float(cutoff), window, dtype)
    g = store.get(key)
    if g is None:
        span = chunk_of(edges)
        if span is None:
            g = _tables(edges, cutoff, window, dtype)
        else:
            parent, e0, e1 = span
            g = _chunk_tables(geometry(parent, cutoff, window, dtype), edges, e0, e1)
        store[key] = g
    return g


def _device_ok(x: Any) -> bool:
    """Device tensors of the ops' element types under ``"1"`` and ``"cpu"``;
    CPU tensors never (they run the eager path under every switch value)."""
    if MODE == "0" or x.device.type != "cuda":
        return False
    return x.dtype in (torch.float32, torch.float64)


def _rows_ok(x: Any, heads: int) -> bool:
    """The scores' rows: the element types of _device_ok, or bfloat16 rows on
    the GPU whose heads the fast kernels serve (a power of two up to 16)."""
    if x.dtype == torch.bfloat16:
        return MODE != "0" and x.device.type == "cuda" and heads in (1, 2, 4, 8, 16)
    return _device_ok(x)


def softmax_enabled(mhsa: Any, x: Any, edges: Any) -> bool:
    """Whether the batched attention takes the fused scores-and-softmax op."""
    if not _rows_ok(x, mhsa.num_heads) or mhsa.num_heads > MAX_H:
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
    """The heads' attention weights ``(n_edges, n_heads)`` (reference :400-410);
    bfloat16 rows take float32 tables and give float32 weights."""
    p = plan(mhsa)
    g = geometry(edges, mhsa.cutoff, mhsa.heads[0].window, torch.float32 if q.dtype == torch.bfloat16 else q.dtype)
    scale = float(mhsa.heads[0]._score_scale)
    top = max((n for n, *_ in p.rows), default=0)
    return Softmax.apply(q.contiguous(), k.contiguous(), g.transport_to(top), g.bias, g.inside,
                         descriptors(mhsa, p, q.device), g.row_ptr, g.source, p.heads, scale, max(g.max_degree, 1))


def softmax_eager(p: Plan, q: Tensor, k: Tensor, edges: Any, cutoff: float, window: str, scale: float) -> Tensor:
    """The heads' attention weights ``(n_edges, heads)`` by :func:`eager_ops.softmax`
    on the same geometry tables: the path of a call the fused op declines."""
    from gm_attention_amd.nn import eager_ops

    g = geometry(edges, cutoff, window, q.dtype)
    return eager_ops.softmax(q, k, g.transport, g.bias, g.inside, p.rows, g.row_ptr, g.source, p.heads, scale)


def softmax_head(head: Any, q: Tensor, k: Tensor, edges: Any) -> Tensor:
    """One head's attention weights ``(n_edges,)`` (reference :413-422)."""
    p = plan_head(head)
    g = geometry(edges, head.cutoff, head.window, q.dtype)
    scale = float(head._score_scale)
    top = max((n for n, *_ in p.rows), default=0)
    alpha = Softmax.apply(q.contiguous(), k.contiguous(), g.transport_to(top), g.bias, g.inside,
                          descriptors(head, p, q.device), g.row_ptr, g.source, 1, scale, max(g.max_degree, 1))
    return alpha.reshape(-1)
