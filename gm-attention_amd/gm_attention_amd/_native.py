"""The HIP library behind the fused ops: loading, signatures, and the
extension objects whose entry points carry the reference's names and
argument orders.

``attention()`` stands where the reference's ``gm_fused_attention`` pybind
module stands (``nn/fused/attention_cpu.cpp:256-261``): ``softmax_forward``,
``softmax_backward``, ``conv_forward``, ``conv_backward``.  ``factored()``
stands for ``gm_factored`` (``nn/fused/factored_cpu.cpp:223-234``):
``forward``, ``aggregate``, ``backward``, ``backward_aggregated``.  ``pairs()``
stands for the ``gm_pairs`` modules (``nn/fused/pairs_cpu.cpp:138-148``):
``forward``, ``backward`` of one pair term.  Tensors are
checked with the reference's messages (``attention_cpu.cpp:42-64, 149-171``),
outputs are allocated here through torch's caching allocator, and the raw
pointers go to ``libgmhip.so`` on the current HIP stream.  There is no CPU
driver: a CPU tensor is an error, and a missing library is an error, never a
silent fallback.
"""

from __future__ import annotations

import ctypes
import functools
import weakref
from pathlib import Path
from typing import Any

import torch
from torch import Tensor

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libgmhip.so"

_P = ctypes.c_void_p
_I = ctypes.c_int64
_D = ctypes.c_double

#: C signatures, in include/gm_hip.h order (the return type is int everywhere).
SIGNATURES: dict[str, list[Any]] = {
    "gm_softmax_forward": [_P] * 8 + [_I] * 6 + [_D, _I, _P, _P],
    "gm_softmax_backward": [_P] * 10 + [_I] * 6 + [_D, _I] + [_P] * 9,
    "gm_conv_forward": [_P] * 10 + [_I] * 7 + [_P, _P],
    "gm_conv_backward": [_P] * 11 + [_I] * 7 + [_P] * 7,
    "gm_factored_forward": [_P] * 10 + [_I] * 10 + [_P, _P],
    "gm_factored_aggregate": [_P] * 3 + [_I] * 3 + [_P, _P],
    "gm_factored_backward": [_P] * 14 + [_I] * 9 + [_P] * 5,
    "gm_factored_forward_seg": [_P] * 5 + [_I] + [_P] * 7 + [_I] * 10 + [_P, _P],
    "gm_factored_backward_seg": [_P] * 10 + [_I] + [_P] * 7 + [_I] * 9 + [_P] * 3,
    "gm_pairs_forward": [_P] * 8 + [_I] * 5 + [_P],
    "gm_pairs_backward": [_P] * 11 + [_I] * 6 + [_P],
}

#: fp32-only and host-only entry points (name -> (restype, argtypes)).
SIGNATURES_F32 = {
    "gm_softmax_forward_bf16": (ctypes.c_int, [_P] * 8 + [_I] * 6 + [_D, _I, _P, _P]),
    "gm_softmax_backward_bf16": (ctypes.c_int, [_P] * 10 + [_I] * 6 + [_D, _I] + [_P] * 9),
    "gm_radial_trunk_forward_f32": (ctypes.c_int, [_P] * 4 + [_I] * 4 + [_D, _P, _P]),
    "gm_radial_trunk_backward_f32": (ctypes.c_int, [_P] * 5 + [_I] * 4 + [_D, _P, _P, _P]),
    "gm_radial_trunk_partials": (ctypes.c_int64, [_I]),
    "gm_radial_trunk_forward_bf16": (ctypes.c_int, [_P] * 4 + [_I] * 4 + [_D, _P, _P]),
    "gm_radial_trunk_backward_bf16": (ctypes.c_int, [_P] * 5 + [_I] * 4 + [_D, _P, _P, _P]),
    "gm_node_mix_forward_f32": (ctypes.c_int, [_P, _I, _P, _I, _I, _I, _P, _P]),
    "gm_node_mix_backward_input_f32": (ctypes.c_int, [_P, _P, _I, _I, _I, _P, _I, _P]),
    "gm_node_mix_weight_partials": (ctypes.c_int64, [_I, _I, _I]),
    "gm_node_mix_backward_weight_f32": (ctypes.c_int, [_P, _I, _P, _I, _I, _I, _P, _P, _P]),
    "gm_node_mix_backward_weight_noalloc_f32": (ctypes.c_int, [_P, _I, _P, _I, _I, _I, _P, _P]),
    "gm_node_mix_forward_bf16": (ctypes.c_int, [_P, _I, _P, _I, _I, _I, _P, _P]),
    "gm_node_mix_backward_weight_bf16": (ctypes.c_int, [_P, _I, _P, _I, _I, _I, _P, _P, _P]),
    "gm_node_mix_backward_weight_bf16_bf16": (ctypes.c_int, [_P, _I, _P, _I, _I, _I, _P, _P, _P]),
    "gm_node_mix_backward_weight_f32_bf16": (ctypes.c_int, [_P, _I, _P, _I, _I, _I, _P, _P, _P]),
    "gm_xcd_block_map": (ctypes.c_int, [_I, ctypes.c_int, _P, _I, ctypes.c_int, _P]),
    "gm_factored_forward_grouped_f32": (ctypes.c_int, [_P] * 5 + [_I] + [_P] * 7 + [_I] * 10 + [_P] * 3 + [_I, _D]
                                        + [_P, _P]),
    "gm_factored_backward_grouped_f32": (ctypes.c_int, [_P] * 10 + [_I] + [_P] * 7 + [_I] * 10 + [_P] * 3 + [_I, _D]
                                         + [_I] + [_P] * 3),
    "gm_factored_backward_grouped_ld_f32": (ctypes.c_int, [_P, _I] + [_P] * 9 + [_I] + [_P] * 7 + [_I] * 10
                                            + [_P] * 3 + [_I, _D] + [_I] + [_P] * 3),
    "gm_factored_aggregate_gather_f32": (ctypes.c_int, [_P] * 4 + [_I] * 3 + [_P, _P]),
    "gm_factored_lane_tables": (ctypes.c_int, [_P] + [_I] * 6 + [_P] * 3),
    "gm_factored_lanes_fixed": (ctypes.c_int, [_P] + [_I] * 6 + [_P]),
    "gm_factored_aggregate_heads_f32": (ctypes.c_int, [_P] * 4 + [_I] * 5 + [_P, _P]),
    "gm_factored_aggregate_heads_bf16": (ctypes.c_int, [_P] * 4 + [_I] * 5 + [_P, _P]),
    "gm_factored_forward_grouped_bf16": (ctypes.c_int, [_P] * 5 + [_I] + [_P] * 7 + [_I] * 10 + [_P, _P]),
    "gm_factored_backward_grouped_ld_bf16": (ctypes.c_int, [_P, _I] + [_P] * 9 + [_I] + [_P] * 7 + [_I] * 10 + [_I]
                                             + [_P] * 3),
    "gm_gather_transpose_f32": (ctypes.c_int, [_P, _P, _I, _I, _P, _P]),
    "gm_scatter_transpose_f32": (ctypes.c_int, [_P, _P, _I, _I, _P, _P]),
    "gm_conv_radial_partial_row": (ctypes.c_int64, []),
    "gm_conv_radial_backward_groups": (ctypes.c_int64, [_I]),
    "gm_conv_radial_workspace_rows": (ctypes.c_int64, [_I]),
    "gm_conv_radial_forward_f32": (ctypes.c_int, [_P] * 6 + [_I, _D] + [_P] * 6 + [_I] * 7 + [_P] * 4),
    "gm_conv_radial_backward_f32": (ctypes.c_int, [_P] * 8 + [_I, _D] + [_P] * 7 + [_I] * 7 + [_P, _P, _I] + [_P] * 4),
    "gm_radius_workspace_doubles": (ctypes.c_int64, [_I, _I]),
    "gm_radius_row_ptr_f64": (ctypes.c_int, [_P, _I, _P, _I, _D, _P, _P, _P]),
    "gm_radius_edges_f64": (ctypes.c_int, [_P, _I, _P, _I, _D, _P, _P, _I, _P, _P]),
    "gm_geodesic_distances_f64": (ctypes.c_int, [_P] * 3 + [_I] * 3 + [_P, _P]),
    "gm_edge_tables_f64": (ctypes.c_int, [_P] * 6 + [_I] * 4 + [_P] * 7 + [_P]),
    "gm_layer_norm_partial_rows": (ctypes.c_int64, [_I]),
    "gm_ffn_partial_rows": (ctypes.c_int64, [_I]),
    "gm_ffn_forward_bf16": (ctypes.c_int, [_P, _I, _I, _I, _D, ctypes.c_int] + [_P] * 12),
    "gm_ffn_backward_bf16": (ctypes.c_int, [_P, _P, _I, _I, _I, _D, ctypes.c_int] + [_P] * 20),
    **{f"gm_layer_norm_forward_{sfx}": (ctypes.c_int, [_P] * 3 + [_I] * 4 + [_P, _P, _D] + [_P] * 4)
       for sfx in ("f32", "f64", "bf16")},
    **{f"gm_layer_norm_backward_{sfx}": (ctypes.c_int, [_P] * 5 + [_I] * 4 + [_P] * 2 + [_P] * 4)
       for sfx in ("f32", "f64", "bf16")},
    **{f"gm_gate_forward_{sfx}": (ctypes.c_int, [_P] * 2 + [_I] * 4 + [_P, _P, _I, _P, _P])
       for sfx in ("f32", "f64", "bf16")},
    **{f"gm_gate_backward_{sfx}": (ctypes.c_int, [_P] * 3 + [_I] * 4 + [_P, _P, _I] + [_P] * 3)
       for sfx in ("f32", "f64", "bf16")},
}


class NativeLibraryError(RuntimeError):
    """libgmhip.so is missing or cannot be loaded."""


@functools.cache
def library() -> ctypes.CDLL:
    """Load libgmhip.so (after torch, so it binds to torch's HIP runtime)."""
    if not LIB_PATH.exists():
        raise NativeLibraryError(
            f"{LIB_PATH} is not built: run `python gm-attention_amd/build.py` (hipcc --offload-arch=gfx950)"
        )
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as error:
        raise NativeLibraryError(f"cannot load {LIB_PATH}: {error}") from error
    lib.gm_last_error.restype = ctypes.c_char_p
    lib.gm_last_error.argtypes = []
    lib.gm_abi_version.restype = ctypes.c_int
    for stem, args in SIGNATURES.items():
        for suffix in ("_f32", "_f64"):
            fn = getattr(lib, stem + suffix)
            fn.restype = ctypes.c_int
            fn.argtypes = args
    for name, (res, args) in SIGNATURES_F32.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _call(name: str, *args: Any) -> None:
    status = getattr(library(), name)(*args)
    if status != 0:
        message = library().gm_last_error().decode()
        raise RuntimeError(f"{name}: {message}")


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _suffix(dtype: torch.dtype) -> str:
    if dtype == torch.float32:
        return "_f32"
    if dtype == torch.float64:
        return "_f64"
    raise RuntimeError(f"libgmhip supports float32 and float64, got {dtype}")


def _row_suffix(dtype: torch.dtype) -> str:
    """The softmax entry points' suffix: bfloat16 rows have their own (float32 tables)."""
    return "_bf16" if dtype == torch.bfloat16 else _suffix(dtype)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def _require_device(*tensors: Tensor) -> None:
    first = tensors[0]
    if first.device.type != "cuda":
        raise RuntimeError(
            "libgmhip runs on the GPU only: the tensors are on the CPU (this build has no CPU driver)"
        )
    for t in tensors:
        _check(t.is_contiguous(), "every tensor must be contiguous")
        _check(t.device == first.device, "every tensor must live on the same device")


_HOST_DESC: dict[tuple, tuple[Any, Tensor]] = {}


def host_desc(desc: Tensor) -> Tensor:
    """A CPU int64 copy of a descriptor table, cached per device tensor (its
    identity and version), so a layer's descriptor is copied to the host once."""
    if desc.device.type == "cpu":
        return desc.contiguous()
    key = (id(desc), desc.data_ptr(), desc._version)
    held = _HOST_DESC.get(key)
    if held is not None and held[0]() is desc:
        return held[1]
    copy = desc.detach().to("cpu").contiguous()
    for stale in [k for k, (ref, _) in _HOST_DESC.items() if ref() is None]:
        del _HOST_DESC[stale]
    _HOST_DESC[key] = (weakref.ref(desc), copy)
    return copy


# ---------------------------------------------------------------- source groups

_GROUPS: dict[tuple, tuple[Any, tuple[Tensor, Tensor, Tensor]]] = {}


def source_major(source: Tensor, row_ptr: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """``(src_ptr, src_order, target)``: every node's run of edges in the
    edges sorted (stably) by source, and each edge's target.  The transposed
    CSR the backward passes walk instead of adding atomically; built on the
    device once per edge set and cached against the ``source`` tensor."""
    n_nodes = row_ptr.shape[0] - 1
    key = (id(source), source.data_ptr(), source.numel(), source._version, row_ptr.data_ptr(), n_nodes)
    held = _GROUPS.get(key)
    if held is not None and held[0]() is source:
        return held[1]
    device = source.device
    if source.numel() == 0:
        result = (torch.zeros(n_nodes + 1, dtype=torch.int64, device=device),
                  torch.zeros(0, dtype=torch.int64, device=device), torch.zeros(0, dtype=torch.int64, device=device))
    else:
        order = torch.argsort(source, stable=True)
        counts = torch.bincount(source, minlength=n_nodes)
        src_ptr = torch.zeros(n_nodes + 1, dtype=torch.int64, device=device)
        torch.cumsum(counts, dim=0, out=src_ptr[1:])
        degrees = row_ptr[1:] - row_ptr[:-1]
        target = torch.repeat_interleave(torch.arange(n_nodes, device=device), degrees)
        result = (src_ptr.contiguous(), order.contiguous(), target.contiguous())
    for stale in [k for k, (ref, _) in _GROUPS.items() if ref() is None]:
        del _GROUPS[stale]
    _GROUPS[key] = (weakref.ref(source), result)
    return result


_GROUPED_TABLES: dict[tuple, tuple[Any, Any, tuple[Tensor, Tensor, Tensor]]] = {}


def source_grouped_tables(source: Tensor, row_ptr: Tensor, transport: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """``(target_s, inv, transport_s)`` for the per-source backward passes:
    each edge's target (int32) and transport row in the source grouping's
    order, and every edge's place in that order (int32).  Built on the device
    once per edge set and transport table, cached against both tensors."""
    src_ptr, src_order, target = source_major(source, row_ptr)
    key = (id(source), source.data_ptr(), source._version, id(transport), transport.data_ptr(), transport._version,
           tuple(transport.shape))
    held = _GROUPED_TABLES.get(key)
    if held is not None and held[0]() is source and held[1]() is transport:
        return held[2]
    _check(row_ptr.shape[0] - 1 < 2**31 and source.shape[0] < 2**31,
           "the source-grouped streams index nodes and edges in 32 bits")
    target_s = target.index_select(0, src_order).to(torch.int32)
    inv = torch.empty(source.shape[0], dtype=torch.int32, device=source.device)
    inv[src_order] = torch.arange(source.shape[0], dtype=torch.int32, device=source.device)
    transport_s = transport.index_select(0, src_order).contiguous()
    result = (target_s.contiguous(), inv, transport_s)
    for stale in [k for k, (a, b, _) in _GROUPED_TABLES.items() if a() is None or b() is None]:
        del _GROUPED_TABLES[stale]
    _GROUPED_TABLES[key] = (weakref.ref(source), weakref.ref(transport), result)
    while len(_GROUPED_TABLES) > 8:
        del _GROUPED_TABLES[next(iter(_GROUPED_TABLES))]
    return result


# ---------------------------------------------------------------- attention


class AttentionExtension:
    """The reference's ``gm_fused_attention`` module surface on libgmhip."""

    with_cuda = True  # the device path exists (HIP on ROCm); the attribute name is the reference's

    # ---- scores and softmax (attention_cpu.cpp:149-252) ----

    @staticmethod
    def _check_softmax(q: Tensor, k: Tensor, transport: Tensor, bias: Tensor, inside: Tensor, desc: Tensor,
                       row_ptr: Tensor, source: Tensor, H: int) -> None:
        _check(q.dim() == 2, "q must be (n_nodes, D)")
        _require_device(q, k, transport, bias, inside, row_ptr, source)
        _check(desc.is_contiguous(), "every tensor must be contiguous")
        n, e = q.shape[0], source.shape[0]
        _check(k.dtype == q.dtype, "q and k must share a dtype")
        # bfloat16 rows read float32 tables (and give float32 weights and gradients)
        table = torch.float32 if q.dtype == torch.bfloat16 else q.dtype
        for t in (transport, bias):
            _check(t.dtype == table, "the tables must be q's dtype (float32 for bfloat16 rows)")
        _check(k.shape == q.shape, "q and k must share a shape")
        _check(1 <= H <= 16, "at most 16 heads")
        _check(transport.dim() == 3 and transport.shape[0] == e and transport.shape[2] == 2,
               "transport must be (n_edges, orders, 2)")
        _check(bias.dim() == 1 and bias.shape[0] == e, "bias must be (n_edges,)")
        _check(inside.dtype == torch.uint8 and inside.shape == bias.shape, "inside must be uint8 (n_edges,)")
        _check(desc.dtype == torch.int64 and desc.dim() == 2 and desc.shape[1] == 5 and desc.shape[0] <= 8,
               "desc must be int64 (F <= 8, 5)")
        _check(row_ptr.dtype == torch.int64 and row_ptr.dim() == 1 and row_ptr.shape[0] == n + 1,
               "row_ptr must be int64 (n_nodes + 1,)")
        _check(source.dtype == torch.int64 and source.dim() == 1, "source must be int64 (n_edges,)")
        _check(q.shape[1] >= 1, "D must be positive")

    def softmax_forward(self, q: Tensor, k: Tensor, transport: Tensor, bias: Tensor, inside: Tensor, desc: Tensor,
                        row_ptr: Tensor, source: Tensor, H: int, scale: float, deg_max: int) -> Tensor:
        """alpha (n_edges, H): the heads' neighbourhood softmax of the transported scores."""
        self._check_softmax(q, k, transport, bias, inside, desc, row_ptr, source, H)
        alpha = torch.empty(source.shape[0], H, dtype=transport.dtype, device=q.device)
        if q.shape[0] == 0:
            return alpha
        hd = host_desc(desc)
        _call("gm_softmax_forward" + _row_suffix(q.dtype), _ptr(q), _ptr(k), _ptr(transport), _ptr(bias), _ptr(inside),
              hd.data_ptr(), _ptr(row_ptr), _ptr(source), q.shape[0], source.shape[0], q.shape[1], transport.shape[1],
              hd.shape[0], H, float(scale), int(deg_max), _ptr(alpha), _stream(q.device))
        return alpha

    def softmax_backward(self, dalpha: Tensor, q: Tensor, k: Tensor, transport: Tensor, bias: Tensor, inside: Tensor,
                         desc: Tensor, row_ptr: Tensor, source: Tensor, alpha: Tensor, H: int, scale: float,
                         deg_max: int) -> list[Tensor]:
        """[dq, dk] from d alpha and the saved alpha (dk gathered per source, no atomics)."""
        self._check_softmax(q, k, transport, bias, inside, desc, row_ptr, source, H)
        for t in (alpha, dalpha):
            _check(t.is_contiguous() and t.dim() == 2 and t.shape[0] == source.shape[0] and t.shape[1] == H
                   and t.dtype == transport.dtype,
                   "alpha and dalpha must be contiguous (n_edges, H) in the tables' dtype")
        # the gradients in the arithmetic's dtype (float32 for bfloat16 rows)
        dq = torch.empty(q.shape, dtype=transport.dtype, device=q.device)
        dk = torch.empty(q.shape, dtype=transport.dtype, device=q.device)
        if q.shape[0] == 0:
            return [dq, dk]
        src_ptr, src_order, _ = source_major(source, row_ptr)
        target_s, inv, transport_s = source_grouped_tables(source, row_ptr, transport.contiguous())
        ds = torch.empty(source.shape[0], H, dtype=transport.dtype, device=q.device)
        hd = host_desc(desc)
        _call("gm_softmax_backward" + _row_suffix(q.dtype), _ptr(dalpha), _ptr(q), _ptr(k), _ptr(transport), _ptr(bias),
              _ptr(inside), hd.data_ptr(), _ptr(row_ptr), _ptr(source), _ptr(alpha), q.shape[0], source.shape[0],
              q.shape[1], transport.shape[1], hd.shape[0], H, float(scale), int(deg_max), _ptr(src_ptr),
              _ptr(src_order), _ptr(target_s), _ptr(inv), _ptr(transport_s), _ptr(ds), _ptr(dq), _ptr(dk),
              _stream(q.device))
        return [dq, dk]

    # ---- depthwise convolution (attention_cpu.cpp:42-145) ----

    @staticmethod
    def _check_conv(v: Tensor, rc: Tensor, cc: Tensor, transport: Tensor, angular: Tensor, rho: Tensor,
                    weights: Tensor, desc: Tensor, row_ptr: Tensor, source: Tensor, A0: int, W: int) -> None:
        _check(v.dim() == 2, "v must be (n_nodes, D)")
        _require_device(v, rc, cc, transport, angular, rho, weights, row_ptr, source)
        _check(desc.is_contiguous(), "every tensor must be contiguous")
        n, e = v.shape[0], source.shape[0]
        for t in (rc, cc, transport, angular, rho, weights):
            _check(t.dtype == v.dtype, "v, the coefficients, the weights and the tables must share a dtype")
        _check(rc.numel() == e * A0, "rc must hold (1, n_edges, a_0) entries")
        _check(cc.numel() == e * W, "cc must hold (1, n_edges, W) entries")
        _check(transport.dim() == 3 and transport.shape[0] == e and transport.shape[2] == 2,
               "transport must be (n_edges, orders, 2)")
        _check(angular.shape == transport.shape, "angular must match transport's shape")
        _check(rho.dim() == 1 and rho.shape[0] == e and weights.shape == rho.shape, "rho and weights must be (n_edges,)")
        _check(desc.dtype == torch.int64 and desc.dim() == 2 and desc.shape[1] == 5 and desc.shape[0] <= 8,
               "desc must be int64 (F <= 8, 5)")
        _check(row_ptr.dtype == torch.int64 and row_ptr.dim() == 1 and row_ptr.shape[0] == n + 1,
               "row_ptr must be int64 (n_nodes + 1,)")
        _check(source.dtype == torch.int64 and source.dim() == 1, "source must be int64 (n_edges,)")
        _check(v.shape[1] >= 1, "D must be positive")

    def conv_forward(self, v: Tensor, rc: Tensor, cc: Tensor, transport: Tensor, angular: Tensor, rho: Tensor,
                     weights: Tensor, desc: Tensor, row_ptr: Tensor, source: Tensor, A0: int, W: int) -> Tensor:
        """out (n_nodes, D) = sum over each target's edges of weight * C_e(tau v_j)."""
        self._check_conv(v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, A0, W)
        out = torch.empty_like(v)
        if v.shape[0] == 0:
            return out
        hd = host_desc(desc)
        _call("gm_conv_forward" + _suffix(v.dtype), _ptr(v), _ptr(rc), _ptr(cc), _ptr(transport), _ptr(angular),
              _ptr(rho), _ptr(weights), hd.data_ptr(), _ptr(row_ptr), _ptr(source), v.shape[0], source.shape[0],
              v.shape[1], transport.shape[1], hd.shape[0], int(A0), int(W), _ptr(out), _stream(v.device))
        return out

    def conv_backward(self, g: Tensor, v: Tensor, rc: Tensor, cc: Tensor, transport: Tensor, angular: Tensor,
                      rho: Tensor, weights: Tensor, desc: Tensor, row_ptr: Tensor, source: Tensor, A0: int,
                      W: int) -> list[Tensor]:
        """[dv, drc, dcc] from the output gradient (one pass per source node, no atomics)."""
        self._check_conv(v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, A0, W)
        _check(g.shape == v.shape and g.is_contiguous() and g.dtype == v.dtype,
               "g must be contiguous, shaped and typed as v")
        dv = torch.empty_like(v)
        drc = torch.empty_like(rc)
        dcc = torch.empty_like(cc)
        if v.shape[0] == 0:
            dv.zero_()
            return [dv, drc, dcc]
        src_ptr, src_order, target = source_major(source, row_ptr)
        hd = host_desc(desc)
        _call("gm_conv_backward" + _suffix(v.dtype), _ptr(g), _ptr(v), _ptr(rc), _ptr(cc), _ptr(transport),
              _ptr(angular), _ptr(rho), _ptr(weights), hd.data_ptr(), _ptr(row_ptr), _ptr(source), v.shape[0],
              source.shape[0], v.shape[1], transport.shape[1], hd.shape[0], int(A0), int(W), _ptr(src_ptr),
              _ptr(src_order), _ptr(target), _ptr(dv), _ptr(drc), _ptr(dcc), _stream(v.device))
        return [dv, drc, dcc]


@functools.cache
def attention() -> AttentionExtension:
    library()  # raises when the library is absent
    return AttentionExtension()


# ---------------------------------------------------------------- factored kernel

MAX_K, MAX_OUT, MAX_BM, MAX_C, FACT_DESC = 20, 128, 32, 320, 8


def _fcheck(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError("gm_factored: " + message)


_HOST_DESC32: dict[tuple, tuple[Any, Tensor]] = {}


def host_desc32(desc: Tensor) -> Tensor:
    """A CPU int32 copy of a factored descriptor table, cached per device tensor."""
    if desc.device.type == "cpu":
        return desc.contiguous()
    key = (id(desc), desc.data_ptr(), desc._version)
    held = _HOST_DESC32.get(key)
    if held is not None and held[0]() is desc:
        return held[1]
    copy = desc.detach().to("cpu").contiguous()
    for stale in [k for k, (ref, _) in _HOST_DESC32.items() if ref() is None]:
        del _HOST_DESC32[stale]
    _HOST_DESC32[key] = (weakref.ref(desc), copy)
    return copy


class FactoredExtension:
    """The reference's ``gm_factored`` module surface on libgmhip."""

    with_cuda = True

    @staticmethod
    def _check_common(h: Tensor, zc: Tensor, zr: Tensor, angular: Tensor, transport: Tensor, rho: Tensor,
                      desc: Tensor, source: Tensor, d_out: int) -> None:
        """The checks of factored_cpu.cpp:37-58, with the same messages."""
        _fcheck(h.dim() == 2 and h.is_contiguous(), "h must be a contiguous (n_edges, k - 1) tensor")
        _fcheck(zc.dim() == 4 and zc.shape[3] == 2 and zc.is_contiguous(),
                "zc must be a contiguous (n_nodes, k, wc, 2) tensor")
        _fcheck(zr.dim() == 3 and zr.is_contiguous(), "zr must be a contiguous (n_nodes, k, wr) tensor")
        _fcheck(zc.shape[1] == h.shape[1] + 1 and zr.shape[1] == h.shape[1] + 1,
                "zc and zr must have k = h's width + 1 (the constant feature)")
        _fcheck(zc.shape[0] == zr.shape[0], "zc and zr must have the same node count")
        _fcheck(angular.dim() == 3 and angular.shape[2] == 2 and angular.is_contiguous()
                and angular.shape[0] == h.shape[0], "angular must be a contiguous (n_edges, n_f, 2) tensor")
        _fcheck(transport.shape == angular.shape and transport.is_contiguous(), "transport must match angular")
        _fcheck(rho.dim() == 1 and rho.is_contiguous() and rho.shape[0] == h.shape[0],
                "rho must be a contiguous (n_edges,) tensor")
        _fcheck(desc.dim() == 2 and desc.shape[1] == FACT_DESC and desc.dtype == torch.int32 and desc.is_contiguous(),
                "desc must be a contiguous int32 (n_blocks, 8) tensor")
        _fcheck(source.dim() == 1 and source.shape[0] == h.shape[0] and source.dtype == torch.int64
                and source.is_contiguous(), "source must be a contiguous int64 (n_edges,) tensor")
        _fcheck(h.shape[1] + 1 <= MAX_K, "k exceeds MAX_K")
        _fcheck(1 <= d_out <= MAX_OUT, "d_out must be in [1, MAX_OUT]")
        _fcheck(2 * zc.shape[2] + zr.shape[2] <= MAX_C, "2 wc + wr exceeds MAX_C")
        for t in (zc, zr, angular, transport, rho):
            _fcheck(t.dtype == h.dtype, "every floating tensor must share h's dtype")
            _fcheck(t.device == h.device, "every tensor must be on h's device")
        _fcheck(desc.device == h.device and source.device == h.device, "desc and source must be on h's device")
        if h.device.type != "cuda":
            raise RuntimeError("libgmhip runs on the GPU only: the tensors are on the CPU (this build has no CPU driver)")

    @staticmethod
    def _groups(order: Tensor, group_ptr: Tensor, group_source: Tensor, n_edges: int) -> None:
        _fcheck(order.dtype == torch.int64 and order.dim() == 1 and order.shape[0] == n_edges and order.is_contiguous(),
                "order must be a contiguous int64 (n_edges,) tensor")
        _fcheck(group_source.dtype == torch.int64 and group_source.dim() == 1 and group_source.is_contiguous(),
                "group_source must be a contiguous int64 (n_groups,) tensor")
        _fcheck(group_ptr.dtype == torch.int64 and group_ptr.dim() == 1 and group_ptr.is_contiguous()
                and group_ptr.shape[0] == group_source.shape[0] + 1,
                "group_ptr must be a contiguous int64 (n_groups + 1,) tensor")
        for t in (order, group_ptr, group_source):
            _fcheck(t.device.type == "cuda", "order and the groups must be device tensors")

    def forward(self, h: Tensor, zc: Tensor, zr: Tensor, angular: Tensor, transport: Tensor, rho: Tensor, desc: Tensor,
                source: Tensor, order: Tensor, group_ptr: Tensor, group_source: Tensor, d_out: int,
                max_bm: int) -> Tensor:
        """The rows ``(n_edges, d_out)``: every edge's message in the flat output layout."""
        self._check_common(h, zc, zr, angular, transport, rho, desc, source, d_out)
        out = torch.empty(h.shape[0], d_out, dtype=h.dtype, device=h.device)
        _fcheck(1 <= max_bm <= MAX_BM, "max_bm must be in [1, MAX_BM]")
        if h.shape[0] == 0:
            return out
        self._groups(order, group_ptr, group_source, h.shape[0])
        hd = host_desc32(desc)
        _call("gm_factored_forward" + _suffix(h.dtype), _ptr(h), _ptr(zc), _ptr(zr), _ptr(angular), _ptr(transport),
              _ptr(rho), hd.data_ptr(), _ptr(order), _ptr(group_ptr), _ptr(group_source), zc.shape[0], h.shape[0],
              group_source.shape[0], h.shape[1] + 1, zc.shape[2], zr.shape[2], angular.shape[1], hd.shape[0],
              int(d_out), int(max_bm), _ptr(out), _stream(h.device))
        return out

    def aggregate(self, rows: Tensor, weights: Tensor, row_ptr: Tensor) -> Tensor:
        """``(n_targets, d_out)``: each target's weighted sum of its rows."""
        _fcheck(rows.dim() == 2 and rows.is_contiguous() and 1 <= rows.shape[1] <= MAX_OUT,
                "rows must be a contiguous (n_edges, d_out <= MAX_OUT) tensor")
        _fcheck(weights.dim() == 1 and weights.is_contiguous() and weights.shape[0] == rows.shape[0]
                and weights.dtype == rows.dtype, "weights must be a contiguous (n_edges,) tensor in the rows' dtype")
        _fcheck(row_ptr.dim() == 1 and row_ptr.is_contiguous() and row_ptr.shape[0] >= 1 and row_ptr.dtype == torch.int64,
                "row_ptr must be a contiguous int64 (n_targets + 1,) tensor")
        _fcheck(weights.device == rows.device and row_ptr.device == rows.device,
                "every tensor must be on the rows' device")
        if rows.device.type != "cuda":
            raise RuntimeError("libgmhip runs on the GPU only: the tensors are on the CPU (this build has no CPU driver)")
        n_targets = row_ptr.shape[0] - 1
        out = torch.empty(n_targets, rows.shape[1], dtype=rows.dtype, device=rows.device)
        if n_targets == 0:
            return out
        _call("gm_factored_aggregate" + _suffix(rows.dtype), _ptr(rows), _ptr(weights), _ptr(row_ptr), n_targets,
              rows.shape[0], rows.shape[1], _ptr(out), _stream(rows.device))
        return out

    def _backward(self, g: Tensor, target: Tensor | None, weights: Tensor | None, rows: Tensor | None, h: Tensor,
                  zc: Tensor, zr: Tensor, angular: Tensor, transport: Tensor, rho: Tensor, desc: Tensor,
                  source: Tensor, order: Tensor, group_ptr: Tensor, group_source: Tensor) -> list[Tensor]:
        _fcheck(g.dim() == 2 and g.is_contiguous() and g.dtype == h.dtype and g.device == h.device,
                "g must be a contiguous (rows, d_out) tensor in h's dtype")
        self._check_common(h, zc, zr, angular, transport, rho, desc, source, g.shape[1])
        aggregated = target is not None
        if aggregated:
            _fcheck(target.dim() == 1 and target.shape[0] == h.shape[0] and target.dtype == torch.int64
                    and target.is_contiguous() and target.device == h.device,
                    "target must be a contiguous int64 (n_edges,) tensor")
            _fcheck(weights.dim() == 1 and weights.shape[0] == h.shape[0] and weights.is_contiguous()
                    and weights.dtype == h.dtype and weights.device == h.device,
                    "weights must be a contiguous (n_edges,) tensor in h's dtype")
            _fcheck(rows.dim() == 2 and rows.shape[0] == h.shape[0] and rows.shape[1] == g.shape[1]
                    and rows.is_contiguous() and rows.dtype == h.dtype and rows.device == h.device,
                    "rows must be a contiguous (n_edges, d_out) tensor in h's dtype")
        else:
            _fcheck(g.shape[0] == h.shape[0], "g must have one row per edge")
        dh = torch.empty_like(h)
        dzc = torch.zeros_like(zc)
        dzr = torch.zeros_like(zr)
        dweights = torch.empty_like(weights) if aggregated else None
        if h.shape[0] == 0:
            return [dh, dzc, dzr] + ([dweights] if aggregated else [])
        self._groups(order, group_ptr, group_source, h.shape[0])
        hd = host_desc32(desc)
        _call("gm_factored_backward" + _suffix(h.dtype), _ptr(g), _ptr(target) if aggregated else None,
              _ptr(weights) if aggregated else None, _ptr(rows) if aggregated else None, _ptr(h), _ptr(zc), _ptr(zr),
              _ptr(angular), _ptr(transport), _ptr(rho), hd.data_ptr(), _ptr(order), _ptr(group_ptr),
              _ptr(group_source), zc.shape[0], h.shape[0], group_source.shape[0], h.shape[1] + 1, zc.shape[2],
              zr.shape[2], angular.shape[1], hd.shape[0], g.shape[1], _ptr(dh), _ptr(dzc), _ptr(dzr),
              _ptr(dweights) if aggregated else None, _stream(h.device))
        return [dh, dzc, dzr] + ([dweights] if aggregated else [])

    def backward(self, g: Tensor, h: Tensor, zc: Tensor, zr: Tensor, angular: Tensor, transport: Tensor, rho: Tensor,
                 desc: Tensor, source: Tensor, order: Tensor, group_ptr: Tensor,
                 group_source: Tensor) -> list[Tensor]:
        """[dh, dzc, dzr] from the rows' gradient ``g (n_edges, d_out)``."""
        return self._backward(g, None, None, None, h, zc, zr, angular, transport, rho, desc, source, order, group_ptr,
                              group_source)

    def backward_aggregated(self, g: Tensor, target: Tensor, weights: Tensor, rows: Tensor, h: Tensor, zc: Tensor,
                            zr: Tensor, angular: Tensor, transport: Tensor, rho: Tensor, desc: Tensor,
                            source: Tensor, order: Tensor, group_ptr: Tensor, group_source: Tensor) -> list[Tensor]:
        """[dh, dzc, dzr, dweights] from the targets' gradient ``g (n_targets, d_out)``."""
        if h.shape[0] == 0:
            return [torch.empty_like(h), torch.zeros_like(zc), torch.zeros_like(zr), torch.empty_like(weights)]
        _fcheck(target.numel() == h.shape[0], "target must list every edge")
        return self._backward(g, target, weights, rows, h, zc, zr, angular, transport, rho, desc, source, order,
                              group_ptr, group_source)


@functools.cache
def factored() -> FactoredExtension:
    library()
    return FactoredExtension()


# ---------------------------------------------------------------- mix runs and the radial trunk


class MixRuns:
    """Host arrays describing up to four runs of packed mix columns: run r
    covers ``width[r]`` columns, column c of node j at mix t at
    ``z[r] + j * node_stride[r] + t * t_stride[r] + (c - c_r)`` (elements)."""

    def __init__(self, runs: list[tuple[Tensor, int, int, int]], grads: list[Tensor] | None = None):
        n = len(runs)
        _fcheck(1 <= n <= 4, "between 1 and 4 mix runs")
        self.keep = [t for t, *_ in runs] + (grads or [])
        self.z = (ctypes.c_void_p * n)(*[t.data_ptr() for t, *_ in runs])
        self.dz = (ctypes.c_void_p * n)(*[g.data_ptr() for g in grads]) if grads is not None else None
        self.node_stride = (ctypes.c_int64 * n)(*[r[1] for r in runs])
        self.t_stride = (ctypes.c_int64 * n)(*[r[2] for r in runs])
        self.width = (ctypes.c_int64 * n)(*[r[3] for r in runs])
        self.n = n


def factored_forward_seg(h: Tensor, runs: MixRuns, n_nodes: int, angular: Tensor, transport: Tensor, rho: Tensor,
                         desc: Tensor, order: Tensor, group_ptr: Tensor, group_source: Tensor, K: int, wc: int, wr: int,
                         d_out: int, max_bm: int) -> Tensor:
    """The rows ``(n_edges, d_out)`` with the mixes read from ``runs``."""
    out = torch.empty(h.shape[0], d_out, dtype=h.dtype, device=h.device)
    if h.shape[0] == 0:
        return out
    E = h.shape[0]
    _edge_stream(h, E, 16, "h")
    _index_vector(order, E, "order")
    _grouping(group_ptr, group_source, None)
    _edge_stream(rho, E, 1, "rho")
    hd = host_desc32(desc)
    _call("gm_factored_forward_seg" + _suffix(h.dtype), _ptr(h), ctypes.cast(runs.z, ctypes.c_void_p),
          ctypes.cast(runs.node_stride, ctypes.c_void_p), ctypes.cast(runs.t_stride, ctypes.c_void_p),
          ctypes.cast(runs.width, ctypes.c_void_p), runs.n, _ptr(angular), _ptr(transport), _ptr(rho), hd.data_ptr(),
          _ptr(order), _ptr(group_ptr), _ptr(group_source), n_nodes, h.shape[0], group_source.shape[0], K, wc, wr,
          angular.shape[1], hd.shape[0], d_out, max_bm, _ptr(out), _stream(h.device))
    return out


def factored_backward_seg(g: Tensor, target: Tensor, weights: Tensor, rows: Tensor, h: Tensor, runs: MixRuns,
                          n_nodes: int, angular: Tensor, transport: Tensor, rho: Tensor, desc: Tensor, order: Tensor,
                          group_ptr: Tensor, group_source: Tensor, K: int, wc: int, wr: int,
                          dh: Tensor) -> Tensor:
    """dh written into ``dh``, the mix gradients into the runs' gradient
    arrays (zeroed by the caller); returns dweights."""
    dweights = torch.empty_like(weights)
    if h.shape[0] == 0:
        return dweights
    E = h.shape[0]
    for t, width, name in ((h, 16, "h"), (dh, 16, "dh"), (rho, 1, "rho"), (weights, 1, "weights"),
                           (rows, g.shape[1], "rows")):
        _edge_stream(t, E, width, name)
    _index_vector(target, E, "target")
    _index_vector(order, E, "order")
    _grouping(group_ptr, group_source, None)
    _check(g.dim() == 2 and g.is_contiguous(), "g must be a contiguous (n_targets, d_out) tensor")
    hd = host_desc32(desc)
    _call("gm_factored_backward_seg" + _suffix(h.dtype), _ptr(g), _ptr(target), _ptr(weights), _ptr(rows), _ptr(h),
          ctypes.cast(runs.z, ctypes.c_void_p), ctypes.cast(runs.dz, ctypes.c_void_p),
          ctypes.cast(runs.node_stride, ctypes.c_void_p), ctypes.cast(runs.t_stride, ctypes.c_void_p),
          ctypes.cast(runs.width, ctypes.c_void_p), runs.n, _ptr(angular), _ptr(transport), _ptr(rho),
          hd.data_ptr(), _ptr(order), _ptr(group_ptr), _ptr(group_source), n_nodes, h.shape[0],
          group_source.shape[0], K, wc, wr, angular.shape[1], hd.shape[0], g.shape[1], _ptr(dh), _ptr(dweights),
          _stream(h.device))
    return dweights


def _trunk_checks(rho: Tensor, weight: Tensor, bias: Tensor | None, centers: Tensor) -> None:
    _check(rho.dtype == torch.float32 and rho.dim() == 1 and rho.is_contiguous(), "rho must be a contiguous float32 vector")
    _check(weight.dtype == torch.float32 and weight.dim() == 3 and weight.is_contiguous(),
           "weight must be a contiguous float32 (H, T, B) tensor")
    H, T, B = weight.shape
    _check(bias is None or (bias.dtype == torch.float32 and bias.is_contiguous() and tuple(bias.shape) == (H, T)),
           "bias must be a contiguous float32 (H, T) tensor")
    _check(centers.dtype == torch.float32 and centers.is_contiguous() and tuple(centers.shape) == (B,),
           "centers must be a contiguous float32 (B,) tensor")


def radial_trunk_forward(rho: Tensor, weight: Tensor, bias: Tensor | None, centers: Tensor, width: float,
                         dtype: torch.dtype | None = None) -> Tensor:
    """``h (H, E, T)``: every head's SiLU(W b(rho) + c) over the Gaussian basis
    of rho^2, in rho's dtype or ``dtype`` (bfloat16: float32 arithmetic, each
    feature rounded to nearest even as it is stored)."""
    _trunk_checks(rho, weight, bias, centers)
    H, T, B = weight.shape
    dtype = rho.dtype if dtype is None else dtype
    _check(dtype in (torch.float32, torch.bfloat16), "the trunk features are float32 or bfloat16")
    h = torch.empty(H, rho.shape[0], T, dtype=dtype, device=rho.device)
    if rho.shape[0] == 0:
        return h
    name = "gm_radial_trunk_forward_bf16" if dtype == torch.bfloat16 else "gm_radial_trunk_forward_f32"
    _call(name, _ptr(rho), _ptr(weight), _ptr(bias) if bias is not None else None,
          _ptr(centers), rho.shape[0], H, T, B, float(width), _ptr(h), _stream(rho.device))
    return h


def radial_trunk_backward(dh: Tensor, rho: Tensor, weight: Tensor, bias: Tensor | None, centers: Tensor,
                          width: float) -> tuple[Tensor, Tensor]:
    """(dweight (H, T, B), dbias (H, T)) summed over the edges in a fixed order;
    ``dh`` float32 or bfloat16."""
    _trunk_checks(rho, weight, bias, centers)
    H, T, B = weight.shape
    _check(dh.dtype in (torch.float32, torch.bfloat16) and dh.is_contiguous() and tuple(dh.shape) == (H, rho.shape[0], T),
           "dh must be contiguous float32 or bfloat16 (H, E, T)")
    P = T * B + T
    lib = library()
    blocks = int(lib.gm_radial_trunk_partials(rho.shape[0]))
    partial = torch.empty(max(blocks, 1) * H * P, dtype=torch.float32, device=rho.device)
    dparams = torch.empty(H, P, dtype=torch.float32, device=rho.device)
    name = "gm_radial_trunk_backward_bf16" if dh.dtype == torch.bfloat16 else "gm_radial_trunk_backward_f32"
    _call(name, _ptr(dh), _ptr(rho), _ptr(weight), _ptr(bias) if bias is not None else None,
          _ptr(centers), rho.shape[0], H, T, B, float(width), _ptr(partial), _ptr(dparams), _stream(rho.device))
    return dparams[:, : T * B].reshape(H, T, B), dparams[:, T * B:]


def _column_view(v: Tensor) -> tuple[int, int]:
    """(rows, leading dimension) of a 2-D float32 (or bfloat16) view whose rows
    are evenly strided and whose columns are contiguous (a column slice of flat rows)."""
    _check(v.dim() == 2 and v.dtype in (torch.float32, torch.bfloat16) and v.device.type == "cuda",
           "node vectors must be a 2-D float32 or bfloat16 tensor on the GPU")
    _check(v.stride(1) == 1 or v.shape[1] == 1, "node vectors must have contiguous columns")
    return v.shape[0], (v.stride(0) if v.shape[0] > 1 else v.shape[1])


def node_mix_forward(v: Tensor, m: Tensor) -> Tensor:
    """``v (N, w) @ m (w, C)`` on MFMA: every head's node mixes for one input
    frequency (``v`` may be a column slice of the flat node rows)."""
    N, ldv = _column_view(v)
    w, C = m.shape
    _check(v.shape[1] == w and m.is_contiguous() and m.dtype == torch.float32 and m.device == v.device,
           "the mixing matrix must be a contiguous float32 (w, C) on the node vectors' device")
    out = torch.empty(N, C, dtype=torch.float32, device=v.device)
    name = "gm_node_mix_forward_bf16" if v.dtype == torch.bfloat16 else "gm_node_mix_forward_f32"
    _call(name, _ptr(v), max(ldv, w), _ptr(m), N, w, C, _ptr(out), _stream(v.device))
    return out


def node_mix_backward_input(dmix: Tensor, m: Tensor, dv: Tensor) -> None:
    """``dv (N, w) = dmix (N, C) @ m^T`` written into ``dv`` (a column slice of a
    flat gradient is fine: its leading dimension is passed)."""
    N, lddv = _column_view(dv)
    w, C = m.shape
    _require_device(dmix, m)
    _check(dmix.shape == (N, C) and dv.shape[1] == w, "dmix must be (N, C) for m (w, C) and dv (N, w)")
    _call("gm_node_mix_backward_input_f32", _ptr(dmix), _ptr(m), N, w, C, _ptr(dv), max(lddv, w), _stream(dv.device))


def node_mix_backward_weight(v: Tensor, dmix: Tensor) -> Tensor:
    """``v^T (w, N) @ dmix (N, C)`` summed over row ranges in a fixed order."""
    N, ldv = _column_view(v)
    w = v.shape[1]
    _require_device(dmix)
    C = dmix.shape[1]
    _check(dmix.shape[0] == N, "dmix must have the node vectors' rows")
    _check(dmix.dtype in (torch.float32, torch.bfloat16) and dmix.is_contiguous(),
           "dmix must be contiguous float32 or bfloat16")
    lib = library()
    partial = torch.empty(max(int(lib.gm_node_mix_weight_partials(N, w, C)), 1), dtype=torch.float32,
                          device=dmix.device)
    dm = torch.empty(w, C, dtype=torch.float32, device=dmix.device)
    vs = "bf16" if v.dtype == torch.bfloat16 else "f32"
    name = f"gm_node_mix_backward_weight_{vs}" + ("_bf16" if dmix.dtype == torch.bfloat16 else "")
    _call(name, _ptr(v), max(ldv, w), _ptr(dmix), N, w, C, _ptr(partial), _ptr(dm), _stream(dmix.device))
    return dm


def _index_vector(t: Tensor, n: int | None, name: str, dtype: torch.dtype = torch.int64) -> None:
    """An index tensor the kernels read as contiguous entries of ``dtype`` (``n`` of them when given):
    a wider or shorter one would send them past its end."""
    if t.dtype != dtype or t.dim() != 1 or not t.is_contiguous() or (n is not None and t.shape[0] != n):
        raise ValueError(f"{name} must be a contiguous {str(dtype).replace('torch.', '')} vector"
                         + (f" of {n} entries" if n is not None else ""))


def _edge_stream(t: Tensor | None, n_edges: int, width: int, name: str) -> None:
    """A per-edge stream in the grouping's order: contiguous (n_edges, width) (or (n_edges,) for width 1)."""
    if t is None:
        return
    shape = (n_edges,) if width == 1 else (n_edges, width)
    if tuple(t.shape) != shape or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {shape} tensor")


def _grouping(group_ptr: Tensor, group_source: Tensor, group_order: Tensor | None) -> None:
    _index_vector(group_source, None, "group_source")
    _index_vector(group_ptr, group_source.shape[0] + 1, "group_ptr")
    _check_order(group_order, group_source)


def _check_order(group_order: Tensor | None, group_source: Tensor) -> None:
    if group_order is None:
        return
    if (group_order.dtype != torch.int64 or not group_order.is_contiguous()
            or group_order.shape != group_source.shape or group_order.device != group_source.device):
        raise ValueError("group_order must be a contiguous int64 permutation of the groups, on their device")


class FusedTrunk:
    """A head's radial trunk for the lane-owned grouped kernels to evaluate from
    ``rho_g`` themselves: ``w (16, nb)`` and ``b (16,)`` (or None) on the
    device, the basis centres (host floats) and width."""

    def __init__(self, w: Tensor, b: Tensor | None, centers: list[float], width: float):
        _check(w.dim() == 2 and w.shape[0] == 16 and 1 <= w.shape[1] <= 8 and w.is_contiguous()
               and w.dtype == torch.float32, "the fused trunk's weight must be a contiguous float32 (16, nb <= 8)")
        _check(b is None or (b.shape == (16,) and b.is_contiguous() and b.dtype == torch.float32),
               "the fused trunk's bias must be a contiguous float32 (16,)")
        _check(len(centers) == w.shape[1], "one basis centre per basis function")
        self.w, self.b, self.width = w, b, float(width)
        self.centers = (ctypes.c_float * 8)(*centers)
        self.nb = w.shape[1]

    def args(self) -> list:
        return [_ptr(self.w), _ptr(self.b), ctypes.addressof(self.centers), self.nb, self.width]


_NO_TRUNK = [None, None, None, 0, 0.0]


def factored_forward_grouped(h_g: Tensor | None, runs: MixRuns, n_nodes: int, phase_g: Tensor, rho_g: Tensor,
                             zw_g: Tensor | None, pa: int, pt: int, desc: Tensor, group_ptr: Tensor,
                             group_source: Tensor, group_order: Tensor | None, K: int, wc: int, wr: int,
                             d_out: int, out: Tensor | None = None, trunk: FusedTrunk | None = None) -> Tensor:
    """The rows in the grouping's order, every per-edge stream read in that order
    (into ``out`` (n_edges, d_out) when given).  With ``trunk`` the kernels
    evaluate h from ``rho_g`` and ``h_g`` may be None.  A bfloat16 ``h_g``
    gives bfloat16 rows (plans with compiled-in lane slots, :func:`lanes_fixed`;
    float32 arithmetic)."""
    n_edges = rho_g.shape[0]
    if h_g is None and trunk is None:
        raise ValueError("h_g is required without a fused trunk")
    b16 = h_g is not None and h_g.dtype == torch.bfloat16
    row_dtype = torch.bfloat16 if b16 else rho_g.dtype
    if out is None:
        out = torch.empty(n_edges, d_out, dtype=row_dtype, device=rho_g.device)
    elif out.shape != (n_edges, d_out) or not out.is_contiguous() or out.dtype != row_dtype:
        raise ValueError("out must be a contiguous (n_edges, d_out) tensor in h's dtype")
    if n_edges == 0:
        return out
    _grouping(group_ptr, group_source, group_order)
    _edge_stream(h_g, n_edges, 16, "h_g")
    _edge_stream(rho_g, n_edges, 1, "rho_g")
    hd = host_desc32(desc)
    if b16:
        _check(trunk is None, "bfloat16 trunk features are read, not evaluated in the kernels")
        _call("gm_factored_forward_grouped_bf16", _ptr(h_g), ctypes.cast(runs.z, ctypes.c_void_p),
              ctypes.cast(runs.node_stride, ctypes.c_void_p), ctypes.cast(runs.t_stride, ctypes.c_void_p),
              ctypes.cast(runs.width, ctypes.c_void_p), runs.n, _ptr(phase_g), _ptr(rho_g), _ptr(zw_g), hd.data_ptr(),
              _ptr(group_ptr), _ptr(group_source), _ptr(group_order), n_nodes, n_edges, group_source.shape[0], K, wc,
              wr, pa, pt, hd.shape[0], d_out, _ptr(out), _stream(rho_g.device))
        return out
    _call("gm_factored_forward_grouped_f32", _ptr(h_g), ctypes.cast(runs.z, ctypes.c_void_p),
          ctypes.cast(runs.node_stride, ctypes.c_void_p), ctypes.cast(runs.t_stride, ctypes.c_void_p),
          ctypes.cast(runs.width, ctypes.c_void_p), runs.n, _ptr(phase_g), _ptr(rho_g), _ptr(zw_g), hd.data_ptr(),
          _ptr(group_ptr), _ptr(group_source), _ptr(group_order), n_nodes, n_edges, group_source.shape[0], K, wc,
          wr, pa, pt, hd.shape[0], d_out, *(trunk.args() if trunk is not None else _NO_TRUNK), _ptr(out),
          _stream(rho_g.device))
    return out


def factored_backward_grouped(g: Tensor, target_g: Tensor, weights_g: Tensor, rows_g: Tensor, h_g: Tensor | None,
                              runs: MixRuns, n_nodes: int, phase_g: Tensor, rho_g: Tensor, zw_g: Tensor | None,
                              pa: int, pt: int, desc: Tensor, group_ptr: Tensor, group_source: Tensor,
                              group_order: Tensor | None, K: int, wc: int, wr: int, dh_g: Tensor,
                              dweights: Tensor | None = None, trunk: FusedTrunk | None = None,
                              accumulate: bool = False) -> Tensor:
    """dh (grouping order) into ``dh_g``, the mix gradients into the runs'
    gradient arrays; returns dweights in the grouping's order (into
    ``dweights`` when given).  ``g`` (n_targets, d_out) may be a view with
    rows further apart (one head of the heads' gradient), read in place.
    With ``trunk`` the kernels evaluate h from
    ``rho_g`` and ``h_g`` may be None.  ``accumulate``: dh and dweights are
    added to ``dh_g`` and ``dweights`` (which must then be given) instead of
    written.  With bfloat16 ``h_g`` the rows and ``dh_g`` are bfloat16 too
    (float32 arithmetic)."""
    if accumulate and dweights is None:
        raise ValueError("accumulate needs the dweights to add to")
    if h_g is None and trunk is None:
        raise ValueError("h_g is required without a fused trunk")
    if dweights is None:
        dweights = torch.empty_like(weights_g)
    elif dweights.shape != weights_g.shape or not dweights.is_contiguous() or dweights.dtype != weights_g.dtype:
        raise ValueError("dweights must be a contiguous tensor shaped like weights_g")
    n_edges = rho_g.shape[0]
    if n_edges == 0:
        return dweights
    _grouping(group_ptr, group_source, group_order)
    _index_vector(target_g, n_edges, "target_g")
    _edge_stream(weights_g, n_edges, 1, "weights_g")
    _edge_stream(rows_g, n_edges, g.shape[1], "rows_g")
    _edge_stream(h_g, n_edges, 16, "h_g")
    _edge_stream(dh_g, n_edges, 16, "dh_g")
    _edge_stream(rho_g, n_edges, 1, "rho_g")
    hd = host_desc32(desc)
    # g may be one head's columns of a wider gradient array, read in place (rows g_ld floats apart)
    g_ld = g.stride(0) if g.dim() == 2 and g.stride(1) == 1 else -1
    if g_ld != g.shape[1] and not (g_ld >= g.shape[1] and g_ld % 2 == 0 and g.data_ptr() % 8 == 0):
        g, g_ld = g.contiguous(), g.shape[1]
    if h_g is not None and h_g.dtype == torch.bfloat16:
        _check(trunk is None and rows_g.dtype == torch.bfloat16 and dh_g.dtype == torch.bfloat16,
               "bfloat16 trunk features go with bfloat16 rows and dh (no fused trunk)")
        _call("gm_factored_backward_grouped_ld_bf16", _ptr(g), g_ld, _ptr(target_g), _ptr(weights_g), _ptr(rows_g),
              _ptr(h_g), ctypes.cast(runs.z, ctypes.c_void_p), ctypes.cast(runs.dz, ctypes.c_void_p),
              ctypes.cast(runs.node_stride, ctypes.c_void_p), ctypes.cast(runs.t_stride, ctypes.c_void_p),
              ctypes.cast(runs.width, ctypes.c_void_p), runs.n, _ptr(phase_g), _ptr(rho_g), _ptr(zw_g), hd.data_ptr(),
              _ptr(group_ptr), _ptr(group_source), _ptr(group_order), n_nodes, n_edges, group_source.shape[0], K,
              wc, wr, pa, pt, hd.shape[0], g.shape[1], int(accumulate), _ptr(dh_g), _ptr(dweights),
              _stream(rho_g.device))
        return dweights
    _call("gm_factored_backward_grouped_ld_f32", _ptr(g), g_ld, _ptr(target_g), _ptr(weights_g), _ptr(rows_g), _ptr(h_g),
          ctypes.cast(runs.z, ctypes.c_void_p), ctypes.cast(runs.dz, ctypes.c_void_p),
          ctypes.cast(runs.node_stride, ctypes.c_void_p), ctypes.cast(runs.t_stride, ctypes.c_void_p),
          ctypes.cast(runs.width, ctypes.c_void_p), runs.n, _ptr(phase_g), _ptr(rho_g), _ptr(zw_g), hd.data_ptr(),
          _ptr(group_ptr), _ptr(group_source), _ptr(group_order), n_nodes, n_edges, group_source.shape[0], K,
          wc, wr, pa, pt, hd.shape[0], g.shape[1], *(trunk.args() if trunk is not None else _NO_TRUNK),
          int(accumulate), _ptr(dh_g), _ptr(dweights), _stream(rho_g.device))
    return dweights


def lane_tables(desc: Tensor, wc: int, wr: int, d_out: int, pa: int, pt: int) -> tuple[int, list[int], list[int]]:
    """The grouped kernels' lane-owned slot tables for a plan: (slot count,
    per-slot words, slot column -> packed column with 255 for padding); a
    count of 0 means the plan takes the generic grouped kernels."""
    hd = host_desc32(desc)
    n = ctypes.c_int32(0)
    slot = (ctypes.c_uint32 * 16)()
    slotcol = (ctypes.c_uint8 * 128)()
    _call("gm_factored_lane_tables", hd.data_ptr(), hd.shape[0], wc, wr, d_out, pa, pt, ctypes.byref(n), slot, slotcol)
    return n.value, list(slot), list(slotcol)


def lanes_fixed(desc: Tensor, wc: int, wr: int, d_out: int, pa: int, pt: int) -> bool:
    """Whether a plan's lane slots are one of the compiled-in tables (the
    kernels that also take bfloat16 streams)."""
    hd = host_desc32(desc)
    fixed = ctypes.c_int32(0)
    _call("gm_factored_lanes_fixed", hd.data_ptr(), hd.shape[0], wc, wr, d_out, pa, pt, ctypes.byref(fixed))
    return bool(fixed.value)


def aggregate_heads(rows: Tensor, inv: Tensor, alpha: Tensor, row_ptr: Tensor, split: int = 1) -> Tensor:
    """``out[i, h] = sum_e alpha[e, h // split] rows[h, inv[e]]`` over each
    target's edges: rows ``(H, E, d_out)`` (float32, or bfloat16 widened as
    read), alpha ``(E, H / split)``; ``(N, H, d_out)`` float32 out."""
    H, E, d_out = rows.shape
    n_targets = row_ptr.shape[0] - 1
    out = torch.empty(n_targets, H, d_out, dtype=torch.float32, device=rows.device)
    if split < 1 or H % split or rows.dtype not in (torch.float32, torch.bfloat16) or alpha.dtype != torch.float32 \
            or alpha.shape != (E, H // split):
        raise ValueError("rows (H, E, d_out; float32 or bfloat16) and alpha (E, H / split; float32), split dividing H")
    if not (rows.is_contiguous() and alpha.is_contiguous() and inv.is_contiguous() and row_ptr.is_contiguous()):
        raise ValueError("rows, alpha, inv and row_ptr must be contiguous")
    if inv.dtype != torch.int64 or row_ptr.dtype != torch.int64 or inv.shape != (E,):
        raise ValueError("inv must be int64 (E,) and row_ptr int64")
    if n_targets == 0:
        return out
    name = "gm_factored_aggregate_heads_bf16" if rows.dtype == torch.bfloat16 else "gm_factored_aggregate_heads_f32"
    _call(name, _ptr(rows), _ptr(inv), _ptr(alpha), _ptr(row_ptr), n_targets, E, H,
          d_out, split, _ptr(out), _stream(rows.device))
    return out


def gather_transpose(src: Tensor, perm: Tensor) -> Tensor:
    """``dst_t[h, g] = src[perm[g], h]``: ``(n, width)`` in, ``(width, n)`` out."""
    n, width = src.shape
    if src.dtype != torch.float32 or not src.is_contiguous() or perm.shape != (n,) or not perm.is_contiguous():
        raise ValueError("src must be a contiguous float32 (n, width) tensor and perm a contiguous (n,) index")
    _index_vector(perm, n, "perm")
    out = torch.empty(width, n, dtype=src.dtype, device=src.device)
    _call("gm_gather_transpose_f32", _ptr(src), _ptr(perm), n, width, _ptr(out), _stream(src.device))
    return out


def scatter_transpose(src_t: Tensor, perm: Tensor) -> Tensor:
    """``dst[perm[g], h] = src_t[h, g]``: ``(width, n)`` in, ``(n, width)`` out."""
    width, n = src_t.shape
    if src_t.dtype != torch.float32 or not src_t.is_contiguous() or perm.shape != (n,) or not perm.is_contiguous():
        raise ValueError("src_t must be a contiguous float32 (width, n) tensor and perm a contiguous (n,) index")
    _index_vector(perm, n, "perm")
    out = torch.empty(n, width, dtype=src_t.dtype, device=src_t.device)
    _call("gm_scatter_transpose_f32", _ptr(src_t), _ptr(perm), n, width, _ptr(out), _stream(src_t.device))
    return out


def aggregate_gather(rows_g: Tensor, inv: Tensor, weights: Tensor, row_ptr: Tensor) -> Tensor:
    """``out_i = sum_e weights[e] rows_g[inv[e]]`` over each target's edges."""
    n_targets = row_ptr.shape[0] - 1
    out = torch.empty(n_targets, rows_g.shape[1], dtype=rows_g.dtype, device=rows_g.device)
    if n_targets == 0:
        return out
    _index_vector(row_ptr, n_targets + 1, "row_ptr")
    _index_vector(inv, None, "inv")
    _edge_stream(weights, inv.shape[0], 1, "weights")
    _call("gm_factored_aggregate_gather_f32", _ptr(rows_g), _ptr(inv), _ptr(weights), _ptr(row_ptr), n_targets,
          rows_g.shape[0], rows_g.shape[1], _ptr(out), _stream(rows_g.device))
    return out


# ---------------------------------------------------------------- pair terms of the general kernel

PAIRS_MATRIX_COMPLEX, PAIRS_U_REAL, PAIRS_CONJ_U, PAIRS_OUT_REAL = 1, 2, 4, 8
PAIRS_MAX_MULT, PAIRS_MAX_TRUNK = 16, 16


def _pcheck(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError("gm_pairs: " + message)


def _real_view(t: Tensor) -> Tensor:
    return torch.view_as_real(t) if t.is_complex() else t


class PairsExtension:
    """``gm_pairs``' entry points (reference nn/fused/pairs_cpu.cpp:88-148):
    one pair term per call, accumulating into caller-allocated outputs.  An
    empty tensor stands for an absent ``bias``, ``pre``, ``post`` or ``scale``."""

    with_cuda = True

    @staticmethod
    def _check(hidden: Tensor, weight: Tensor, u: Tensor, out: Tensor, a: int, b: int, flags: int) -> int:
        trunk = hidden.shape[1]
        _pcheck(1 <= a <= PAIRS_MAX_MULT and 1 <= b <= PAIRS_MAX_MULT, "block dimensions must be in 1..16")
        _pcheck(1 <= trunk <= PAIRS_MAX_TRUNK, "trunk width must be in 1..16")
        _pcheck(hidden.is_contiguous() and weight.is_contiguous() and u.is_contiguous() and out.is_contiguous(),
                "hidden, weight, u and out must be contiguous")
        width = (2 if flags & PAIRS_MATRIX_COMPLEX else 1) * a * b
        _pcheck(weight.dim() == 2 and weight.shape[0] == width and weight.shape[1] == trunk,
                "weight must be (width, trunk)")
        _pcheck(u.dim() == 2 and out.dim() == 2 and u.shape[1] == a and out.shape[1] == b,
                "u must be (n_edges, a) and out (n_edges, b)")
        _pcheck(u.shape[0] == hidden.shape[0] and out.shape[0] == hidden.shape[0], "n_edges mismatch")
        _pcheck(bool(flags & PAIRS_U_REAL) == (not u.is_complex()), "u must be real iff U_REAL")
        _pcheck(bool(flags & PAIRS_OUT_REAL) == (not out.is_complex()), "out must be real iff OUT_REAL")
        _pcheck(_real_view(u).dtype == hidden.dtype and weight.dtype == hidden.dtype
                and _real_view(out).dtype == hidden.dtype, "every tensor must share the hidden dtype")
        if hidden.device.type != "cuda":
            raise RuntimeError("libgmhip runs on the GPU only: the tensors are on the CPU (this build has no CPU driver)")
        return trunk

    @staticmethod
    def _optional(t: Tensor, n: int, complex_: bool, dtype: torch.dtype, what: str) -> int | None:
        if t is None or t.numel() == 0:
            return None
        _pcheck(t.is_contiguous() and t.shape[0] == n and t.is_complex() == complex_
                and _real_view(t).dtype == dtype, f"{what} must be a contiguous (n_edges,) tensor")
        return t.data_ptr()

    def forward(self, hidden: Tensor, weight: Tensor, bias: Tensor, u: Tensor, pre: Tensor, post: Tensor,
                scale: Tensor, out: Tensor, a: int, b: int, flags: int) -> None:
        trunk = self._check(hidden, weight, u, out, a, b, flags)
        n = hidden.shape[0]
        if n == 0:
            return
        _call("gm_pairs_forward" + _suffix(hidden.dtype), hidden.data_ptr(), weight.data_ptr(),
              self._optional(bias, weight.shape[0], False, hidden.dtype, "bias"), u.data_ptr(),
              self._optional(pre, n, True, hidden.dtype, "pre"), self._optional(post, n, True, hidden.dtype, "post"),
              self._optional(scale, n, False, hidden.dtype, "scale"), out.data_ptr(), n, int(a), int(b), trunk,
              int(flags), _stream(hidden.device))

    def backward(self, hidden: Tensor, weight: Tensor, bias: Tensor, u: Tensor, pre: Tensor, post: Tensor,
                 scale: Tensor, grad_out: Tensor, grad_u: Tensor, grad_hidden: Tensor, grad_k: Tensor, a: int, b: int,
                 flags: int) -> None:
        trunk = self._check(hidden, weight, u, grad_out, a, b, flags)
        n = hidden.shape[0]
        _pcheck(grad_u.is_contiguous() and grad_hidden.is_contiguous(), "grad_u and grad_hidden must be contiguous")
        _pcheck(grad_u.shape == u.shape and grad_u.dtype == u.dtype and grad_hidden.shape == hidden.shape
                and grad_hidden.dtype == hidden.dtype, "grad_u and grad_hidden must match u and hidden")
        _pcheck(grad_k.dim() == 2 and grad_k.shape[1] == n and grad_k.shape[0] == weight.shape[0]
                and grad_k.stride(1) == 1 and grad_k.stride(0) >= n and grad_k.dtype == hidden.dtype,
                "grad_k must be (width, n_edges) with unit column stride")
        if n == 0:
            return
        _call("gm_pairs_backward" + _suffix(hidden.dtype), hidden.data_ptr(), weight.data_ptr(),
              self._optional(bias, weight.shape[0], False, hidden.dtype, "bias"), u.data_ptr(),
              self._optional(pre, n, True, hidden.dtype, "pre"), self._optional(post, n, True, hidden.dtype, "post"),
              self._optional(scale, n, False, hidden.dtype, "scale"), grad_out.data_ptr(), grad_u.data_ptr(),
              grad_hidden.data_ptr(), grad_k.data_ptr(), grad_k.stride(0), n, int(a), int(b), trunk, int(flags),
              _stream(hidden.device))


@functools.cache
def pairs() -> PairsExtension:
    library()  # raises when the library is absent
    return PairsExtension()


# ---------------------------------------------------------------- depthwise conv, radial heads in the walk

RADIAL_TILES_SCALAR, RADIAL_TILES_COMPLEX = 2, 16


def _conv_radial_checks(v: Tensor, rf: Tensor, rbias: Tensor, rb: Tensor | None, w1: Tensor, b1: Tensor | None,
                        centers: list[float], transport: Tensor, angular: Tensor, rho: Tensor, weights: Tensor,
                        row_ptr: Tensor, source: Tensor, tiles: Tensor) -> None:
    """The walk's arguments as the kernels read them: the readout's operand tables
    of the compiled tile count, the per-edge streams of the CSR's edges, the host tile table."""
    _check(v.dim() == 2 and v.is_contiguous(), "v must be a contiguous (N, D) tensor")
    row = int(library().gm_conv_radial_partial_row())
    nt = (row - 16 * 8 - 16) // (256 + 16)  # coefficient tiles: the partial row holds dR, its bias column, W1, b1
    for t, numel, name in ((rf, nt * 256, "rf"), (rbias, nt * 16, "rbias"), (rb, nt * 256, "rb")):
        if t is not None:
            _check(t.dtype == torch.float32 and t.is_contiguous() and t.numel() == numel,
                   f"{name} must be a contiguous float32 table of {numel} entries")
    nb = len(centers)
    _check(w1.dtype == torch.float32 and w1.is_contiguous() and tuple(w1.shape) == (16, nb),
           f"w1 must be a contiguous float32 (16, {nb}) tensor")
    _check(b1 is None or (b1.dtype == torch.float32 and b1.is_contiguous() and tuple(b1.shape) == (16,)),
           "b1 must be a contiguous float32 (16,) tensor")
    n, E = v.shape[0], source.shape[0]
    _index_vector(row_ptr, n + 1, "row_ptr")
    _index_vector(source, E, "source")
    for t, name in ((rho, "rho"), (weights, "weights")):
        _check(t.dtype == torch.float32 and t.is_contiguous() and tuple(t.shape) == (E,),
               f"{name} must be a contiguous float32 ({E},) tensor")
    for t, name in ((transport, "transport"), (angular, "angular")):
        _check(t.dtype == torch.float32 and t.is_contiguous() and t.dim() == 3 and t.shape[0] == E
               and t.shape[2] == 2 and tuple(t.shape) == tuple(transport.shape),
               f"{name} must be a contiguous float32 (E, orders, 2) tensor shaped like transport")
    _check(tiles.device.type == "cpu" and tiles.dtype == torch.int32 and tiles.is_contiguous() and tiles.dim() == 2
           and tiles.shape[0] == 2, "tiles must be a contiguous host int32 (2, nc) table")


def conv_radial_forward(v: Tensor, rf: Tensor, rbias: Tensor, w1: Tensor, b1: Tensor | None, centers: list[float], width: float,
                        transport: Tensor, angular: Tensor, rho: Tensor, weights: Tensor, row_ptr: Tensor,
                        source: Tensor, a0: int, ns: int, tiles: Tensor) -> Tensor:
    """``out (N, D)``: the depthwise walk with the radial heads evaluated per
    edge from ``rho`` (``gm_conv_radial_forward_f32``).  ``rf`` is the packed
    readout in the kernel's A-operand layout, ``tiles`` a host int32 (2, nc)
    table of the complex tiles' frequencies and first columns."""
    _require_device(v, rf, rbias, w1, transport, angular, rho, weights, row_ptr, source)
    _check(v.dtype == torch.float32 and v.data_ptr() % 16 == 0, "v must be 16-byte aligned float32")
    _conv_radial_checks(v, rf, rbias, None, w1, b1, centers, transport, angular, rho, weights, row_ptr, source, tiles)
    out = torch.empty_like(v)
    if v.shape[0] == 0:
        return out
    cen = (ctypes.c_float * 8)(*centers)
    _call("gm_conv_radial_forward_f32", _ptr(v), _ptr(rf), _ptr(rbias), _ptr(w1), _ptr(b1), ctypes.addressof(cen), len(centers),
          float(width), _ptr(transport), _ptr(angular), _ptr(rho), _ptr(weights), _ptr(row_ptr), _ptr(source),
          v.shape[0], source.shape[0], v.shape[1], transport.shape[1], int(a0), int(ns), tiles.shape[1],
          tiles[0].data_ptr(), tiles[1].data_ptr(), _ptr(out), _stream(v.device))
    return out


def conv_radial_backward(g: Tensor, v: Tensor, rf: Tensor, rbias: Tensor, rb: Tensor, w1: Tensor, b1: Tensor | None,
                         centers: list[float], width: float, transport: Tensor, angular: Tensor, rho: Tensor,
                         weights: Tensor, source: Tensor, row_ptr: Tensor, a0: int, ns: int,
                         tiles: Tensor) -> tuple[Tensor, Tensor]:
    """``(dv, grad)``: the input gradient and the parameter-gradient row
    (``gm_conv_radial_partial_row()`` floats: dR in lane layout, its bias
    column, W1, b1), summed over per-wave partial rows in a fixed order."""
    _require_device(g, v, rf, rbias, rb, w1, transport, angular, rho, weights, row_ptr, source)
    _check(g.shape == v.shape and g.dtype == v.dtype and g.data_ptr() % 16 == 0 and v.data_ptr() % 16 == 0,
           "g must be shaped and typed as v, both 16-byte aligned")
    _check(g.is_contiguous(), "g must be contiguous")
    _conv_radial_checks(v, rf, rbias, rb, w1, b1, centers, transport, angular, rho, weights, row_ptr, source, tiles)
    src_ptr, src_order, target = source_major(source, row_ptr)
    n = v.shape[0]
    dv = torch.empty_like(v)
    row = int(library().gm_conv_radial_partial_row())
    # one resident round (two 4-wave workgroups per CU at the kernels' register use), a
    # multiple of 8: one share of the sources per XCD
    n_blocks = max(8, min(512, (n + 3) // 4 // 8 * 8))
    rows = int(library().gm_conv_radial_workspace_rows(n_blocks))  # partial rows of every tile group + slices
    partial = torch.empty(rows, row, dtype=torch.float32, device=v.device)
    grad = torch.empty(row, dtype=torch.float32, device=v.device)
    cen = (ctypes.c_float * 8)(*centers)
    _call("gm_conv_radial_backward_f32", _ptr(g), _ptr(v), _ptr(rf), _ptr(rbias), _ptr(rb), _ptr(w1), _ptr(b1),
          ctypes.addressof(cen), len(centers), float(width), _ptr(transport), _ptr(angular), _ptr(rho),
          _ptr(weights), _ptr(src_ptr), _ptr(src_order), _ptr(target), n, source.shape[0], v.shape[1],
          transport.shape[1], int(a0), int(ns), tiles.shape[1], tiles[0].data_ptr(), tiles[1].data_ptr(), n_blocks,
          _ptr(partial), _ptr(dv), _ptr(grad), _stream(v.device))
    return dv, grad


# ---------------------------------------------------------------- neighbourhoods and edge geometry


def _geo_nodes(x: Tensor, name: str) -> None:
    _require_device(x)
    _check(x.dtype == torch.float64 and x.dim() == 2 and x.shape[1] == 3 and x.shape[0] > 0,
           f"{name} must be a non-empty (n, 3) float64 tensor")


def radius_edges(targets: Tensor, sources: Tensor, limit: float) -> tuple[Tensor, Tensor]:
    """``(edge_index (2, E), row_ptr (n_targets + 1))``: every pair with
    ``atan2(|p x q|, clamp(<p, q>)) <= limit``, target-major, source-minor."""
    _geo_nodes(targets, "targets")
    _geo_nodes(sources, "sources")
    _check(targets.device == sources.device, "targets and sources must live on the same device")
    nt, ns = targets.shape[0], sources.shape[0]
    device = targets.device
    for x, name in ((targets, "targets"), (sources, "sources")):
        drift = float(((x * x).sum(dim=1) - 1.0).abs().max())
        _check(drift <= 1e-14, f"{name} must be unit vectors to 1e-14 (|p|^2 - 1 reaches {drift:.3g})")
    workspace = torch.empty(int(library().gm_radius_workspace_doubles(nt, ns)), dtype=torch.float64, device=device)
    row_ptr = torch.empty(nt + 1, dtype=torch.int64, device=device)
    stream = _stream(device)
    _call("gm_radius_row_ptr_f64", _ptr(targets), nt, _ptr(sources), ns, float(limit), _ptr(workspace),
          _ptr(row_ptr), stream)
    n_edges = int(row_ptr[-1])  # sizes the edge list (one host sync)
    edge_index = torch.empty(2, n_edges, dtype=torch.int64, device=device)
    _call("gm_radius_edges_f64", _ptr(targets), nt, _ptr(sources), ns, float(limit), _ptr(workspace), _ptr(row_ptr),
          n_edges, _ptr(edge_index), stream)
    return edge_index, row_ptr


def geodesic_distances(targets: Tensor, sources: Tensor, edge_index: Tensor) -> Tensor:
    """``atan2(|p x q|, clamp(<p, q>))`` per edge in float64 (the membership rule's distance)."""
    _geo_nodes(targets, "targets")
    _geo_nodes(sources, "sources")
    _require_device(targets, sources, edge_index)
    _check(edge_index.dtype == torch.int64 and edge_index.dim() == 2 and edge_index.shape[0] == 2,
           "edge_index must be a (2, E) int64 tensor")
    out = torch.empty(edge_index.shape[1], dtype=torch.float64, device=targets.device)
    _call("gm_geodesic_distances_f64", _ptr(targets), _ptr(sources), _ptr(edge_index), edge_index.shape[1],
          targets.shape[0], sources.shape[0], _ptr(out), _stream(targets.device))
    return out


def edge_tables(targets: Tensor, target_frames: Tensor, sources: Tensor, source_frames: Tensor,
                source_quadrature: Tensor, edge_index: Tensor, max_frequency: int) -> dict[str, Tensor]:
    """Per-edge geometry in float64: ``log_coordinates (E, 2)``, ``distances``,
    ``polar_angles``, ``transport_angles``, ``tangent_quadrature_weights`` (E)
    and the phase tables ``(E, K + 1, 2)`` (real, imaginary)."""
    _geo_nodes(targets, "targets")
    _geo_nodes(sources, "sources")
    _require_device(targets, target_frames, sources, source_frames, source_quadrature, edge_index)
    nt, ns = targets.shape[0], sources.shape[0]
    _check(target_frames.dtype == torch.float64 and tuple(target_frames.shape) == (nt, 3, 2),
           "target_frames must be (n_targets, 3, 2) float64")
    _check(source_frames.dtype == torch.float64 and tuple(source_frames.shape) == (ns, 3, 2),
           "source_frames must be (n_sources, 3, 2) float64")
    _check(source_quadrature.dtype == torch.float64 and tuple(source_quadrature.shape) == (ns,),
           "source_quadrature must be (n_sources,) float64")
    _check(edge_index.dtype == torch.int64 and edge_index.dim() == 2 and edge_index.shape[0] == 2,
           "edge_index must be a (2, E) int64 tensor")
    E, K = edge_index.shape[1], int(max_frequency)
    kw = dict(dtype=torch.float64, device=targets.device)
    out = dict(log_coordinates=torch.empty(E, 2, **kw), distances=torch.empty(E, **kw),
               polar_angles=torch.empty(E, **kw), transport_angles=torch.empty(E, **kw),
               tangent_quadrature_weights=torch.empty(E, **kw), angular_phases=torch.empty(E, K + 1, 2, **kw),
               transport_phases=torch.empty(E, K + 1, 2, **kw))
    _call("gm_edge_tables_f64", _ptr(targets), _ptr(target_frames), _ptr(sources), _ptr(source_frames),
          _ptr(source_quadrature), _ptr(edge_index), E, nt, ns, K, *(_ptr(t) for t in out.values()),
          _stream(targets.device))
    return out


# ---------------------------------------------------------------- transformer block pointwise operators


_PW_SUFFIX = {torch.float32: "f32", torch.float64: "f64", torch.bfloat16: "bf16"}


class PointwiseLayout:
    """A field type's flat layout as the pointwise entry points take it (host arrays)."""

    def __init__(self, field_type: Any):
        self.D = field_type.dimension
        self.a0 = field_type.multiplicity(0) if 0 in field_type else 0
        nonzero = [(n, field_type.multiplicity(n)) for n in field_type.frequencies if n != 0]
        slices = field_type.slices()
        self.nf = len(nonzero)
        self.offsets = (ctypes.c_int64 * max(1, self.nf))(*[slices[n].start for n, _ in nonzero])
        self.mults = (ctypes.c_int64 * max(1, self.nf))(*[m for _, m in nonzero])
        self.G = sum(m for _, m in nonzero)

    def args(self) -> tuple:
        return (self.D, self.a0, self.nf, ctypes.cast(self.offsets, _P), ctypes.cast(self.mults, _P))


def _pointers(ts: list[Tensor]) -> Any:
    """A host array of the tensors' device pointers (kept alive by the caller's reference)."""
    return (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])


def _ffn_check_weights(A: int, B: int, w1t: list[Tensor], wg: Tensor, w2t: list[Tensor]) -> None:
    for f, (a, b) in enumerate(((A, B), (2 * A, 2 * B), (2 * A, 2 * B))):
        _check(w1t[f].dtype == torch.bfloat16 and w1t[f].shape == (b, a) and w1t[f].is_contiguous(),
               f"w1t[{f}] must be a contiguous ({b}, {a}) bfloat16 block")
        _check(w2t[f].dtype == torch.bfloat16 and w2t[f].shape == (a, b) and w2t[f].is_contiguous(),
               f"w2t[{f}] must be a contiguous ({a}, {b}) bfloat16 block")
    _check(wg.dtype == torch.bfloat16 and wg.shape == (2 * B, B) and wg.is_contiguous(),
           f"wg must be a contiguous ({2 * B}, {B}) bfloat16 matrix")


def _ffn_check_params(x: Tensor, A: int, B: int, gamma: Tensor, beta: Tensor | None, b1: Tensor | None,
                      bg: Tensor | None, b2: Tensor | None) -> None:
    _require_device(x, gamma)
    _check(x.dtype == torch.bfloat16 and x.dim() == 2 and x.shape[1] == 5 * A and x.is_contiguous(),
           f"x must be contiguous (N, {5 * A}) bfloat16 rows")
    for name, t, n in (("gamma", gamma, 5 * A), ("beta", beta, A), ("b1", b1, B), ("bg", bg, 2 * B), ("b2", b2, A)):
        _check(t is None or (t.dtype == torch.float32 and t.shape == (n,) and t.is_contiguous()),
               f"{name} must be a contiguous ({n},) float32 vector")


def ffn_forward(x: Tensor, A: int, B: int, eps: float, double_sigmoid: bool, gamma: Tensor, beta: Tensor | None,
                w1t: list[Tensor], b1: Tensor | None, wg: Tensor, bg: Tensor | None, w2t: list[Tensor],
                b2: Tensor | None) -> tuple[Tensor, Tensor, Tensor]:
    """``(x + y, mean, inv_d)``: the block's fused feed-forward on bfloat16 rows (``gm_ffn_forward_bf16``)."""
    _ffn_check_params(x, A, B, gamma, beta, b1, bg, b2)
    _ffn_check_weights(A, B, w1t, wg, w2t)
    n = x.shape[0]
    out = torch.empty_like(x)
    mean = torch.empty(n, dtype=torch.float32, device=x.device)
    inv_d = torch.empty(n, dtype=torch.float32, device=x.device)
    p1, p2 = _pointers(w1t), _pointers(w2t)
    _call("gm_ffn_forward_bf16", _ptr(x), n, A, B, float(eps), int(double_sigmoid), _ptr(gamma), _ptr(beta),
          ctypes.cast(p1, _P), _ptr(b1), _ptr(wg), _ptr(bg), ctypes.cast(p2, _P), _ptr(b2), _ptr(out), _ptr(mean),
          _ptr(inv_d), _stream(x.device))
    return out, mean, inv_d


def ffn_backward(dz: Tensor, x: Tensor, A: int, B: int, eps: float, double_sigmoid: bool, gamma: Tensor,
                 beta: Tensor | None, w1t: list[Tensor], w1n: list[Tensor], b1: Tensor | None, wg: Tensor,
                 wgt: Tensor, bg: Tensor | None, w2t: list[Tensor], w2n: list[Tensor], mean: Tensor,
                 inv_d: Tensor) -> dict[str, Any]:
    """The fused feed-forward's backward (``gm_ffn_backward_bf16``): ``dx`` and the
    factors of the parameter gradients (``xhat``, ``hidden0``, ``outs``,
    ``dhidden``, ``dpre``), with ``dgb`` = (dgamma | dbeta) summed over the tiles."""
    _ffn_check_params(x, A, B, gamma, beta, b1, bg, None)
    _ffn_check_weights(A, B, w1t, wg, w2t)
    for f, (a, b) in enumerate(((A, B), (2 * A, 2 * B), (2 * A, 2 * B))):
        _check(w1n[f].dtype == torch.bfloat16 and w1n[f].shape == (a, b) and w1n[f].is_contiguous(),
               f"w1n[{f}] must be a contiguous ({a}, {b}) bfloat16 block")
        _check(w2n[f].dtype == torch.bfloat16 and w2n[f].shape == (b, a) and w2n[f].is_contiguous(),
               f"w2n[{f}] must be a contiguous ({b}, {a}) bfloat16 block")
    _check(wgt.dtype == torch.bfloat16 and wgt.shape == (B, 2 * B) and wgt.is_contiguous(),
           f"wgt must be a contiguous ({B}, {2 * B}) bfloat16 matrix")
    _require_device(dz, mean, inv_d)
    _check(dz.dtype == torch.bfloat16 and dz.shape == x.shape and dz.is_contiguous(), "dz must match x")
    n, dev = x.shape[0], x.device
    f32 = dict(dtype=torch.float32, device=dev)
    dx = torch.empty_like(x)
    xhat = torch.empty_like(x)
    bf = dict(dtype=torch.bfloat16, device=dev)
    hidden0 = torch.empty(n, B, **f32)
    outs = [torch.empty(n, w, **bf) for w in (B, 2 * B, 2 * B)]
    dhidden = [torch.empty(n, w, **bf) for w in (B, 2 * B, 2 * B)]
    dpre = torch.empty(n, 2 * B, **bf)
    partial = torch.empty(max(int(library().gm_ffn_partial_rows(n)), 1), 6 * A, **f32)
    arrays = [_pointers(w1t), _pointers(w1n), _pointers(w2t), _pointers(w2n), _pointers(outs), _pointers(dhidden)]
    p1t, p1n, p2t, p2n, po, pd = (ctypes.cast(a, _P) for a in arrays)
    _call("gm_ffn_backward_bf16", _ptr(dz), _ptr(x), n, A, B, float(eps), int(double_sigmoid), _ptr(gamma),
          _ptr(beta), p1t, p1n, _ptr(b1), _ptr(wg), _ptr(wgt), _ptr(bg), p2t, p2n, _ptr(mean), _ptr(inv_d),
          _ptr(dx), _ptr(xhat), _ptr(hidden0), po, pd, _ptr(dpre), _ptr(partial), _stream(dev))
    dgb = partial[: int(library().gm_ffn_partial_rows(n))].sum(0) if n > 0 else torch.zeros(6 * A, **f32)
    return dict(dx=dx, xhat=xhat, hidden0=hidden0, outs=outs, dhidden=dhidden, dpre=dpre, dgb=dgb)


def param_dtype(dtype: torch.dtype) -> torch.dtype:
    """The parameter (and statistics) dtype of the pointwise entry points for rows of ``dtype``."""
    return torch.float64 if dtype == torch.float64 else torch.float32


def _pw_check(x: Tensor, layout: PointwiseLayout) -> str:
    _require_device(x)
    _check(x.dtype in _PW_SUFFIX, f"the pointwise operators take float32, float64 or bfloat16 rows, got {x.dtype}")
    _check(x.dim() == 2 and x.shape[1] == layout.D and x.is_contiguous(), f"rows must be contiguous (n_nodes, {layout.D})")
    return _PW_SUFFIX[x.dtype]


def layer_norm_forward(x: Tensor, gamma: Tensor, beta: Tensor | None, layout: PointwiseLayout,
                       eps: float) -> tuple[Tensor, Tensor, Tensor]:
    """``(y, mean, inv_d)``: the merged equivariant layer normalization of the rows ``x``."""
    sfx = _pw_check(x, layout)
    pd = param_dtype(x.dtype)
    _require_device(x, gamma, *(() if beta is None else (beta,)))
    _check(gamma.dtype == pd and gamma.shape == (layout.D,) and gamma.is_contiguous(), f"gamma must be ({layout.D},) {pd}")
    _check(beta is None or (beta.dtype == pd and beta.shape == (layout.a0,) and beta.is_contiguous()),
           f"beta must be ({layout.a0},) {pd}")
    n = x.shape[0]
    y = torch.empty_like(x)
    mean = torch.empty(n, dtype=pd, device=x.device)
    inv_d = torch.empty(n, dtype=pd, device=x.device)
    _call(f"gm_layer_norm_forward_{sfx}", _ptr(x), _ptr(gamma), _ptr(beta), n, *layout.args(), float(eps), _ptr(y),
          _ptr(mean), _ptr(inv_d), _stream(x.device))
    return y, mean, inv_d


def layer_norm_backward(gy: Tensor, x: Tensor, gamma: Tensor, mean: Tensor, inv_d: Tensor,
                        layout: PointwiseLayout) -> tuple[Tensor, Tensor]:
    """``(dx, dparams)`` with ``dparams = (dgamma (D), dbeta (a0))`` summed over the nodes in a fixed order."""
    sfx = _pw_check(x, layout)
    _require_device(gy, x, gamma, mean, inv_d)
    _check(gy.dtype == x.dtype and gy.shape == x.shape and gy.is_contiguous(), "gy must match x (contiguous)")
    pd = param_dtype(x.dtype)
    n = x.shape[0]
    _check(gamma.dtype == pd and gamma.shape == (layout.D,) and gamma.is_contiguous(), f"gamma must be ({layout.D},) {pd}")
    for t, name in ((mean, "mean"), (inv_d, "inv_d")):
        _check(t.dtype == pd and t.shape == (n,) and t.is_contiguous(), f"{name} must be ({n},) {pd}")
    rows = int(library().gm_layer_norm_partial_rows(n))
    partial = torch.empty(rows, layout.D + layout.a0, dtype=pd, device=x.device)
    dparams = torch.empty(layout.D + layout.a0, dtype=pd, device=x.device)
    dx = torch.empty_like(x)
    _call(f"gm_layer_norm_backward_{sfx}", _ptr(gy), _ptr(x), _ptr(gamma), _ptr(mean), _ptr(inv_d), n, *layout.args(),
          _ptr(dx), _ptr(partial), _ptr(dparams), _stream(x.device))
    return dx, dparams


def gate_forward(h: Tensor, pre: Tensor, layout: PointwiseLayout, double_sigmoid: bool) -> Tensor:
    """SiLU on the scalar entries, every copy scaled by its gate ``act(pre)``."""
    sfx = _pw_check(h, layout)
    _require_device(h, pre)
    _check(pre.dtype == h.dtype and tuple(pre.shape) == (h.shape[0], layout.G) and pre.is_contiguous(),
           f"pre must be contiguous (n_nodes, {layout.G})")
    y = torch.empty_like(h)
    _call(f"gm_gate_forward_{sfx}", _ptr(h), _ptr(pre), h.shape[0], *layout.args(), int(double_sigmoid), _ptr(y),
          _stream(h.device))
    return y


def gate_backward(gy: Tensor, h: Tensor, pre: Tensor, layout: PointwiseLayout,
                  double_sigmoid: bool) -> tuple[Tensor, Tensor]:
    """``(dh, dpre)``: the gate's direct gradient and the pre-activations' gradient."""
    sfx = _pw_check(h, layout)
    _require_device(gy, h, pre)
    _check(gy.dtype == h.dtype and gy.shape == h.shape and gy.is_contiguous(), "gy must match h (contiguous)")
    _check(pre.dtype == h.dtype and tuple(pre.shape) == (h.shape[0], layout.G) and pre.is_contiguous(),
           f"pre must be contiguous (n_nodes, {layout.G})")
    dh = torch.empty_like(h)
    dpre = torch.empty_like(pre)
    _call(f"gm_gate_backward_{sfx}", _ptr(gy), _ptr(h), _ptr(pre), h.shape[0], *layout.args(), int(double_sigmoid),
          _ptr(dh), _ptr(dpre), _stream(h.device))
    return dh, dpre
