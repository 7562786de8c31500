"""ctypes binding of oracle/_ref/libgmref.so: the reference's own header-only
CPU arithmetic (nn/fused/attention.h, factored.h) behind oracle/ref_driver.cpp.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  ``available()`` is False
where the library was not built (it needs the reference checkout to build).
"""

from __future__ import annotations

import ctypes
import functools
from pathlib import Path

import torch
from torch import Tensor

LIB = Path(__file__).resolve().parent / "_ref" / "libgmref.so"


def available() -> bool:
    return LIB.exists()


@functools.cache
def lib() -> ctypes.CDLL:
    return ctypes.CDLL(str(LIB))


def _p(t: Tensor | None):
    return None if t is None or t.numel() == 0 else ctypes.c_void_p(t.data_ptr())


def _sfx(t: Tensor) -> str:
    return "f64" if t.dtype == torch.float64 else "f32"


def _i(*xs):
    return [ctypes.c_int64(int(x)) for x in xs]


def softmax_forward(q, k, transport, bias, inside, desc, row_ptr, source, H, scale, first=0, last=None) -> Tensor:
    N, D, E = q.shape[0], q.shape[1], source.shape[0]
    alpha = torch.zeros(E, H, dtype=q.dtype)
    last = N if last is None else last
    getattr(lib(), "ref_softmax_forward_" + _sfx(q))(
        _p(q), _p(k), _p(transport), _p(bias), _p(inside), _p(desc), _p(row_ptr), _p(source),
        *_i(N, E, D, transport.shape[1], desc.shape[0], H), ctypes.c_double(scale), _p(alpha), *_i(first, last))
    return alpha


def softmax_backward(dalpha, q, k, transport, desc, row_ptr, source, alpha, H, scale, first=0, last=None):
    N, D, E = q.shape[0], q.shape[1], source.shape[0]
    dq, dk = torch.zeros_like(q), torch.zeros_like(q)
    last = N if last is None else last
    getattr(lib(), "ref_softmax_backward_" + _sfx(q))(
        _p(dalpha), _p(q), _p(k), _p(transport), _p(desc), _p(row_ptr), _p(source), _p(alpha),
        *_i(N, E, D, transport.shape[1], desc.shape[0], H), ctypes.c_double(scale), _p(dq), _p(dk), *_i(first, last))
    return dq, dk


def conv_forward(v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, A0, W) -> Tensor:
    N, D, E = v.shape[0], v.shape[1], source.shape[0]
    out = torch.zeros_like(v)
    getattr(lib(), "ref_conv_forward_" + _sfx(v))(
        _p(v), _p(rc), _p(cc), _p(transport), _p(angular), _p(rho), _p(weights), _p(desc), _p(row_ptr), _p(source),
        *_i(N, E, D, transport.shape[1], desc.shape[0], A0, W), _p(out))
    return out


def conv_backward(g, v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, A0, W):
    N, D, E = v.shape[0], v.shape[1], source.shape[0]
    dv, drc, dcc = torch.zeros_like(v), torch.zeros_like(rc), torch.zeros_like(cc)
    getattr(lib(), "ref_conv_backward_" + _sfx(v))(
        _p(g), _p(v), _p(rc), _p(cc), _p(transport), _p(angular), _p(rho), _p(weights), _p(desc), _p(row_ptr),
        _p(source), *_i(N, E, D, transport.shape[1], desc.shape[0], A0, W), _p(dv), _p(drc), _p(dcc))
    return dv, drc, dcc


def factored_forward(h, zc, zr, angular, transport, rho, desc, source, d_out) -> Tensor:
    E = h.shape[0]
    out = torch.zeros(E, d_out, dtype=h.dtype)
    getattr(lib(), "ref_factored_forward_" + _sfx(h))(
        _p(h), _p(zc), _p(zr), _p(angular), _p(transport), _p(rho), _p(desc), _p(source),
        *_i(E, h.shape[1] + 1, zc.shape[2], zr.shape[2], angular.shape[1], desc.shape[0], d_out), _p(out))
    return out


def factored_aggregate(rows, weights, row_ptr) -> Tensor:
    N = row_ptr.shape[0] - 1
    out = torch.zeros(N, rows.shape[1], dtype=rows.dtype)
    getattr(lib(), "ref_factored_aggregate_" + _sfx(rows))(_p(rows), _p(weights), _p(row_ptr), *_i(N, rows.shape[1]),
                                                            _p(out))
    return out


def factored_backward(g, target, weights, rows, h, zc, zr, angular, transport, rho, desc, source):
    """The aggregated backward: (dh, dzc, dzr, dweights)."""
    E = h.shape[0]
    dh, dzc, dzr = torch.zeros_like(h), torch.zeros_like(zc), torch.zeros_like(zr)
    dweights = torch.zeros_like(weights)
    getattr(lib(), "ref_factored_backward_" + _sfx(h))(
        _p(g), _p(target), _p(weights), _p(rows), _p(h), _p(zc), _p(zr), _p(angular), _p(transport), _p(rho),
        _p(desc), _p(source), *_i(zc.shape[0], E, h.shape[1] + 1, zc.shape[2], zr.shape[2], angular.shape[1],
                                   desc.shape[0], rows.shape[1]), _p(dh), _p(dzc), _p(dzr), _p(dweights))
    return dh, dzc, dzr, dweights
