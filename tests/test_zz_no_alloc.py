"""The no-allocation entry point gm_node_mix_backward_weight_noalloc_f32
(partials in the library's own device array) against the workspace entry
point gm_node_mix_backward_weight_f32, both called through the C ABI: two
calls in a row on one GPU, the second smaller, each within fp32 summation
tolerance of the workspace form (the two sum the row splits in different
orders) and of a float64 product; two calls on two streams issued back to
back (ordered by the library's event, not by the caller); and a size beyond
the array rejected with a message before anything is launched."""

import ctypes

import pytest
import torch

from gm_attention_amd import _native

pytestmark = pytest.mark.gpu


def _workspace_form(lib, v, ldv, dmix, N, w, C, stream):
    partial = torch.empty(max(int(lib.gm_node_mix_weight_partials(N, w, C)), 1), device=v.device)
    dm = torch.empty(w, C, device=v.device)
    assert lib.gm_node_mix_backward_weight_f32(v.data_ptr(), ldv, dmix.data_ptr(), N, w, C, partial.data_ptr(),
                                               dm.data_ptr(), stream) == 0, lib.gm_last_error()
    return dm


def _noalloc_form(lib, v, ldv, dmix, N, w, C, stream):
    dm = torch.full((w, C), float("nan"), device=v.device)
    assert lib.gm_node_mix_backward_weight_noalloc_f32(v.data_ptr(), ldv, dmix.data_ptr(), N, w, C, dm.data_ptr(),
                                                       stream) == 0, lib.gm_last_error()
    return dm


@pytest.mark.parametrize("first,second", [((524288 // 8, 64, 5440), (777, 20, 100)),
                                          ((40000, 128, 2176), (129, 64, 68))])
def test_no_alloc_weight_gradient_matches_the_workspace_form_twice(first, second, cuda):
    lib = _native.library()
    stream = torch.cuda.current_stream(cuda).cuda_stream
    for N, w, C in (first, second):
        print(f"no-alloc dM N={N} w={w} C={C}", flush=True)
        g = torch.Generator().manual_seed(N + w + C)
        rows = torch.randn(N, w + 7, generator=g).to(cuda)
        dmix = torch.randn(N, C, generator=g).to(cuda)
        v = rows[:, 3:3 + w]
        want = _workspace_form(lib, v, w + 7, dmix, N, w, C, stream)
        got = _noalloc_form(lib, v, w + 7, dmix, N, w, C, stream)
        torch.cuda.synchronize()
        exact = (v.double().T @ dmix.double()).cpu()
        scale = float(exact.abs().max())
        assert not bool(torch.isnan(got).any())
        assert float((got.double().cpu() - want.double().cpu()).abs().max()) <= 2e-6 * scale
        assert float((got.double().cpu() - exact).abs().max()) <= 2e-6 * scale


def test_no_alloc_calls_on_two_streams_do_not_race(cuda):
    """Two calls on two streams, issued with no synchronisation between them:
    the second stream waits for the first call's kernels before it writes the
    shared partials, so both results match the workspace form."""
    lib = _native.library()
    shapes = [(524288 // 4, 64, 5440), (300000, 64, 4000)]
    inputs = []
    for N, w, C in shapes:
        g = torch.Generator().manual_seed(N + C)
        inputs.append((torch.randn(N, w, generator=g).to(cuda), torch.randn(N, C, generator=g).to(cuda)))
    main = torch.cuda.current_stream(cuda)
    wants = [_workspace_form(lib, v, w, dmix, N, w, C, main.cuda_stream)
             for (v, dmix), (N, w, C) in zip(inputs, shapes)]
    outs = [torch.full((w, C), float("nan"), device=cuda) for (N, w, C) in shapes]
    streams = [torch.cuda.Stream(cuda), torch.cuda.Stream(cuda)]
    torch.cuda.synchronize()
    print("no-alloc dM on two streams", flush=True)
    for s, (v, dmix), (N, w, C), out in zip(streams, inputs, shapes, outs):
        assert lib.gm_node_mix_backward_weight_noalloc_f32(v.data_ptr(), w, dmix.data_ptr(), N, w, C, out.data_ptr(),
                                                           s.cuda_stream) == 0, lib.gm_last_error()
    torch.cuda.synchronize()
    for got, want in zip(outs, wants):
        scale = float(want.abs().max())
        assert float((got - want).abs().max()) <= 2e-6 * scale


def test_no_alloc_weight_gradient_rejects_what_the_array_cannot_hold(cuda):
    """w = 128, C = 65540: one row split's partial needs 8.4 M floats > 2^23;
    the check runs before any launch."""
    lib = _native.library()
    v = torch.zeros(4, 128, device=cuda)
    dmix = torch.zeros(4, 65540, device=cuda)
    dm = torch.zeros(128, 65540, device=cuda)
    status = lib.gm_node_mix_backward_weight_noalloc_f32(v.data_ptr(), 128, dmix.data_ptr(), 4, 128, 65540,
                                                         dm.data_ptr(), torch.cuda.current_stream(cuda).cuda_stream)
    assert status == 1
    assert b"too large for the no-allocation weight gradient" in lib.gm_last_error()
    assert ctypes.c_int(status).value == 1
