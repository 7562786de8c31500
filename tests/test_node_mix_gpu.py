"""The node-mix MFMA kernels (gm_node_mix_*: every head's node products
X_n M_n, the reference's einsum at nn/kernels.py:575-603, and their two
gradients) against float64 torch products of the same float32 inputs, on
column slices of flat rows as the layers pass them, over widths that fill,
pad and span the kernels' 16/32/64/128 width classes, mix widths with partial
column tiles, and node counts with partial row tiles."""

import pytest
import torch

import problems

from gm_attention_amd import _native

pytestmark = pytest.mark.gpu

CASES = [  # (N, D, column offset, w, C)
    (1, 8, 0, 8, 4),
    (63, 20, 4, 16, 68),
    (64, 160, 32, 64, 5440),
    (129, 160, 0, 32, 2720),
    (5000, 160, 96, 64, 5440),
    (777, 40, 3, 20, 100),
    (300, 384, 128, 128, 2176),
    (200, 100, 1, 99, 12),
]


def _inputs(N, D, off, w, C, seed):
    g = torch.Generator().manual_seed(seed)
    rows = torch.randn(N, D, generator=g, dtype=torch.float64).float()
    m = torch.randn(w, C, generator=g, dtype=torch.float64).float()
    dmix = torch.randn(N, C, generator=g, dtype=torch.float64).float()
    return rows, m, dmix


def _close(got, want, name, tol):
    got, want = got.double().cpu(), want.double()
    problems.report_strict(got, want, name)
    scale = want.abs().max().clamp_min(1.0)
    err = float((got - want).abs().max() / scale)
    assert err <= tol, f"{name}: error {err:.3e} of the largest entry"


@pytest.mark.parametrize("case", CASES)
def test_node_mix_kernels_match_float64_products(case, cuda):
    N, D, off, w, C = case
    print(f"node mix N={N} w={w} C={C}", flush=True)
    rows, m, dmix = _inputs(N, D, off, w, C, sum(case))
    v = rows[:, off:off + w].double()
    rd, md, dd = rows.to(cuda), m.to(cuda), dmix.to(cuda)
    out = _native.node_mix_forward(rd[:, off:off + w], md)
    _close(out, v @ m.double(), "mix", 2e-6)
    dx = torch.full((N, D), 7.0, device=cuda)
    _native.node_mix_backward_input(dd, md, dx[:, off:off + w])
    _close(dx[:, off:off + w], dmix.double() @ m.double().T, "dv", 5e-6)
    untouched = torch.cat([dx[:, :off], dx[:, off + w:]], dim=1)
    assert bool((untouched == 7.0).all()), "the input gradient wrote outside its columns"
    dm = _native.node_mix_backward_weight(rd[:, off:off + w], dd)
    _close(dm, v.T @ dmix.double(), "dM", 5e-6)


def test_node_mix_backward_weight_is_deterministic(cuda):
    rows, m, dmix = _inputs(4096, 64, 0, 64, 1088, 3)
    v, dd = rows.to(cuda), dmix.to(cuda)
    first = _native.node_mix_backward_weight(v, dd)
    second = _native.node_mix_backward_weight(v, dd)
    assert torch.equal(first, second)


def test_node_mixes_function_gradients_match_torch(cuda):
    """The autograd Function over three frequencies' column slices of one
    flat field: the mixes and both gradients against float64 autograd."""
    from gm_attention_amd.nn.node_products import NodeMixes

    g = torch.Generator().manual_seed(11)
    N, columns = 999, ((0, 32), (32, 64), (96, 64))
    rows = torch.randn(N, 160, generator=g, dtype=torch.float64)
    mats = [torch.randn(w, c, generator=g, dtype=torch.float64) for (_, w), c in zip(columns, (2720, 5440, 5440))]
    probes = [torch.randn(N, m.shape[1], generator=g, dtype=torch.float64) for m in mats]
    r64 = rows.clone().requires_grad_(True)
    m64 = [m.clone().requires_grad_(True) for m in mats]
    want = [r64[:, o:o + w] @ m for (o, w), m in zip(columns, m64)]
    sum((y * p).sum() for y, p in zip(want, probes)).backward()
    r32 = rows.float().to(cuda).requires_grad_(True)
    m32 = [m.float().to(cuda).requires_grad_(True) for m in mats]
    got = NodeMixes.apply(r32, columns, *m32)
    sum((y * p.float().to(cuda)).sum() for y, p in zip(got, probes)).backward()
    for y, ref in zip(got, want):
        _close(y.detach(), ref.detach(), "mix", 2e-6)
    _close(r32.grad, r64.grad, "dx", 5e-6)
    for a, b in zip(m32, m64):
        _close(a.grad, b.grad, "dM", 5e-6)


def test_node_mixes_sharing_columns_add_their_input_gradients(cuda):
    """Two products reading the same columns (as the real block and the
    promoted complex blocks both read x_0) and one reading others."""
    from gm_attention_amd.nn.node_products import NodeMixes

    g = torch.Generator().manual_seed(5)
    N, columns = 700, ((0, 16), (0, 16), (16, 32))
    rows = torch.randn(N, 48, generator=g, dtype=torch.float64)
    mats = [torch.randn(w, c, generator=g, dtype=torch.float64) for (_, w), c in zip(columns, (68, 136, 544))]
    probes = [torch.randn(N, m.shape[1], generator=g, dtype=torch.float64) for m in mats]
    r64 = rows.clone().requires_grad_(True)
    sum(((r64[:, o:o + w] @ m) * p).sum() for (o, w), m, p in zip(columns, mats, probes)).backward()
    r32 = rows.float().to(cuda).requires_grad_(True)
    got = NodeMixes.apply(r32, columns, *[m.float().to(cuda) for m in mats])
    sum((y * p.float().to(cuda)).sum() for y, p in zip(got, probes)).backward()
    _close(r32.grad, r64.grad, "dx", 5e-6)
