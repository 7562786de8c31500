"""Zero-sized inputs through the native entry points: no edges, no nodes, or
targets without edges.  Each entry point must return normally (no launch of
an empty grid) with outputs of the right shape, and reductions over nothing
(the trunk's and the node mixes' parameter gradients, the aggregate of a
target without edges) must be exactly zero."""

import pytest
import torch

from gm_attention_amd import _native

pytestmark = pytest.mark.gpu


def trunk_params(cuda, H=8, T=16, B=8):
    g = torch.Generator().manual_seed(0)
    weight = torch.randn(H, T, B, generator=g).to(cuda)
    bias = torch.randn(H, T, generator=g).to(cuda)
    centers = torch.linspace(0.0, 1.0, B).to(cuda)
    return weight, bias, centers


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_trunk_without_edges(dtype, cuda):
    weight, bias, centers = trunk_params(cuda)
    rho = torch.zeros(0, device=cuda)
    h = _native.radial_trunk_forward(rho, weight, bias, centers, 0.2, dtype)
    assert h.shape == (8, 0, 16) and h.dtype == dtype
    dw, db = _native.radial_trunk_backward(torch.zeros(8, 0, 16, dtype=dtype, device=cuda), rho, weight, bias,
                                           centers, 0.2)
    torch.cuda.synchronize()
    assert dw.shape == (8, 16, 8) and db.shape == (8, 16)
    assert torch.count_nonzero(dw) == 0 and torch.count_nonzero(db) == 0


@pytest.mark.parametrize("w", [32, 64])
def test_node_mixes_without_nodes(w, cuda):
    C = 5 * 16
    m = torch.randn(w, C, device=cuda)
    v = torch.zeros(0, w, device=cuda)
    out = _native.node_mix_forward(v, m)
    assert out.shape == (0, C)
    dv = torch.zeros(0, w, device=cuda)
    _native.node_mix_backward_input(torch.zeros(0, C, device=cuda), m, dv)
    dm = _native.node_mix_backward_weight(v, torch.zeros(0, C, device=cuda))
    torch.cuda.synchronize()
    assert dm.shape == (w, C) and torch.count_nonzero(dm) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_aggregate_of_targets_without_edges(dtype, cuda):
    H, d_out = 8, 20
    # no edges at all: every target's sum is empty
    row_ptr = torch.zeros(7, dtype=torch.int64, device=cuda)
    out = _native.aggregate_heads(torch.zeros(H, 0, d_out, dtype=dtype, device=cuda),
                                  torch.zeros(0, dtype=torch.int64, device=cuda), torch.zeros(0, H, device=cuda),
                                  row_ptr)
    torch.cuda.synchronize()
    assert out.shape == (6, H, d_out) and torch.count_nonzero(out) == 0
    # no targets
    out = _native.aggregate_heads(torch.zeros(H, 0, d_out, dtype=dtype, device=cuda),
                                  torch.zeros(0, dtype=torch.int64, device=cuda), torch.zeros(0, H, device=cuda),
                                  torch.zeros(1, dtype=torch.int64, device=cuda))
    assert out.shape == (0, H, d_out)


def test_aggregate_refuses_32_bit_indices(cuda):
    """inv holds each edge's place in the source grouping as int64 (the kernel reads 8 bytes an edge)."""
    with pytest.raises(ValueError):
        _native.aggregate_heads(torch.zeros(8, 3, 20, device=cuda), torch.zeros(3, dtype=torch.int32, device=cuda),
                                torch.zeros(3, 8, device=cuda), torch.tensor([0, 3], device=cuda))


def test_transposes_refuse_32_bit_permutations(cuda):
    """The grouping's permutation is read as int64 entries."""
    perm = torch.arange(5, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError):
        _native.gather_transpose(torch.zeros(5, 8, device=cuda), perm)
    with pytest.raises(ValueError):
        _native.scatter_transpose(torch.zeros(8, 5, device=cuda), perm)
