"""Host-side pieces of the fused feed-forward (no GPU): the per-frequency
blocks it hands the kernels are the SO2Linear layers' flat matrices
(reference nn/linear.py:130-190), and the predicate declines what the
kernels do not serve."""

import types

import torch

from gm_attention_amd.nn import ffn
from gm_attention_amd.nn.linear import SO2Linear, block_matrix
from gm_attention_amd.nn.nonlinearities import SO2ScalarGatedNonlinearity
from gm_attention_amd.nn.normalization import SO2Dropout, SO2LayerNorm
from gm_attention_amd.representations.field_type import SO2FieldType


def _block(a: int, b: int):
    ft = SO2FieldType({0: a, 1: a, 2: a})
    hft = SO2FieldType({0: b, 1: b, 2: b})
    return types.SimpleNamespace(norm2=SO2LayerNorm(ft), linear1=SO2Linear(ft, hft),
                                 activation=SO2ScalarGatedNonlinearity(hft), linear2=SO2Linear(hft, ft),
                                 mlp_dropout=SO2Dropout(ft, p=0.0), field_type=ft, hidden_field_type=hft)


def test_blocks_are_the_flat_matrix_blocks():
    torch.manual_seed(0)
    blk = _block(32, 128)
    for lin in (blk.linear1, blk.linear2):
        m = block_matrix(lin)
        sin, sout = lin.field_type_in.slices(), lin.field_type_out.slices()
        for f in (0, 1, 2):
            assert torch.equal(ffn._real_block(lin, f), m[sin[f], sout[f]])
        # and nothing outside the blocks
        mask = torch.zeros_like(m, dtype=torch.bool)
        for f in (0, 1, 2):
            mask[sin[f], sout[f]] = True
        assert float(m[~mask].abs().max()) == 0.0


def test_the_complex_block_is_a_complex_product():
    """Frequency 1's block acts on interleaved (re, im) pairs as the complex weights do."""
    torch.manual_seed(1)
    lin = SO2Linear(SO2FieldType({0: 2, 1: 3}), SO2FieldType({0: 4, 1: 5}))
    x = torch.randn(7, 3, 2)
    want = torch.view_as_real(torch.einsum("ba,na->nb", torch.view_as_complex(lin.weight["1"].detach()),
                                           torch.view_as_complex(x)))
    got = (x.reshape(7, 6) @ ffn._real_block(lin, 1).detach()).reshape(7, 5, 2)
    assert torch.allclose(got, want, atol=1e-6)


def test_predicate_declines_what_the_kernels_do_not_serve():
    x = torch.zeros(16, 160, dtype=torch.bfloat16)
    assert not ffn.serves(_block(32, 128), x)  # CPU rows
    assert ffn._uniform(SO2FieldType({0: 32, 1: 32, 2: 32}), ffn.A_SERVED) == 32
    assert ffn._uniform(SO2FieldType({0: 32, 1: 32}), ffn.A_SERVED) is None  # frequency 2 missing
    assert ffn._uniform(SO2FieldType({0: 32, 1: 16, 2: 32}), ffn.A_SERVED) is None  # uneven copies
    assert ffn._uniform(SO2FieldType({0: 96, 1: 96, 2: 96}), ffn.B_SERVED) is None  # no kernel for 96
