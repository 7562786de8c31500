"""The row-blocked weight gradient of the projections (nn.linear.RowsMatmul):
x^T g summed over blocks of rows equals the direct product, remainder rows
included, and the Function passes gradcheck."""

import pytest
import torch

from gm_attention_amd.nn.linear import RowsMatmul, blocked_gram


@pytest.mark.parametrize("rows,block", [(10, 4), (8192 * 3 + 17, 8192), (64, 64), (63, 64)])
def test_blocked_gram_is_the_gram_product(rows, block):
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, 7, dtype=torch.float64, generator=g)
    y = torch.randn(rows, 5, dtype=torch.float64, generator=g)
    torch.testing.assert_close(blocked_gram(x, y, block), x.t() @ y, rtol=1e-12, atol=1e-12)


def test_rows_matmul_gradcheck():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(37, 6, dtype=torch.float64, generator=g, requires_grad=True)
    w = torch.randn(6, 4, dtype=torch.float64, generator=g, requires_grad=True)
    assert torch.autograd.gradcheck(RowsMatmul.apply, (x, w))
