"""The grouped path's helper ops on the GPU: the all-heads aggregate
(gm_factored_aggregate_heads_f32) against a float64 sum in CSR order, and the
gather/scatter transposes (gm_gather_transpose_f32 / gm_scatter_transpose_f32)
bit-exact against indexing."""

import pytest
import torch

import problems

from gm_attention_amd import _native

pytestmark = pytest.mark.gpu


def csr(degrees):
    row_ptr = torch.zeros(len(degrees) + 1, dtype=torch.long)
    row_ptr[1:] = torch.cumsum(torch.tensor(degrees, dtype=torch.long), 0)
    return row_ptr


@pytest.mark.parametrize("H,d_out,split", [(8, 20, 1), (2, 12, 1), (3, 6, 1), (1, 1, 1), (16, 20, 2), (32, 20, 2),
                                           (16, 16, 4), (40, 7, 2), (64, 16, 1)])
def test_aggregate_heads_matches_a_csr_sum(H, d_out, split, cuda):
    """fp32: within 1e-5 of the largest |value| (sums of up to 70 products);
    row heads h share alpha's column h // split; the 16-byte kernels take one
    to four pieces a lane, other widths the scalar kernel."""
    g = torch.Generator().manual_seed(H * 100 + d_out)
    degrees = [0, 1, 5, 70, 3, 0, 17, 8, 64, 9]  # empty targets, one edge, more than one step of eight
    row_ptr = csr(degrees)
    E = int(row_ptr[-1])
    rows = torch.randn(H, E, d_out, generator=g)
    alpha = torch.rand(E, H // split, generator=g)
    inv = torch.randperm(E, generator=g)
    wide = alpha.repeat_interleave(split, dim=1)
    want = torch.zeros(len(degrees), H, d_out, dtype=torch.float64)
    for i in range(len(degrees)):
        for e in range(int(row_ptr[i]), int(row_ptr[i + 1])):
            want[i] += wide[e].double()[:, None] * rows[:, inv[e]].double()
    got = _native.aggregate_heads(rows.to(cuda), inv.to(cuda), alpha.to(cuda), row_ptr.to(cuda), split).cpu().double()
    problems.report_strict(got, want, "aggregate")
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5 * float(want.abs().max()))


@pytest.mark.parametrize("n", [1000, 9483, 100003])
@pytest.mark.parametrize("width", [1, 4, 8, 13])
def test_gather_and_scatter_transposes_are_exact(width, n, cuda):
    """Rows 0 .. n-1 in 256-row blocks that each XCD takes as a contiguous range:
    fewer blocks than XCDs, a block count that does not divide among them and a
    ragged last block all move every row exactly once."""
    g = torch.Generator().manual_seed(width + n)
    src = torch.randn(n, width, generator=g)
    perm = torch.randperm(n, generator=g)
    t = _native.gather_transpose(src.to(cuda), perm.to(cuda)).cpu()
    assert torch.equal(t, src[perm].t().contiguous())
    back = _native.scatter_transpose(t.to(cuda), perm.to(cuda)).cpu()
    assert torch.equal(back, src)
