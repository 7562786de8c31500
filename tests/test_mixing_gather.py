"""The mix matrices' signed gather (nn/fused_factored.py ``_SignedGather``):
its values and its parameter gradient equal those of plain indexing
(``flat[index] * sign`` under autograd) on maps with repeated parameters,
negated and zero entries; no GPU needed."""

import torch

from gm_attention_amd.nn import fused_factored


def _maps(n, shapes, seed):
    g = torch.Generator().manual_seed(seed)
    maps = []
    for shape in shapes:
        index = torch.randint(0, n, shape, generator=g)
        sign = torch.randint(-1, 2, shape, generator=g).to(torch.float64)  # -1, 0 or 1
        maps.append((index, sign))
    return maps


def test_signed_gather_matches_indexing():
    torch.manual_seed(0)
    n = 97
    maps = _maps(n, [(5, 40), (7, 33), (3, 128)], seed=1)
    flat = torch.randn(n, dtype=torch.float64, requires_grad=True)
    want = [flat[i] * s for i, s in maps]
    upstream = [torch.randn_like(w) for w in want]
    want_grad, = torch.autograd.grad(want, flat, upstream)

    flat2 = flat.detach().clone().requires_grad_(True)
    got = fused_factored._SignedGather.apply(flat2, dict(maps=maps))
    for a, b in zip(got, want, strict=True):
        assert torch.equal(a, b.detach())
    got_grad, = torch.autograd.grad(got, flat2, upstream)
    assert torch.allclose(got_grad, want_grad, rtol=0, atol=1e-12)
    # a parameter no map reads gets zero
    unused = torch.ones(n, dtype=torch.bool)
    for i, s in maps:
        unused[i[s != 0]] = False
    assert torch.all(got_grad[unused] == 0)


def test_signed_gather_plan_is_reused_and_unused_outputs_count_zero():
    n = 31
    maps = _maps(n, [(4, 10), (2, 9)], seed=2)
    plan = dict(maps=maps)
    flat = torch.randn(n, dtype=torch.float64, requires_grad=True)
    a, b = fused_factored._SignedGather.apply(flat, plan)
    a.sum().backward()  # b takes no gradient
    want = torch.zeros(n, dtype=torch.float64).index_add_(0, maps[0][0].reshape(-1), maps[0][1].reshape(-1))
    assert torch.allclose(flat.grad, want, rtol=0, atol=1e-12)
    assert "order" in plan and "cols" in plan
    flat.grad = None
    a, b = fused_factored._SignedGather.apply(flat, plan)
    (2 * b).sum().backward()
    want = torch.zeros(n, dtype=torch.float64).index_add_(0, maps[1][0].reshape(-1), 2 * maps[1][1].reshape(-1))
    assert torch.allclose(flat.grad, want, rtol=0, atol=1e-12)


def test_signed_gather_many_uses_takes_the_segment_sum():
    """More uses of a parameter than the padded columns hold: the segment-sum form."""
    n = 5
    maps = _maps(n, [(9, 40)], seed=3)  # 360 positions over 5 parameters: about 72 uses each
    flat = torch.randn(n, dtype=torch.float64, requires_grad=True)
    want = [flat[i] * s for i, s in maps]
    up = [torch.randn_like(w) for w in want]
    want_grad, = torch.autograd.grad(want, flat, up)
    plan = dict(maps=maps)
    got = fused_factored._SignedGather.apply(flat, plan)
    got_grad, = torch.autograd.grad(got, flat, up)
    assert "cols" not in plan
    assert torch.allclose(got_grad, want_grad, rtol=0, atol=1e-12)
