"""The bfloat16 per-edge streams of a bfloat16 block's value kernels: the
trunk features h, the value rows and dh stored in bfloat16 with float32
arithmetic (gm_radial_trunk_*_bf16, gm_factored_{forward,backward}_grouped
*_bf16, gm_factored_aggregate_heads_bf16).

Each entry is checked against its float32 twin on the same (exactly widened)
inputs: the arithmetic is the same, so a bfloat16 output is the float32
result rounded to nearest even and a float32 output agrees to float32
rounding.  In the layer the grouped calls are shadowed by the float32 entries
call by call, and the whole attention is compared with its float32-stream
form (GM_BF16_STREAMS=0) within the bfloat16 bar."""

import copy

import pytest
import torch

import problems
from gm_attention_amd import _native
from gm_attention_amd.nn import fused_factored
from gm_attention_amd.nn.attention import SO2MHSA
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def rounded_from(got_b16, want_f32, name):
    """``got_b16`` is ``want_f32`` rounded to bfloat16, up to one bfloat16 unit
    where ``want_f32`` itself differs from the twin's by float32 rounding:
    |got - want| <= 2^-8 |want| + 1e-30 everywhere, and equal to torch's
    rounding of ``want`` in all but a 1e-4 fraction of entries."""
    g, w = got_b16.float().cpu(), want_f32.float().cpu()
    assert bool(((g - w).abs() <= w.abs() * 2.0 ** -8 + 1e-30).all()), f"{name}: not within a bfloat16 unit"
    mismatched = float((got_b16.cpu() != want_f32.cpu().to(BF16)).float().mean())
    assert mismatched <= 1e-4, f"{name}: {mismatched:.2e} of the entries round differently"


def test_trunk_features_in_bfloat16_are_the_float32_ones_rounded(cuda):
    g = torch.Generator().manual_seed(3)
    E, H, B = 5003, 8, 8  # not a multiple of the 16-edge tile
    rho = torch.rand(E, generator=g).to(cuda)
    weight = torch.randn(H, 16, B, generator=g).to(cuda)
    bias = torch.randn(H, 16, generator=g).to(cuda)
    centers = torch.linspace(0.0, 1.0, B).to(cuda)
    h32 = _native.radial_trunk_forward(rho, weight, bias, centers, 0.2)
    h16 = _native.radial_trunk_forward(rho, weight, bias, centers, 0.2, BF16)
    assert h16.dtype == BF16 and h16.shape == h32.shape
    assert torch.equal(h16, h32.to(BF16))
    dh16 = torch.randn(H, E, 16, generator=g).to(cuda, BF16)
    dw16, db16 = _native.radial_trunk_backward(dh16, rho, weight, bias, centers, 0.2)
    dw32, db32 = _native.radial_trunk_backward(dh16.float(), rho, weight, bias, centers, 0.2)
    torch.testing.assert_close(dw16, dw32, rtol=1e-6, atol=1e-6 * float(dw32.abs().max()))
    torch.testing.assert_close(db16, db32, rtol=1e-6, atol=1e-6 * float(db32.abs().max()))


@pytest.mark.parametrize("H,d_out,split", [(8, 20, 1), (16, 20, 2), (4, 12, 1)])
def test_aggregate_of_bfloat16_rows_equals_the_float32_sum_of_the_widened_rows(H, d_out, split, cuda):
    g = torch.Generator().manual_seed(H + d_out)
    degrees = torch.tensor([0, 1, 5, 70, 3, 0, 17, 8, 64, 9])
    row_ptr = torch.zeros(len(degrees) + 1, dtype=torch.long)
    row_ptr[1:] = torch.cumsum(degrees, 0)
    E = int(row_ptr[-1])
    rows = torch.randn(H, E, d_out, generator=g).to(BF16)
    alpha = torch.rand(E, H // split, generator=g)
    inv = torch.randperm(E, generator=g)
    args = (inv.to(cuda), alpha.to(cuda), row_ptr.to(cuda), split)
    got = _native.aggregate_heads(rows.to(cuda), *args)
    want = _native.aggregate_heads(rows.float().to(cuda), *args)
    assert got.dtype == torch.float32 and torch.equal(got, want)


def mhsa_case(nlat=16, nlon=32, batch=2):
    disc = problems.discretization(nlat, nlon)
    edges = disc.edge_geometry.tile(batch, n_sources=disc.n_nodes)
    torch.manual_seed(0)
    mhsa = SO2MHSA(SO2FieldType({0: 32, 1: 32, 2: 32}), 8, cutoff=disc.coverage_radius, window="hard",
                   batched=True, dtype=torch.float64)
    n = edges.row_ptr.shape[0] - 1
    x = problems.normal((n, mhsa.field_type_in.dimension), 1).to(BF16)
    return mhsa, x, edges


def run(module, flat, edges, probe):
    leaf = flat.clone().requires_grad_(True)
    module.zero_grad(set_to_none=True)
    out = module(SO2FeatureField.from_flat(module.field_type_in, leaf), edges).to_flat()
    (out.float() * probe).sum().backward()
    return out.detach(), leaf.grad, {k: p.grad for k, p in module.named_parameters() if p.grad is not None}


def test_grouped_calls_on_bfloat16_streams_match_their_float32_twins(cuda, monkeypatch):
    """The 8-head {0:32,1:32,2:32} attention (the block's) on bfloat16 rows,
    16x32, two samples: every grouped forward and backward call runs on
    bfloat16 streams, and each equals the float32 entry on the widened
    streams (rows and dh: the float32 results rounded; dweights to float32
    rounding)."""
    monkeypatch.setattr(fused_factored, "BF16_STREAMS", True)
    mhsa, x, edges = mhsa_case()
    gpu = copy.deepcopy(mhsa).to(cuda, torch.float32)
    e32 = edges.to(cuda, torch.float32)
    probe = problems.normal(tuple(x.shape), 7).float().to(cuda)
    real_fwd, real_bwd = _native.factored_forward_grouped, _native.factored_backward_grouped
    calls = {"forward": 0, "backward": 0}

    def forward(h_g, *args, out=None, **kwargs):
        assert h_g.dtype == BF16, "the trunk features are not bfloat16"
        got = real_fwd(h_g, *args, out=out, **kwargs)
        want = real_fwd(h_g.float(), *args, **kwargs)
        rounded_from(got, want, "rows")
        calls["forward"] += 1
        return got

    def backward(g, target_g, weights_g, rows_g, h_g, *args, dweights=None, accumulate=False, **kwargs):
        assert h_g.dtype == BF16 and rows_g.dtype == BF16
        dh_g = args[-1]
        dh_before = dh_g.float().clone()
        dw_before = None if dweights is None else dweights.clone()
        got_dw = real_bwd(g, target_g, weights_g, rows_g, h_g, *args, dweights=dweights, accumulate=accumulate,
                          **kwargs)
        dh32 = dh_before.clone()
        want_dw = real_bwd(g, target_g, weights_g, rows_g.float(), h_g.float(), *args[:-1], dh32,
                           dweights=None if dw_before is None else dw_before.clone(), accumulate=accumulate, **kwargs)
        rounded_from(dh_g, dh32, "dh")
        scale = float(want_dw.abs().max())
        assert float((got_dw - want_dw).abs().max()) <= 1e-6 * scale, "dweights"
        calls["backward"] += 1
        return got_dw

    monkeypatch.setattr(_native, "factored_forward_grouped", forward)
    monkeypatch.setattr(_native, "factored_backward_grouped", backward)
    print("bf16 streams 16x32 B=2: grouped calls against float32 twins", flush=True)
    run(gpu, x.to(cuda), e32, probe)
    assert calls == {"forward": 8, "backward": 8}


def test_attention_on_bfloat16_streams_is_within_the_bfloat16_bar_of_float32_streams(cuda, monkeypatch):
    """The same attention with the streams in bfloat16 and in float32
    (GM_BF16_STREAMS=0): output and input gradient within 2e-2 of the largest
    entry, parameter gradients within 2e-2 in norm (the block's bar; the key
    biases' gradients vanish and are not compared)."""
    mhsa, x, edges = mhsa_case()
    gpu = copy.deepcopy(mhsa).to(cuda, torch.float32)
    e32 = edges.to(cuda, torch.float32)
    probe = problems.normal(tuple(x.shape), 7).float().to(cuda)
    results = {}
    for on in (True, False):
        monkeypatch.setattr(fused_factored, "BF16_STREAMS", on)
        print(f"bf16 streams {on}: attention 16x32 B=2", flush=True)
        results[on] = run(gpu, x.to(cuda), e32, probe)
    (o16, dx16, dp16), (o32, dx32, dp32) = results[True], results[False]
    for name, g, w in (("out", o16, o32), ("dx", dx16, dx32)):
        err = float((g.float() - w.float()).abs().max()) / float(w.float().abs().max())
        print(f"  {name}: {err:.2e} of the largest entry", flush=True)
        assert err <= 2e-2, name
    assert set(dp16) == set(dp32)
    for k in dp32:
        # the softmax is invariant to a key bias (it adds q.b to every score of a target): its
        # gradient is zero in exact arithmetic and rounding noise of the bfloat16 rows in both forms
        if k.endswith("key.bias"):
            continue
        w, g = dp32[k].double(), dp16[k].double()
        assert float((g - w).norm()) / float(w.norm()) <= 2e-2, k
