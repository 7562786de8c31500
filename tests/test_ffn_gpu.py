"""The fused feed-forward (gm_ffn_forward_bf16 / gm_ffn_backward_bf16) against
the float64 oracle (oracle.modules.layer_norm, linear and gated composed as
the reference's block composes them after the mixer, nn/blocks.py:326-349):

* bfloat16 rows of {0:32,1:32,2:32}, the hidden field {0:B,1:B,2:B} for B = 128
  (the C4 block, ffn_multiplier 4) and 64 (ffn_multiplier 2), both gates
  (SiLU and 2 sigmoid), nonzero gains, norm bias and layer and gate biases, a
  node count that is no multiple of the 16-node tile;
* out = x + linear2(act(linear1(norm2(x)))) and its input gradient within 2e-2
  of the largest entry, every parameter gradient within 2e-2 in norm (the
  bfloat16 bars of the C4 block test), against float64 on the same rounded
  input and parameters; the products run in bfloat16 with float32
  accumulation, as the separate passes' GEMMs do;
* the fused pass serves exactly the shapes it claims (predicate)."""

import types

import pytest
import torch

from gm_attention_amd.nn import ffn
from gm_attention_amd.nn.linear import SO2Linear
from gm_attention_amd.nn.nonlinearities import SO2ScalarGatedNonlinearity
from gm_attention_amd.nn.normalization import SO2Dropout, SO2LayerNorm
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import modules

pytestmark = pytest.mark.gpu

D64 = torch.float64


def _block(B: int, gate: str, dtype, device):
    ft = SO2FieldType({0: 32, 1: 32, 2: 32})
    hft = SO2FieldType({0: B, 1: B, 2: B})
    kw = dict(dtype=dtype, device=device)
    return types.SimpleNamespace(
        norm2=SO2LayerNorm(ft, **kw), linear1=SO2Linear(ft, hft, **kw),
        activation=SO2ScalarGatedNonlinearity(hft, gate=gate, **kw), linear2=SO2Linear(hft, ft, **kw),
        mlp_dropout=SO2Dropout(ft, p=0.0), field_type=ft, hidden_field_type=hft)


def _modules(blk):
    return [blk.norm2, blk.linear1, blk.activation, blk.linear2]


def _params(blk):
    return {f"{i}.{k}": p for i, m in enumerate(_modules(blk)) for k, p in m.named_parameters()}


@pytest.mark.parametrize("B,gate", [(128, "double_sigmoid"), (128, "silu"), (64, "double_sigmoid")])
def test_fused_ffn_matches_the_oracle(cuda, B, gate):
    print(f"fused FFN A=32 B={B} gate={gate} N=1000", flush=True)
    ref = _block(B, gate, D64, "cpu")
    g = torch.Generator().manual_seed(11)
    with torch.no_grad():  # every parameter random (gains near 1, weights ~ 1 / sqrt(fan-in)), float32 values
        for name, p in _params(ref).items():
            base = 1.0 if name.startswith("0.gamma") else 0.0
            scale = 0.18 if name.startswith("1.weight") else (0.09 if name.startswith("3.weight") else 0.3)
            p.copy_((base + scale * torch.randn(p.shape, generator=g, dtype=D64)).float().double())
    gpu = _block(B, gate, torch.float32, cuda)
    for mr, mg in zip(_modules(ref), _modules(gpu), strict=True):
        mg.load_state_dict({k: v.float() for k, v in mr.state_dict().items()})
    n, ft = 1000, ref.field_type
    x = torch.randn(n, ft.dimension, generator=g, dtype=D64).to(torch.bfloat16)
    probe = torch.randn(n, ft.dimension, generator=g, dtype=D64)

    # float64 oracle on the rounded input
    leaf = x.double().requires_grad_(True)
    xs = dict(SO2FeatureField.from_flat(ft, leaf).coefficients)
    normed = modules.layer_norm(ref.norm2, xs)
    hidden = modules.linear(ref.linear1, normed, ref.hidden_field_type)
    y = modules.linear(ref.linear2, modules.gated(ref.activation, hidden), ft)
    want = leaf + modules.flat(y)
    (want * probe).sum().backward()
    want_grads = {k: p.grad for k, p in _params(ref).items()}

    # the fused pass
    xg = x.to(cuda).requires_grad_(True)
    assert ffn.serves(gpu, xg)
    got = ffn.forward(gpu, xg)
    assert got.dtype == torch.bfloat16
    (got.double() * probe.to(cuda)).sum().backward()

    for name, gv, wv in (("out", got.detach(), want.detach()), ("dx", xg.grad, leaf.grad)):
        gv, wv = gv.double().cpu(), wv.double().cpu()
        err = float((gv - wv).abs().max()) / float(wv.abs().max())
        print(f"  {name}: error {err:.2e} of the largest entry", flush=True)
        assert err <= 2e-2, f"{name}: error {err:.3e} of the largest entry"
    for name, p in _params(gpu).items():
        gv, wv = p.grad.double().cpu(), want_grads[name]
        err = float((gv - wv).norm()) / max(float(wv.norm()), 1e-30)
        print(f"  d{name}: error {err:.2e} in norm", flush=True)
        assert err <= 2e-2, f"d{name}: error {err:.3e} in norm"


def test_fused_ffn_predicate(cuda):
    blk = _block(128, "double_sigmoid", torch.float32, cuda)
    x = torch.zeros(16, 160, dtype=torch.bfloat16, device=cuda)
    assert ffn.serves(blk, x)
    assert not ffn.serves(blk, x.float())  # float32 rows keep the separate passes
    assert not ffn.serves(blk, x.cpu())
    blk.mlp_dropout = SO2Dropout(blk.field_type, p=0.1)  # a training dropout sits between linear2 and the sum
    assert not ffn.serves(blk, x)
    blk.mlp_dropout.eval()
    assert ffn.serves(blk, x)
    wide = _block(96, "silu", torch.float32, cuda)
    assert not ffn.serves(wide, x)
