"""The transformer block's oracle (oracle.modules.layer_norm, gated,
block_forward) pinned on the CPU:

* the layer norm of a scalar-only field is torch's LayerNorm, of a field with
  one nonzero frequency torch's RMSNorm over its coordinates (no centring
  there), and with a zero second frequency the pooled variance halves (the
  mean over present frequencies, reference normalization.py:170-176);
* the gate with zero weights and biases is the identity on copies under
  2 sigmoid and zero under SiLU, SiLU on the scalars; a constant gate bias
  scales every copy by act(bias);
* the layer norm, the gate and the whole block (both mixers) are gauge
  equivariant under random frame rotations;
* the package's torch paths for CPU tensors (the modules' reference
  arithmetic, the flat block-diagonal SO2Linear) equal the oracle."""

import math

import pytest
import torch
import torch.nn.functional as F

import problems
from gm_attention_amd.discretization.discretization import SphericalDiscretization
from gm_attention_amd.discretization.frames import build_tangent_frames, rotate_tangent_frames
from gm_attention_amd.discretization.grid import build_equiangular_grid
from gm_attention_amd.nn.blocks import SO2TransformerBlock
from gm_attention_amd.nn.linear import SO2Linear, flat_forward
from gm_attention_amd.nn.nonlinearities import SO2ScalarGatedNonlinearity
from gm_attention_amd.nn.normalization import SO2LayerNorm
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import modules

D64 = torch.float64


def field_of(ft, n, seed):
    return {f: problems.normal((n, m) if f == 0 else (n, m, 2), seed + f) for f, m in ft.items()}


def randomise(module, seed=3):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in module.parameters():
            p.copy_(torch.randn(p.shape, generator=g, dtype=D64))


def rotate(x, theta):
    out = {}
    for f, t in x.items():
        if f == 0:
            out[f] = t
        else:
            out[f] = torch.view_as_real(torch.view_as_complex(t.contiguous()) * torch.polar(
                torch.ones_like(theta), f * theta).unsqueeze(-1))
    return out


def test_layer_norm_of_scalars_is_torch_layer_norm():
    ft = SO2FieldType({0: 12})
    norm = SO2LayerNorm(ft, eps=1e-3, dtype=D64)
    randomise(norm)
    x = field_of(ft, 9, 0)
    want = F.layer_norm(x[0], (12,), weight=norm.gamma["0"], bias=norm.beta, eps=1e-3)
    torch.testing.assert_close(modules.layer_norm(norm, x)[0], want, rtol=1e-12, atol=1e-12)


def test_layer_norm_of_one_frequency_is_rms_norm():
    ft = SO2FieldType({2: 5})
    norm = SO2LayerNorm(ft, eps=1e-3, dtype=D64)
    randomise(norm)
    x = field_of(ft, 9, 1)
    flat = x[2].reshape(9, 10)
    want = F.rms_norm(flat, (10,), weight=norm.gamma["2"].repeat_interleave(2), eps=1e-3).reshape(9, 5, 2)
    torch.testing.assert_close(modules.layer_norm(norm, x)[2], want, rtol=1e-12, atol=1e-12)


def test_layer_norm_pools_the_variance_over_present_frequencies():
    ft = SO2FieldType({0: 6, 1: 4})
    norm = SO2LayerNorm(ft, eps=1e-3, dtype=D64)
    randomise(norm)
    x = field_of(ft, 7, 2)
    x[1] = torch.zeros_like(x[1])
    out = modules.layer_norm(norm, x)
    want = math.sqrt(2.0) * norm.gamma["0"] * F.layer_norm(x[0], (6,), eps=2e-3) + norm.beta
    torch.testing.assert_close(out[0], want, rtol=1e-12, atol=1e-12)
    assert float(out[1].detach().abs().max()) == 0.0


@pytest.mark.parametrize("gate", ["silu", "double_sigmoid"])
def test_gate_special_cases(gate):
    ft = SO2FieldType({0: 5, 1: 3, 2: 2})
    act = SO2ScalarGatedNonlinearity(ft, gate=gate, dtype=D64)
    x = field_of(ft, 8, 4)
    with torch.no_grad():
        for lin in act.gates.values():
            lin.weight.zero_()
            lin.bias.zero_()
    out = modules.gated(act, x)
    torch.testing.assert_close(out[0], F.silu(x[0]), rtol=1e-14, atol=0)
    for f in (1, 2):
        torch.testing.assert_close(out[f], x[f] if gate == "double_sigmoid" else torch.zeros_like(x[f]))
    with torch.no_grad():
        for lin in act.gates.values():
            lin.bias.fill_(0.7)
    scale = 2 * torch.sigmoid(torch.tensor(0.7, dtype=D64)) if gate == "double_sigmoid" else F.silu(
        torch.tensor(0.7, dtype=D64))
    out = modules.gated(act, x)
    for f in (1, 2):
        torch.testing.assert_close(out[f], scale * x[f], rtol=1e-14, atol=1e-14)


def test_norm_and_gate_are_gauge_equivariant():
    ft = SO2FieldType({0: 4, 1: 3, 2: 5})
    norm = SO2LayerNorm(ft, dtype=D64)
    act = SO2ScalarGatedNonlinearity(ft, gate="double_sigmoid", dtype=D64)
    randomise(norm)
    randomise(act, 5)
    x = field_of(ft, 11, 6)
    theta = problems.normal((11,), 7)
    for fn in (lambda v: modules.layer_norm(norm, v), lambda v: modules.gated(act, v)):
        a = fn(rotate(x, theta))
        b = rotate(fn(x), theta)
        for f in a:
            torch.testing.assert_close(a[f], b[f], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("mixer", ["attention", "convolution"])
def test_block_oracle_is_gauge_equivariant(mixer):
    nlat, nlon = 8, 16
    grid = build_equiangular_grid(nlat, nlon)
    cutoff = 3.0 * math.pi / (nlat - 1)
    frames = build_tangent_frames(grid.nodes)
    theta = torch.rand(grid.n_nodes, dtype=D64, generator=torch.Generator().manual_seed(4)) * 2 * math.pi
    base = SphericalDiscretization.from_grid(grid, cutoff, frames=frames).edge_geometry
    turned = SphericalDiscretization.from_grid(grid, cutoff, frames=rotate_tangent_frames(frames, theta)).edge_geometry
    torch.manual_seed(0)
    ft = SO2FieldType({0: 4, 1: 4, 2: 4})
    block = SO2TransformerBlock(ft, 2, ffn_multiplier=2, cutoff=cutoff, n_radial_basis=4, mixer=mixer, dtype=D64)
    randomise(block, 9)
    with torch.no_grad():  # keep the scores moderate
        for p in block.parameters():
            p.mul_(0.3)
    x = field_of(ft, grid.n_nodes, 8)
    y = modules.block_forward(block, x, base)
    # the field in the rotated gauge: coefficients by rho(r_{-theta})
    y_turned = modules.block_forward(block, rotate(x, -theta), turned)
    want = rotate(y, -theta)
    for f in y:
        torch.testing.assert_close(y_turned[f], want[f], rtol=1e-9, atol=1e-9)
    assert max(float((y[f] - want[f]).abs().max()) for f in (1, 2)) > 1e-3


def test_host_paths_equal_the_oracle():
    ft = SO2FieldType({0: 6, 1: 4, 2: 2})
    hidden = SO2FieldType({0: 12, 1: 8, 2: 4})
    norm = SO2LayerNorm(ft, dtype=D64)
    act = SO2ScalarGatedNonlinearity(hidden, gate="double_sigmoid", dtype=D64)
    lin = SO2Linear(ft, hidden, dtype=D64)
    for m in (norm, act, lin):
        randomise(m, 11)
    x = field_of(ft, 10, 12)
    xf = SO2FeatureField(ft, x)
    for got, want in ((norm(xf), modules.layer_norm(norm, x)),):
        for f in want:
            torch.testing.assert_close(got[f], want[f], rtol=1e-12, atol=1e-12)
    h = modules.linear(lin, x, hidden)
    torch.testing.assert_close(flat_forward(lin, xf.to_flat()), modules.flat(h), rtol=1e-12, atol=1e-12)
    got = act(SO2FeatureField(hidden, h))
    want = modules.gated(act, h)
    for f in want:
        torch.testing.assert_close(got[f], want[f], rtol=1e-12, atol=1e-12)
