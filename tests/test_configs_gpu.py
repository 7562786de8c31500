"""The benchmark configurations' own layer shapes on the HIP path against the
oracle, at grid sizes the float64 oracle finishes in seconds:

* C2 / the headline layer: ``SO2MHSA(batched=True)``, field {0:32,1:32,2:32}
  (D = 160), 8 heads, hard window, radius 3 row spacings, float32, two
  samples of 16x32 and of 24x48, the output, the input's gradient and every
  parameter's gradient;
* C1: the 4-head {0:16,1:16,2:16} layer (D = 80) on one 32x64 sample, forward;
* C3: ``SO2Convolution(depthwise=True, n_radial_basis=4)`` on {0:32,1:32,2:32},
  hard window, radius 3 row spacings, the radial heads inside the walk,
  two samples of 16x32 and of 24x48, every gradient;
* C4: ``SO2TransformerBlock(ffn_multiplier=4)`` with 8 heads on
  {0:32,1:32,2:32} (160 -> 640 -> 160), bfloat16 rows and float32
  parameters, two 16x32 samples, against the float64 block on the same
  rounded inputs.

The oracle evaluates the value kernels in the factored order (the node
products gathered to the edges), which the regrouping identity pins to the
per-edge readout (tests/test_oracle_factored.py).

Tolerances (float32): the output and the input gradient elementwise within
1e-5 |want| + 1e-6 (the ratio is printed); a parameter gradient, a sum over every edge or node whose entries
can cancel to far below the summands, within 1e-5 of its norm and of its
largest entry (the elementwise figure is printed: the reference's own eager
path in float32 reaches 8.7x the elementwise bound on these sums at 16x32,
with norm errors near 5e-7).  bfloat16: within 2e-2
of the largest entry (elementwise and per parameter gradient in norm)."""

import pytest
import torch

import problems
from gm_attention_amd.nn import ffn
from gm_attention_amd.nn.attention import SO2MHSA, batched_flat_serves
from gm_attention_amd.nn.blocks import SO2TransformerBlock
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import modules

pytestmark = pytest.mark.gpu

D64 = torch.float64


def strict_report(got, want):
    """Largest |got - want| / (1e-5 |want| + 1e-6): at most 1 meets the
    north star's elementwise bound."""
    got, want = got.detach().double().cpu(), want.detach().double().cpu()
    return float(((got - want).abs() / (1e-5 * want.abs() + 1e-6)).max())


def assert_strict(got, want, name, bound=1.0):
    r = strict_report(got, want)
    assert r <= bound, f"{name}: |got - want| reaches {r:.2f} x (1e-5 |want| + 1e-6)"


def assert_reduction(got, want, name):
    got, want = got.detach().double().cpu(), want.detach().double().cpu()
    if float(want.abs().max()) < 1e-6:  # an identically vanishing gradient (a key bias under the softmax)
        assert float(got.abs().max()) <= 1e-5, f"{name}: {float(got.abs().max()):.3e} where the gradient vanishes"
        return
    err = float((got - want).norm() / want.norm())
    peak = float((got - want).abs().max() / want.abs().max())
    print(f"  {name}: norm {err:.2e} peak {peak:.2e} elementwise {strict_report(got, want):.2f}", flush=True)
    assert err <= 1e-5 and peak <= 1e-5, f"{name}: relative error {err:.3e}, peak {peak:.3e}"


def mhsa_case(field, heads, nlat, nlon, batch, seed=0):
    disc = problems.discretization(nlat, nlon)
    edges = disc.edge_geometry.tile(batch, n_sources=disc.n_nodes) if batch > 1 else disc.edge_geometry
    torch.manual_seed(seed)
    mhsa = SO2MHSA(SO2FieldType(field), heads, cutoff=disc.coverage_radius, window="hard", batched=True, dtype=D64)
    # the oracle sees the float32-rounded parameters, inputs and geometry the GPU sees
    mhsa.load_state_dict({k: v.float().double() for k, v in mhsa.state_dict().items()})
    n = edges.row_ptr.shape[0] - 1
    x = problems.normal((n, mhsa.field_type_in.dimension), seed + 1).float().double()
    return mhsa, x, edges


def run_mhsa(module, flat, edges, probe, *, oracle, backward=True):
    leaf = flat.clone().requires_grad_(backward)
    module.zero_grad(set_to_none=True)
    if oracle:
        x = SO2FeatureField.from_flat(module.field_type_in, leaf).coefficients
        out = modules.flat(modules.mhsa_forward(module, x, edges, 1e-5, messages="factored"))
    else:
        out = module(SO2FeatureField.from_flat(module.field_type_in, leaf), edges).to_flat()
    if not backward:
        return out.detach(), None, {}
    (out.double() * probe.to(out.device)).sum().backward()
    return out.detach(), leaf.grad, {n: p.grad for n, p in module.named_parameters() if p.grad is not None}


def compare_mhsa(mhsa, x, edges, cuda, backward=True):
    from gm_attention_amd.nn import eager_ops

    probe = problems.normal(x.shape, 7)
    want = run_mhsa(mhsa, x, edges.to(None, torch.float32).to(None, D64), probe, oracle=True, backward=backward)
    gpu = SO2MHSA(mhsa.field_type_in, len(mhsa.heads), cutoff=mhsa.cutoff, window="hard", batched=True,
                  dtype=torch.float32, device=cuda)
    gpu.load_state_dict({k: v.float() for k, v in mhsa.state_dict().items()})
    before = dict(eager_ops.calls)
    got = run_mhsa(gpu, x.to(cuda, torch.float32), edges.to(cuda, torch.float32), probe.to(cuda), oracle=False,
                   backward=backward)
    assert eager_ops.calls == before, "part of the layer fell back to the eager path"
    print(f"  out elementwise {strict_report(got[0], want[0]):.2f}", flush=True)
    assert_strict(got[0], want[0], "out")
    if not backward:
        return
    print(f"  dx elementwise {strict_report(got[1], want[1]):.2f}", flush=True)
    assert_strict(got[1], want[1], "dx")
    assert set(got[2]) == set(want[2]) and len(want[2]) > 0
    for name in want[2]:
        assert_reduction(got[2][name], want[2][name], f"d{name}")


@pytest.mark.parametrize("grid", [(16, 32), (24, 48)])
def test_c2_layer_matches_the_oracle(grid, cuda):
    """The headline layer: 8 heads on {0:32,1:32,2:32}, two samples, float32,
    every gradient (at 24x48 the softmax and aggregate deal their blocks to
    the XCDs in chunks)."""
    print(f"C2 layer {grid} B=2", flush=True)
    mhsa, x, edges = mhsa_case({0: 32, 1: 32, 2: 32}, 8, *grid, batch=2)
    assert mhsa.field_type_in.dimension == 160
    compare_mhsa(mhsa, x, edges, cuda)


def test_c1_layer_forward_matches_the_oracle(cuda):
    """C1: 4 heads on {0:16,1:16,2:16}, one 32x64 sample, forward."""
    print("C1 layer 32x64 B=1", flush=True)
    mhsa, x, edges = mhsa_case({0: 16, 1: 16, 2: 16}, 4, 32, 64, batch=1)
    assert mhsa.field_type_in.dimension == 80 and edges.source_index.shape[0] == 172288
    compare_mhsa(mhsa, x, edges, cuda, backward=False)


@pytest.mark.parametrize("grid", [(16, 32), (24, 48)])
def test_c3_convolution_matches_the_oracle(grid, cuda):
    """C3: the depthwise steerable convolution with 4 radial functions on
    {0:32,1:32,2:32}, two samples, float32 with the radial heads evaluated in
    the walk, against the float64 oracle on the same rounded parameters and
    inputs: the output and the input gradient at the north star's
    elementwise bound, every parameter gradient as the sums they are."""
    from gm_attention_amd.nn import depthwise_radial
    from gm_attention_amd.nn.convolution import SO2Convolution

    print(f"C3 convolution {grid} B=2", flush=True)
    disc = problems.discretization(*grid)
    edges = disc.edge_geometry.tile(2, n_sources=disc.n_nodes)
    ft = SO2FieldType({0: 32, 1: 32, 2: 32})
    torch.manual_seed(0)
    conv = SO2Convolution(ft, ft, cutoff=disc.coverage_radius, window="hard", depthwise=True, n_radial_basis=4,
                          dtype=D64)
    conv.load_state_dict({k: v.float().double() for k, v in conv.state_dict().items()})
    n = edges.row_ptr.shape[0] - 1
    x = problems.normal((n, ft.dimension), 1).float().double()
    probe = problems.normal(x.shape, 7)

    def run(module, flat, eds, oracle):
        leaf = flat.clone().requires_grad_(True)
        module.zero_grad(set_to_none=True)
        if oracle:
            out = modules.flat(modules.conv_forward(module, dict(SO2FeatureField.from_flat(ft, leaf).coefficients),
                                                    eds, 1e-5))
        else:
            out = module(SO2FeatureField.from_flat(ft, leaf), eds).to_flat()
        (out.double() * probe.to(out.device)).sum().backward()
        return out.detach(), leaf.grad, {k: p.grad for k, p in module.named_parameters() if p.grad is not None}

    want = run(conv, x, edges.to(None, torch.float32).to(None, D64), True)
    gpu = SO2Convolution(ft, ft, cutoff=disc.coverage_radius, window="hard", depthwise=True, n_radial_basis=4,
                         dtype=torch.float32, device=cuda)
    gpu.load_state_dict({k: v.float() for k, v in conv.state_dict().items()})
    e32 = edges.to(cuda, torch.float32)
    assert depthwise_radial.eligible(gpu.kernel, SO2FeatureField.from_flat(ft, x.to(cuda, torch.float32)), e32)
    got = run(gpu, x.to(cuda, torch.float32), e32, False)
    print(f"  out elementwise {strict_report(got[0], want[0]):.2f}", flush=True)
    assert_strict(got[0], want[0], "out")
    print(f"  dx elementwise {strict_report(got[1], want[1]):.2f}", flush=True)
    assert_strict(got[1], want[1], "dx")
    assert set(got[2]) == set(want[2]) and len(want[2]) > 0
    for name in want[2]:
        assert_reduction(got[2][name], want[2][name], f"d{name}")


def test_c4_block_in_bfloat16_is_within_2e2(cuda):
    """C4: the 8-head block with the 160 -> 640 -> 160 feed-forward, bfloat16
    rows and float32 parameters, two 16x32 samples, against the float64
    oracle block on the same rounded input and parameters."""
    print("C4 block 16x32 B=2 bf16", flush=True)
    disc = problems.discretization(16, 32)
    edges = disc.edge_geometry.tile(2, n_sources=disc.n_nodes)
    ft = SO2FieldType({0: 32, 1: 32, 2: 32})
    torch.manual_seed(0)
    block = SO2TransformerBlock(ft, 8, ffn_multiplier=4, cutoff=disc.coverage_radius, mixer="attention",
                                attention_batched=True, dtype=D64)
    assert block.hidden_field_type.dimension == 640
    with torch.no_grad():  # nonzero biases and gains everywhere
        for p in block.parameters():
            p.add_(0.1 * torch.randn_like(p))
    block.load_state_dict({k: v.float().double() for k, v in block.state_dict().items()})
    n = edges.row_ptr.shape[0] - 1
    x = problems.normal((n, ft.dimension), 1).to(torch.bfloat16).double()
    probe = problems.normal(x.shape, 7)

    def run(module, flat, eds, oracle):
        leaf = flat.clone().requires_grad_(True)
        module.zero_grad(set_to_none=True)
        if oracle:
            xs = dict(SO2FeatureField.from_flat(ft, leaf).coefficients)
            out = modules.flat(modules.block_forward(module, xs, eds, 1e-5, messages="factored"))
        else:
            out = module(SO2FeatureField.from_flat(ft, leaf), eds).to_flat()
        (out.double() * probe.to(out.device)).sum().backward()
        return out.detach(), leaf.grad, {k: p.grad for k, p in module.named_parameters() if p.grad is not None}

    want = run(block, x, edges.to(None, torch.float32).to(None, D64), True)
    gpu = SO2TransformerBlock(ft, 8, ffn_multiplier=4, cutoff=disc.coverage_radius, mixer="attention",
                              attention_batched=True, dtype=torch.float32, device=cuda)
    gpu.load_state_dict({k: v.float() for k, v in block.state_dict().items()})
    # the bfloat16 rows go into the fused attention as they are (bf16 scores and node-mix kernels)
    assert batched_flat_serves(gpu.attention, SO2FeatureField.from_flat(ft, x.to(cuda, torch.bfloat16)),
                               edges.to(cuda, torch.float32))
    # and the feed-forward runs as the fused pass (LN -> SO2Linear -> gate -> SO2Linear on bf16 MFMA)
    assert ffn.serves(gpu, x.to(cuda, torch.bfloat16))
    got = run(gpu, x.to(cuda, torch.bfloat16), edges.to(cuda, torch.float32), False)
    assert got[0].dtype == torch.bfloat16 and got[1].dtype == torch.bfloat16
    for name, g, w in (("out", got[0], want[0]), ("dx", got[1], want[1])):
        g, w = g.double().cpu(), w.double().cpu()
        err = float((g - w).abs().max()) / float(w.abs().max())
        print(f"  {name}: bf16 error {err:.2e} of the largest entry", flush=True)
        assert err <= 2e-2, f"{name}: bf16 error {err:.3e} of the largest entry"
    assert set(got[2]) == set(want[2])
    for k in want[2]:
        w, g = want[2][k].double(), got[2][k].double().cpu()
        if float(w.abs().max()) < 1e-6:
            continue
        err = float((g - w).norm()) / float(w.norm())
        assert err <= 2e-2, f"d{k}: bf16 relative error {err:.3e}"


def test_grouped_backward_reads_head_columns_in_place(cuda, monkeypatch):
    """The grouped factored backward reads each head's gradient rows as a view
    of the heads' (N, H, d_out) gradient (rows H d_out floats apart): every
    gradient is bit-identical to the call on contiguous copies."""
    import copy

    from gm_attention_amd import _native

    mhsa, x, edges = mhsa_case({0: 32, 1: 32, 2: 32}, 8, 16, 32, batch=2)
    gpu = copy.deepcopy(mhsa).to(cuda, torch.float32)
    e32 = edges.to(cuda, torch.float32)
    flat = x.float().to(cuda)
    probe = problems.normal(tuple(flat.shape), 11).to(cuda)
    seen = []
    real = _native.factored_backward_grouped

    def spy(g, *args, **kwargs):
        seen.append(g.is_contiguous())
        return real(g, *args, **kwargs)

    monkeypatch.setattr(_native, "factored_backward_grouped", spy)
    out, dx, dp = run_mhsa(gpu, flat, e32, probe, oracle=False)
    assert seen and not any(seen), "the heads' gradient rows were copied before the call"

    def contiguous(g, *args, **kwargs):
        return real(g.contiguous(), *args, **kwargs)

    monkeypatch.setattr(_native, "factored_backward_grouped", contiguous)
    out2, dx2, dp2 = run_mhsa(gpu, flat, e32, probe, oracle=False)
    assert torch.equal(out, out2) and torch.equal(dx, dx2)
    assert set(dp) == set(dp2)
    for name in dp:
        assert torch.equal(dp[name], dp2[name]), name
