"""The attention layers (SO2MHSA batched and per head, SO2Attention chunked) on
the HIP path against the oracle (oracle.modules.mhsa_forward: the
reference's eager head-by-head attention in float64), with the input field's
and every parameter's gradient; and gauge equivariance under random frame
rotations (the reference's pattern: tests/nn/test_attention_batched.py:105).
"""

import math

import pytest
import torch

import problems
from gm_attention_amd.discretization.discretization import SphericalDiscretization
from gm_attention_amd.discretization.frames import build_tangent_frames, rotate_tangent_frames
from gm_attention_amd.discretization.grid import build_equiangular_grid
from gm_attention_amd.nn.attention import SO2Attention, SO2MHSA
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import modules

pytestmark = pytest.mark.gpu


def close(got, want, dtype, name, reduction=False, scaled=False):
    """float64: 1e-10.  float32: |got - want| <= 1e-5 |want| + 1e-6
    elementwise, the north star's bound; with ``scaled`` the absolute term is
    1e-6 max(1, max|want|), for the tests whose inputs reach entries of 5 to
    70, where the long float32 sums that cancel leave absolute errors of about
    1e-6 of the largest entry on entries near zero (each such caller says what
    it measured against the unscaled bound).  A parameter gradient
    (``reduction``, a sum over every edge or node) instead within 1e-5 of its
    norm and 1e-5 of its largest entry."""
    want, got = want.detach().double().cpu(), got.detach().double().cpu()
    if dtype == torch.float32 and reduction:
        err = (got - want).norm() / want.norm().clamp_min(1e-30)
        peak = (got - want).abs().max() / want.abs().max().clamp_min(1e-30)
        if want.abs().max() < 1e-6:  # an identically zero gradient (e.g. a key bias under the softmax)
            assert got.abs().max() <= 1e-5, f"{name}: {got.abs().max():.3e} where the gradient vanishes"
        else:
            assert err <= 1e-5 and peak <= 1e-5, f"{name}: relative error {err:.3e}, peak {peak:.3e}"
        return
    if dtype == torch.float64:
        torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10, msg=lambda m, name=name: f"{name}: {m}")
    else:
        problems.report_strict(got, want, name)
        scale = max(1.0, float(want.abs().max())) if scaled else 1.0
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6 * scale, msg=lambda m, name=name: f"{name}: {m}")


def build(field, heads, window, batch, nlat=10, nlon=20, seed=0):
    disc = problems.discretization(nlat, nlon)
    edges = disc.edge_geometry.tile(batch, n_sources=disc.n_nodes) if batch > 1 else disc.edge_geometry
    torch.manual_seed(seed)
    mhsa = SO2MHSA(SO2FieldType(field), heads, cutoff=disc.coverage_radius, window=window, dtype=torch.float64)
    n = edges.row_ptr.shape[0] - 1
    x = problems.normal((n, mhsa.field_type_in.dimension), seed + 1)
    return mhsa, x, edges


def run(module, flat, edges, probe, *, oracle=False, chunk=None, tolerance=None):
    leaf_flat = flat.clone().requires_grad_(True)
    x = SO2FeatureField.from_flat(module.field_type_in, leaf_flat)
    leaf = x.coefficients
    module.zero_grad(set_to_none=True)
    if oracle:
        out = modules.flat(modules.mhsa_forward(module, leaf, edges, tolerance))
    elif chunk is not None:
        out = module.forward_chunked(x, edges, chunk_size=chunk).to_flat()
    else:
        out = module(x, edges).to_flat()
    (out * probe.to(out.device, out.dtype)).sum().backward()
    return out.detach(), {"x": leaf_flat.grad}, {n: p.grad for n, p in module.named_parameters()
                                                  if p.grad is not None}


CASES = [({0: 8, 1: 8, 2: 8}, 4, "hard", 2), ({0: 4, 1: 4, 2: 4}, 2, "quartic", 1), ({0: 6, 1: 3}, 3, "hard", 1),
         # heads of {0: 8, 1: 8, 2: 8}: float32 runs the grouped kernels on two shares of each head's copies
         ({0: 16, 1: 16, 2: 16}, 2, "hard", 1)]


@pytest.mark.parametrize("batched", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("case", CASES)
def test_mhsa_matches_the_oracle(case, dtype, batched, cuda):
    field, heads, window, batch = case
    print(f"mhsa {case} {dtype} batched={batched}", flush=True)
    mhsa, x, edges = build(field, heads, window, batch)
    mhsa.batched = batched
    probe = problems.normal(x.shape, 7)
    if dtype == torch.float32:  # the oracle sees the same rounded parameters, inputs and geometry
        mhsa.load_state_dict({k: v.float().double() for k, v in mhsa.state_dict().items()})
        x = x.float().double()
        edges_o = edges.to(None, torch.float32).to(None, torch.float64)
    else:
        edges_o = edges
    # the hard window admits an edge by the tested dtype's slack (1e-5 in float32), as the fused path does
    want = run(mhsa, x, edges_o, probe, oracle=True, tolerance=1e-5 if dtype == torch.float32 else None)
    gpu = SO2MHSA(mhsa.field_type_in, heads, cutoff=mhsa.cutoff, window=window, batched=batched, dtype=dtype,
                  device=cuda)
    gpu.load_state_dict({k: v.to(dtype) for k, v in mhsa.state_dict().items()})
    got = run(gpu, x.to(cuda, dtype), edges.to(cuda, dtype), probe)
    close(got[0], want[0], dtype, "out")
    for f in want[1]:
        close(got[1][f], want[1][f], dtype, f"dx[{f}]")
    assert set(got[2]) == set(want[2])
    for n in want[2]:
        close(got[2][n], want[2][n], dtype, f"d{n}", reduction=True)


def test_mhsa_float32_with_blocks_dealt_in_chunks_matches_the_oracle(cuda):
    """Two samples of a 24x48 grid: enough blocks (576 for the softmax and the
    aggregate, 2304 groups) that the kernels deal them to the XCDs in 32-block
    chunks, which they do here because two samples make the contiguous eighths
    uneven (the polar quarters hold most edges); float32 batched against the
    oracle, every gradient."""
    field, heads, window, batch = {0: 8, 1: 8, 2: 8}, 2, "hard", 2
    mhsa, x, edges = build(field, heads, window, batch, nlat=24, nlon=48)
    assert edges.row_ptr.shape[0] - 1 == 2 * 24 * 48
    mhsa.batched = True
    probe = problems.normal(x.shape, 7)
    mhsa.load_state_dict({k: v.float().double() for k, v in mhsa.state_dict().items()})
    x = x.float().double()
    want = run(mhsa, x, edges.to(None, torch.float32).to(None, torch.float64), probe, oracle=True, tolerance=1e-5)
    gpu = SO2MHSA(mhsa.field_type_in, heads, cutoff=mhsa.cutoff, window=window, batched=True, dtype=torch.float32,
                  device=cuda)
    gpu.load_state_dict({k: v.float() for k, v in mhsa.state_dict().items()})
    got = run(gpu, x.to(cuda, torch.float32), edges.to(cuda, torch.float32), probe)
    close(got[0], want[0], torch.float32, "out")
    for f in want[1]:
        close(got[1][f], want[1][f], torch.float32, f"dx[{f}]")
    assert set(got[2]) == set(want[2])
    for n in want[2]:
        close(got[2][n], want[2][n], torch.float32, f"d{n}", reduction=True)


def test_chunked_equals_whole(cuda):
    mhsa, x, edges = build({0: 8, 1: 8, 2: 8}, 4, "hard", 2)
    gpu = mhsa.to(cuda)
    gpu.train()
    e = edges.to(cuda, torch.float64)
    probe = problems.normal(x.shape, 7)
    whole = run(gpu, x.to(cuda), e, probe)
    chunked = run(gpu, x.to(cuda), e, probe, chunk=37)
    close(chunked[0], whole[0], torch.float64, "out")
    for f in whole[1]:
        close(chunked[1][f], whole[1][f], torch.float64, f"dx[{f}]")
    for n in whole[2]:
        close(chunked[2][n], whole[2][n], torch.float64, f"d{n}")


@pytest.mark.parametrize("window", ["hard", "quartic"])
def test_gauge_equivariance_under_random_frame_rotations(window, cuda):
    """Rotating every node's frame by theta_i and transforming the input by
    rho(r_{-theta}) transforms the output the same way."""
    nlat, nlon = 10, 20
    grid = build_equiangular_grid(nlat, nlon)
    cutoff = 3.0 * math.pi / (nlat - 1)
    frames = build_tangent_frames(grid.nodes)
    theta = torch.rand(grid.n_nodes, dtype=torch.float64, generator=torch.Generator().manual_seed(4)) * 2 * math.pi
    base = SphericalDiscretization.from_grid(grid, cutoff, frames=frames)
    turned = SphericalDiscretization.from_grid(grid, cutoff, frames=rotate_tangent_frames(frames, theta))
    assert torch.equal(base.edge_geometry.edge_index, turned.edge_geometry.edge_index)
    torch.manual_seed(0)
    field = SO2FieldType({0: 8, 1: 8, 2: 8})
    mhsa = SO2MHSA(field, 4, cutoff=cutoff, window=window, batched=True, dtype=torch.float64, device=cuda)
    x = SO2FeatureField.from_flat(field, problems.normal((grid.n_nodes, field.dimension), 1).to(cuda))
    with torch.no_grad():
        y = mhsa(x, base.edge_geometry.to(cuda, torch.float64))
        y_turned = mhsa(x.gauge_transform(theta.to(cuda)), turned.edge_geometry.to(cuda, torch.float64))
    expected = y.gauge_transform(theta.to(cuda))
    torch.testing.assert_close(y_turned.to_flat(), expected.to_flat(), rtol=1e-9, atol=1e-9)
    # and the output is not trivially invariant
    assert float((y.to_flat() - expected.to_flat()).abs().max()) > 1e-3


def test_single_head_attention_matches_the_oracle(cuda):
    mhsa, x, edges = build({0: 4, 1: 4, 2: 4}, 1, "quartic", 1)
    head = mhsa.heads[0]
    probe = problems.normal((x.shape[0], head.field_type_out.dimension), 3)

    # the head's type and score scale derived by the oracle from the input type and head count
    fin = mhsa.field_type_in
    attn = modules.head_type({f: fin.multiplicity(f) for f in fin.frequencies}, len(mhsa.heads))

    def run_head(module, flat, eds, oracle):
        xx = SO2FeatureField.from_flat(mhsa.field_type_in, flat.clone().requires_grad_(True))
        module.zero_grad(set_to_none=True)
        if oracle:
            q = modules.linear(module.query, xx.coefficients, attn)
            k = modules.linear(module.key, xx.coefficients, attn)
            alpha = modules.softmax_weights(q, k, eds, module.cutoff, module.window, 1, modules.score_scale(attn))[:, 0]
            msgs = modules.readout_messages(module.value, xx.coefficients, eds.source_index, eds.distances,
                                            eds.angular_phases, eds.transport_phases)
            out = torch.segment_reduce(alpha.unsqueeze(-1) * modules.flat(msgs), "sum", offsets=eds.row_ptr, axis=0)
        else:
            out = module(xx, eds).to_flat()
        (out * probe.to(out.device)).sum().backward()
        return out.detach(), {n: p.grad for n, p in module.named_parameters() if p.grad is not None}

    want = run_head(head, x, edges, True)
    gpu = SO2Attention(mhsa.field_type_in, head.field_type_attn, head.field_type_out, cutoff=head.cutoff,
                       window="quartic", dtype=torch.float64, device=cuda)
    gpu.load_state_dict(head.state_dict())
    got = run_head(gpu, x.to(cuda), edges.to(cuda, torch.float64), False)
    close(got[0], want[0], torch.float64, "out")
    for n in want[1]:
        close(got[1][n], want[1][n], torch.float64, f"d{n}")


def test_mhsa_float32_on_the_run_kernels_matches_the_oracle(cuda, monkeypatch):
    """The batched layer with the grouped kernels switched off (every head on
    the mix-run kernels), float32, against the oracle."""
    monkeypatch.setenv("GM_FACTORED_GROUPED", "0")
    test_mhsa_matches_the_oracle(CASES[0], torch.float32, True, cuda)


def test_mhsa_float32_with_largest_first_groups_matches_the_oracle(cuda, monkeypatch):
    """The grouped kernels launched in largest-first group order (an explicit
    group_order permutation), float32, against the oracle."""
    monkeypatch.setenv("GM_FACTORED_LPT", "1")
    test_mhsa_matches_the_oracle(CASES[0], torch.float32, True, cuda)


LANE_CASES = [({0: 8, 1: 8, 2: 8}, 2, "hard", 2), ({0: 16, 1: 8, 2: 8}, 2, "quartic", 1), ({0: 8, 1: 8}, 2, "hard", 1)]


@pytest.mark.parametrize("form", ["fixed", "runtime", "generic"])
@pytest.mark.parametrize("case", LANE_CASES)
def test_mhsa_float32_on_the_lane_kernels_matches_the_oracle(case, form, cuda, monkeypatch):
    """Heads with four (or eight) copies per frequency on the grouped kernels'
    lane-owned output form: with compile-time slot words where the plan has
    them ("fixed"), with the words as kernel arguments
    (GM_FACTORED_STATIC=0), and on the generic grouped form
    (GM_FACTORED_LANES=0); float32 batched, against the oracle."""
    monkeypatch.setenv("GM_FACTORED_STATIC", "0" if form == "runtime" else "1")
    monkeypatch.setenv("GM_FACTORED_LANES", "0" if form == "generic" else "1")
    test_mhsa_matches_the_oracle(case, torch.float32, True, cuda)


@pytest.mark.parametrize("case", LANE_CASES)
@pytest.mark.parametrize("form", ["fixed", "runtime"])
def test_mhsa_float32_lanes_with_the_trunk_in_the_kernels_matches_the_oracle(case, form, cuda, monkeypatch):
    """The lane-owned kernels evaluating each head's radial trunk themselves
    (GM_FACTORED_TRUNK=1: no h tensor; the trunk's gradient from the dh they
    write), float32 batched, against the oracle; the plans take the lane form."""
    from gm_attention_amd.nn import fused_factored

    monkeypatch.setattr(fused_factored, "FUSED_TRUNK", True)
    monkeypatch.setenv("GM_FACTORED_STATIC", "0" if form == "runtime" else "1")
    mhsa, _, _ = build(case[0], case[1], "hard", 1)
    kernel = mhsa.heads[0].value
    hp = fused_factored.heads_plan(kernel)
    ok, pa, pt = fused_factored.grouped_eligible(hp, torch.float32, 17)
    assert ok and fused_factored._lanes_apply(kernel, hp, pa, pt)
    test_mhsa_matches_the_oracle(case, torch.float32, True, cuda)


def test_mhsa_with_the_fused_switches_off_takes_the_eager_path_on_the_gpu(cuda, monkeypatch):
    """GM_FUSED_ATTENTION=0, GM_FUSED_FACTORED=0 (the reference's defaults):
    device tensors run the eager path (nn/eager_ops, as the reference's
    layers fall back at attention.py:880-886), float64, against the oracle."""
    from gm_attention_amd.nn import eager_ops, fused_attention, fused_factored

    monkeypatch.setattr(fused_attention, "MODE", "0")
    monkeypatch.setattr(fused_factored, "MODE", "0")
    before = eager_ops.calls.get("softmax", 0)
    test_mhsa_matches_the_oracle(CASES[0], torch.float64, True, cuda)
    assert eager_ops.calls.get("softmax", 0) > before


@pytest.mark.parametrize("case", [({0: 8, 1: 8, 2: 8}, 2, "hard", 2), ({0: 16, 1: 16, 2: 16}, 2, "quartic", 2),
                                  ({0: 8, 1: 8}, 2, "hard", 1)])
def test_staged_mixes_backward_equals_the_register_staged_one(case, cuda, monkeypatch):
    """The lane-owned backward with its mixes staged by direct-to-LDS loads
    (the default for the compiled-in slot tables) against the same kernel
    staging them by register loads and LDS writes (GM_FACTORED_ZDMA=0): the
    same tiles in the same order, so every output and gradient agrees to
    float32 rounding (the two instantiations' instruction selection may fuse
    a multiply-add differently), on a 24x48 grid whose groups span one to
    many tiles; the second case's heads run as two shares, the second adding
    into dh and dweights."""
    field, heads, window, batch = case
    mhsa, x, edges = build(field, heads, window, batch, nlat=24, nlon=48)
    mhsa = mhsa.to(cuda, torch.float32)
    probe = problems.normal((x.shape[0], mhsa.field_type_in.dimension), 5)
    results = []
    for stream in ("1", "0"):
        monkeypatch.setenv("GM_FACTORED_ZDMA", stream)
        print(f"staged-mix backward {case} GM_FACTORED_ZDMA={stream}", flush=True)
        results.append(run(mhsa, x.to(cuda, torch.float32), edges.to(cuda, torch.float32), probe))

    def near(got, want, name):
        scale = float(want.abs().max())
        err = float((got - want).abs().max())
        assert err <= 1e-6 * scale, f"{name}: {err:.3e} of {scale:.3e}"

    near(results[0][0], results[1][0], "out")
    near(results[0][1]["x"], results[1][1]["x"], "x")
    assert set(results[0][2]) == set(results[1][2])
    scale = max(float(g.abs().max()) for g in results[1][2].values())
    for n in results[1][2]:  # sums over every edge or node
        if n.endswith("key.bias"):
            # the softmax is invariant to a key bias: its gradient vanishes in exact arithmetic and holds
            # float32 rounding noise in both forms (up to about 1e-6 with the fp32 matrix products)
            for r in results:
                assert float(r[2][n].abs().max()) <= 1e-5 * scale, f"{n}: {float(r[2][n].abs().max()):.3e}"
            continue
        close(results[0][2][n], results[1][2][n], torch.float32, n, reduction=True)
