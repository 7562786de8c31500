"""The C5 stage's model (nn/segformer.GmSegformer: restrictions, attention +
Mix-FFN blocks per level, convolution readouts, the fusion decoder and the
head) on the CPU in float64 against the oracle's composition
(oracle.modules.segformer_forward, which restates the reference's
experiments/stanford_2d3ds/model.py from the oracle's layer functions), with
the input's and every parameter's gradient; the low-pass restriction's
closed forms; and the stage hierarchy's and the model's argument checks."""

import math

import pytest
import torch

import problems
from gm_attention_amd.nn.segformer import (GmSegformer, LowPassRestriction, SO2DropPath, build_stage_hierarchy,
                                           stage_radii)
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import modules

D64 = torch.float64
IMG, STAGES = (12, 24), ((8, 16), (5, 10))


def small_model(types, heads, radii, dtype=D64, device=None, seed=0, **kw):
    torch.manual_seed(seed)
    model = GmSegformer(in_channels=4, num_classes=13, stage_field_types=[SO2FieldType(t) for t in types],
                        heads=heads, depths=(1, 1), merge_cutoffs=radii.merge, attention_cutoffs=radii.attention,
                        mix_cutoffs=radii.mix, interpolate_cutoffs=radii.interpolate, readout_cutoffs=radii.readout,
                        readout_channels=(8, 8), decoder_channels=8, n_radial_basis=4, dtype=dtype, device=device,
                        **kw)
    with torch.no_grad():  # nonzero biases and gains away from one everywhere
        for p in model.parameters():
            p.add_(0.05 * torch.randn_like(p))
    return model


def run(model, x0, hierarchy, probe, oracle=False, tolerance=None, messages="readout"):
    leaf = x0.clone().requires_grad_(True)
    model.zero_grad(set_to_none=True)
    if oracle:
        out = modules.segformer_forward(model, leaf, hierarchy, tolerance, messages)
    else:
        out = model(SO2FeatureField(model.input_field_type, {0: leaf}), hierarchy)[0]
    (out * probe.to(out.device, out.dtype)).sum().backward()
    return out.detach(), leaf.grad, {n: p.grad for n, p in model.named_parameters() if p.grad is not None}


def test_model_matches_the_oracle_composition():
    radii = stage_radii(STAGES)
    h = build_stage_hierarchy(IMG, STAGES, radii).tile(2)
    model = small_model([{0: 8, 1: 8, 2: 8}, {0: 8, 1: 4, 2: 8}], (2, 4), radii, normalized_mix=True,
                        normalized_readout=True)
    model.eval()
    n0 = h.levels[0].n_nodes
    x0 = torch.rand(n0, 4, generator=torch.Generator().manual_seed(1), dtype=D64)
    probe = problems.normal((n0, 13), 2)
    got = run(model, x0, h, probe)
    want = run(model, x0, h, probe, oracle=True, messages="factored")
    torch.testing.assert_close(got[0], want[0], rtol=1e-10, atol=1e-11)
    torch.testing.assert_close(got[1], want[1], rtol=1e-10, atol=1e-11)
    assert set(got[2]) == set(want[2])
    for name in want[2]:
        torch.testing.assert_close(got[2][name], want[2][name], rtol=1e-9, atol=1e-11, msg=name)


def test_low_pass_reproduces_constants_and_a_brute_force_sum():
    """Scalar constants pass unchanged (the denominator is the numerator's
    weight sum); on a tiny hop the restriction equals the double loop."""
    radii = stage_radii(STAGES)
    h = build_stage_hierarchy(IMG, STAGES, radii)
    edges = h.up_edges[0]
    lp = LowPassRestriction(SO2FieldType({0: 3}), cutoff=radii.interpolate[0])
    n_src = h.levels[1].n_nodes
    const = torch.full((n_src, 3), 2.5, dtype=D64)
    out = lp(SO2FeatureField(lp.field_type, {0: const}), edges)[0]
    covered = torch.segment_reduce((edges.distances < lp.cutoff).to(D64), "sum", offsets=edges.row_ptr) > 0
    assert bool(covered.all())
    torch.testing.assert_close(out, torch.full_like(out, 2.5), rtol=1e-14, atol=1e-14)
    x = problems.normal((n_src, 3), 5)
    got = lp(SO2FeatureField(lp.field_type, {0: x}), edges)[0]
    rp, src, d, q = edges.row_ptr.tolist(), edges.source_index.tolist(), edges.distances.tolist(), \
        edges.tangent_quadrature_weights.tolist()
    for i in range(0, len(rp) - 1, 37):
        num, den = [0.0, 0.0, 0.0], 0.0
        for e in range(rp[i], rp[i + 1]):
            w = max(0.0, 1.0 - (d[e] / lp.cutoff) ** 2) ** 2 * q[e]
            den += w
            for c in range(3):
                num[c] += w * float(x[src[e], c])
        want = torch.tensor([v / max(den, 1e-12) for v in num], dtype=D64)
        torch.testing.assert_close(got[i], want, rtol=1e-12, atol=1e-13)
    assert torch.allclose(modules.low_pass(lp, x, edges), got, rtol=1e-13, atol=1e-14)


def test_drop_path_is_the_identity_in_evaluation_and_rescales_in_training():
    drop = SO2DropPath(0.25)
    ft = SO2FieldType({0: 2, 1: 1})
    x = SO2FeatureField.from_flat(ft, torch.ones(5, ft.dimension, dtype=D64))
    drop.eval()
    assert drop(x) is x
    drop.train()
    torch.manual_seed(0)
    seen = {float(drop(x).to_flat()[0, 0]) for _ in range(64)}
    assert seen == {0.0, 1.0 / 0.75}
    with pytest.raises(ValueError, match="0 <= p < 1"):
        SO2DropPath(1.0)


def test_model_and_hierarchy_argument_checks():
    radii = stage_radii(STAGES)
    with pytest.raises(ValueError, match="one entry per stage"):
        GmSegformer(in_channels=4, num_classes=13, stage_field_types=[SO2FieldType({0: 4})], heads=(1, 1),
                    depths=(1,), merge_cutoffs=radii.merge[:1], attention_cutoffs=radii.attention[:1],
                    mix_cutoffs=radii.mix[:1], interpolate_cutoffs=radii.interpolate[:1],
                    readout_cutoffs=radii.readout[:1], readout_channels=(4,))
    with pytest.raises(ValueError, match="must be positive"):
        stage_radii(STAGES, mix_rows=0.0)
    assert math.isclose(radii.attention[1], 3 * math.pi / 4)
    h = build_stage_hierarchy(IMG, STAGES, radii)
    assert len(h.lateral_edges) == 1 and h.depth == 2
    model = small_model([{0: 4, 1: 4}, {0: 4, 1: 4}], (1, 1), radii)
    deep = build_stage_hierarchy(IMG, ((8, 16), (6, 12), (5, 10)), stage_radii(((8, 16), (6, 12), (5, 10))))
    x = SO2FeatureField(model.input_field_type, {0: torch.zeros(deep.levels[0].n_nodes, 4, dtype=D64)})
    with pytest.raises(ValueError, match="3 hops, the model 2 stages"):
        model(x, deep)
