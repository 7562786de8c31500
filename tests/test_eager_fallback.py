"""The layers' eager path (nn/eager_ops: what a call the fused predicates
decline runs, as the reference falls back to its eager layers at
nn/attention.py:880-886 and nn/convolution.py:297-308) on CPU tensors in
float64 against the oracle: batched and per-head MHSA, the general and the
depthwise convolution, the transformer block, the encoder hop and the value
kernel's per-edge readout, forward and every gradient; and
SO2DepthwiseKernel.forward's per-edge messages."""

import math

import pytest
import torch

import problems
from gm_attention_amd.nn import eager_ops
from gm_attention_amd.nn.attention import SO2MHSA
from gm_attention_amd.nn.blocks import EquiEncode, SO2TransformerBlock
from gm_attention_amd.nn.convolution import SO2Convolution
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import modules

D64 = torch.float64


def _grads(module, leaf, out, seed=7):
    probe = problems.normal(out.shape, seed)
    module.zero_grad(set_to_none=True)
    (out * probe).sum().backward()
    return leaf.grad.clone(), {n: p.grad.clone() for n, p in module.named_parameters() if p.grad is not None}


def _compare(got, want, tol=1e-10):
    torch.testing.assert_close(got[0], want[0], rtol=tol, atol=tol)
    torch.testing.assert_close(got[1], want[1], rtol=tol, atol=tol)
    assert set(got[2]) == set(want[2])
    for name in want[2]:
        torch.testing.assert_close(got[2][name], want[2][name], rtol=tol, atol=tol, msg=name)


def _run(module, ft, flat, edges, oracle_fn):
    results = []
    for use_oracle in (False, True):
        leaf = flat.clone().requires_grad_(True)
        if use_oracle:
            out = modules.flat(oracle_fn(module, dict(SO2FeatureField.from_flat(ft, leaf).coefficients), edges))
        else:
            out = module(SO2FeatureField.from_flat(ft, leaf), edges).to_flat()
        results.append((out.detach(), *_grads(module, leaf, out)))
    return results


@pytest.mark.parametrize("batched", [True, False])
def test_mhsa_on_the_cpu_takes_the_eager_path(batched):
    edges = problems.discretization(10, 20).edge_geometry
    ft = SO2FieldType({0: 4, 1: 4, 2: 4})
    torch.manual_seed(0)
    mhsa = SO2MHSA(ft, 2, cutoff=problems.discretization(10, 20).coverage_radius, window="quartic", batched=batched,
                   dtype=D64)
    before = dict(eager_ops.calls)
    got, want = _run(mhsa, ft, problems.normal((edges.row_ptr.shape[0] - 1, ft.dimension), 1), edges,
                     modules.mhsa_forward)
    _compare(got, want)
    assert eager_ops.calls.get("softmax", 0) > before.get("softmax", 0)
    assert eager_ops.calls.get("factored", 0) > before.get("factored", 0)


@pytest.mark.parametrize("depthwise", [True, False])
def test_convolution_on_the_cpu_takes_the_eager_path(depthwise):
    disc = problems.discretization(10, 20)
    ft = SO2FieldType({0: 4, 1: 3, 2: 2})
    torch.manual_seed(1)
    conv = SO2Convolution(ft, ft, cutoff=disc.coverage_radius, depthwise=depthwise, n_radial_basis=4,
                          self_interaction="linear", normalize=depthwise, dtype=D64)
    got, want = _run(conv, ft, problems.normal((disc.n_nodes, ft.dimension), 2), disc.edge_geometry,
                     modules.conv_forward)
    _compare(got, want)


def test_transformer_block_on_the_cpu_takes_the_eager_path():
    disc = problems.discretization(10, 20)
    ft = SO2FieldType({0: 8, 1: 8, 2: 8})
    torch.manual_seed(2)
    block = SO2TransformerBlock(ft, 2, ffn_multiplier=2, cutoff=disc.coverage_radius, n_radial_basis=4,
                                attention_batched=True, dtype=D64)
    with torch.no_grad():
        for p in block.parameters():
            p.add_(0.1 * torch.randn_like(p))
    got, want = _run(block, ft, problems.normal((disc.n_nodes, ft.dimension), 3), disc.edge_geometry,
                     modules.block_forward)
    _compare(got, want)


def test_encoder_hop_on_the_cpu_takes_the_eager_path():
    from test_encode_gpu import levels

    h = levels()
    edges = h.down_edges[0]
    fin, fout = SO2FieldType({0: 2, 1: 2, 2: 2}), SO2FieldType({0: 5, 1: 3, 2: 4})
    torch.manual_seed(3)
    enc = EquiEncode(fin, fout, cutoff=1.5 * math.pi / 8, n_radial_basis=4, dtype=D64)
    got, want = _run(enc, fin, problems.normal((h.levels[0].n_nodes, fin.dimension), 4), edges,
                     lambda m, x, e: modules.encode_forward(m.integral, x, e))
    _compare(got, want)


def test_value_kernel_readout_and_depthwise_messages_on_edges():
    """The per-edge readout (SO2SteerableKernel.forward) and the depthwise
    kernel's per-edge messages on gathered fields against the oracle."""
    disc = problems.discretization(10, 20)
    edges = disc.edge_geometry
    ft = SO2FieldType({0: 3, 1: 2, 2: 2})
    torch.manual_seed(4)
    conv = SO2Convolution(ft, ft, cutoff=disc.coverage_radius, depthwise=False, n_radial_basis=4, dtype=D64)
    x = SO2FeatureField.from_flat(ft, problems.normal((disc.n_nodes, ft.dimension), 5))
    gathered = SO2FeatureField(ft, {f: t.index_select(0, edges.source_index) for f, t in x.coefficients.items()})
    got = conv.kernel(gathered, edges)
    want = modules.readout_messages(conv.kernel, x.coefficients, edges.source_index, edges.distances,
                                    edges.angular_phases, edges.transport_phases)
    for f in want:
        torch.testing.assert_close(got[f], want[f], rtol=1e-11, atol=1e-12)
    dw = SO2Convolution(ft, ft, cutoff=disc.coverage_radius, depthwise=True, n_radial_basis=4, dtype=D64).kernel
    got = dw(gathered, edges)
    want = modules.depthwise_layer_messages(dw, x.coefficients, edges)
    for f in want:
        torch.testing.assert_close(got[f], want[f], rtol=1e-11, atol=1e-12)


@pytest.mark.parametrize("readout", [False, True])
def test_cpu_switch_value_runs_cpu_tensors(monkeypatch, readout):
    """``GM_FUSED_{ATTENTION,FACTORED,PAIRS}=cpu`` means "on everywhere" in the
    reference (fused_attention.py:43-60, fused_factored.py:50-51,
    fused_pairs.py:39-40): CPU tensors must run, not raise.  This build has no
    CPU driver, so under ``"cpu"`` they take the eager path, in both value
    orders (``GM_FACTORED_KERNEL``: factored, or the per-edge readout the
    fused pair terms serve on the GPU)."""
    from gm_attention_amd.nn import fused_attention, fused_factored, fused_pairs, kernels

    for mod in (fused_attention, fused_factored, fused_pairs):
        monkeypatch.setattr(mod, "MODE", "cpu")
    monkeypatch.setattr(kernels, "FACTORED", not readout)
    disc = problems.discretization(10, 20)
    ft = SO2FieldType({0: 4, 1: 4, 2: 4})
    torch.manual_seed(5)
    mhsa = SO2MHSA(ft, 2, cutoff=disc.coverage_radius, window="hard", batched=True, dtype=D64)
    flat = problems.normal((disc.n_nodes, ft.dimension), 6)
    got, want = _run(mhsa, ft, flat, disc.edge_geometry, modules.mhsa_forward)
    _compare(got, want)
    for depthwise in (True, False):
        conv = SO2Convolution(ft, ft, cutoff=disc.coverage_radius, depthwise=depthwise, n_radial_basis=4, dtype=D64)
        got, want = _run(conv, ft, flat, disc.edge_geometry, modules.conv_forward)
        _compare(got, want)
    # the predicates decline CPU tensors under "cpu" and admit device tensors
    x = SO2FeatureField.from_flat(ft, flat)
    assert not fused_attention.softmax_enabled(mhsa, flat, disc.edge_geometry)
    assert not fused_attention.enabled_depthwise(conv, flat, disc.edge_geometry)
    assert not fused_pairs.enabled(mhsa.heads[0].value, x, disc.edge_geometry)
    assert fused_factored.declined(mhsa.heads[0].value, x, disc.edge_geometry) != ""
