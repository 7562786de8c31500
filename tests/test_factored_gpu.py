"""The HIP factored kernel (fused_factored.Factored / FactoredAggregate and the
kernel's forward_factored_aggregated) against the oracle on the same inputs.

* op level: oracle.eager.factored_rows / factored_aggregate in float64 on the
  op's inputs rounded to the tested dtype, gradients by autograd;
* module level: the product kernel on cuda against the per-edge readout
  (oracle.modules.readout_messages) weighted and segment-summed, float64 on
  the CPU, for the output, the input field's and every parameter's gradient.

Tolerances: float64 1e-10; float32 rtol 1e-5 with atol 1e-6 times the
tensor's largest magnitude (a sum of K products per entry rounds at the
scale of the tensor, not of the entry).
"""

import pytest
import torch

import problems
from gm_attention_amd.nn import fused_factored
from gm_attention_amd.nn.kernels import SO2SteerableKernel
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
from oracle import eager, modules

pytestmark = pytest.mark.gpu

CONFIGS = [
    ({0: 32, 1: 32, 2: 32}, {0: 4, 1: 4, 2: 4}, True),  # one head of the 8-head attention at {0:32,1:32,2:32}
    ({0: 16, 1: 16, 2: 16}, {0: 8, 1: 8, 2: 8}, True),
    ({0: 4, 1: 3, 2: 2}, {0: 3, 1: 2, 2: 2}, False),
    ({0: 4}, {0: 5, 1: 3, 2: 2}, True),
    ({0: 4, 1: 3, 2: 2}, {0: 3}, True),
    ({1: 3}, {2: 2}, True),
    ({0: 18, 1: 6, 2: 6}, {0: 24, 1: 8, 2: 8}, True),
    ({0: 24, 1: 8, 2: 8}, {0: 32, 1: 8, 2: 8}, True),  # 2 wc + wr = 320, the widest admitted
]


def close(got, want, dtype, name, reduction=False):
    """float64: 1e-10.  float32: |got - want| <= 1e-5 |want| + 1e-6 max|want|
    elementwise; a parameter gradient (``reduction``, a sum over every edge or
    node) instead within 1e-5 of its norm and 1e-5 of its largest entry."""
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
        scale = max(1.0, float(want.abs().max())) if want.numel() else 1.0
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6 * scale, msg=lambda m, name=name: f"{name}: {m}")


def setup(fin, fout, bias, dtype, nlat=12, nlon=24, batch=1, seed=0):
    disc = problems.discretization(nlat, nlon)
    edges = disc.edge_geometry.tile(batch, n_sources=disc.n_nodes) if batch > 1 else disc.edge_geometry
    torch.manual_seed(seed)
    kernel = SO2SteerableKernel(SO2FieldType(fin), SO2FieldType(fout), cutoff=disc.coverage_radius, n_radial_basis=8,
                                radial_hidden_features=[16], bias=bias, dtype=torch.float64)
    n = edges.row_ptr.shape[0] - 1
    x = SO2FeatureField.from_flat(kernel.field_type_in, problems.normal((n, kernel.field_type_in.dimension), seed + 1))
    return kernel, x, edges


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("fin,fout,bias", CONFIGS)
def test_the_op_matches_the_oracle(fin, fout, bias, dtype, cuda):
    print(f"factored op {fin}->{fout} {dtype}", flush=True)
    kernel, x, edges = setup(fin, fout, bias, torch.float64)
    with torch.no_grad():
        i = fused_factored.inputs(kernel, x, edges, None)
    p = i.plan
    rnd = lambda t: t.to(dtype).double()
    h64, zc64, zr64 = rnd(i.h), rnd(i.zc), rnd(i.zr)
    ang64, tr64, rho64 = rnd(i.angular), rnd(i.transport), rnd(i.rho)
    w64 = rnd(torch.rand(edges.n_edges, dtype=torch.float64, generator=torch.Generator().manual_seed(3)))
    g64 = rnd(problems.normal((edges.row_ptr.shape[0] - 1, p.d_out), 4))
    ge64 = rnd(problems.normal((edges.n_edges, p.d_out), 5))
    rows_desc = [b.row() for b in p.blocks]
    # oracle
    leaves = [t.clone().requires_grad_(True) for t in (h64, zc64, zr64, w64)]
    rows_o = eager.factored_rows(*leaves[:3], ang64, tr64, rho64, rows_desc, i.source, p.d_out)
    agg_o = eager.factored_aggregate(rows_o, leaves[3], edges.row_ptr)
    grads_rows_o = torch.autograd.grad(rows_o, leaves[:3], ge64, retain_graph=True, allow_unused=True,
                                       materialize_grads=True)
    grads_agg_o = torch.autograd.grad(agg_o, leaves, g64, allow_unused=True, materialize_grads=True)
    # HIP
    dev = lambda t: t.to(dtype).to(cuda)
    order, ptr, gsrc = (t.to(cuda) for t in fused_factored.source_groups(i.source))
    consts = (dev(ang64), dev(tr64), dev(rho64), i.desc.to(cuda), i.source.to(cuda))
    h, zc, zr, w = (dev(t).requires_grad_(True) for t in (h64, zc64, zr64, w64))
    rows = fused_factored.Factored.apply(h, zc, zr, *consts, order, ptr, gsrc, p.d_out, p.max_bm)
    grads_rows = torch.autograd.grad(rows, (h, zc, zr), dev(ge64), allow_unused=True, materialize_grads=True)
    agg = fused_factored.FactoredAggregate.apply(h, zc, zr, w, *consts, edges.target_index.to(cuda),
                                                 edges.row_ptr.to(cuda), order, ptr, gsrc, p.d_out, p.max_bm)
    grads_agg = torch.autograd.grad(agg, (h, zc, zr, w), dev(g64), allow_unused=True, materialize_grads=True)
    close(rows, rows_o, dtype, "rows")
    close(agg, agg_o, dtype, "aggregate")
    for name, a, b in zip(("dh", "dzc", "dzr"), grads_rows, grads_rows_o):
        close(a, b, dtype, name)
    for name, a, b in zip(("dh", "dzc", "dzr", "dweights"), grads_agg, grads_agg_o):
        close(a, b, dtype, "aggregated " + name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("fin,fout,bias", CONFIGS[:3])
def test_the_kernel_matches_the_readout(fin, fout, bias, dtype, cuda):
    """forward_factored_aggregated on the GPU (node products, trunk, fused op)
    against the per-edge readout weighted and segment-summed, with the input
    field's and every parameter's gradient."""
    print(f"factored kernel {fin}->{fout} {dtype}", flush=True)
    kernel, x, edges = setup(fin, fout, bias, torch.float64, nlat=10, nlon=20, batch=2)
    weights = torch.rand(edges.n_edges, dtype=torch.float64, generator=torch.Generator().manual_seed(8))
    probe = problems.normal((edges.row_ptr.shape[0] - 1, kernel.field_type_out.dimension), 9)

    def run(kern, field, eds, w, fused):
        field = SO2FeatureField(field.field_type, {f: v.clone().requires_grad_(True)
                                                   for f, v in field.coefficients.items()})
        w = w.clone().requires_grad_(True)
        kern.zero_grad(set_to_none=True)
        if fused:
            out = kern.forward_factored_aggregated(field, eds, w).to_flat()
        else:
            msgs = modules.readout_messages(kern, field.coefficients, eds.source_index, eds.distances,
                                            eds.angular_phases, eds.transport_phases)
            flat = SO2FeatureField(kern.field_type_out, msgs).to_flat()
            out = torch.segment_reduce(w.unsqueeze(-1) * flat, "sum", offsets=eds.row_ptr, axis=0)
        (out * probe.to(out.device, out.dtype)).sum().backward()
        return (out.detach(), {f: field[f].grad for f in field.frequencies},
                {n: p.grad for n, p in kern.named_parameters() if p.grad is not None}, w.grad)

    want = run(kernel, x, edges, weights, fused=False)
    gpu_kernel = SO2SteerableKernel(kernel.field_type_in, kernel.field_type_out, cutoff=kernel.radial_basis.cutoff,
                                    n_radial_basis=8, radial_hidden_features=[16], bias=bias, dtype=dtype, device=cuda)
    gpu_kernel.load_state_dict({k: v.to(dtype) for k, v in kernel.state_dict().items()})
    got = run(gpu_kernel, x.to(cuda, dtype), edges.to(cuda, dtype), weights.to(cuda, dtype), fused=True)
    if dtype == torch.float32:  # compare with the oracle on the same rounded parameters and inputs
        kernel.load_state_dict({k: v.to(dtype).double() for k, v in kernel.state_dict().items()})
        want = run(kernel, x.to(dtype=dtype).to(dtype=torch.float64), edges.to(None, dtype).to(None, torch.float64),
                   weights.to(dtype).double(), fused=False)
    close(got[0], want[0], dtype, "out")
    for f in want[1]:
        close(got[1][f], want[1][f], dtype, f"dx[{f}]")
    assert set(got[2]) == set(want[2]) and got[2]
    for n in want[2]:
        close(got[2][n], want[2][n], dtype, f"d{n}", reduction=True)
    close(got[3], want[3], dtype, "dweights")
