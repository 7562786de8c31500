"""Benchmark of gm-attention's fused hot path on one MI355X.

Default workload (the north-star shape): one ``SO2MHSA(batched=True)`` layer,
forward + backward (input and every parameter gradient), on the equiangular
256x512 grid, batch 4 (a 4-fold disjoint union: 524,288 query points,
62,963,712 edges), field {0: 32, 1: 32, 2: 32} (160 reals per point), 8
heads, geodesic radius 3 row spacings, hard window, float32.  The layer runs
the stacked query/key projections, the fused scores-and-softmax op, every
head's node products, radial trunk and fused factored value aggregation,
and the output projection.  Inputs and the upstream gradient are N(0, 1),
resident in HBM before the timed region.

``--workload geometry`` times the GPU build of one 256x512 sample's
neighbourhoods, CSR and per-edge geometry (float64 lattice membership, tables
in float64) from the grid's nodes and frames resident on the device; its CPU
baseline is the host builder (KD-tree + exact filter + torch arithmetic).

``--workload c1`` and ``--workload c2`` run BASELINE's attention rows: C1 the
same layer forward only on the 32x64 grid, batch 1, field {0: 16, 1: 16, 2:
16}, 4 heads; C2 forward + backward on the 128x256 grid, batch 4, the
headline's field and heads.  C1 is launch-bound (2,048 query points): its
timed steps are replays of the step captured once in a HIP graph, checked
equal to an eager step first (``--no-graph``: eager steps); its ops are timed
on eager steps.

``--workload block`` runs the C4 configuration: one
``SO2TransformerBlock(ffn_multiplier=4)`` (pre-norm: batched 8-head SO2MHSA,
then the 160 -> 640 -> 160 gated feed-forward), forward + backward with every
gradient, at 256x512, batch 2, with bfloat16 rows and float32 parameters: the
attention's Q/K projections, scores and node mixes read the bfloat16 rows and
compute from the node mixes on in float32; the feed-forward (layer norm,
SO2Linear, gate, SO2Linear, residual) is one bf16-MFMA kernel per direction.

``--workload encoder`` runs the C5 stage model end to end (``GmSegformer``:
restrictions 128x256 ({0: 4}) -> 64x128 ({0: 64, 1: 64, 2: 64}) -> 32x64
({0: 128, 1: 128, 2: 128}), an 8-head then a 16-head block, readouts, fusion
decoder, 13-class head and cross-entropy), batch 8, forward + backward with
every gradient, float32; ``--workload hops`` times its two restrictions alone.

The default run also measures the other configurations (C1, C2, C3 ``conv``,
C4 ``block``, C5 ``encoder`` and the GPU ``geometry`` build), each in a
process of its own after the headline measurement, and reports their rates,
step times, roofline objects, op coverage and (C1, C2, C3) CPU baselines under
``other_workloads`` in the same JSON line (``--no-other-workloads`` skips
them).

``--workload softmax`` times the scores-and-softmax op alone (forward +
backward) on the same shape.  ``--workload conv`` times the depthwise steerable
convolution layer (``SO2Convolution(depthwise=True, n_radial_basis=4)``,
forward + backward with every parameter gradient) on the same grid, batch
and field: the C3 configuration.

Prints one JSON line.  Every native entry point the layers call (the
softmax, the radial trunk, the node mixes, the factored forward, aggregate
and backward, the gather/scatter transposes, the depthwise walks, the block's
pointwise kernels) and the flat projections' GEMMs are timed live with HIP
events on the stream they launch on, each call's algorithmic bytes and FLOPs
computed from its arguments; ``ops_coverage`` says how much of the step they
account for.  The roofline entry is the op with the largest share of the
step: the larger of its HBM time and its FP32 matrix time over its measured
time.  The CPU baseline is the eager PyTorch restatement of the reference's
path (oracle/, the factored order) on a bounded sample of the same workload on
this host's cores, extrapolated per edge.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from collections import defaultdict
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "gm-attention_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
NLAT, NLON, BATCH, HEADS = 256, 512, 4, 8
FIELD = {0: 32, 1: 32, 2: 32}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads() -> int:
    """Threads for the CPU baselines: the box's CPU share for one GPU (16), or
    fewer where the host has fewer.  The GPU boxes report many more cores in
    os.cpu_count() than one GPU's job may use (OMP_NUM_THREADS is 16 there);
    torch on all of them would oversubscribe the share, not add cores."""
    return min(16, os.cpu_count() or 1)


def cpu_model() -> str:
    """The host CPU's model name (as lscpu reports it, from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------- algorithmic cost per launch
#
# Each native entry point the layers call is timed with HIP events on its
# stream, and its algorithmic cost is computed from the call's own arguments:
# every tensor crossing the op boundary read or written once (int64 indices,
# the rows' element size, transport orders 0..2 as (cos, sin) pairs), and the
# multiply-adds of the contraction (x2 FLOPs).  An op's roofline is the larger
# of its HBM time (bytes / 8 TB/s) and its FP32 matrix time (FLOPs / 157.3
# TFLOP/s) over its measured time.


def _es(t) -> int:
    return t.element_size()


def cost_softmax_forward(a, kw, out):
    q, k, transport, bias, inside, desc, row_ptr, source, H = a[:9]
    E, N, D = source.shape[0], q.shape[0], q.shape[1]
    return E * (8 + 24 + 4 + 1 + 4 * H) + N * (2 * D * _es(q) + 8), E * 2.0 * D


def cost_softmax_backward(a, kw, out):
    dalpha, q, k, transport, bias, inside, desc, row_ptr, source, alpha, H = a[:11]
    E, N, D = source.shape[0], q.shape[0], q.shape[1]
    return E * (8 + 24 + 8 * H) + N * (2 * D * _es(q) + 8 * D + 8), E * 4.0 * D


def _factored_shape(K, wc, wr):
    return K, 2 * wc + wr, wc


def cost_factored_forward_grouped(a, kw, out):
    h_g, runs, n_nodes, phase_g, rho_g = a[:5]
    K, C, wc = _factored_shape(*a[12:15])
    d_out = a[15]
    E = rho_g.shape[0]
    es = _es(h_g) if h_g is not None else 4  # bfloat16 streams: h and the rows at 2 bytes
    h_bytes = es * (K - 1) if h_g is not None else 4
    return E * (h_bytes + 16 + es * d_out) + n_nodes * 4 * K * C, E * (2.0 * K * C + 8 * wc)


def cost_factored_backward_grouped(a, kw, out):
    g, target_g, weights_g, rows_g, h_g, runs, n_nodes, phase_g, rho_g = a[:9]
    K, C, wc = _factored_shape(*a[16:19])
    d_out = g.shape[1]
    E = rho_g.shape[0]
    es = _es(h_g) if h_g is not None else 4  # bfloat16 streams: h, the rows and dh at 2 bytes
    h_bytes = es * (K - 1) if h_g is not None else 4
    per_edge = h_bytes + 16 + 4 + 8 + 4 * d_out + es * d_out + es * (K - 1) + 4
    return E * per_edge + 2 * n_nodes * 4 * K * C, E * (4.0 * K * C + 8 * wc)


def cost_factored_forward(a, kw, out):
    h, zc, zr = a[:3]
    E, N, K, wc, wr = h.shape[0], zc.shape[0], zc.shape[1], zc.shape[2], zr.shape[2]
    C, d_out = 2 * wc + wr, a[11]
    return E * (4 * h.shape[1] + 48 + 4 + 8 + 4 * d_out) + N * 4 * K * C, E * (2.0 * K * C + 8 * wc)


def cost_factored_backward_aggregated(a, kw, out):
    g, target, weights, rows, h, zc, zr = a[:7]
    E, N, K, wc, wr = h.shape[0], zc.shape[0], zc.shape[1], zc.shape[2], zr.shape[2]
    C, d_out = 2 * wc + wr, g.shape[1]
    return (E * (8 + 4 + 4 * d_out + 8 * h.shape[1] + 48 + 4 + 8 + 4 * d_out + 4) + 2 * N * 4 * K * C,
            E * (4.0 * K * C + 8 * wc))


def cost_factored_aggregate(a, kw, out):
    rows, weights, row_ptr = a[:3]
    E, d_out = rows.shape
    return E * (4 * d_out + 4) + (row_ptr.shape[0] - 1) * (4 * d_out + 8), E * 2.0 * d_out


def cost_aggregate_heads(a, kw, out):
    rows, inv, alpha, row_ptr = a[:4]
    H, E, d_out = rows.shape
    N = row_ptr.shape[0] - 1
    return E * (8 + 4 * alpha.shape[1] + _es(rows) * H * d_out) + N * (4 * H * d_out + 8), E * 2.0 * H * d_out


def cost_trunk_forward(a, kw, out):
    rho, weight = a[:2]
    H, T, B = weight.shape
    E = rho.shape[0]
    dtype = a[5] if len(a) > 5 else kw.get("dtype")  # the features' storage type (None: rho's, float32)
    es = dtype.itemsize if dtype is not None else 4
    return E * (4 + es * H * T), E * H * (2.0 * T * B + 20 * T)


def cost_trunk_backward(a, kw, out):
    dh, rho, weight = a[:3]
    H, T, B = weight.shape
    E = rho.shape[0]
    return E * (4 + _es(dh) * H * T), E * H * (4.0 * T * B + 30 * T)


def cost_node_mix_forward(a, kw, out):
    v, m = a[:2]
    (N, w), C = v.shape, m.shape[1]
    return N * (w * _es(v) + 4 * C) + 4 * w * C, 2.0 * N * w * C


def cost_node_mix_backward_input(a, kw, out):
    dmix, m = a[:2]
    (N, C), w = dmix.shape, m.shape[0]
    return N * (4 * C + 4 * w) + 4 * w * C, 2.0 * N * w * C


def cost_node_mix_backward_weight(a, kw, out):
    v, dmix = a[:2]
    (N, w), C = v.shape, dmix.shape[1]
    return N * (w * _es(v) + C * _es(dmix)) + 4 * w * C, 2.0 * N * w * C


def cost_gather_transpose(a, kw, out):
    src = a[0]
    n, width = src.shape
    return n * (8 + 2 * 4 * width), 0.0


def cost_scatter_transpose(a, kw, out):
    src_t = a[0]
    width, n = src_t.shape
    return n * (8 + 2 * 4 * width), 0.0


def cost_projection_forward(a, kw, out):
    ctx, x, m = a[:3]
    (N, din), dout = x.shape, m.shape[1]
    return N * (din + dout) * _es(x) + 4 * din * dout, 2.0 * N * din * dout


def cost_projection_backward(a, kw, out):
    ctx, g = a[:2]
    x, m = ctx.saved_tensors
    (N, din), dout = x.shape, m.shape[1]
    return N * (2 * din + dout) * _es(x) + 8 * din * dout, 4.0 * N * din * dout


def cost_conv_forward(a, kw, out):
    v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, A0, W = a[:12]
    E, (N, D) = source.shape[0], v.shape
    return E * (8 + 4 * A0 + 4 * W + 48 + 8) + N * (8 * D + 8), E * 12.0 * D


def cost_conv_backward(a, kw, out):
    g, v, rc, cc = a[:4]
    source, A0, W = a[10], a[11], a[12]
    E, (N, D) = source.shape[0], v.shape
    return E * (16 + 8 * (A0 + W) + 48 + 8) + N * (12 * D + 16), E * 24.0 * D


def _radial_width(v, a0):
    D = v.shape[1]
    return a0, 4 * (D - a0) // 2


def cost_conv_radial_forward(a, kw, out):
    v, source, a0 = a[0], a[12], a[13]
    A0, W = _radial_width(v, a0)
    E, (N, D) = source.shape[0], v.shape
    return E * (8 + 48 + 8) + N * (8 * D + 8), E * (2.0 * 17 * (A0 + W) + 12 * D)


def cost_conv_radial_backward(a, kw, out):
    g, v, source, a0 = a[0], a[1], a[13], a[15]
    A0, W = _radial_width(v, a0)
    E, (N, D) = source.shape[0], v.shape
    return E * (16 + 48 + 8) + N * (12 * D + 16), E * (6.0 * 17 * (A0 + W) + 24 * D)


def cost_layer_norm_forward(a, kw, out):
    x = a[0]
    return 2 * x.numel() * _es(x) + 8 * x.shape[0], 0.0


def cost_layer_norm_backward(a, kw, out):
    gy = a[0]
    return 3 * gy.numel() * _es(gy) + 8 * gy.shape[0], 0.0


def cost_gate_forward(a, kw, out):
    h, pre = a[:2]
    return (2 * h.numel() + pre.numel()) * _es(h), 0.0


def cost_gate_backward(a, kw, out):
    gy, h, pre = a[:3]
    return (3 * h.numel() + 2 * pre.numel()) * _es(h), 0.0


def _ffn_flops(N, A, B):
    # per node: LN, the first linear (frequency 0: A x B; frequencies 1, 2: complex 2A x 2B each),
    # the gate's linear, the second linear back (B x A, 2B x 2A complex)
    return 2.0 * N * (A * B + 2 * (2 * A) * (2 * B) + 2 * B * B + B * A + 2 * (2 * B) * (2 * A))


def cost_ffn_forward(a, kw, out):
    x, A, B = a[:3]
    return x.shape[0] * (2 * x.shape[1] * _es(x) + 8), _ffn_flops(x.shape[0], A, B)


def cost_ffn_backward(a, kw, out):
    dz, x, A, B = a[:4]
    return x.shape[0] * (4 * x.shape[1] * _es(x) + 16), 1.65 * _ffn_flops(x.shape[0], A, B)


def roofline(nbytes: float, flops: float, seconds: float) -> dict:
    """The op's roofline: the larger of its HBM time and its FP32 matrix time
    over its measured time (``bound`` names which)."""
    t_hbm = nbytes / (HBM_PEAK_GBS * 1e9)
    t_mfma = flops / (FP32_PEAK_TFLOPS * 1e12)
    both = {"frac_hbm": t_hbm / seconds, "frac_mfma": t_mfma / seconds}
    if t_mfma > t_hbm:
        achieved = flops / seconds / 1e12
        return {"bound": "mfma", "achieved": achieved, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / FP32_PEAK_TFLOPS, **both}
    achieved = nbytes / seconds / 1e9
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
            **both}


# ---------------------------------------------------------------- live op timing


class OpTimer:
    """Wraps the native entry points with HIP events on the launching stream
    (torch's current stream, the one every entry point launches on) and sums
    each call's algorithmic bytes and FLOPs."""

    def __init__(self):
        self.events = defaultdict(list)
        self.cost = defaultdict(lambda: [0.0, 0.0])
        self.enabled = False

    def wrap(self, obj, name, label, cost=None, static=False):
        import torch

        if not hasattr(obj, name):
            return
        inner = getattr(obj, name)

        def timed(*args, **kwargs):
            if not self.enabled:
                return inner(*args, **kwargs)
            if cost is not None:  # from the arguments, before the call (a backward's saved tensors go with it)
                b, f = cost(args, kwargs, None)
                self.cost[label][0] += b
                self.cost[label][1] += f
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            out = inner(*args, **kwargs)
            end.record()
            self.events[label].append((start, end))
            return out

        setattr(obj, name, staticmethod(timed) if static else timed)

    def wrap_layers(self):
        """Every native entry point the attention, convolution, block and
        encoder layers reach, plus the flat projections' GEMMs."""
        from gm_attention_amd import _native
        from gm_attention_amd.nn import linear

        att, fac = _native.attention(), _native.factored()
        for obj, name, label, cost in (
                (att, "softmax_forward", "softmax_forward", cost_softmax_forward),
                (att, "softmax_backward", "softmax_backward", cost_softmax_backward),
                (att, "conv_forward", "conv_forward", cost_conv_forward),
                (att, "conv_backward", "conv_backward", cost_conv_backward),
                (fac, "forward", "factored_forward", cost_factored_forward),
                (fac, "aggregate", "factored_aggregate", cost_factored_aggregate),
                (fac, "backward_aggregated", "factored_backward_aggregated", cost_factored_backward_aggregated),
                (_native, "factored_forward_grouped", "factored_forward", cost_factored_forward_grouped),
                (_native, "factored_backward_grouped", "factored_backward_aggregated", cost_factored_backward_grouped),
                (_native, "aggregate_heads", "factored_aggregate", cost_aggregate_heads),
                (_native, "radial_trunk_forward", "radial_trunk_forward", cost_trunk_forward),
                (_native, "radial_trunk_backward", "radial_trunk_backward", cost_trunk_backward),
                (_native, "node_mix_forward", "node_mix_forward", cost_node_mix_forward),
                (_native, "node_mix_backward_input", "node_mix_backward_input", cost_node_mix_backward_input),
                (_native, "node_mix_backward_weight", "node_mix_backward_weight", cost_node_mix_backward_weight),
                (_native, "gather_transpose", "gather_transpose", cost_gather_transpose),
                (_native, "scatter_transpose", "scatter_transpose", cost_scatter_transpose),
                (_native, "conv_radial_forward", "conv_radial_forward", cost_conv_radial_forward),
                (_native, "conv_radial_backward", "conv_radial_backward", cost_conv_radial_backward),
                (_native, "layer_norm_forward", "layer_norm_forward", cost_layer_norm_forward),
                (_native, "layer_norm_backward", "layer_norm_backward", cost_layer_norm_backward),
                (_native, "gate_forward", "gate_forward", cost_gate_forward),
                (_native, "gate_backward", "gate_backward", cost_gate_backward),
                (_native, "ffn_forward", "ffn_forward", cost_ffn_forward),
                (_native, "ffn_backward", "ffn_backward", cost_ffn_backward)):
            self.wrap(obj, name, label, cost)
        self.wrap(linear.FlatLinear, "forward", "projection_forward", cost_projection_forward, static=True)
        self.wrap(linear.FlatLinear, "backward", "projection_backward", cost_projection_backward, static=True)

    def summary(self, steps: int) -> dict[str, dict[str, float]]:
        out = {}
        for label, pairs in self.events.items():
            times = [s.elapsed_time(e) for s, e in pairs]
            total_s = sum(times) * 1e-3
            nbytes, flops = self.cost[label]
            rec = {"launches_per_step": len(times) / steps, "avg_ms": sum(times) / len(times),
                   "ms_per_step": sum(times) / steps, "bytes_per_launch": nbytes / len(times),
                   "flops_per_launch": flops / len(times)}
            if total_s > 0:
                rec["GB/s"] = nbytes / total_s / 1e9
                rec["TFLOP/s"] = flops / total_s / 1e12
                r = roofline(nbytes, flops, total_s)
                rec["bound"], rec["frac"] = r["bound"], r["frac"]
            out[label] = rec
        return out

    def line_roofline(self, ops: dict, dominant: str, workload_tag: str) -> dict:
        """The dominant op's roofline object for the JSON line, with the
        counter-measured traffic per launch where a profile holds it."""
        rec = ops[dominant]
        n = rec["launches_per_step"]
        r = roofline(rec["bytes_per_launch"] * n, rec["flops_per_launch"] * n, rec["ms_per_step"] * 1e-3)
        traffic_file = ROOT / "profiles" / f"{dominant}_{workload_tag}_traffic.json"
        r["traffic"] = json.loads(traffic_file.read_text()).get("bytes_per_launch") if traffic_file.exists() else None
        r["kernel"] = dominant
        r["algorithmic_per_launch"] = {"bytes": rec["bytes_per_launch"], "flops": rec["flops_per_launch"]}
        r["launches_per_step"] = n
        return r


def ops_coverage(ops: dict, ms_per_step: float) -> dict:
    """How much of the step the timed entry points account for; the rest is
    torch's own kernels (copies, index gathers, sums, the allocator) and host time."""
    total = sum(v["ms_per_step"] for v in ops.values())
    return {"ops_ms_per_step": total, "step_ms": ms_per_step, "fraction": total / ms_per_step,
            "other_ms_per_step": ms_per_step - total}


# ---------------------------------------------------------------- problem


#: The attention configurations: the north-star shape (the headline) and BASELINE's C1 and C2.
LAYERS = {
    "attention": dict(nlat=NLAT, nlon=NLON, batch=BATCH, heads=HEADS, field=FIELD, backward=True,
                      metric="attn fwd+bwd query-points/s at 256x512 B=4", tag="ns"),
    "c2": dict(nlat=128, nlon=256, batch=4, heads=8, field=FIELD, backward=True,
               metric="attn fwd+bwd query-points/s at 128x256 B=4 (C2)", tag="c2"),
    "c1": dict(nlat=32, nlon=64, batch=1, heads=4, field={0: 16, 1: 16, 2: 16}, backward=False,
               metric="attn fwd query-points/s at 32x64 B=1 (C1)", tag="c1"),
}


def build_edges(device, batch: int = BATCH, nlat: int = NLAT, nlon: int = NLON):
    import torch

    from gm_attention_amd.discretization.edge_geometry import compute_edge_geometry
    from gm_attention_amd.discretization.frames import build_tangent_frames
    from gm_attention_amd.discretization.grid import build_equiangular_grid

    t0 = time.time()
    cutoff = 3.0 * math.pi / (nlat - 1)
    grid = build_equiangular_grid(nlat, nlon)
    edges = compute_edge_geometry(grid, build_tangent_frames(grid.nodes), cutoff)
    log(f"geometry {nlat}x{nlon}: {edges.n_edges} edges per sample in {time.time() - t0:.1f}s")
    tiled = edges.to(device, torch.float32).tile(batch, n_sources=grid.n_nodes)
    return edges, tiled, cutoff


def cpu_baseline_attention(edges, cutoff, mhsa_gpu, budget_edges: int, cfg: dict | None = None):
    """The eager restatement of one SO2MHSA layer (``oracle.modules.mhsa_forward``,
    the factored order as under GM_FACTORED_KERNEL=1, per-head types and scales
    derived by the oracle) forward (+ backward when the configuration has it)
    in float32 on the host's cores (at most 16 threads, one GPU's share of the
    box), over one sample's nodes and the edges of a mixed sample of its
    targets: the first (pole) targets and whole equator rows.  The node-side
    work (projections, node products) always covers the sample's nodes; the
    edge-side work scales with the sampled edges.  Three sample sizes give
    both costs by least squares, extrapolated to the step's nodes and edges.
    A sample with fewer edges than the budget is timed whole (one point)."""
    import torch

    from gm_attention_amd.nn.attention import SO2MHSA
    from gm_attention_amd.representations.field_type import SO2FeatureField
    from oracle import modules

    cfg = cfg or LAYERS["attention"]
    nlat, nlon = cfg["nlat"], cfg["nlon"]
    threads = cpu_threads()
    torch.set_num_threads(threads)
    row_ptr = edges.row_ptr
    n = row_ptr.shape[0] - 1
    mhsa = SO2MHSA(mhsa_gpu.field_type_in, cfg["heads"], cutoff=cutoff, window="hard", batched=True,
                   dtype=torch.float32)
    mhsa.load_state_dict({k: v.detach().cpu() for k, v in mhsa_gpu.state_dict().items()})
    fin = mhsa.field_type_in
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(n, fin.dimension, generator=gen).requires_grad_(cfg["backward"])
    g = torch.randn(n, fin.dimension, generator=gen)

    def sample(budget):
        if budget >= edges.n_edges:
            return edges.to(None, torch.float32)
        pole_last = max(1, int(torch.searchsorted(row_ptr, torch.tensor(budget // 2)).item()))
        eq_first = (nlat // 2) * nlon
        eq_last = eq_first + nlon
        while int(row_ptr[eq_last] - row_ptr[eq_first]) < budget // 2 and eq_last + nlon <= n:
            eq_last += nlon
        sel = torch.cat([torch.arange(int(row_ptr[a]), int(row_ptr[b])) for a, b in ((0, pole_last), (eq_first, eq_last))])
        return edges.select(sel, n_nodes=n).to(None, torch.float32)

    def step(sub):
        xs = SO2FeatureField.from_flat(fin, x).coefficients
        out = modules.flat(modules.mhsa_forward(mhsa, xs, sub, messages="factored"))
        if cfg["backward"]:
            (out * g).sum().backward()
            x.grad = None
            mhsa.zero_grad(set_to_none=True)

    budgets = (budget_edges // 4, budget_edges // 2, budget_edges) if edges.n_edges > budget_edges else (edges.n_edges,)
    points = []
    for budget in budgets:
        sub = sample(budget)
        with torch.set_grad_enabled(cfg["backward"]):
            step(sub)  # warm-up
            t0 = time.perf_counter()
            step(sub)
        points.append((sub.n_edges, time.perf_counter() - t0))
    if len(points) == 1:  # the whole sample: no extrapolation in edges
        return dict(per_edge=0.0, per_sample_nodes=points[0][1], points=points, threads=threads, whole=True)
    # least squares t = per_sample_nodes + per_edge e over the three samples
    k = len(points)
    me = sum(e for e, _ in points) / k
    mt = sum(t for _, t in points) / k
    per_edge = sum((e - me) * (t - mt) for e, t in points) / sum((e - me) ** 2 for e, _ in points)
    per_sample_nodes = max(0.0, mt - per_edge * me)
    return dict(per_edge=per_edge, per_sample_nodes=per_sample_nodes, points=points, threads=threads, whole=False)


def attention_baseline_line(b: dict, cfg: dict, N: int, E: int, batch: int) -> dict:
    """The CPU baseline's entry of the JSON line from ``cpu_baseline_attention``'s result."""
    direction = "fwd+bwd" if cfg["backward"] else "fwd"
    grid = f"{cfg['nlat']}x{cfg['nlon']}"
    if b["whole"]:
        cpu_step = b["per_sample_nodes"] * batch
        e, t = b["points"][0]
        how = (f"on one whole {grid} sample ({e} edges) in {t:.2f}s, the rate on that sample"
               + (f" x {batch} samples" if batch > 1 else ""))
    else:
        cpu_step = b["per_sample_nodes"] * batch + b["per_edge"] * E
        pts = "; ".join(f"{e} edges in {t:.2f}s" for e, t in b["points"])
        how = (f"on one {grid} sample's nodes with the edges of its first (pole) targets and equator rows, three "
               f"sizes: {pts}; the least-squares fit {b['per_sample_nodes']:.2f}s per sample's nodes + "
               f"{b['per_edge'] * 1e6:.1f}us per edge, extrapolated to {batch} samples and {E} edges")
    return {"value": N / cpu_step, "unit": "query-points/s", "cores": b["threads"], "kind": "port",
            "cpu_model": cpu_model(), "host_cpu_count": os.cpu_count(),
            "sample": (f"oracle eager SO2MHSA {direction} (oracle.modules.mhsa_forward, factored order, float32, "
                       f"torch on {b['threads']} threads) {how}")}


def cpu_baseline_ffn(block_gpu, n_nodes: int):
    """The block's node-wise part (both layer norms, the two SO2Linear layers and
    the gate, oracle.modules) forward + backward in float32 on the host's cores
    (at most 16 threads) over one 256x512 sample's nodes: seconds per sample."""
    import torch

    from gm_attention_amd.nn.blocks import SO2TransformerBlock
    from gm_attention_amd.representations.field_type import SO2FeatureField
    from oracle import modules

    threads = cpu_threads()
    torch.set_num_threads(threads)
    ft = block_gpu.field_type
    block = SO2TransformerBlock(ft, HEADS, ffn_multiplier=4, cutoff=1.0, attention_batched=True, dtype=torch.float32)
    block.load_state_dict({k: v.detach().cpu() for k, v in block_gpu.state_dict().items()})
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(n_nodes, ft.dimension, generator=gen).requires_grad_(True)
    g = torch.randn(n_nodes, ft.dimension, generator=gen)

    def step():
        xs = SO2FeatureField.from_flat(ft, x).coefficients
        a = modules.layer_norm(block.norm1, xs)
        h = modules.linear(block.linear1, modules.layer_norm(block.norm2, a), block.hidden_field_type)
        out = modules.flat(modules.linear(block.linear2, modules.gated(block.activation, h), ft))
        (out * g).sum().backward()
        x.grad = None
        block.zero_grad(set_to_none=True)

    step()
    t0 = time.perf_counter()
    step()
    return time.perf_counter() - t0, threads


def cpu_baseline_conv(edges, cutoff, conv_gpu, budget_edges: int):
    """The eager restatement (oracle.modules.conv_forward) of the depthwise
    layer's forward + backward in float32 on the host's cores (at most 16
    threads) over the targets of a mixed sample (the first, pole, targets
    and whole equator rows) of one 256x512 sample; the layer has no node-side
    work beyond the gather, so the time per edge is extrapolated to the step."""
    import torch

    from gm_attention_amd.nn.convolution import SO2Convolution
    from gm_attention_amd.representations.field_type import SO2FeatureField
    from oracle import modules

    threads = cpu_threads()
    torch.set_num_threads(threads)
    row_ptr = edges.row_ptr
    n = row_ptr.shape[0] - 1
    conv = SO2Convolution(conv_gpu.field_type_in, conv_gpu.field_type_out, cutoff=cutoff, depthwise=True,
                          n_radial_basis=conv_gpu.kernel.radial_basis.n_basis, dtype=torch.float32)
    conv.load_state_dict({k: v.detach().cpu() for k, v in conv_gpu.state_dict().items()})
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(n, conv.field_type_in.dimension, generator=gen).requires_grad_(True)
    g = torch.randn(n, conv.field_type_in.dimension, generator=gen)
    pole_last = max(1, int(torch.searchsorted(row_ptr, torch.tensor(budget_edges // 2)).item()))
    eq_first = (NLAT // 2) * NLON
    eq_last = eq_first + NLON
    while int(row_ptr[eq_last] - row_ptr[eq_first]) < budget_edges // 2 and eq_last + NLON <= n:
        eq_last += NLON
    sel = torch.cat([torch.arange(int(row_ptr[a]), int(row_ptr[b])) for a, b in ((0, pole_last), (eq_first, eq_last))])
    sub = edges.select(sel, n_nodes=n).to(None, torch.float32)

    def step():
        xs = SO2FeatureField.from_flat(conv.field_type_in, x).coefficients
        out = modules.flat(modules.conv_forward(conv, xs, sub))
        (out * g).sum().backward()
        x.grad = None
        conv.zero_grad(set_to_none=True)

    step()
    t0 = time.perf_counter()
    step()
    dt = time.perf_counter() - t0
    return dict(per_edge=dt / sub.n_edges, edges=sub.n_edges, seconds=dt, threads=threads)


def run_geometry(args) -> None:
    """One step = the whole edge-geometry build of one 256x512 sample: degree
    walk, prefix sum, edge walk (gm_radius_*), then the per-edge tables
    (gm_edge_tables_f64).  The step reads E back to size the edge list."""
    import torch

    from gm_attention_amd import _native
    from gm_attention_amd.discretization import edge_geometry as eg
    from gm_attention_amd.discretization.frames import build_tangent_frames
    from gm_attention_amd.discretization.grid import build_equiangular_grid

    device = torch.device("cuda:0")
    cutoff = 3.0 * math.pi / (NLAT - 1)
    grid = build_equiangular_grid(NLAT, NLON, device=device)
    frames = build_tangent_frames(grid.nodes)
    timer = OpTimer()
    timer.wrap(_native, "radius_edges", "radius_edges")
    timer.wrap(_native, "edge_tables", "edge_tables")
    n_edges = 0
    for _ in range(args.warmup):
        n_edges = eg.compute_edge_geometry(grid, frames, cutoff).n_edges
    torch.cuda.synchronize()
    timer.enabled = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        n_edges = eg.compute_edge_geometry(grid, frames, cutoff).n_edges
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timer.enabled = False
    ms_per_step = 1e3 * elapsed / args.steps
    ops = timer.summary(args.steps)
    log(f"step {ms_per_step:.2f} ms; ops: " + ", ".join(f"{k} {v['ms_per_step']:.2f} ms" for k, v in ops.items()))
    E, N, K = n_edges, grid.n_nodes, 4
    # tables: edge_index in (16 B), log map, distance, polar, transport, quadrature and both phase tables out
    table_bytes = E * (16 + 8 * (2 + 4) + 2 * 16 * (K + 1))
    avg_s = ops["edge_tables"]["avg_ms"] * 1e-3
    roof = {"bound": "hbm", "achieved": table_bytes / avg_s / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    traffic_file = ROOT / "profiles" / "edge_tables_ns_traffic.json"
    roof["traffic"] = json.loads(traffic_file.read_text()).get("bytes_per_launch") if traffic_file.exists() else None
    roof["kernel"] = "edge_tables"
    roof["algorithmic_per_launch"] = {"bytes": table_bytes, "flops": None}
    roof["note"] = ("radius_edges (the two box walks) is the larger share of the step; it is bound by float64 VALU "
                    "issue and LDS latency, so neither the HBM nor the MFMA roofline applies to it")
    baseline = None
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        torch.set_num_threads(threads)
        host = build_equiangular_grid(NLAT, NLON)
        hframes = build_tangent_frames(host.nodes)
        t0 = time.perf_counter()
        candidates = eg.radius_edges(host.exact_nodes, cutoff, exact=True, workers=threads)
        keep = eg.geodesic_distances(host.exact_nodes, candidates) <= cutoff + eg.EXACT_SLACK
        edges_cpu = eg.edge_geometry_from_index(host.nodes, hframes, host.quadrature_weights, candidates[:, keep],
                                                N, K)
        seconds = time.perf_counter() - t0
        baseline = {"value": edges_cpu.n_edges / seconds, "unit": "edges/s", "cores": threads, "kind": "port", "cpu_model": cpu_model(),
                    "sample": (f"the host builder on one whole 256x512 sample ({edges_cpu.n_edges} edges): scipy "
                               f"cKDTree ball query ({threads} workers), float64 exact filter and torch per-edge "
                               f"arithmetic ({threads} threads) in {seconds:.2f}s")}
        log(f"cpu baseline: {baseline['value']:.3g} edges/s ({baseline['sample']})")
    op_rates = {name: {k: (round(x, 4) if isinstance(x, float) else x) for k, x in v.items()}
                for name, v in ops.items()}
    line = {
        "metric": "edge-geometry build edges/s at 256x512 (one sample)",
        "value": E / (ms_per_step * 1e-3),
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic: the equiangular grid's nodes, tangent frames and quadrature weights",
        "config": {"workload": "neighbourhoods within 3 row spacings, CSR and per-edge geometry (max frequency 4)",
                   "grid": f"{NLAT}x{NLON} equiangular", "nodes": N, "edges": E},
        "roofline": roof,
        "ops": op_rates,
        "cpu_baseline": baseline,
    }
    print(json.dumps(line))


C5_IMG, C5_STAGES, C5_BATCH = (128, 256), ((64, 128), (32, 64)), 8
C5_TYPES, C5_HEADS = ({0: 64, 1: 64, 2: 64}, {0: 128, 1: 128, 2: 128}), (8, 16)


def run_stage(args) -> None:
    """One step = the C5 model forward and backward: per stage the learned
    restriction (EquiEncode) and its norm, one GmSegformer block (8 / 16-head
    SO2MHSA, depthwise steerable Mix-FFN), the stage norm; the readout
    convolutions, the fusion decoder's interpolations and the 13-class head on
    the 128x256 input grid; cross-entropy against random labels."""
    import torch

    from gm_attention_amd.nn import eager_ops
    from gm_attention_amd.nn.segformer import GmSegformer, build_stage_hierarchy, stage_radii
    from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

    device = torch.device("cuda:0")
    t0 = time.time()
    radii = stage_radii(C5_STAGES)
    h = build_stage_hierarchy(C5_IMG, C5_STAGES, radii, device=device).tile(C5_BATCH).to(device, torch.float32)
    n0 = h.levels[0].n_nodes
    down = [e.n_edges for e in h.down_edges]
    local = [h.levels[i + 1].discretization.n_edges for i in range(len(C5_STAGES))]
    log(f"hierarchy {C5_IMG} -> {C5_STAGES}, batch {C5_BATCH}: {n0} input points, restriction edges {down}, "
        f"stage edges {local} in {time.time() - t0:.1f}s")
    torch.manual_seed(0)
    model = GmSegformer(in_channels=4, num_classes=13, stage_field_types=[SO2FieldType(t) for t in C5_TYPES],
                        heads=C5_HEADS, depths=(1, 1), merge_cutoffs=radii.merge, attention_cutoffs=radii.attention,
                        mix_cutoffs=radii.mix, interpolate_cutoffs=radii.interpolate, readout_cutoffs=radii.readout,
                        readout_channels=(32, 32), decoder_channels=32, n_radial_basis=8, dtype=torch.float32,
                        device=device)
    timer = OpTimer()
    timer.wrap_layers()
    gen = torch.Generator(device=device).manual_seed(1)
    x0 = torch.rand(n0, 4, device=device, generator=gen).requires_grad_(True)
    labels = torch.randint(0, 13, (n0,), device=device, generator=gen)

    def step():
        logits = model(SO2FeatureField(model.input_field_type, {0: x0}), h)[0]
        torch.nn.functional.cross_entropy(logits, labels).backward()

    def clear():
        x0.grad = None
        model.zero_grad(set_to_none=True)

    before = dict(eager_ops.calls)
    for _ in range(args.warmup):
        step()
        clear()
    if eager_ops.calls != before:
        raise RuntimeError(f"part of the C5 model ran on the eager path: {eager_ops.calls}")
    torch.cuda.synchronize()
    timer.enabled = True
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
        clear()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t1
    timer.enabled = False
    ms_per_step = 1e3 * elapsed / args.steps
    ops = timer.summary(args.steps)
    log(f"step {ms_per_step:.2f} ms; ops: " + ", ".join(f"{k} {v['ms_per_step']:.2f} ms" for k, v in ops.items()))
    dominant = max(ops, key=lambda k: ops[k]["ms_per_step"])
    line = {
        "metric": "C5 stage fwd+bwd fine-points/s at 128x256 B=8",
        "value": n0 / (ms_per_step * 1e-3),
        "unit": "fine-points/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: U(0,1) 4-channel input, uniform random labels of 13 classes, random-init weights, "
                "equiangular grids",
        "config": {"workload": ("GmSegformer encoder stages + fusion decoder: 128x256 {0:4} -> EquiEncode -> 64x128 "
                                "{0:64,1:64,2:64} (8-head SO2MHSA + depthwise Mix-FFN block) -> EquiEncode -> 32x64 "
                                "{0:128,1:128,2:128} (16-head block); readouts, fusion decoder, 13-class head, "
                                "cross-entropy; input and every parameter gradient"),
                   "batch": C5_BATCH, "fine_points": n0, "restriction_edges": down, "stage_edges": local},
        "roofline": timer.line_roofline(ops, dominant, "c5"),
        "ops": {name: {k: (round(x, 4) if isinstance(x, float) else x) for k, x in v.items()}
                for name, v in ops.items()},
        "ops_coverage": ops_coverage(ops, ms_per_step),
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_stage(model),
    }
    print(json.dumps(line))


def cpu_baseline_stage(model_gpu) -> dict:
    """The oracle's composition of the C5 model (oracle.modules.segformer_forward,
    factored order) forward + backward with cross-entropy, float32, on the
    host's cores (all of them), on the same model's widths and heads over a
    32x64 input grid (stages 16x32 and 8x16), batch 1: the rate measured on
    that sample, not extrapolated (the oracle's cost grows faster than the
    points with the grid, so the full 128x256 x 8 rate would be lower)."""
    import torch

    from gm_attention_amd.nn.segformer import GmSegformer, build_stage_hierarchy, stage_radii
    from gm_attention_amd.representations.field_type import SO2FieldType
    from oracle import modules

    threads = cpu_threads()
    torch.set_num_threads(threads)
    img = (32, 64)
    stages = ((16, 32), (8, 16))
    radii = stage_radii(stages)
    h = build_stage_hierarchy(img, stages, radii).to(None, torch.float32)
    model = GmSegformer(in_channels=4, num_classes=13, stage_field_types=[SO2FieldType(t) for t in C5_TYPES],
                        heads=C5_HEADS, depths=(1, 1), merge_cutoffs=radii.merge, attention_cutoffs=radii.attention,
                        mix_cutoffs=radii.mix, interpolate_cutoffs=radii.interpolate, readout_cutoffs=radii.readout,
                        readout_channels=(32, 32), decoder_channels=32, n_radial_basis=8, dtype=torch.float32)
    model.load_state_dict({k: v.detach().cpu() for k, v in model_gpu.state_dict().items()})
    n0 = h.levels[0].n_nodes
    gen = torch.Generator().manual_seed(3)
    x0 = torch.rand(n0, 4, generator=gen).requires_grad_(True)
    labels = torch.randint(0, 13, (n0,), generator=gen)
    t0 = time.perf_counter()
    out = modules.segformer_forward(model, x0, h, None, "factored")
    torch.nn.functional.cross_entropy(out, labels).backward()
    dt = time.perf_counter() - t0
    log(f"cpu baseline: C5 oracle at {img} batch 1: {dt:.2f}s on {threads} threads")
    return {"value": n0 / dt, "unit": "fine-points/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": (f"oracle composition of the C5 model (same widths, heads and radii in row spacings) fwd+bwd "
                       f"with cross-entropy, float32, torch on {threads} threads, on a {img[0]}x{img[1]} input grid "
                       f"(stages 16x32, 8x16), batch 1: {n0} points in {dt:.2f}s, the rate on that sample (not "
                       "extrapolated)")}


def run_encoder(args) -> None:
    """One step = both restriction hops forward and backward (C5's encoder transfers)."""
    import torch

    from gm_attention_amd.discretization.grid import build_equiangular_grid
    from gm_attention_amd.discretization.hierarchy import build_grid_hierarchy
    from gm_attention_amd.nn import fused_factored
    from gm_attention_amd.nn.blocks import EquiEncode
    from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType
    from oracle import modules

    device = torch.device("cuda:0")
    shapes = [(128, 256), (64, 128), (32, 64)]
    cutoffs = [2.0 * math.pi / (shapes[1][0] - 1), 2.0 * math.pi / (shapes[2][0] - 1)]
    t0 = time.time()
    h1 = build_grid_hierarchy([build_equiangular_grid(*s, device=device) for s in shapes], ["equiangular"] * 3, shapes,
                              restrict_cutoffs=cutoffs, interpolate_cutoffs=cutoffs, local_cutoffs=[None, None, None])
    h = h1.tile(8)
    down = [e.to(device, torch.float32) for e in h.down_edges]
    log(f"hierarchy {shapes}: down edges {[e.n_edges for e in down]} (batch 8) in {time.time() - t0:.1f}s")
    types = [SO2FieldType({0: 4}), SO2FieldType({0: 64, 1: 64, 2: 64}), SO2FieldType({0: 128, 1: 128, 2: 128})]
    torch.manual_seed(0)
    encs = [EquiEncode(types[k], types[k + 1], cutoff=cutoffs[k], n_radial_basis=8, dtype=torch.float32, device=device)
            for k in range(2)]
    timer = OpTimer()
    timer.wrap_layers()
    n0 = h.levels[0].n_nodes
    gen = torch.Generator(device=device).manual_seed(1)
    x = torch.rand(n0, types[0].dimension, device=device, generator=gen).requires_grad_(True)
    upstream = torch.randn(h.levels[2].n_nodes, types[2].dimension, device=device, generator=gen)

    def step():
        y = encs[0](SO2FeatureField.from_flat(types[0], x), down[0])
        z = encs[1](y, down[1])._rows()
        torch.autograd.backward(z, upstream)

    def clear():
        x.grad = None
        for e in encs:
            e.zero_grad(set_to_none=True)

    for _ in range(args.warmup):
        step()
        clear()
    torch.cuda.synchronize()
    timer.enabled = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
        clear()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timer.enabled = False
    ms_per_step = 1e3 * elapsed / args.steps
    ops = timer.summary(args.steps)
    log(f"step {ms_per_step:.2f} ms; ops: " + ", ".join(f"{k} {v['ms_per_step']:.2f} ms" for k, v in ops.items()))
    dominant = max(ops, key=lambda k: ops[k]["ms_per_step"])
    roof = timer.line_roofline(ops, dominant, "hops")
    roof["note"] = "the op's launches (output tiles of both hops) differ in size: bytes and FLOPs summed per call"
    baseline = None
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        torch.set_num_threads(threads)
        total, parts = 0.0, []
        for k, (enc, e) in enumerate(zip(encs, down)):
            host = EquiEncode(types[k], types[k + 1], cutoff=cutoffs[k], n_radial_basis=8, dtype=torch.float32)
            host.load_state_dict({n: v.detach().cpu() for n, v in enc.state_dict().items()})
            one = h1.down_edges[k].to("cpu")
            n_t = max(1, int(torch.searchsorted(one.row_ptr, torch.tensor(args.cpu_budget_edges // 8)).item()))
            sub = one.select(torch.arange(int(one.row_ptr[n_t])), n_nodes=n_t).to(None, torch.float32)
            xs = torch.randn(h1.levels[k].n_nodes, types[k].dimension).requires_grad_(True)
            g = torch.randn(n_t, types[k + 1].dimension)

            def cpu_step():
                out = modules.flat(modules.encode_forward(host.integral, dict(
                    SO2FeatureField.from_flat(types[k], xs).coefficients), sub))
                (out * g).sum().backward()
                xs.grad = None
                host.zero_grad(set_to_none=True)

            cpu_step()
            t1 = time.perf_counter()
            cpu_step()
            dt = time.perf_counter() - t1
            total += dt / sub.n_edges * e.n_edges
            parts.append(f"hop {k + 1}: {sub.n_edges} edges in {dt:.2f}s")
        baseline = {"value": n0 / total, "unit": "fine-points/s", "cores": threads, "kind": "port", "cpu_model": cpu_model(),
                    "sample": (f"oracle eager EquiEncode fwd+bwd (per-edge readout, float32, torch on {threads} "
                               f"threads) over the first targets of one sample per hop ({'; '.join(parts)}), "
                               f"extrapolated per edge to both hops' {down[0].n_edges} + {down[1].n_edges} edges")}
        log(f"cpu baseline: {baseline['value']:.1f} fine-points/s ({baseline['sample']})")
    line = {
        "metric": "encoder restriction hops fwd+bwd fine-points/s at 128x256 B=8",
        "value": n0 / (ms_per_step * 1e-3),
        "unit": "fine-points/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: U(0,1) scalar input, N(0,1) upstream gradient, random-init weights, equiangular grids",
        "config": {"workload": ("EquiEncode 128x256 {0:4} -> 64x128 {0:64,1:64,2:64} -> 32x64 {0:128,1:128,2:128}, "
                                "quartic window, radius 2 coarse row spacings, n_radial_basis 8; input and every "
                                "parameter gradient"),
                   "batch": 8, "fine_points": n0, "edges": [e.n_edges for e in down],
                   "tiles": [len(fused_factored.tiles(e.integral.kernel) or ()) for e in encs]},
        "roofline": roof,
        "ops": {name: {k: (round(x, 4) if isinstance(x, float) else x) for k, x in v.items()}
                for name, v in ops.items()},
        "ops_coverage": ops_coverage(ops, ms_per_step),
        "cpu_baseline": baseline,
    }
    print(json.dumps(line))


#: The other configurations the default run measures after the headline: (workload, timed steps, with its
#: CPU baseline, extra arguments).  C1 and C2 are BASELINE's attention rows, conv is C3, block C4, encoder C5.
OTHER_WORKLOADS = (("c1", 10, True, ()), ("c2", 5, True, ("--cpu-budget-edges", "100000")), ("conv", 5, True, ()),
                   ("block", 5, False, ()), ("encoder", 3, False, ()), ("geometry", 5, False, ()))


def other_workloads() -> dict:
    """Every other configuration's line, from a child process each (warm-up 2, a few timed steps; the CPU
    baseline where OTHER_WORKLOADS asks for it): rate, step time, roofline and op coverage, or the error it
    ended with."""
    import subprocess

    out = {}
    for name, steps, cpu, extra in OTHER_WORKLOADS:
        log(f"other workload: {name} ({steps} steps{', CPU baseline' if cpu else ''})")
        cmd = [sys.executable, str(Path(__file__).resolve()), "--workload", name, "--steps", str(steps), "--warmup",
               "2", *extra] + ([] if cpu else ["--no-cpu-baseline"])
        try:
            run = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
        except subprocess.TimeoutExpired:
            out[name] = {"error": "timed out after 300 s"}
            continue
        lines = [x for x in run.stdout.splitlines() if x.startswith("{")]
        if run.returncode != 0 or not lines:
            tail = (run.stderr or run.stdout).strip().splitlines()[-1:] or [""]
            out[name] = {"error": f"exit {run.returncode}: {tail[0][:300]}"}
            continue
        rec = json.loads(lines[-1])
        out[name] = {k: rec.get(k) for k in ("metric", "value", "unit", "ms_per_step", "steps", "dtype", "roofline",
                                             "ops_coverage", "cpu_baseline")}
        log(f"{name}: {rec.get('ms_per_step')} ms per step")
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", choices=("attention", "c1", "c2", "softmax", "conv", "geometry", "block", "encoder",
                                           "hops"), default="attention")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-workloads", action="store_true",
                    help="the default attention run skips measuring the other configurations")
    ap.add_argument("--cpu-budget-edges", type=int, default=200_000)
    ap.add_argument("--no-graph", action="store_true",
                    help="time the forward-only C1 layer as eager steps instead of HIP graph replays")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB between two device buffers three times (the reference reading for the "
                         "HBM traffic counters) and exit")
    args = ap.parse_args()
    if args.calibrate_copy:
        import torch

        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": 4 * n, "copy_bytes_written": 4 * n, "launches": 3}))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: every run here has one MI355X; "
                                   "run with --gpus 1 (the multi-GPU sharding is a design note, not built)"}))
        sys.exit(2)

    if args.workload == "geometry":
        run_geometry(args)
        return
    if args.workload == "hops":
        run_encoder(args)
        return
    if args.workload == "encoder":
        run_stage(args)
        return
    run_layer(args)


def capture_step(step):
    """``step`` captured in a HIP graph (torch.cuda.CUDAGraph) after two steps on a side stream, or None
    when capture fails or the first two replays differ from an eager step (the graph replays exactly the
    eager kernels: any difference means something in the step cannot be replayed)."""
    import torch

    try:
        want = step().detach().clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = step()
        for _ in range(2):
            graph.replay()
            torch.cuda.synchronize()
            if not torch.equal(out, want):
                log("graph replay differs from the eager step: timing eager steps")
                return None
    except RuntimeError as exc:
        log(f"graph capture failed ({exc}): timing eager steps")
        return None
    return graph.replay


def run_layer(args) -> None:
    """The attention layer at a configuration of ``LAYERS`` (the headline,
    C1, C2), the scores-and-softmax op alone, the C3 depthwise convolution or
    the C4 block, each on its equiangular grid and batch."""
    import torch

    from gm_attention_amd.nn import fused_attention
    from gm_attention_amd.nn.attention import SO2MHSA
    from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

    device = torch.device("cuda:0")
    cfg = dict(LAYERS.get(args.workload, LAYERS["attention"]))
    if args.workload == "block":
        cfg.update(batch=2, tag="c4")
    timer = OpTimer()
    timer.wrap_layers()
    batch = cfg["batch"]
    edges_cpu, edges, cutoff = build_edges(device, batch, cfg["nlat"], cfg["nlon"])
    N = edges.row_ptr.shape[0] - 1
    E = edges.n_edges
    field = SO2FieldType(cfg["field"])
    D = field.dimension
    heads = cfg["heads"]
    torch.manual_seed(0)
    mhsa = SO2MHSA(field, heads, cutoff=cutoff, window="hard", batched=True, dtype=torch.float32, device=device)
    gen = torch.Generator(device=device).manual_seed(1)
    x_flat = torch.randn(N, D, device=device, generator=gen).requires_grad_(cfg["backward"])
    upstream = torch.randn(N, D, device=device, generator=gen)
    g = fused_attention.geometry(edges, cutoff, "hard", torch.float32)
    log(f"problem: N={N} E={E} D={D} H={heads} max_degree={g.max_degree}")
    module = mhsa  # the module whose parameter gradients the loop clears
    grid = f"{cfg['nlat']}x{cfg['nlon']}"

    if args.workload == "block":
        from gm_attention_amd.nn.blocks import SO2TransformerBlock

        torch.manual_seed(0)
        block = SO2TransformerBlock(field, heads, ffn_multiplier=4, cutoff=cutoff, window="hard",
                                    attention_batched=True, dtype=torch.float32, device=device)
        module = block
        mhsa = block.attention
        x_flat = x_flat.detach().to(torch.bfloat16).requires_grad_(True)
        upstream = upstream.to(torch.bfloat16)

        def step():
            y = block.forward_flat(x_flat, edges)
            torch.autograd.backward(y, upstream)
        workload = ("SO2TransformerBlock(ffn_multiplier=4) fwd+bwd: layer norm, batched 8-head SO2MHSA (bf16 Q/K "
                    "projections, scores reading bf16 q and k, node mixes reading bf16 rows, float32 from the mixes "
                    "on), residual, then the fused feed-forward (layer norm, SO2Linear 160->640, scalar gate, "
                    "SO2Linear 640->160, residual: one bf16-MFMA kernel per direction); bf16 rows, float32 "
                    "parameters; input and every parameter gradient")
    elif args.workload in LAYERS:
        def step():
            x = SO2FeatureField.from_flat(field, x_flat)
            y = mhsa(x, edges)._rows()
            if cfg["backward"]:
                torch.autograd.backward(y, upstream)
            return y
        workload = (f"SO2MHSA(batched) {'fwd+bwd' if cfg['backward'] else 'fwd'}: stacked Q/K projections, fused "
                    f"scores+softmax, {heads} heads of node products + radial trunk + fused factored value "
                    "aggregation, output projection" + ("; input and every parameter gradient" if cfg["backward"]
                                                        else ""))
    elif args.workload == "conv":
        from gm_attention_amd.nn.convolution import SO2Convolution

        torch.manual_seed(0)
        conv = SO2Convolution(field, field, cutoff=cutoff, window="hard", depthwise=True, n_radial_basis=4,
                              dtype=torch.float32, device=device)
        module = conv

        def step():
            x = SO2FeatureField.from_flat(field, x_flat)
            y = conv(x, edges)._rows()
            torch.autograd.backward(y, upstream)
        workload = ("SO2Convolution(depthwise=True, n_radial_basis=4) fwd+bwd: radial trunk and readout heads, "
                    "fused depthwise walk (transport, coefficient products, weighting, segment sum); input and "
                    "every parameter gradient")
    else:
        p = fused_attention.plan(mhsa)
        desc = fused_attention.descriptors(mhsa, p, device)
        scale = float(mhsa.heads[0]._score_scale)
        q = torch.randn(N, D, device=device, generator=gen).requires_grad_(True)
        k = torch.randn(N, D, device=device, generator=gen).requires_grad_(True)
        dalpha = torch.randn(E, heads, device=device, generator=gen)
        transport = g.transport_to(2)

        def step():
            alpha = fused_attention.Softmax.apply(q, k, transport, g.bias, g.inside, desc, g.row_ptr, g.source, heads,
                                                  scale, g.max_degree)
            torch.autograd.backward(alpha, dalpha)
        workload = "Softmax.apply fwd+bwd: neighbourhood scores + softmax over CSR (gauge-transported keys)"

    def clear():
        module.zero_grad(set_to_none=True)
        x_flat.grad = None

    # A forward-only layer (C1) is launch-bound: its step is captured once in a HIP graph and replayed
    # (every kernel still runs each replay, on the resident inputs); its ops are timed on eager steps.
    graphed = args.workload in LAYERS and not cfg["backward"] and not args.no_graph
    with torch.set_grad_enabled(cfg["backward"] or args.workload not in LAYERS):
        for _ in range(args.warmup):
            step()
            clear()
        torch.cuda.synchronize()
        timer.enabled = True
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
            clear()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        timer.enabled = False
        if graphed:
            replay = capture_step(step)
            if replay is None:
                graphed = False
            else:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(args.steps):
                    replay()
                torch.cuda.synchronize()
                elapsed = time.perf_counter() - t0
    ms_per_step = 1e3 * elapsed / args.steps
    if graphed:
        workload += "; the step captured once in a HIP graph and replayed (ops timed on eager steps)"
    ops = timer.summary(args.steps)
    log(f"step {ms_per_step:.2f} ms; ops: " + ", ".join(f"{k} {v['ms_per_step']:.2f} ms" for k, v in ops.items()))
    dominant = max(ops, key=lambda k: ops[k]["ms_per_step"])
    roof = timer.line_roofline(ops, dominant, cfg["tag"])

    baseline = None
    if not args.no_cpu_baseline and args.workload in LAYERS:
        b = cpu_baseline_attention(edges_cpu, cutoff, mhsa, args.cpu_budget_edges, cfg)
        baseline = attention_baseline_line(b, cfg, N, E, batch)
        log(f"cpu baseline: {baseline['value']:.1f} qp/s ({baseline['sample']})")
    elif not args.no_cpu_baseline and args.workload == "block":
        b = cpu_baseline_attention(edges_cpu, cutoff, mhsa, args.cpu_budget_edges, cfg)
        ffn_s, _ = cpu_baseline_ffn(block, N // batch)
        cpu_step = (b["per_sample_nodes"] + ffn_s) * batch + b["per_edge"] * E
        pts = ", ".join(f"{e} edges in {t:.2f}s" for e, t in b["points"])
        baseline = {"value": N / cpu_step, "unit": "query-points/s", "cores": b["threads"], "kind": "port",
                    "cpu_model": cpu_model(), "host_cpu_count": os.cpu_count(),
                    "sample": (f"oracle eager block fwd+bwd in float32 (torch on {b['threads']} threads): the "
                               f"SO2MHSA as in the attention workload ({pts}; "
                               f"{b['per_sample_nodes']:.2f}s per sample's nodes + "
                               f"{b['per_edge'] * 1e6:.1f}us per edge) plus both layer norms, the feed-forward and "
                               f"the gate over one sample's {N // batch} nodes in {ffn_s:.2f}s, extrapolated to "
                               f"{batch} samples and {E} edges")}
        log(f"cpu baseline: {baseline['value']:.1f} qp/s ({baseline['sample']})")
    elif not args.no_cpu_baseline and args.workload == "conv":
        b = cpu_baseline_conv(edges_cpu, cutoff, conv, args.cpu_budget_edges)
        baseline = {"value": N / (b["per_edge"] * E), "unit": "query-points/s", "cores": b["threads"], "kind": "port",
                    "cpu_model": cpu_model(), "host_cpu_count": os.cpu_count(),
                    "sample": (f"oracle eager SO2Convolution(depthwise) fwd+bwd (float32, torch on {b['threads']} "
                               f"threads) over the edges of one 256x512 sample's first (pole) targets and equator "
                               f"rows: {b['edges']} edges in {b['seconds']:.2f}s, {b['per_edge'] * 1e6:.2f}us per "
                               f"edge, extrapolated to {E} edges")}
        log(f"cpu baseline: {baseline['value']:.1f} qp/s ({baseline['sample']})")

    # the whole step's HBM traffic (every kernel's FETCH_SIZE + WRITE_SIZE of one steady-state step, measured
    # with rocprofv3) over this run's step time: the layer's achieved HBM bandwidth
    hbm = None
    step_file = ROOT / "profiles" / f"{args.workload}_ns_step_traffic.json"
    if step_file.exists():
        step_bytes = json.loads(step_file.read_text())["step_bytes"]
        achieved = step_bytes / (ms_per_step * 1e-3) / 1e9
        hbm = {"achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
               "step_traffic": step_bytes, "source": str(step_file.relative_to(ROOT))}
    metric = cfg["metric"] if args.workload in LAYERS else {
        "softmax": "attn scores+softmax fwd+bwd query-points/s at 256x512 B=4",
        "conv": "depthwise conv fwd+bwd query-points/s at 256x512 B=4",
        "block": "transformer block fwd+bwd query-points/s at 256x512 B=2"}[args.workload]
    line = {
        "metric": metric,
        "value": N / (ms_per_step * 1e-3),
        "unit": "query-points/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.workload == "block" else "f32",
        "data": "synthetic: N(0,1) input field and upstream gradient, random-init weights, equiangular grid geometry",
        "config": {"workload": workload, "grid": f"{grid} equiangular", "batch": batch,
                   "field": "{" + ",".join(f"{f}:{m}" for f, m in cfg["field"].items()) + "}", "heads": heads,
                   "radius": "3 row spacings", "window": "hard", "query_points": N, "edges": E,
                   "max_degree": g.max_degree},
        "roofline": roof,
        "hbm_step": hbm,
        "ops": {name: {k: (round(x, 4) if isinstance(x, float) else x) for k, x in v.items()}
                for name, v in ops.items()},
        "ops_coverage": ops_coverage(ops, ms_per_step) if not graphed else {
            "note": "the ops are timed on eager steps; the step time is of graph replays, without launch gaps"},
        "cpu_baseline": baseline,
    }
    if args.workload == "attention" and not args.no_other_workloads:
        # the headline's tensors go back to the device before the other configurations run beside this process
        del x_flat, upstream, mhsa, module
        import gc

        gc.collect()
        torch.cuda.empty_cache()
        line["other_workloads"] = other_workloads()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
