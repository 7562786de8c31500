// The depthwise steerable convolution with its radial heads evaluated inside
// the walk (CDNA4, gfx950): no per-edge coefficient tensor in either direction.
//
// Per edge e = (i <- j) with r = rho_e = d_e / cutoff, s = r^2:
//   b_k(e)   = exp(-((s - mu_k) / sigma)^2 / 2)                 k < NB  (Gaussian basis)
//   pre_t(e) = sum_k W1[t, k] b_k(e) + b1[t],  h_t = SiLU(pre_t)   t < 16  (the shared trunk)
//   C(e)     = R (h_0..h_15, 1)^T                                  (the readout heads, bias as column 16)
// and per copy of the field, with z = e^{i n gamma_e} v_j (transport),
//   scalar copy a:       m = C_a v_j,a
//   complex copy of n:   m = A z + r^{2n} e^{2 i n phi_e} B conj(z),   (A, B) = C's rows (Ar, Ai, Br, Bi)
//   out_i = sum_e w_e m_e.
// (The reference: nn/depthwise.py:147-193 and :206-238 -- the readout
// materialised per edge by torch products, then fused/attention.h:167-232 on
// it.)  R's rows are ordered in 16-row tiles: scalar tiles first (row a =
// copy a), then complex tiles of four copies, copy q of a tile owning rows
// 4q..4q+3 = (Ar, Ai, Br, Bi); every complex tile holds one frequency.
//
// MFMA mapping (v_mfma_f32_16x16x4f32: lane l supplies A[l%16][l/16],
// B[l/16][l%16] and holds D[4(l/16)+r][l%16]): lane (q = l/16, c = l%16)
// works on edge c of a 16-edge tile and computes trunk features 4q..4q+3 of
// it; the coefficient product D_m = R_m (w H~) over k-steps s = 0..4 (k =
// 4q + s, then the bias row) leaves the lane rows 4q..4q+3 of tile m for its
// edge: four scalar copies or one complex copy, whose message it forms at
// once.  Forward: one wave per target node, lanes accumulate their edge
// column's messages, a 16-lane butterfly per target.  Backward: persistent
// waves over SOURCE nodes (the transposed CSR): per edge tile the same
// coefficients, then dC (the coefficients' gradient) and dv in registers,
// dh~ = R^T dC on MFMA (D layout = the lane's own trunk features), and
// dR += dC h~^T on MFMA with dC and h~ transposed through the wave's LDS;
// per wave the parameter gradients end in a partial row, and a second kernel
// sums the rows in a fixed order (deterministic, no atomics).
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "common.hpp"
#include "split.hpp"

namespace gm {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kRNS = 2;            // scalar tiles: up to 32 scalar copies
constexpr int kRNC = 16;           // complex tiles: up to 64 complex copies
constexpr int kRNT = kRNS + kRNC;  // coefficient tiles
constexpr int kRWaves = 4;         // waves per workgroup
constexpr int kRThreads = kRWaves * kWave;
constexpr int kRMaxBasis = 8;
constexpr int kRChunk = 1;         // backward: coefficient tiles per LDS hand-over
// The backward's tile groups: kRGroup consecutive slots each; a group runs
// only when it holds a live tile.
constexpr int kRGroup = 9;
constexpr int kRGroups = (kRNT + kRGroup - 1) / kRGroup;
// per-wave partial row of the backward: dR in lane layout, the bias column, W1 and b1
constexpr int kRPartDR = kRNT * 256;
constexpr int kRPartDB = kRNT * 16;
constexpr int kRPartW1 = 16 * kRMaxBasis + 16;
constexpr int kRPart = kRPartDR + kRPartDB + kRPartW1;

struct RadialConvArgs {
  const float* v;          // (N, D)
  const float* rf;         // (kRNT, 4, 64): A operand of the coefficient product
  const float* rbias;      // (kRNT * 16,): the readout's bias column
  const float* rb;         // (kRNT, 4, 64): A operand of dh~ = R^T dC
  const float* w1;         // (16, NB)
  const float* b1;         // (16,) or null
  const float* transport;  // (E, orders, 2)
  const float* angular;    // (E, orders, 2)
  const float* rho;        // (E,)
  const float* weights;    // (E,)
  const int64_t* row_ptr;  // (N + 1,)
  const int64_t* source;   // (E,)
  const float* g;          // (N, D) backward
  const int64_t* src_ptr;  // (N + 1,) backward: edges grouped by source
  const int64_t* src_order;
  const int64_t* target;
  float* out;      // (N, D)
  float* dv;       // (N, D)
  int64_t n_nodes;
  int D, orders, ns, nc, a0;
  float inv_width;
  float centers[kRMaxBasis];
  int tile_n[kRNC];    // frequency of complex tile m
  int tile_col[kRNC];  // flat column of its copy 0 (copy q at + 2q)
};

__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// A wave's LDS operations run in order; handing data between its lanes
// needs only a compiler ordering point at wavefront scope.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float2 ld2(const float* p) { return *reinterpret_cast<const float2*>(p); }

// One edge as a lane sees it: the source (or target), weight, transport
// phases of orders 1 and 2 and the angular factors r^{2n} e^{2 i n phi}
// (e^{2 i n phi} as loaded; with_radius applies r^{2n}).
struct EdgeView {
  int64_t node;
  float w, r;
  float2 t1, t2, p1, p2;
};

__device__ __forceinline__ EdgeView edge_view(const RadialConvArgs& a, int64_t e, int64_t node, bool live) {
  EdgeView v;
  v.node = node;
  v.w = live ? a.weights[e] : 0.f;
  v.r = a.rho[e];
  const float* tr = a.transport + e * a.orders * 2;
  const float* an = a.angular + e * a.orders * 2;
  v.t1 = ld2(tr + 2);
  v.t2 = ld2(tr + 4);
  v.p1 = ld2(an + 4);
  v.p2 = ld2(an + 8);
  return v;
}

// The view with its angular factors scaled by r^2 and r^4.  Kept apart from
// edge_view so that a view requested a tile ahead leaves its loads in flight
// until the tile that uses it.
__device__ __forceinline__ EdgeView with_radius(EdgeView v) {
  const float r2 = v.r * v.r, r4 = r2 * r2;
  v.p1 = make_float2(r2 * v.p1.x, r2 * v.p1.y);
  v.p2 = make_float2(r4 * v.p2.x, r4 * v.p2.y);
  return v;
}

// The lane's trunk features k = 4q + s (s < 4) of its edge: pre-activations,
// SiLU outputs and (for the backward) the basis.
template <int NB>
__device__ __forceinline__ void trunk_of(const RadialConvArgs& a, const float* w1s, float r, int q, float (&bas)[NB],
                                         float (&pre)[4], float (&h)[4]) {
  const float s = r * r;
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const float z = (s - a.centers[k]) * a.inv_width;
    bas[k] = fexp(-0.5f * z * z);
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = 4 * q + u;
    float p = w1s[16 * kRMaxBasis + t];
#pragma unroll
    for (int k = 0; k < NB; ++k) p = fmaf(w1s[t * kRMaxBasis + k], bas[k], p);
    pre[u] = p;
    h[u] = p * frcp(1.f + fexp(-p));
  }
}

__device__ __forceinline__ void load_tables(const RadialConvArgs& a, float* rf_s, float* rb_s, float* bias_s, float* w1s,
                                            int nb) {
  if (rf_s)
    for (int i = threadIdx.x; i < kRNT * 4 * 64; i += kRThreads) rf_s[i] = a.rf[i];
  for (int i = threadIdx.x; i < kRNT * 16; i += kRThreads) bias_s[i] = a.rbias[i];
  if (rb_s)
    for (int i = threadIdx.x; i < kRNT * 4 * 64; i += kRThreads) rb_s[i] = a.rb[i];
  for (int i = threadIdx.x; i < 16 * kRMaxBasis; i += kRThreads) {
    const int t = i / kRMaxBasis, k = i % kRMaxBasis;
    w1s[i] = k < nb ? a.w1[t * nb + k] : 0.f;
  }
  if (threadIdx.x < 16) w1s[16 * kRMaxBasis + threadIdx.x] = a.b1 ? a.b1[threadIdx.x] : 0.f;
}

// The lane's rows 4q..4q+3 of coefficient tile m for its edge, times the
// edge's weight: w (R_m h~) = w bias + R_m (w h) over the four k-steps k = 4q + s.
__device__ __forceinline__ floatx4 coefficients(const float* rf_s, const float* bias_s, int m, int lane, int q, float w,
                                                const float (&bv)[4]) {
  const float4 b = *reinterpret_cast<const float4*>(bias_s + m * 16 + 4 * q);
  floatx4 d = floatx4{w * b.x, w * b.y, w * b.z, w * b.w};
#pragma unroll
  for (int s = 0; s < 4; ++s) d = mfma16(rf_s[(m * 4 + s) * 64 + lane], bv[s], d);
  return d;
}

// The coefficient product as split-bf16 products (split.hpp): R_m's rows c,
// features 4q..4q+3 -- a lane's four contraction indices -- split once per
// workgroup into the A operand pieces (hm, hl), held in LDS; w h~'s features
// 4q..4q+3 of the lane's edge split once per edge tile into the B pieces,
// shared by every tile.  Three bf16 instructions a tile instead of four fp32
// ones, in fp32 accuracy.  A tile's pieces are stored as its 64 lanes' hm,
// then their hl, so consecutive lanes read consecutive 16-byte pieces (no
// bank conflicts).
struct SplitTile {
  u32x4 hm, hl;
};

__device__ __forceinline__ void load_split(const RadialConvArgs& a, SplitTile* rs_s) {
  u32x4* pieces = reinterpret_cast<u32x4*>(rs_s);
  for (int i = threadIdx.x; i < kRNT * kWave; i += kRThreads) {
    const int m = i / kWave, l = i % kWave;
    const SplitA sa = split_a(a.rf[(m * 4 + 0) * 64 + l], a.rf[(m * 4 + 1) * 64 + l], a.rf[(m * 4 + 2) * 64 + l],
                              a.rf[(m * 4 + 3) * 64 + l]);
    pieces[2 * kWave * m + l] = sa.hm;
    pieces[2 * kWave * m + kWave + l] = sa.hl;
  }
}

__device__ __forceinline__ floatx4 coefficients_split(const SplitTile* rs_s, const float* bias_s, int m, int lane,
                                                      int q, float w, const SplitB& hb) {
  const float4 b = *reinterpret_cast<const float4*>(bias_s + m * 16 + 4 * q);
  const u32x4* pieces = reinterpret_cast<const u32x4*>(rs_s) + 2 * kWave * m;
  return mfma_split(SplitA{pieces[lane], pieces[kWave + lane]}, hb, floatx4{w * b.x, w * b.y, w * b.z, w * b.w});
}

// The tile's coefficients for the lane's edge: fp32 MFMA from rf_s, or the split products from rs_s.
template <bool SPLIT>
__device__ __forceinline__ floatx4 coefficients_of(const float* rf_s, const SplitTile* rs_s, const float* bias_s, int m,
                                                   int lane, int q, float w, const float (&bv)[4], const SplitB& hb) {
  if constexpr (SPLIT)
    return coefficients_split(rs_s, bias_s, m, lane, q, w, hb);
  else
    return coefficients(rf_s, bias_s, m, lane, q, w, bv);
}

// Whether coefficient tile slot m holds copies (uniform).
__device__ __forceinline__ bool tile_live(const RadialConvArgs& a, int m) {
  return m < kRNS ? m < a.ns : m - kRNS < a.nc;
}

// Coefficient tile m's source values for the lane: a scalar tile's four, a
// complex tile's pair in x and y (zeros for a dead tile or absent copies).
__device__ __forceinline__ float4 tile_x(const RadialConvArgs& a, int m, int q, const float* vj) {
  if (m < kRNS) {
    const int col = 16 * m + 4 * q;
    if (m < a.ns && col < a.a0) return *reinterpret_cast<const float4*>(vj + col);
  } else if (m - kRNS < a.nc) {
    const float2 x = ld2(vj + a.tile_col[m - kRNS] + 2 * q);
    return make_float4(x.x, x.y, 0.f, 0.f);
  }
  return make_float4(0.f, 0.f, 0.f, 0.f);
}

template <int NB, bool SPLIT>
__global__ __launch_bounds__(kRThreads) __attribute__((amdgpu_waves_per_eu(SPLIT ? 4 : 1))) void
conv_radial_forward_kernel(RadialConvArgs a) {
  __shared__ float rf_s[SPLIT ? 1 : kRNT * 4 * 64];
  __shared__ __attribute__((aligned(16))) SplitTile rs_s[SPLIT ? kRNT * kWave : 1];
  __shared__ __attribute__((aligned(16))) float bias_s[kRNT * 16];
  __shared__ float w1s[16 * kRMaxBasis + 16];
  if constexpr (SPLIT) {
    load_split(a, rs_s);
    load_tables(a, nullptr, nullptr, bias_s, w1s, NB);
  } else {
    load_tables(a, rf_s, nullptr, bias_s, w1s, NB);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, c = lane & 15, q = lane >> 4;
  const int64_t i = xcd_block(blockIdx.x, gridDim.x) * kRWaves + (threadIdx.x >> 6);
  if (i >= a.n_nodes) return;
  float accs[kRNS][4], accc[kRNC][2];
#pragma unroll
  for (int m = 0; m < kRNS; ++m) accs[m][0] = accs[m][1] = accs[m][2] = accs[m][3] = 0.f;
#pragma unroll
  for (int m = 0; m < kRNC; ++m) accc[m][0] = accc[m][1] = 0.f;
  const int64_t e0 = a.row_ptr[i], e1 = a.row_ptr[i + 1];
  // the next tile's edge rows and sources are requested while this tile computes
  EdgeView nxt;
  if (e0 < e1) {
    const int64_t e = e0 + c < e1 ? e0 + c : e0;
    nxt = edge_view(a, e, a.source[e], e0 + c < e1);
  }
  for (int64_t base = e0; base < e1; base += 16) {
    const EdgeView ev = with_radius(nxt);
    if (base + 16 < e1) {
      const bool live = base + 16 + c < e1;
      const int64_t e = live ? base + 16 + c : e0;
      nxt = edge_view(a, e, a.source[e], live);
    }
    float bas[NB], pre[4], h[4];
    trunk_of<NB>(a, w1s, ev.r, q, bas, pre, h);
    float bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) bv[u] = ev.w * h[u];
    SplitB hb{};
    if constexpr (SPLIT) hb = split_b(bv[0], bv[1], bv[2], bv[3]);
    const float* vj = a.v + ev.node * a.D;
#pragma unroll
    for (int m = 0; m < kRNS; ++m) {
      const float4 x = tile_x(a, m, q, vj);
      if (m < a.ns) {
      const floatx4 d = coefficients_of<SPLIT>(rf_s, rs_s, bias_s, m, lane, q, ev.w, bv, hb);
      const int col = 16 * m + 4 * q;
      if (col < a.a0) {
        accs[m][0] = fmaf(d[0], x.x, accs[m][0]);
        accs[m][1] = fmaf(d[1], x.y, accs[m][1]);
        accs[m][2] = fmaf(d[2], x.z, accs[m][2]);
        accs[m][3] = fmaf(d[3], x.w, accs[m][3]);
      }
      }
    }
#pragma unroll
    for (int m = 0; m < kRNC; ++m) {
      const float4 x = tile_x(a, kRNS + m, q, vj);
      if (m < a.nc) {
      const floatx4 d = coefficients_of<SPLIT>(rf_s, rs_s, bias_s, kRNS + m, lane, q, ev.w, bv, hb);
      const bool one = a.tile_n[m] == 1;
      const float tc = one ? ev.t1.x : ev.t2.x, ts = one ? ev.t1.y : ev.t2.y;
      const float pr = one ? ev.p1.x : ev.p2.x, pi = one ? ev.p1.y : ev.p2.y;
      const float zr = tc * x.x - ts * x.y, zi = tc * x.y + ts * x.x;
      const float bzr = d[2] * zr + d[3] * zi, bzi = d[3] * zr - d[2] * zi;  // B conj(z)
      accc[m][0] += (d[0] * zr - d[1] * zi) + (pr * bzr - pi * bzi);
      accc[m][1] += (d[0] * zi + d[1] * zr) + (pr * bzi + pi * bzr);
      }
    }
  }
  // sum each copy over the 16 edge lanes of its row, then lane c = 0 stores
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) {
#pragma unroll
    for (int m = 0; m < kRNS; ++m)
#pragma unroll
      for (int u = 0; u < 4; ++u) accs[m][u] += __shfl_xor(accs[m][u], off, kWave);
#pragma unroll
    for (int m = 0; m < kRNC; ++m) {
      accc[m][0] += __shfl_xor(accc[m][0], off, kWave);
      accc[m][1] += __shfl_xor(accc[m][1], off, kWave);
    }
  }
  if (c != 0) return;
  float* oi = a.out + i * a.D;
#pragma unroll
  for (int m = 0; m < kRNS; ++m) {
    const int col = 16 * m + 4 * q;
    if (m < a.ns && col < a.a0)
      *reinterpret_cast<float4*>(oi + col) = make_float4(accs[m][0], accs[m][1], accs[m][2], accs[m][3]);
  }
#pragma unroll
  for (int m = 0; m < kRNC; ++m)
    if (m < a.nc) *reinterpret_cast<float2*>(oi + a.tile_col[m] + 2 * q) = make_float2(accc[m][0], accc[m][1]);
}

// A coefficient tile's source values and target gradient pieces for the lane
// (a scalar tile's four, a complex tile's pair in x and y), requested a tile
// ahead of their use so the walk does not wait a round trip per tile.
struct TileIn {
  float4 x, g;
};

__device__ __forceinline__ TileIn tile_in(const RadialConvArgs& a, int m, int q, const float* vj, const float* gt) {
  TileIn t{make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
  if (m < kRNS) {
    const int col = 16 * m + 4 * q;
    if (m < a.ns && col < a.a0) {
      t.x = *reinterpret_cast<const float4*>(vj + col);
      t.g = *reinterpret_cast<const float4*>(gt + col);
    }
  } else if (m - kRNS < a.nc) {
    const int col = a.tile_col[m - kRNS] + 2 * q;
    const float2 x = ld2(vj + col), g = ld2(gt + col);
    t.x = make_float4(x.x, x.y, 0.f, 0.f);
    t.g = make_float4(g.x, g.y, 0.f, 0.f);
  }
  return t;
}

// The backward of one coefficient tile for the lane's edge: the coefficients
// again (times w), the copy's value gradient into dv, and the coefficients'
// gradient dC (rows 4q..4q+3, D layout), from the tile's pieces `in`.
template <bool SPLIT>
__device__ __forceinline__ void tile_dc(const RadialConvArgs& a, const float* rf_s, const SplitTile* rs_s,
                                        const float* bias_s, int m, int lane, int q, const EdgeView& ev,
                                        const float (&bv)[4], const SplitB& hb, const TileIn& in,
                                        float (&dv)[4], float (&dc)[4]) {
  const floatx4 d = coefficients_of<SPLIT>(rf_s, rs_s, bias_s, m, lane, q, ev.w, bv, hb);
  if (m < kRNS) {
    const int col = 16 * m + 4 * q;
    dc[0] = dc[1] = dc[2] = dc[3] = 0.f;
    if (col < a.a0) {
      const float4 x = in.x;
      const float4 gv = in.g;
      dv[0] = fmaf(d[0], gv.x, dv[0]);
      dv[1] = fmaf(d[1], gv.y, dv[1]);
      dv[2] = fmaf(d[2], gv.z, dv[2]);
      dv[3] = fmaf(d[3], gv.w, dv[3]);
      dc[0] = ev.w * gv.x * x.x;
      dc[1] = ev.w * gv.y * x.y;
      dc[2] = ev.w * gv.z * x.z;
      dc[3] = ev.w * gv.w * x.w;
    }
    return;
  }
  const int mc = m - kRNS;
  const bool one = a.tile_n[mc] == 1;
  const float2 x = make_float2(in.x.x, in.x.y), gv = make_float2(in.g.x, in.g.y);
  const float tc = one ? ev.t1.x : ev.t2.x, ts = one ? ev.t1.y : ev.t2.y;
  const float pr = one ? ev.p1.x : ev.p2.x, pi = one ? ev.p1.y : ev.p2.y;
  const float zr = tc * x.x - ts * x.y, zi = tc * x.y + ts * x.x;
  // dz = conj(wA) g + p (wB) conj(g);  dv += conj(tau) dz
  const float bgr = d[2] * gv.x + d[3] * gv.y, bgi = d[3] * gv.x - d[2] * gv.y;
  const float dzr = (d[0] * gv.x + d[1] * gv.y) + (pr * bgr - pi * bgi);
  const float dzi = (d[0] * gv.y - d[1] * gv.x) + (pr * bgi + pi * bgr);
  dv[0] += tc * dzr + ts * dzi;
  dv[1] += tc * dzi - ts * dzr;
  // dA = w g conj(z);  dB = w (g conj(p)) z
  const float xr = gv.x * pr + gv.y * pi, xi = gv.y * pr - gv.x * pi;
  dc[0] = ev.w * (gv.x * zr + gv.y * zi);
  dc[1] = ev.w * (gv.y * zr - gv.x * zi);
  dc[2] = ev.w * (xr * zr - xi * zi);
  dc[3] = ev.w * (xr * zi + xi * zr);
}

// The backward over the coefficient tiles [T0, T1) (slots: scalar tiles
// 0..kRNS-1, then the complex tiles).  Each group of tiles is one launch with
// its own accumulators, so a wave holds dR, the bias column and dv for its
// tiles only; the per-edge work (loads, trunk, h~ transpose) is repeated per
// group, and the trunk's gradient, linear in dh~, is each group's share.
// The backward's walk for the coefficient tiles [T0, T1) (slots: scalar tiles
// 0..kRNS-1, then the complex tiles), for one wave: sources j_lo + lw, + nwx,
// ... of its XCD's eighth, its dR, bias column and dv accumulated for those
// tiles only, its partial row at `part_row`.
// Rows of the wave's 16 x 16 hand-over tile in LDS, padded to 20 floats: a
// 16-byte write's set of 8 lanes (c = 0..7 or 8..15 of one lane row) then meets
// 8 distinct bank quads (at 16 floats lanes c and c + 4 share one), and the
// 4-byte reads of a half-wave (rows 4 s + q, q = 0, 1) stay in distinct banks.
constexpr int kTRow = 20;

template <int NB, int T0, int T1, bool SPLIT>
__device__ __forceinline__ void backward_walk(const RadialConvArgs& a, float* partial, const float* rf_s,
                                              const SplitTile* rs_s, const float* rb_s, const float* bias_s,
                                              const float* w1s, float* T, int64_t gw, int64_t lw, int64_t nwx) {
  constexpr int G = T1 - T0;
  const int lane = threadIdx.x & 63, c = lane & 15, q = lane >> 4;
  // Workgroups go round-robin to the eight XCDs (gridDim.x is a multiple of 8): XCD x
  // walks the x-th eighth of the sources, so its waves' targets (rows of g) share its L2.
  const int64_t xcd = blockIdx.x & 7;
  const int64_t j_lo = a.n_nodes * xcd / 8, j_hi = a.n_nodes * (xcd + 1) / 8;
  floatx4 dr[G];
  float db[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    dr[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    db[i] = 0.f;
  }
  float dw1[4][NB], db1[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    db1[u] = 0.f;
#pragma unroll
    for (int k = 0; k < NB; ++k) dw1[u][k] = 0.f;
  }
  for (int64_t j = j_lo + lw; j < j_hi; j += nwx) {
    float dvx[G][4];  // scalar tiles use four, complex tiles two
#pragma unroll
    for (int i = 0; i < G; ++i) dvx[i][0] = dvx[i][1] = dvx[i][2] = dvx[i][3] = 0.f;
    const float* vj = a.v + j * a.D;
    const int64_t g0 = a.src_ptr[j], g1 = a.src_ptr[j + 1];
    for (int64_t base = g0; base < g1; base += 16) {
      const bool live = base + c < g1;
      const int64_t e = a.src_order[live ? base + c : g0];
      const EdgeView ev = with_radius(edge_view(a, e, a.target[e], live));
      float bas[NB], pre[4], h[4];
      trunk_of<NB>(a, w1s, ev.r, q, bas, pre, h);
      float bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) bv[u] = ev.w * h[u];
      SplitB hb{};
      if constexpr (SPLIT) hb = split_b(bv[0], bv[1], bv[2], bv[3]);
      // h~^T for dR's B operand: ht[s] = h_c(edge 4s + q)
      wave_sync();
      *reinterpret_cast<float4*>(T + c * kTRow + 4 * q) = make_float4(h[0], h[1], h[2], h[3]);
      wave_sync();
      float ht[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) ht[s] = T[(4 * s + q) * kTRow + c];
      const float* gt = a.g + ev.node * a.D;
      floatx4 dh[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
      static_assert(kRChunk == 1, "the tiles' pieces are requested one tile ahead");
      TileIn in_next = tile_in(a, T0, q, vj, gt);
      // kRChunk tiles at a time: dC and dh~ += R^T dC from the D layout, then dC through the
      // wave's LDS into the A-operand layout dC[row c][edge 4s + q] (one hand-over per
      // chunk), the bias column sums and dR += dC h~^T
#pragma unroll
      for (int i0 = 0; i0 < G; i0 += kRChunk) {
        float dcs[kRChunk][4];
        const TileIn in = in_next;
        if (i0 + 1 < G) in_next = tile_in(a, T0 + i0 + 1, q, vj, gt);
#pragma unroll
        for (int p = 0; p < kRChunk; ++p) {
          const int i = i0 + p, m = T0 + i;
          if (i < G && tile_live(a, m)) {
            tile_dc<SPLIT>(a, rf_s, rs_s, bias_s, m, lane, q, ev, bv, hb, in, dvx[i], dcs[p]);
#pragma unroll
            for (int r = 0; r < 4; ++r) dh[i & 1] = mfma16(rb_s[(m * 4 + r) * 64 + lane], dcs[p][r], dh[i & 1]);
          }
        }
        wave_sync();
#pragma unroll
        for (int p = 0; p < kRChunk; ++p) {
          const int i = i0 + p;
          if (i < G && tile_live(a, T0 + i))
            *reinterpret_cast<float4*>(T + p * 16 * kTRow + c * kTRow + 4 * q) =
                make_float4(dcs[p][0], dcs[p][1], dcs[p][2], dcs[p][3]);
        }
        wave_sync();
#pragma unroll
        for (int p = 0; p < kRChunk; ++p) {
          const int i = i0 + p;
          if (i < G && tile_live(a, T0 + i)) {
            float at[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) at[s] = T[p * 16 * kTRow + (4 * s + q) * kTRow + c];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              db[i] += at[s];
              dr[i] = mfma16(at[s], ht[s], dr[i]);
            }
          }
        }
      }
      // the trunk's backward for the lane's features 4q + u of its edge (this group's share of dh~)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float sg = frcp(1.f + fexp(-pre[u]));
        const float dp = (dh[0][u] + dh[1][u]) * sg * (1.f + pre[u] * (1.f - sg));
        db1[u] += dp;
#pragma unroll
        for (int k = 0; k < NB; ++k) dw1[u][k] = fmaf(dp, bas[k], dw1[u][k]);
      }
    }
    // dv_j for this group's copies: each summed over the 16 edge lanes of its row
#pragma unroll
    for (int off = 1; off < 16; off <<= 1)
#pragma unroll
      for (int i = 0; i < G; ++i)
#pragma unroll
        for (int u = 0; u < ((T0 + i) < kRNS ? 4 : 2); ++u) dvx[i][u] += __shfl_xor(dvx[i][u], off, kWave);
    if (c == 0) {
      float* dvj = a.dv + j * a.D;
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int m = T0 + i;
        if (m < kRNS) {
          const int col = 16 * m + 4 * q;
          if (m < a.ns && col < a.a0)
            *reinterpret_cast<float4*>(dvj + col) = make_float4(dvx[i][0], dvx[i][1], dvx[i][2], dvx[i][3]);
        } else if (m - kRNS < a.nc) {
          *reinterpret_cast<float2*>(dvj + a.tile_col[m - kRNS] + 2 * q) = make_float2(dvx[i][0], dvx[i][1]);
        }
      }
    }
  }
  // this wave's partial row: dR in lane layout and the bias column for its tiles (zero for
  // the other groups' tiles), its share of W1 and b1
  float* part = partial + gw * kRPart;
#pragma unroll
  for (int m = 0; m < kRNT; ++m) {
    floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
    float b = 0.f;
#pragma unroll
    for (int i = 0; i < G; ++i)
      if (T0 + i == m) {
        v = dr[i];
        b = db[i];
      }
    *reinterpret_cast<float4*>(part + m * 256 + lane * 4) = make_float4(v[0], v[1], v[2], v[3]);
    b += __shfl_xor(b, 16, kWave);
    b += __shfl_xor(b, 32, kWave);
    if (q == 0) part[kRPartDR + m * 16 + c] = b;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    float b = db1[u];
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) b += __shfl_xor(b, off, kWave);
    if (c == 0) part[kRPartDR + kRPartDB + 16 * kRMaxBasis + 4 * q + u] = b;
#pragma unroll
    for (int k = 0; k < kRMaxBasis; ++k) {
      float w = k < NB ? dw1[u][k < NB ? k : 0] : 0.f;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) w += __shfl_xor(w, off, kWave);
      if (c == 0) part[kRPartDR + kRPartDB + (4 * q + u) * kRMaxBasis + k] = w;
    }
  }
}

// Each group of tiles as a launch of its own: every wave walks its sources for
// the group's tiles; the per-edge work (loads, trunk, h~ transpose) is repeated
// per launch, and the trunk's gradient, linear in dh~, is each group's share.
template <int NB, int T0, int T1, bool SPLIT>
__global__ __launch_bounds__(kRThreads) void conv_radial_backward_kernel(RadialConvArgs a, float* partial) {
  __shared__ float rf_s[SPLIT ? 1 : kRNT * 4 * 64];
  __shared__ __attribute__((aligned(16))) SplitTile rs_s[SPLIT ? kRNT * kWave : 1];
  __shared__ float rb_s[kRNT * 4 * 64];
  __shared__ __attribute__((aligned(16))) float bias_s[kRNT * 16];
  __shared__ float w1s[16 * kRMaxBasis + 16];
  __shared__ __attribute__((aligned(16))) float tr_s[kRWaves][kRChunk * 16 * kTRow];
  if constexpr (SPLIT) {
    load_split(a, rs_s);
    load_tables(a, nullptr, rb_s, bias_s, w1s, NB);
  } else {
    load_tables(a, rf_s, rb_s, bias_s, w1s, NB);
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6;
  backward_walk<NB, T0, T1, SPLIT>(a, partial, rf_s, rs_s, rb_s, bias_s, w1s, tr_s[wave],
                                   (int64_t)blockIdx.x * kRWaves + wave,
                                   (int64_t)(blockIdx.x >> 3) * kRWaves + wave, (int64_t)(gridDim.x >> 3) * kRWaves);
}

// Both tile groups in one launch: the waves of a workgroup go in pairs, the
// even wave walking a source for the first group's tiles and the odd one for
// the second's, so the pair reads each edge's streams and rows within moments
// of each other (the second read hits the caches) instead of once per launch.
template <int NB, bool SPLIT>
__global__ __launch_bounds__(kRThreads) void conv_radial_backward_paired(RadialConvArgs a, float* partial) {
  __shared__ float rf_s[SPLIT ? 1 : kRNT * 4 * 64];
  __shared__ __attribute__((aligned(16))) SplitTile rs_s[SPLIT ? kRNT * kWave : 1];
  __shared__ float rb_s[kRNT * 4 * 64];
  __shared__ __attribute__((aligned(16))) float bias_s[kRNT * 16];
  __shared__ float w1s[16 * kRMaxBasis + 16];
  __shared__ __attribute__((aligned(16))) float tr_s[kRWaves][kRChunk * 16 * kTRow];
  if constexpr (SPLIT) {
    load_split(a, rs_s);
    load_tables(a, nullptr, rb_s, bias_s, w1s, NB);
  } else {
    load_tables(a, rf_s, rb_s, bias_s, w1s, NB);
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6;
  constexpr int kPairs = kRWaves / 2;
  const int64_t gw = (int64_t)blockIdx.x * kRWaves + wave;
  const int64_t lw = (int64_t)(blockIdx.x >> 3) * kPairs + (wave >> 1), nwx = (int64_t)(gridDim.x >> 3) * kPairs;
  if (wave & 1)
    backward_walk<NB, kRGroup, kRNT, SPLIT>(a, partial, rf_s, rs_s, rb_s, bias_s, w1s, tr_s[wave], gw, lw, nwx);
  else
    backward_walk<NB, 0, kRGroup, SPLIT>(a, partial, rf_s, rs_s, rb_s, bias_s, w1s, tr_s[wave], gw, lw, nwx);
}

// grad[p] = sum over the partial rows w (in order) of partial[w][p], in two
// passes: kRSlices slices of the rows summed in parallel (consecutive threads,
// consecutive columns), then the slices in order.  Deterministic.
constexpr int kRSlices = 32;

__global__ __launch_bounds__(256) void conv_radial_reduce_slices(const float* partial, int64_t n_rows, float* slices) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  const int sl = blockIdx.y;
  if (p >= kRPart) return;
  const int64_t w0 = n_rows * sl / kRSlices, w1 = n_rows * (sl + 1) / kRSlices;
  float acc = 0.f;
  for (int64_t w = w0; w < w1; ++w) acc += partial[w * kRPart + p];
  slices[(int64_t)sl * kRPart + p] = acc;
}

__global__ __launch_bounds__(256) void conv_radial_reduce_kernel(const float* slices, float* grad) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= kRPart) return;
  float acc = 0.f;
#pragma unroll 8
  for (int sl = 0; sl < kRSlices; ++sl) acc += slices[(int64_t)sl * kRPart + p];
  grad[p] = acc;
}


int live_groups(int nc) {
  const int slots = kRNS + nc;
  return (slots + kRGroup - 1) / kRGroup;
}

template <int NB, bool SPLIT>
void launch_backward_groups(const RadialConvArgs& a, float* partial, int64_t rows, int groups, dim3 grid,
                            hipStream_t s) {
  static_assert(kRGroups == 2, "two tile groups");
  hipLaunchKernelGGL((conv_radial_backward_kernel<NB, 0, kRGroup, SPLIT>), grid, dim3(kRThreads), 0, s, a, partial);
  if (groups > 1)
    hipLaunchKernelGGL((conv_radial_backward_kernel<NB, kRGroup, kRNT, SPLIT>), grid, dim3(kRThreads), 0, s, a,
                       partial + rows * kRPart);
}

// GM_CONV_PAIRED=0: the tile groups as launches of their own.
inline bool paired_backward() {
  const char* v = std::getenv("GM_CONV_PAIRED");
  return v == nullptr || v[0] != '0';
}

// The backward's walks; returns the partial rows written (for the reduction).
template <int NB>
int64_t launch_backward_groups(const RadialConvArgs& a, float* partial, int64_t rows, int groups, dim3 grid,
                               hipStream_t s) {
  const bool split = split_products();
  if (groups > 1 && paired_backward()) {
    if (split)
      hipLaunchKernelGGL((conv_radial_backward_paired<NB, true>), grid, dim3(kRThreads), 0, s, a, partial);
    else
      hipLaunchKernelGGL((conv_radial_backward_paired<NB, false>), grid, dim3(kRThreads), 0, s, a, partial);
    return rows;
  }
  if (split)
    launch_backward_groups<NB, true>(a, partial, rows, groups, grid, s);
  else
    launch_backward_groups<NB, false>(a, partial, rows, groups, grid, s);
  return rows * groups;
}

// The forward's split form is held to four waves a SIMD (its registers would
// otherwise allow three): 12.3 ms (fp32) -> 12.8 (split, three waves) -> 11.2 ms
// (split, four waves) at 256x512, B = 4.
template <int NB>
void launch_forward(const RadialConvArgs& a, dim3 grid, hipStream_t s) {
  if (split_products())
    hipLaunchKernelGGL((conv_radial_forward_kernel<NB, true>), grid, dim3(kRThreads), 0, s, a);
  else
    hipLaunchKernelGGL((conv_radial_forward_kernel<NB, false>), grid, dim3(kRThreads), 0, s, a);
}

int prepare(RadialConvArgs& a, const float* v, const float* rf, const float* rbias, const float* rb, const float* w1,
            const float* b1,
            const float* centers_host, int64_t nb, double width, const float* transport, const float* angular,
            const float* rho, const float* weights, const int64_t* row_ptr, const int64_t* source, int64_t n_nodes,
            int64_t n_edges, int64_t D, int64_t orders, int64_t a0, int64_t ns, int64_t nc, const int32_t* tile_n,
            const int32_t* tile_col) {
  a = RadialConvArgs{};
  GM_REQUIRE(n_nodes >= 0 && n_edges >= 0, "sizes must be non-negative");
  GM_REQUIRE(n_nodes < (int64_t(1) << 31) * kRWaves, "too many nodes for one launch");
  GM_REQUIRE(nb == 4 || nb == 6 || nb == 8, "the radial basis must have 4, 6 or 8 functions");
  GM_REQUIRE(width > 0, "the basis width must be positive");
  GM_REQUIRE(ns >= 0 && ns <= kRNS && nc >= 0 && nc <= kRNC, "at most 32 scalar and 64 complex copies");
  GM_REQUIRE(a0 >= 0 && a0 % 4 == 0 && a0 <= 16 * ns && a0 > 16 * (ns - 1), "a_0 must be a multiple of 4 filling ns tiles");
  GM_REQUIRE(orders >= 5, "the phase tables must hold orders 0..4");
  GM_REQUIRE(D % 4 == 0, "D must be a multiple of 4");
  int covered = (int)a0;
  for (int m = 0; m < nc; ++m) {
    GM_REQUIRE(tile_n[m] == 1 || tile_n[m] == 2, "complex tiles hold frequency 1 or 2");
    GM_REQUIRE(tile_col[m] >= a0 && tile_col[m] % 2 == 0 && tile_col[m] + 8 <= D, "a complex tile's columns lie in the field");
    covered += 8;
  }
  GM_REQUIRE(covered == D, "the tiles must cover the flat width D exactly");
  if (n_nodes > 0) GM_REQUIRE(v && rf && rbias && w1 && row_ptr, "v, the tables and row_ptr must be device pointers");
  if (n_edges > 0) GM_REQUIRE(transport && angular && rho && weights && source, "the per-edge tables must be device pointers");
  a.v = v;
  a.rf = rf;
  a.rbias = rbias;
  a.rb = rb;
  a.w1 = w1;
  a.b1 = b1;
  a.transport = transport;
  a.angular = angular;
  a.rho = rho;
  a.weights = weights;
  a.row_ptr = row_ptr;
  a.source = source;
  a.n_nodes = n_nodes;
  a.D = (int)D;
  a.orders = (int)orders;
  a.ns = (int)ns;
  a.nc = (int)nc;
  a.a0 = (int)a0;
  a.inv_width = (float)(1.0 / width);
  for (int k = 0; k < kRMaxBasis; ++k) a.centers[k] = k < nb ? centers_host[k] : 0.f;
  for (int m = 0; m < kRNC; ++m) {
    a.tile_n[m] = m < nc ? tile_n[m] : 0;
    a.tile_col[m] = m < nc ? tile_col[m] : 0;
  }
  return GM_OK;
}

}  // namespace
}  // namespace gm

extern "C" int64_t gm_conv_radial_partial_row(void) { return gm::kRPart; }

extern "C" int64_t gm_conv_radial_backward_groups(int64_t nc) { return gm::live_groups((int)nc); }

// Rows of the backward's workspace for n_blocks workgroups: the partial rows of every
// tile group, then the reduction's slices.
extern "C" int64_t gm_conv_radial_workspace_rows(int64_t n_blocks) {
  return n_blocks * gm::kRWaves * gm::kRGroups + gm::kRSlices;
}

extern "C" int gm_conv_radial_forward_f32(const float* v, const float* rf, const float* rbias, const float* w1,
                                          const float* b1,
                                          const float* centers, int64_t nb, double width, const float* transport,
                                          const float* angular, const float* rho, const float* weights,
                                          const int64_t* row_ptr, const int64_t* source, int64_t n_nodes,
                                          int64_t n_edges, int64_t D, int64_t orders, int64_t a0, int64_t ns,
                                          int64_t nc, const int32_t* tile_n, const int32_t* tile_col, float* out,
                                          void* stream) {
  gm::RadialConvArgs a;
  const int status = gm::prepare(a, v, rf, rbias, nullptr, w1, b1, centers, nb, width, transport, angular, rho, weights,
                                 row_ptr, source, n_nodes, n_edges, D, orders, a0, ns, nc, tile_n, tile_col);
  if (status != GM_OK) return status;
  if (n_nodes == 0) return GM_OK;
  GM_REQUIRE(out, "out must be a device pointer");
  a.out = out;
  const dim3 grid((unsigned)((n_nodes + gm::kRWaves - 1) / gm::kRWaves));
  hipStream_t s = (hipStream_t)stream;
  if (nb == 4)
    gm::launch_forward<4>(a, grid, s);
  else if (nb == 6)
    gm::launch_forward<6>(a, grid, s);
  else
    gm::launch_forward<8>(a, grid, s);
  return gm::check_launch("conv_radial_forward");
}

extern "C" int gm_conv_radial_backward_f32(const float* g, const float* v, const float* rf, const float* rbias,
                                           const float* rb,
                                           const float* w1, const float* b1, const float* centers, int64_t nb,
                                           double width, const float* transport, const float* angular,
                                           const float* rho, const float* weights, const int64_t* src_ptr,
                                           const int64_t* src_order, const int64_t* target, int64_t n_nodes,
                                           int64_t n_edges, int64_t D, int64_t orders, int64_t a0, int64_t ns,
                                           int64_t nc, const int32_t* tile_n, const int32_t* tile_col,
                                           int64_t n_blocks, float* partial, float* dv, float* grad, void* stream) {
  gm::RadialConvArgs a;
  const int status = gm::prepare(a, v, rf, rbias, rb, w1, b1, centers, nb, width, transport, angular, rho, weights, src_ptr,
                                 src_order, n_nodes, n_edges, D, orders, a0, ns, nc, tile_n, tile_col);
  if (status != GM_OK) return status;
  GM_REQUIRE(n_blocks >= 8 && n_blocks <= 65536 && n_blocks % 8 == 0, "n_blocks must be a multiple of 8 in 8..65536");
  GM_REQUIRE(grad && partial, "grad and partial must be device pointers");
  if (n_nodes > 0) GM_REQUIRE(g && dv && rb && src_ptr, "g, dv, rb and src_ptr must be device pointers");
  if (n_edges > 0) GM_REQUIRE(src_order && target, "src_order and target must be device pointers");
  a.g = g;
  a.dv = dv;
  a.src_ptr = src_ptr;
  a.src_order = src_order;
  a.target = target;
  a.row_ptr = nullptr;
  a.source = nullptr;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)n_blocks);
  const int64_t rows = n_blocks * (int64_t)gm::kRWaves;
  const int groups = gm::live_groups((int)nc);
  int64_t written = 0;
  if (nb == 4) {
    written = gm::launch_backward_groups<4>(a, partial, rows, groups, grid, s);
  } else if (nb == 6) {
    written = gm::launch_backward_groups<6>(a, partial, rows, groups, grid, s);
  } else {
    written = gm::launch_backward_groups<8>(a, partial, rows, groups, grid, s);
  }
  int st = gm::check_launch("conv_radial_backward");
  if (st != GM_OK) return st;
  // the slices' sums go to the rows past the partial rows (the caller sizes partial for them)
  float* slices = partial + rows * gm::kRGroups * gm::kRPart;
  hipLaunchKernelGGL(gm::conv_radial_reduce_slices, dim3((gm::kRPart + 255) / 256, gm::kRSlices), dim3(256), 0, s,
                     partial, written, slices);
  hipLaunchKernelGGL(gm::conv_radial_reduce_kernel, dim3((gm::kRPart + 255) / 256), dim3(256), 0, s, slices, grad);
  return gm::check_launch("conv_radial_reduce");
}
