// The value kernels' radial trunk for every head of a layer in one pass
// (CDNA4, gfx950).
//
// Per edge e with r = rho_e = d_e / cutoff and s = r^2:
//   b_k(e)      = exp(-((s - mu_k) / sigma)^2 / 2),  k < B     (the Gaussian basis, shared by the heads)
//   pre_h,t(e)  = sum_k W_h[t, k] b_k(e) + c_h[t],   t < T     (each head's Linear)
//   h_h,t(e)    = pre / (1 + exp(-pre))                        (SiLU)
// and from dh the parameter gradients dW_h = sum_e dpre_h(e) b(e)^T,
// dc_h = sum_e dpre_h(e) with dpre = dh * SiLU'(pre) (the distances are
// geometry and take no gradient).  The reference forms this per head with
// torch ops (nn/kernels.py:191-231 _GaussianRadialBasis, :108-117
// apply_radial_trunk, :605-607 _trunk_hidden; one Linear + SiLU layer).
//
// Both directions: persistent wavefronts over 16-edge tiles, the basis once
// per tile for every head, each head's pre-activations on MFMA.  The forward
// stores SiLU(pre) as whole 1 KB tiles; the backward forms each head's
// (T x B + T) gradient terms on MFMA with the accumulators in registers across
// the wave's tiles, one partial row per wavefront, and a second kernel sums
// the partial rows in a fixed order.  No atomics:
// the parameter gradients are deterministic.
//
// The features (and their gradients) may be kept in bfloat16 (the trunk of a
// bfloat16 block): the forward rounds each feature to nearest even as it
// stores it, the backward widens dh exactly as it loads it; the arithmetic
// stays float32.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.hpp"
#include "split.hpp"

namespace gm {
namespace {

constexpr int kTrunkThreads = 256;

struct TrunkArgs {
  const float* rho;     // (E,)
  const float* weight;  // (H, T, B)
  const float* bias;    // (H, T) or null
  const float* centers; // (B,)
  const float* dh;      // (H, E, T) backward
  float* h;             // (H, E, T) forward
  const uint16_t* dhb;  // (H, E, T) backward, bfloat16 (in place of dh)
  uint16_t* hb;         // (H, E, T) forward, bfloat16 (in place of h)
  float* partial;       // (n_blocks, H, T * B + T) backward
  int64_t n_edges;
  int H, T, B;
  float inv_width;      // 1 / sigma
  int rho_vec4;         // backward: rho 16-byte aligned (4 edges per load)
};

// exp(x) as 2^(x log2 e) on the hardware exponential, and 1 / x on the
// hardware reciprocal (each within about an ulp of the rounded result; the
// trunk's features and gradients then stay within a few 1e-7 relative of
// the precise ones).
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float sigmoid_of(float x) { return fast_rcp(1.f + fast_exp(-x)); }

// The heads' parameters and the basis centres are read-only for the whole
// launch: read through the constant address space, they become uniform
// (scalar) loads and SGPR operands.
typedef const __attribute__((address_space(4))) float* ConstPtr;
__device__ __forceinline__ ConstPtr as_const(const float* p) { return (ConstPtr)p; }

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kTrunkMaxHeads = 8;
constexpr int kTrunkWaves = kTrunkThreads / 64;

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Persistent wavefronts over tiles of 16 edges (tile w, w + W, ... for wave w
// of W).  Lane l = 16 q + c (q = l / 16, c = l % 16) of the 16x16x4 MFMA:
//   pre (feature 4q + r, edge c), r < 4, = D1 = A1 B1 with
//     A1[feature c][basis q + 4s] = W[c][q + 4s] and B1[basis q + 4s][edge c] = b_{q+4s}(edge c), s = 0, 1
//     (the basis once per tile, shared by every head; the bias as the weight of a
//     basis entry that is 1, in the first free slot), so a lane's four
//     features of one edge come from one 16-byte load of its dh row;
//   dp = dh * SiLU'(pre), turned through the wave's LDS tile (feature rows of
//     16 edges padded to 20 floats, so neither the writes nor the 16-byte
//     reads meet in a bank) to
//     B2_j[q][feature c] = dp(feature c, edge 4q + j), j < 4 (one 16-byte LDS read);
//   D2[m][feature c] += sum over j of A2_j B2_j with
//     A2_j[m = c][k = q] = b_c(edge 4q + j) (c < B), 1 at c = B, 0 above,
//   so D2's rows m < B are dW^T and row B is db, accumulated over the wave's
//   tiles in registers for every head.  Edges past the end read dh as zero and add nothing.
// SPLIT: D1 as split-bf16 products (split.hpp), off the fp32 datapath that the
// rest of the tile's arithmetic shares with fp32 MFMA: a lane's contraction
// slots s are basis entries k = 4q + s (the bias at k = B); the heads' A1
// pieces split once per workgroup into LDS, the basis pieces once per tile.
template <int B, bool B16 = false, bool SPLIT = false>
__global__ __launch_bounds__(kTrunkThreads) void trunk_backward_mfma(TrunkArgs a) {
  constexpr int T = 16, P = T * B + T, LDT = T + 4;
  __shared__ __align__(16) float stage[kTrunkWaves][T * LDT];  // per wave: dp as [feature][edge]
  __shared__ __align__(16) u32x4 a1p[SPLIT ? 2 * kTrunkMaxHeads * 64 : 1];  // [head][hm, hl][lane]
  const int lane = threadIdx.x & 63, q = lane >> 4, c = lane & 15, wv = threadIdx.x >> 6;
  if constexpr (SPLIT) {
    for (int i = threadIdx.x; i < kTrunkMaxHeads * 64; i += kTrunkThreads) {
      const int h = i >> 6, l = i & 63, f = l & 15, k0 = 4 * (l >> 4);
      float x[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = k0 + s;
        x[s] = h >= a.H ? 0.f
                        : (k < B ? a.weight[(h * T + f) * B + k] : ((k == B && a.bias) ? a.bias[h * T + f] : 0.f));
      }
      const SplitA sa = split_a(x[0], x[1], x[2], x[3]);
      a1p[128 * h + l] = sa.hm;  // consecutive lanes read consecutive 16-byte pieces
      a1p[128 * h + 64 + l] = sa.hl;
    }
    __syncthreads();
  }
  float* tile_lds = stage[wv];
  const int64_t wave = (int64_t)blockIdx.x * kTrunkWaves + wv;
  const int64_t n_waves = (int64_t)gridDim.x * kTrunkWaves;
  const int64_t n_tiles = (a.n_edges + 15) / 16;
  const ConstPtr centers = as_const(a.centers);
  // A1 operands per head: basis index k = q + 4s takes W[c][k] for k < B, the bias at k = B (its basis
  // entry is 1), zero above; B = 8 puts the bias in a third step (k = 8, lane q = 0)
  float w0[kTrunkMaxHeads], w1[kTrunkMaxHeads], w2[kTrunkMaxHeads];
  floatx4 acc[kTrunkMaxHeads];
  auto a1_weight = [&](int h, int k) {
    if (h >= a.H) return 0.f;
    if (k < B) return a.weight[(h * T + c) * B + k];
    return (k == B && a.bias) ? a.bias[h * T + c] : 0.f;
  };
#pragma unroll
  for (int h = 0; h < kTrunkMaxHeads; ++h) {
    if constexpr (!SPLIT) {
      w0[h] = a1_weight(h, q);
      w1[h] = a1_weight(h, q + 4);
      w2[h] = q == 0 ? a1_weight(h, 8) : 0.f;
    }
    acc[h] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  const float mu0 = q < B ? centers[q] : 0.f, mu1 = q + 4 < B ? centers[q + 4] : 0.f;
  const float mu2 = c < B ? centers[c] : 0.f;
  float mus[4];  // SPLIT: the centres of the lane's basis slots 4q + s
#pragma unroll
  for (int s = 0; s < 4; ++s) mus[s] = 4 * q + s < B ? centers[4 * q + s] : 0.f;
  const float iw = a.inv_width;
  auto gauss = [iw](float r, float mu) {
    const float z = (r * r - mu) * iw;
    return fast_exp(-0.5f * z * z);
  };
  // dh of head h for this lane's edge c of a tile, features 4q..4q+3 (zero past the end),
  // as loaded: four floats, or four bfloat16 in one 8-byte piece (widened where used, so
  // the next tile's loads stay in flight)
  using Raw = typename std::conditional<B16, uint2, float4>::type;
  const int lane_off = c * T + 4 * q;  // the lane's piece within a tile's rows of one head
  auto load_dh = [&](int64_t e0, int h) -> Raw {
    if constexpr (B16) {
      const uint16_t* tile_dh = a.dhb + ((int64_t)h * a.n_edges + e0) * T;  // uniform: a scalar base
      if (e0 + 16 <= a.n_edges) return *reinterpret_cast<const uint2*>(tile_dh + lane_off);
      return e0 + c < a.n_edges ? *reinterpret_cast<const uint2*>(tile_dh + lane_off) : make_uint2(0u, 0u);
    } else {
      const float* tile_dh = a.dh + ((int64_t)h * a.n_edges + e0) * T;  // uniform: a scalar base
      if (e0 + 16 <= a.n_edges)  // every tile but the last: no per-lane test
        return *reinterpret_cast<const float4*>(tile_dh + lane_off);
      return e0 + c < a.n_edges ? *reinterpret_cast<const float4*>(tile_dh + lane_off)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto widen = [](const Raw& v) -> float4 {
    if constexpr (B16)
      return make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
    else
      return v;
  };
  // rho of a tile: edge c (the B1 operand) and edges 4q..4q+3 (the A2 operands)
  auto load_rho = [&](int64_t e0, float& rc, float* r4) {
    rc = e0 + c < a.n_edges ? a.rho[e0 + c] : 0.f;
    if (e0 + 16 <= a.n_edges && a.rho_vec4) {
      const float4 v = *reinterpret_cast<const float4*>(a.rho + e0 + 4 * q);
      r4[0] = v.x;
      r4[1] = v.y;
      r4[2] = v.z;
      r4[3] = v.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) r4[j] = e0 + 4 * q + j < a.n_edges ? a.rho[e0 + 4 * q + j] : 0.f;
    }
  };
  // Loads complete in issue order, so each tile issues the next tile's rho first and then, head by
  // head, the next tile's dh into the register it has just consumed: nothing waited for is younger
  // than what the wave needs next.
  float rc, r4[4];
  load_rho(wave * 16, rc, r4);
  Raw g[kTrunkMaxHeads];
#pragma unroll
  for (int h = 0; h < kTrunkMaxHeads; ++h) g[h] = h < a.H ? load_dh(wave * 16, h) : Raw{};
  for (int64_t tile = wave; tile < n_tiles; tile += n_waves) {
    const int64_t e_next = (tile + n_waves) * 16;
    float rc_next, r4_next[4];
    load_rho(e_next, rc_next, r4_next);
    const float b1_0 = q < B ? gauss(rc, mu0) : (q == B ? 1.f : 0.f);
    const float b1_1 = q + 4 < B ? gauss(rc, mu1) : (q + 4 == B ? 1.f : 0.f);
    const float b1_2 = q == 0 ? 1.f : 0.f;  // the bias step when B = 8
    float a2[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) a2[j] = c < B ? gauss(r4[j], mu2) : (c == B ? 1.f : 0.f);
    SplitB b1p{};
    if constexpr (SPLIT) {
      float x[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) x[s] = 4 * q + s < B ? gauss(rc, mus[s]) : (4 * q + s == B ? 1.f : 0.f);
      b1p = split_b(x[0], x[1], x[2], x[3]);
    }
#pragma unroll
    for (int h = 0; h < kTrunkMaxHeads; ++h) {
      if (h >= a.H) break;
      floatx4 pre;
      if constexpr (SPLIT) {
        pre = mfma_split(SplitA{a1p[128 * h + lane], a1p[128 * h + 64 + lane]}, b1p, floatx4{0.f, 0.f, 0.f, 0.f});
      } else {
        pre = mfma16(w0[h], b1_0, floatx4{0.f, 0.f, 0.f, 0.f});
        pre = mfma16(w1[h], b1_1, pre);
        if (B == 8) pre = mfma16(w2[h], b1_2, pre);
      }
      const float4 gw = widen(g[h]);
      const float gv[4] = {gw.x, gw.y, gw.z, gw.w};
      g[h] = load_dh(e_next, h);
      wave_sync();  // the previous head's LDS reads are done
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sg = sigmoid_of(pre[r]);
        tile_lds[(4 * q + r) * LDT + c] = gv[r] * sg * (1.f + pre[r] * (1.f - sg));
      }
      wave_sync();
      const float4 dp = *reinterpret_cast<const float4*>(tile_lds + c * LDT + 4 * q);  // dp(feature c, edges 4q..4q+3)
      acc[h] = mfma16(a2[0], dp.x, acc[h]);
      acc[h] = mfma16(a2[1], dp.y, acc[h]);
      acc[h] = mfma16(a2[2], dp.z, acc[h]);
      acc[h] = mfma16(a2[3], dp.w, acc[h]);
    }
    rc = rc_next;
#pragma unroll
    for (int j = 0; j < 4; ++j) r4[j] = r4_next[j];
  }
  // this wave's partial row: dW[h][c][m] for D2 rows m < B, db[h][c] for row m = B
  float* out = a.partial + wave * a.H * P;
#pragma unroll
  for (int h = 0; h < kTrunkMaxHeads; ++h) {
    if (h >= a.H) break;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * q + r;
      if (m < B)
        out[h * P + c * B + m] = acc[h][r];
      else if (m == B)
        out[h * P + T * B + c] = acc[h][r];
    }
  }
}

// Persistent wavefronts over 16-edge tiles, as the backward: every head's
// pre-activations (feature 4q + r, edge c) from the same two or three MFMAs
// (the basis once per tile), SiLU in registers, and each lane's four features
// of its edge stored as one 16-byte store (a head's tile is one contiguous 1 KB).
template <int B, bool B16 = false>
__global__ __launch_bounds__(kTrunkThreads) void trunk_forward_mfma(TrunkArgs a) {
  constexpr int T = 16;
  const int lane = threadIdx.x & 63, q = lane >> 4, c = lane & 15;
  const int64_t wave = (int64_t)blockIdx.x * kTrunkWaves + (threadIdx.x >> 6);
  const int64_t n_waves = (int64_t)gridDim.x * kTrunkWaves;
  const int64_t n_tiles = (a.n_edges + 15) / 16;
  const ConstPtr centers = as_const(a.centers);
  float w0[kTrunkMaxHeads], w1[kTrunkMaxHeads], w2[kTrunkMaxHeads];
  auto a1_weight = [&](int h, int k) {
    if (h >= a.H) return 0.f;
    if (k < B) return a.weight[(h * T + c) * B + k];
    return (k == B && a.bias) ? a.bias[h * T + c] : 0.f;
  };
#pragma unroll
  for (int h = 0; h < kTrunkMaxHeads; ++h) {
    w0[h] = a1_weight(h, q);
    w1[h] = a1_weight(h, q + 4);
    w2[h] = q == 0 ? a1_weight(h, 8) : 0.f;
  }
  const float mu0 = q < B ? centers[q] : 0.f, mu1 = q + 4 < B ? centers[q + 4] : 0.f;
  const float iw = a.inv_width;
  auto gauss = [iw](float r, float mu) {
    const float z = (r * r - mu) * iw;
    return fast_exp(-0.5f * z * z);
  };
  const float b1_2 = q == 0 ? 1.f : 0.f;
  float rc = wave * 16 + c < a.n_edges ? a.rho[wave * 16 + c] : 0.f;
  for (int64_t tile = wave; tile < n_tiles; tile += n_waves) {
    const int64_t e0 = tile * 16, e_next = (tile + n_waves) * 16;
    const bool edge_in = e0 + c < a.n_edges;
    const float rn = e_next + c < a.n_edges ? a.rho[e_next + c] : 0.f;  // the next tile's, ahead of the stores
    const float b1_0 = q < B ? gauss(rc, mu0) : (q == B ? 1.f : 0.f);
    const float b1_1 = q + 4 < B ? gauss(rc, mu1) : (q + 4 == B ? 1.f : 0.f);
#pragma unroll
    for (int h = 0; h < kTrunkMaxHeads; ++h) {
      if (h >= a.H) break;
      floatx4 pre = mfma16(w0[h], b1_0, floatx4{0.f, 0.f, 0.f, 0.f});
      pre = mfma16(w1[h], b1_1, pre);
      if (B == 8) pre = mfma16(w2[h], b1_2, pre);
      float4 out;
      out.x = pre[0] * sigmoid_of(pre[0]);
      out.y = pre[1] * sigmoid_of(pre[1]);
      out.z = pre[2] * sigmoid_of(pre[2]);
      out.w = pre[3] * sigmoid_of(pre[3]);
      const int64_t at = ((int64_t)h * a.n_edges + e0 + c) * T + 4 * q;
      if constexpr (B16) {
        if (edge_in) *reinterpret_cast<uint2*>(a.hb + at) = make_uint2(pack_bf16(out.x, out.y), pack_bf16(out.z, out.w));
      } else {
        if (edge_in) *reinterpret_cast<float4*>(a.h + at) = out;
      }
    }
    rc = rn;
  }
}

// out[i] = sum over rows r of partial[r][i]: one workgroup per column, each
// thread summing rows t, t + 256, ... in order, then a fixed tree.
__global__ __launch_bounds__(256) void trunk_reduce_kernel(const float* partial, int64_t rows, int HP, float* out) {
  __shared__ float buf[256];
  const int i = blockIdx.x;
  float s = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += 256) s += partial[r * HP + i];
  buf[threadIdx.x] = s;
  __syncthreads();
  for (int step = 128; step > 0; step >>= 1) {
    if (threadIdx.x < step) buf[threadIdx.x] += buf[threadIdx.x + step];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[i] = buf[0];
}

int prepare(TrunkArgs& a, const float* rho, const float* weight, const float* bias, const float* centers,
            int64_t n_edges, int64_t H, int64_t T, int64_t B, double width) {
  a = TrunkArgs{};
  GM_REQUIRE(n_edges >= 0, "n_edges must be non-negative");
  GM_REQUIRE(H >= 1 && H <= 8, "between 1 and 8 heads");
  GM_REQUIRE((T == 16 && (B == 8 || B == 4 || B == 6)), "this build's trunk kernel takes 16 features over 4, 6 or 8 basis functions");
  GM_REQUIRE(width > 0.0, "the basis width must be positive");
  if (n_edges > 0) GM_REQUIRE(rho && weight && centers, "rho, weight and centers must be device pointers");
  a.rho = rho;
  a.weight = weight;
  a.bias = bias;
  a.centers = centers;
  a.n_edges = n_edges;
  a.H = (int)H;
  a.T = (int)T;
  a.B = (int)B;
  a.inv_width = (float)(1.0 / width);
  return GM_OK;
}

constexpr int64_t kTrunkBlocks = 2048;  // about this many workgroups (waves stride over 16-edge tiles)

// The grid of a pass over n_edges: one tile per wave up to about kTrunkBlocks
// workgroups, in whole rounds of the kernel's resident workgroups (the waves'
// shares differ by at most a tile, so a partial last round would run on a
// fraction of the chip).  The grid (and so the backward's partial rows)
// follows the B = 8 instance's occupancy for every basis size, per storage
// type of the features (the bfloat16 backward holds fewer registers).
// The backward's instance for features of this storage type: the split
// pre-activations unless GM_SPLIT_PRODUCTS=0.
template <int B>
const void* backward_kernel(bool b16) {
  if (split_products())
    return b16 ? (const void*)trunk_backward_mfma<B, true, true> : (const void*)trunk_backward_mfma<B, false, true>;
  return b16 ? (const void*)trunk_backward_mfma<B, true> : (const void*)trunk_backward_mfma<B>;
}

int64_t trunk_blocks(int64_t n_edges, bool forward, bool b16) {
  const int64_t need = (n_edges + 16 * kTrunkWaves - 1) / (16 * kTrunkWaves);  // one tile per wave
  const void* kernel = forward ? (b16 ? (const void*)trunk_forward_mfma<8, true> : (const void*)trunk_forward_mfma<8>)
                               : backward_kernel<8>(b16);
  const int64_t full = whole_rounds(kTrunkBlocks, resident_blocks(kernel, kTrunkThreads));
  return need < full ? (need > 0 ? need : 1) : full;
}

int64_t backward_blocks(int64_t n_edges, bool b16) { return trunk_blocks(n_edges, false, b16); }

template <int B>
void launch(bool forward, const TrunkArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)trunk_blocks(a.n_edges, forward, forward ? a.hb != nullptr : a.dhb != nullptr)),
      block(kTrunkThreads);
  if (forward) {
    if (a.hb)
      hipLaunchKernelGGL((trunk_forward_mfma<B, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((trunk_forward_mfma<B>), grid, block, 0, stream, a);
  } else if (split_products()) {
    if (a.dhb)
      hipLaunchKernelGGL((trunk_backward_mfma<B, true, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((trunk_backward_mfma<B, false, true>), grid, block, 0, stream, a);
  } else {
    if (a.dhb)
      hipLaunchKernelGGL((trunk_backward_mfma<B, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((trunk_backward_mfma<B>), grid, block, 0, stream, a);
  }
}

void launch_any(bool forward, const TrunkArgs& a, hipStream_t stream) {
  if (a.B == 8)
    launch<8>(forward, a, stream);
  else if (a.B == 6)
    launch<6>(forward, a, stream);
  else
    launch<4>(forward, a, stream);
}

}  // namespace
}  // namespace gm

// Partial rows of the backward: one per wavefront of its grid (the larger of the
// float32 and bfloat16 instances' grids).
extern "C" int64_t gm_radial_trunk_partials(int64_t n_edges) {
  const int64_t f = gm::backward_blocks(n_edges, false), b = gm::backward_blocks(n_edges, true);
  return (f > b ? f : b) * gm::kTrunkWaves;
}

namespace gm {
namespace {

// h (float32) or hb (bfloat16): exactly one is given.
int trunk_forward(const float* rho, const float* weight, const float* bias, const float* centers, int64_t n_edges,
                  int64_t H, int64_t T, int64_t B, double width, float* h, uint16_t* hb, void* stream) {
  TrunkArgs a;
  const int status = prepare(a, rho, weight, bias, centers, n_edges, H, T, B, width);
  if (status != GM_OK) return status;
  if (n_edges == 0) return GM_OK;
  if (hb)
    GM_REQUIRE(aligned(hb, 8), "h must be an 8-byte aligned device pointer");
  else
    GM_REQUIRE(h && aligned(h, 16), "h must be a 16-byte aligned device pointer");
  a.h = h;
  a.hb = hb;
  launch_any(true, a, (hipStream_t)stream);
  return check_launch("radial_trunk_forward");
}

// dh (float32) or dhb (bfloat16): exactly one is given.
int trunk_backward(const float* dh, const uint16_t* dhb, const float* rho, const float* weight, const float* bias,
                   const float* centers, int64_t n_edges, int64_t H, int64_t T, int64_t B, double width,
                   float* partial, float* dparams, void* stream) {
  TrunkArgs a;
  const int status = prepare(a, rho, weight, bias, centers, n_edges, H, T, B, width);
  if (status != GM_OK) return status;
  GM_REQUIRE(dparams, "dparams must be a device pointer");
  const int HP = (int)(H * (T * B + T));
  if (n_edges == 0) {
    hipLaunchKernelGGL(trunk_reduce_kernel, dim3(HP), dim3(256), 0, (hipStream_t)stream, partial, (int64_t)0, HP,
                       dparams);
    return check_launch("radial_trunk_backward (empty)");
  }
  if (dhb)
    GM_REQUIRE(aligned(dhb, 8) && partial, "dh (8-byte aligned) and partial must be device pointers");
  else
    GM_REQUIRE(dh && aligned(dh, 16) && partial, "dh (16-byte aligned) and partial must be device pointers");
  a.dh = dh;
  a.dhb = dhb;
  a.partial = partial;
  a.rho_vec4 = aligned(rho, 16);
  launch_any(false, a, (hipStream_t)stream);
  int rc = check_launch("radial_trunk_backward");
  if (rc != GM_OK) return rc;
  hipLaunchKernelGGL(trunk_reduce_kernel, dim3(HP), dim3(256), 0, (hipStream_t)stream, partial,
                     backward_blocks(n_edges, dhb != nullptr) * kTrunkWaves, HP, dparams);
  return check_launch("radial_trunk_backward (reduce)");
}

}  // namespace
}  // namespace gm

extern "C" int gm_radial_trunk_forward_f32(const float* rho, const float* weight, const float* bias,
                                           const float* centers, int64_t n_edges, int64_t H, int64_t T, int64_t B,
                                           double width, float* h, void* stream) {
  return gm::trunk_forward(rho, weight, bias, centers, n_edges, H, T, B, width, h, nullptr, stream);
}

extern "C" int gm_radial_trunk_forward_bf16(const float* rho, const float* weight, const float* bias,
                                            const float* centers, int64_t n_edges, int64_t H, int64_t T, int64_t B,
                                            double width, uint16_t* h, void* stream) {
  GM_REQUIRE(h || n_edges == 0, "h must be a device pointer");
  return gm::trunk_forward(rho, weight, bias, centers, n_edges, H, T, B, width, nullptr, h, stream);
}

extern "C" int gm_radial_trunk_backward_f32(const float* dh, const float* rho, const float* weight, const float* bias,
                                            const float* centers, int64_t n_edges, int64_t H, int64_t T, int64_t B,
                                            double width, float* partial, float* dparams, void* stream) {
  return gm::trunk_backward(dh, nullptr, rho, weight, bias, centers, n_edges, H, T, B, width, partial, dparams, stream);
}

extern "C" int gm_radial_trunk_backward_bf16(const uint16_t* dh, const float* rho, const float* weight,
                                             const float* bias, const float* centers, int64_t n_edges, int64_t H,
                                             int64_t T, int64_t B, double width, float* partial, float* dparams,
                                             void* stream) {
  GM_REQUIRE(dh || n_edges == 0, "dh must be a device pointer");
  return gm::trunk_backward(nullptr, dh, rho, weight, bias, centers, n_edges, H, T, B, width, partial, dparams,
                            stream);
}
