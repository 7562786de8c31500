// The factored kernel's node-side channel mixing (CDNA4, gfx950): every
// head's node mixes Z_t(j) = W_t v_j for one input frequency as one real
// product over the nodes,
//
//   forward   mix (N, C) = v (N, w) M (w, C)
//   backward  dv (N, w)  = dmix M^T            (the node field's gradient)
//             dM (w, C)  = v^T dmix            (the mixing matrix's gradient)
//
// with v the node field's frequency-n reals (w <= 128, a strided view of the
// flat rows) and M the heads' real mixing matrix (every block's complex
// product and input conjugation encoded as reals; C = H K C_n columns).  The
// reference forms the same numbers as one complex einsum("ja,bat->jtb") per
// node vector and block group (nn/kernels.py:575-603, over _block_weights
// :506-536) and their gradients through autograd.
//
// All three are v_mfma_f32_16x16x4f32 products.  Lane l = 16 q + c of the
// MFMA supplies A[c][q] and B[q][c] and holds D[4 q + i][c], i < 4.
//
// * forward: the contraction is short, so each wave keeps its columns of M in
//   registers for the whole launch and streams 64-row tiles of v through LDS;
//   M is the A operand (D = mix^T), so a lane's four D entries are four
//   consecutive columns of one row: one 16-byte store each.
// * input gradient: 128-row tiles, each wave 32 rows over the whole
//   contraction, dmix and M staged per 64-column chunk in LDS; the
//   accumulators restart every four chunks into a running total, so no fp32
//   sum runs sequentially over more than 256 columns.
// * weight gradient: split over row ranges into partial (w, C) matrices, each
//   from 64-row chunks staged in LDS (up to 64-wide vectors: one partial per
//   wave, each wave a quarter of every chunk over the workgroup's whole
//   w x 64 tile, so an operand read feeds four MFMAs); a second pass sums the
//   partials in a fixed order.  No atomics anywhere: results are deterministic.
#include <hip/hip_runtime.h>

#include <mutex>

#include "common.hpp"
#include "split.hpp"

// The weight gradient's partials for gm_node_mix_backward_weight_noalloc_f32:
// 2^23 floats (32 MiB) on every GPU the library runs on, held until the process
// ends.  Host code reaches it only through the per-device address below.
static __device__ __align__(256) float scratch[int64_t(1) << 23];

namespace gm {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kThreads = 256;
// DPP control: rotate right by 8 lanes within each row of 16 (lane c takes lane c ^ 8's value).
constexpr int kDppRowRor8 = 0x128;
constexpr floatx4 kZero4 = {0.f, 0.f, 0.f, 0.f};

// ---------------------------------------------------------------- forward
//
// Workgroup (x, y): columns [x * 64 CT, (x + 1) * 64 CT), wave wv owning CT
// 16-column tiles from col0 = x * 64 CT + 16 CT wv; row tiles y, y + gridDim.y, ...
// Step s of the contraction pairs slot q with k = q (W / 4) + s, so a lane's
// v operands for consecutive steps are consecutive floats of its row (read
// four at a time from LDS).
template <int W, int CT>
__global__ __launch_bounds__(kThreads) void node_mix_forward_kernel(const float* __restrict__ v, int64_t ldv,
                                                                    const float* __restrict__ M, int64_t N, int w,
                                                                    int64_t C, float* __restrict__ out, int vec_v,
                                                                    int vec_out) {
  constexpr int KS = W / 4;    // contraction steps
  constexpr int LDT = W + 4;   // LDS row stride: a 16-lane b128 read covers all 64 banks once
  constexpr int QUADS = 64 * KS;  // 16-byte pieces of a 64-row tile (KS of them a row)
  __shared__ __align__(16) float vt[64 * LDT];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = lane & 15, q = lane >> 4;
  const int64_t col0 = (int64_t)blockIdx.x * (64 * CT) + 16 * CT * wv;
  float mreg[KS][CT];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int k = q * KS + s;
#pragma unroll
    for (int j = 0; j < CT; ++j) {
      const int64_t col = col0 + 16 * j + c;
      mreg[s][j] = (k < w && col < C) ? M[(int64_t)k * C + col] : 0.f;
    }
  }
  const int64_t n_tiles = (N + 63) / 64;
  constexpr int PER = (QUADS + kThreads - 1) / kThreads;
  float4 pre[PER];
  auto fetch = [&](int64_t tile) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      const int row = idx / KS, kq = idx % KS;
      const int64_t r = tile * 64 + row;
      const int k = 4 * kq;
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
      if (idx < QUADS && r < N) {
        const float* src = v + r * ldv + k;
        if (vec_v && k + 3 < w) {
          x = *reinterpret_cast<const float4*>(src);
        } else {
          x.x = k < w ? src[0] : 0.f;
          x.y = k + 1 < w ? src[1] : 0.f;
          x.z = k + 2 < w ? src[2] : 0.f;
          x.w = k + 3 < w ? src[3] : 0.f;
        }
      }
      pre[p] = x;
    }
  };
  if ((int64_t)blockIdx.y < n_tiles) fetch(blockIdx.y);
  for (int64_t tile = blockIdx.y; tile < n_tiles; tile += gridDim.y) {
    __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      if (idx < QUADS) *reinterpret_cast<float4*>(&vt[(idx / KS) * LDT + 4 * (idx % KS)]) = pre[p];
    }
    __syncthreads();
    if (tile + gridDim.y < n_tiles) fetch(tile + gridDim.y);
    const int64_t row0 = tile * 64;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      float b[KS];
#pragma unroll
      for (int s4 = 0; s4 < KS / 4; ++s4) {
        const float4 x = *reinterpret_cast<const float4*>(&vt[(16 * rt + c) * LDT + q * KS + 4 * s4]);
        b[4 * s4] = x.x;
        b[4 * s4 + 1] = x.y;
        b[4 * s4 + 2] = x.z;
        b[4 * s4 + 3] = x.w;
      }
      floatx4 acc[CT];
#pragma unroll
      for (int j = 0; j < CT; ++j) acc[j] = kZero4;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int j = 0; j < CT; ++j) acc[j] = mfma4(mreg[s][j], b[s], acc[j]);
      }
      const int64_t row = row0 + 16 * rt + c;
      if (row < N) {
        float* dst = out + row * C;
#pragma unroll
        for (int j = 0; j < CT; ++j) {
          const int64_t col = col0 + 16 * j + 4 * q;
          if (vec_out && col + 3 < C) {
            *reinterpret_cast<float4*>(dst + col) = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (col + i < C) dst[col + i] = acc[j][i];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------- input gradient
//
// Workgroup x: rows [128 x, 128 x + 128); wave wv rows 32 wv + 16 rt + c
// (rt < 2) as the A operand, M's rows (the w columns of dv) as B.  Chunk
// k-slot mapping: step s = 4 t + i of a chunk pairs slot q with column
// c0 + 16 q + s, so both operands read four consecutive floats of an LDS row.
// Two waves a SIMD: the compiler then keeps the accumulators with the operands
// in VGPRs (measured 3.45 vs 3.66 ms at N = 524288, w = 64, C = 5440).
template <int W>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void node_mix_dinput_kernel(const float* __restrict__ dmix,
                                                                   const float* __restrict__ M, int64_t N, int w,
                                                                   int64_t C, float* __restrict__ dv, int64_t lddv) {
  constexpr int KC = 64, LDD = KC + 4, JW = W / 16;
  constexpr int DQ = 128 * KC / 4 / kThreads;  // 16-byte pieces of the dmix tile per thread: 8
  constexpr int MQ = W * KC / 4 / kThreads;    // of the M tile: W / 16
  __shared__ __align__(16) float dt[128 * LDD];
  __shared__ __align__(16) float mt[W * LDD];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = lane & 15, q = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 128;
  const int64_t n_chunks = (C + KC - 1) / KC;
  float4 pd[DQ], pm[MQ];
  auto fetch = [&](int64_t ch) {
    const int64_t c0 = ch * KC;
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx >> 4, cq = idx & 15;
      const int64_t r = row0 + row, col = c0 + 4 * cq;
      pd[p] = (r < N && col < C) ? *reinterpret_cast<const float4*>(dmix + r * C + col)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int p = 0; p < MQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx >> 4, cq = idx & 15;
      const int64_t col = c0 + 4 * cq;
      pm[p] = (row < w && col < C) ? *reinterpret_cast<const float4*>(M + (int64_t)row * C + col)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  floatx4 acc[2][JW], tot[2][JW];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int j = 0; j < JW; ++j) acc[rt][j] = tot[rt][j] = kZero4;
  fetch(0);
  for (int64_t ch = 0; ch < n_chunks; ++ch) {
    __syncthreads();
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      *reinterpret_cast<float4*>(&dt[(idx >> 4) * LDD + 4 * (idx & 15)]) = pd[p];
    }
#pragma unroll
    for (int p = 0; p < MQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      *reinterpret_cast<float4*>(&mt[(idx >> 4) * LDD + 4 * (idx & 15)]) = pm[p];
    }
    __syncthreads();
    if (ch + 1 < n_chunks) fetch(ch + 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float4 a[2], b[JW];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        a[rt] = *reinterpret_cast<const float4*>(&dt[(32 * wv + 16 * rt + c) * LDD + 16 * q + 4 * t]);
#pragma unroll
      for (int j = 0; j < JW; ++j) b[j] = *reinterpret_cast<const float4*>(&mt[(16 * j + c) * LDD + 16 * q + 4 * t]);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int j = 0; j < JW; ++j) {
          acc[rt][j] = mfma4(a[rt].x, b[j].x, acc[rt][j]);
          acc[rt][j] = mfma4(a[rt].y, b[j].y, acc[rt][j]);
          acc[rt][j] = mfma4(a[rt].z, b[j].z, acc[rt][j]);
          acc[rt][j] = mfma4(a[rt].w, b[j].w, acc[rt][j]);
        }
    }
    if ((ch & 3) == 3 || ch + 1 == n_chunks) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int j = 0; j < JW; ++j) {
          tot[rt][j] += acc[rt][j];
          acc[rt][j] = kZero4;
        }
    }
  }
  // D[4 q + i][c]: dv row row0 + 32 wv + 16 rt + 4 q + i, column 16 j + c
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int j = 0; j < JW; ++j) {
      const int col = 16 * j + c;
      if (col >= w) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t r = row0 + 32 * wv + 16 * rt + 4 * q + i;
        if (r < N) dv[r * lddv + col] = tot[rt][j][i];
      }
    }
}

// ---------------------------------------------------------------- weight gradient
//
// Vectors wider than 64 reals: workgroup (x, y) owns columns [128 x, 128 x + 128)
// (wave wv: 32 wv + 16 jc + c, jc < 2) over rows [y rps, min(N, (y + 1) rps));
// v^T as A (w rows in 16-row tiles), dmix as B.  Step s of a 64-row chunk
// pairs slot q with row 4 s + q (so does the kernel below).
template <int W>
constexpr int dweight_ldv() {
  return (W % 64 == 16 || W % 64 == 48) ? W : W + 16;  // rows 4 s + q land 16 banks apart
}

template <int W>
__global__ __launch_bounds__(kThreads) void node_mix_dweight_kernel(const float* __restrict__ v, int64_t ldv,
                                                                    const float* __restrict__ dmix, int64_t N, int w,
                                                                    int64_t C, int64_t rps, float* __restrict__ partial,
                                                                    int vec_v) {
  constexpr int RC = 64, LDV = dweight_ldv<W>(), LDM = 128 + 16, IW = W / 16;
  constexpr int VQ = (RC * W / 4 + kThreads - 1) / kThreads;  // 16-byte pieces of the v tile per thread
  constexpr int DQ = RC * 128 / 4 / kThreads;                  // of the dmix tile: 8
  __shared__ __align__(16) float vt[RC * LDV];
  __shared__ __align__(16) float dt[RC * LDM];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = lane & 15, q = lane >> 4;
  const int64_t c0 = (int64_t)blockIdx.x * 128;
  const int64_t first = (int64_t)blockIdx.y * rps, last = first + rps < N ? first + rps : N;
  float4 pv[VQ], pd[DQ];
  auto fetch = [&](int64_t r0) {
#pragma unroll
    for (int p = 0; p < VQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx / (W / 4), k = 4 * (idx % (W / 4));
      const int64_t r = r0 + row;
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
      if (idx < RC * W / 4 && r < last) {
        const float* src = v + r * ldv + k;
        if (vec_v && k + 3 < w) {
          x = *reinterpret_cast<const float4*>(src);
        } else {
          x.x = k < w ? src[0] : 0.f;
          x.y = k + 1 < w ? src[1] : 0.f;
          x.z = k + 2 < w ? src[2] : 0.f;
          x.w = k + 3 < w ? src[3] : 0.f;
        }
      }
      pv[p] = x;
    }
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx >> 5, cq = idx & 31;
      const int64_t r = r0 + row, col = c0 + 4 * cq;
      pd[p] = (r < last && col < C) ? *reinterpret_cast<const float4*>(dmix + r * C + col)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  floatx4 acc[IW][2], tot[IW][2];
#pragma unroll
  for (int i = 0; i < IW; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = tot[i][j] = kZero4;
  int64_t chunk = 0;
  if (first < last) fetch(first);
  for (int64_t r0 = first; r0 < last; r0 += RC, ++chunk) {
    __syncthreads();
#pragma unroll
    for (int p = 0; p < VQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      if (idx < RC * W / 4) *reinterpret_cast<float4*>(&vt[(idx / (W / 4)) * LDV + 4 * (idx % (W / 4))]) = pv[p];
    }
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      *reinterpret_cast<float4*>(&dt[(idx >> 5) * LDM + 4 * (idx & 31)]) = pd[p];
    }
    __syncthreads();
    if (r0 + RC < last) fetch(r0 + RC);
#pragma unroll 4
    for (int s = 0; s < RC / 4; ++s) {
      const int row = 4 * s + q;
      float a[IW], b[2];
#pragma unroll
      for (int i = 0; i < IW; ++i) a[i] = vt[row * LDV + 16 * i + c];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = dt[row * LDM + 32 * wv + 16 * j + c];
#pragma unroll
      for (int i = 0; i < IW; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma4(a[i], b[j], acc[i][j]);
    }
    if ((chunk & 15) == 15) {
#pragma unroll
      for (int i = 0; i < IW; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          tot[i][j] += acc[i][j];
          acc[i][j] = kZero4;
        }
    }
  }
  // D[4 q + ii][c]: dM row 16 i + 4 q + ii, column c0 + 32 wv + 16 j + c
  float* out = partial + (int64_t)blockIdx.y * w * C;
#pragma unroll
  for (int i = 0; i < IW; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = c0 + 32 * wv + 16 * j + c;
      if (col >= C) continue;
      const floatx4 sum = tot[i][j] + acc[i][j];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int row = 16 * i + 4 * q + ii;
        if (row < w) out[(int64_t)row * C + col] = sum[ii];
      }
    }
}

// Vectors up to 64 reals wide: workgroup (x, y) owns the whole (w x 64)-column
// tile [64 x, 64 x + 64) over rows [y rps, min(N, (y + 1) rps)); its four waves
// take rows 16 wv .. 16 wv + 15 of each 64-row chunk, each accumulating the whole
// tile (so every operand read feeds four MFMAs), and write one partial each:
// 4 S partial matrices.
template <int W>
__global__ __launch_bounds__(kThreads) void node_mix_dweight_k_kernel(const float* __restrict__ v, int64_t ldv,
                                                                    const float* __restrict__ dmix, int64_t N, int w,
                                                                    int64_t C, int64_t rps, float* __restrict__ partial,
                                                                    int vec_v) {
  constexpr int RC = 64, LDV = dweight_ldv<W>(), LDM = 64 + 16, IW = W / 16;
  constexpr int VQ = (RC * W / 4 + kThreads - 1) / kThreads;
  constexpr int DQ = RC * 64 / 4 / kThreads;  // 4
  __shared__ __align__(16) float vt[RC * LDV];
  __shared__ __align__(16) float dt[RC * LDM];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = lane & 15, q = lane >> 4;
  const int64_t c0 = (int64_t)blockIdx.x * 64;
  const int64_t first = (int64_t)blockIdx.y * rps, last = first + rps < N ? first + rps : N;
  float4 pv[VQ], pd[DQ];
  auto fetch = [&](int64_t r0) {
#pragma unroll
    for (int p = 0; p < VQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx / (W / 4), k = 4 * (idx % (W / 4));
      const int64_t r = r0 + row;
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
      if (idx < RC * W / 4 && r < last) {
        const float* src = v + r * ldv + k;
        if (vec_v && k + 3 < w) {
          x = *reinterpret_cast<const float4*>(src);
        } else {
          x.x = k < w ? src[0] : 0.f;
          x.y = k + 1 < w ? src[1] : 0.f;
          x.z = k + 2 < w ? src[2] : 0.f;
          x.w = k + 3 < w ? src[3] : 0.f;
        }
      }
      pv[p] = x;
    }
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx >> 4, cq = idx & 15;
      const int64_t r = r0 + row, col = c0 + 4 * cq;
      pd[p] = (r < last && col < C) ? *reinterpret_cast<const float4*>(dmix + r * C + col)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  floatx4 acc[IW][4];
#pragma unroll
  for (int i = 0; i < IW; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = kZero4;
  if (first < last) fetch(first);
  for (int64_t r0 = first; r0 < last; r0 += RC) {
    __syncthreads();
#pragma unroll
    for (int p = 0; p < VQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      if (idx < RC * W / 4) *reinterpret_cast<float4*>(&vt[(idx / (W / 4)) * LDV + 4 * (idx % (W / 4))]) = pv[p];
    }
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      *reinterpret_cast<float4*>(&dt[(idx >> 4) * LDM + 4 * (idx & 15)]) = pd[p];
    }
    __syncthreads();
    if (r0 + RC < last) fetch(r0 + RC);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int row = 16 * wv + 4 * s + q;
      float a[IW], b[4];
#pragma unroll
      for (int i = 0; i < IW; ++i) a[i] = vt[row * LDV + 16 * i + c];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = dt[row * LDM + 16 * j + c];
#pragma unroll
      for (int i = 0; i < IW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma4(a[i], b[j], acc[i][j]);
    }
  }
  float* out = partial + ((int64_t)blockIdx.y * 4 + wv) * w * C;
#pragma unroll
  for (int i = 0; i < IW; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = c0 + 16 * j + c;
      if (col >= C) continue;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int row = 16 * i + 4 * q + ii;
        if (row < w) out[(int64_t)row * C + col] = acc[i][j][ii];
      }
    }
}

// ---------------------------------------------------------------- split products
//
// Four consecutive reals k .. k + 3 (< w) of a node vector at src, float32 or
// bfloat16 (widened exactly); vec: 16-byte (8-byte) aligned whole quads.
__device__ __forceinline__ float4 load_v4(const float* src, int k, int w, int vec) {
  if (vec && k + 3 < w) return *reinterpret_cast<const float4*>(src);
  return make_float4(k < w ? src[0] : 0.f, k + 1 < w ? src[1] : 0.f, k + 2 < w ? src[2] : 0.f,
                     k + 3 < w ? src[3] : 0.f);
}
__device__ __forceinline__ float bf16_at(const uint16_t* p) { return __uint_as_float((uint32_t)*p << 16); }
__device__ __forceinline__ float4 load_v4(const uint16_t* src, int k, int w, int vec) {
  if (vec && k + 3 < w) {
    const uint2 u = *reinterpret_cast<const uint2*>(src);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xFFFF0000u));
  }
  return make_float4(k < w ? bf16_at(src) : 0.f, k + 1 < w ? bf16_at(src + 1) : 0.f,
                     k + 2 < w ? bf16_at(src + 2) : 0.f, k + 3 < w ? bf16_at(src + 3) : 0.f);
}
// Four consecutive entries of a mix-gradient row, float32 or bfloat16 (widened
// exactly; 8-byte aligned quads).
__device__ __forceinline__ float4 load_dm4(const float* src) { return *reinterpret_cast<const float4*>(src); }
__device__ __forceinline__ float4 load_dm4(const uint16_t* src) {
  const uint2 u = *reinterpret_cast<const uint2*>(src);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u), __uint_as_float(u.y << 16),
                     __uint_as_float(u.y & 0xFFFF0000u));
}
//
// The same three products for vectors up to 64 reals, with every fp32 product
// formed as six bf16 products on v_mfma_f32_16x16x32_bf16 (three-piece splits,
// fp32 accuracy: split.hpp).  A 16-deep contraction chunk kc gives lane
// (c, q) the indices 16 kc + 4 q + s, s < 4, in both operands.

// The split kernels' tiling by vector width: columns a forward wave owns
// (16 SplitCT), rows an input-gradient wave owns (16 SplitRT) and columns a
// weight-gradient workgroup owns (16 SplitJT); the widest vectors take the
// narrower tiles so the accumulators and held operands stay within a wave's
// registers.
template <int W>
constexpr int SplitCT = W == 128 ? 1 : 2;
template <int W>
constexpr int SplitRT = W == 128 ? 1 : 2;
template <int W>
constexpr int SplitJT = W == 128 ? 2 : 4;

// A SplitB operand from three bf16 planes (four contraction indices each).
__device__ __forceinline__ SplitB split_b_planes(uint2 hi, uint2 mid, uint2 lo) {
  return SplitB{u32x4{hi.x, hi.y, hi.x, hi.y}, u32x4{mid.x, mid.y, mid.x, mid.y}, u32x4{lo.x, lo.y, hi.x, hi.y}};
}

// Four values' three pieces into three bf16 planes at element `at`.
__device__ __forceinline__ void store_planes(uint16_t* plane0, uint16_t* plane1, uint16_t* plane2, int at,
                                             float4 x) {
  const Split4 sp = split4(x.x, x.y, x.z, x.w);
  *reinterpret_cast<uint2*>(plane0 + at) = make_uint2(sp.hi[0], sp.hi[1]);
  *reinterpret_cast<uint2*>(plane1 + at) = make_uint2(sp.mid[0], sp.mid[1]);
  *reinterpret_cast<uint2*>(plane2 + at) = make_uint2(sp.lo[0], sp.lo[1]);
}

// Four values' pieces as the three B operands themselves, one 16-byte record
// each ([hi, hi], [mid, mid], [lo, hi] slot pairs): a wave then reads an
// operand straight into its registers instead of assembling it from planes.
__device__ __forceinline__ void store_operands(uint4* rec, float4 x) {
  const Split4 sp = split4(x.x, x.y, x.z, x.w);
  rec[0] = make_uint4(sp.hi[0], sp.hi[1], sp.hi[0], sp.hi[1]);
  rec[1] = make_uint4(sp.mid[0], sp.mid[1], sp.mid[0], sp.mid[1]);
  rec[2] = make_uint4(sp.lo[0], sp.lo[1], sp.hi[0], sp.hi[1]);
}

__device__ __forceinline__ SplitB load_operands(const uint4* rec) {
  const uint4 hh = rec[0], mm = rec[1], lh = rec[2];
  return SplitB{u32x4{hh.x, hh.y, hh.z, hh.w}, u32x4{mm.x, mm.y, mm.z, mm.w}, u32x4{lh.x, lh.y, lh.z, lh.w}};
}

// Forward: wave wv of workgroup x owns columns x * 64 CT + 16 CT wv + 16 j + c
// (j < CT); the pieces of M at those columns are split once per wave and held
// in registers; each 64-row tile of v is split once per workgroup into LDS, from
// which every wave takes its B operands: for 64 reals as the operands
// themselves (48 bytes a four-value group, rows of W / 4 + 1 groups so neither
// the staging writes nor a 16-lane read meet in a bank), for the other widths
// as three bf16 planes (row stride W + 4 halfwords: a 16-lane 8-byte read
// covers 32 banks once) assembled into operands by each wave.
template <int W, typename V = float>
__global__ __launch_bounds__(kThreads) void node_mix_forward_split(const V* __restrict__ v, int64_t ldv,
                                                                   const float* __restrict__ M, int64_t N, int w,
                                                                   int64_t C, float* __restrict__ out, int vec_v,
                                                                   int vec_out) {
  constexpr int KC = W / 16, CT = SplitCT<W>;
  constexpr int LDP = W + 4;
  constexpr int QUADS = 64 * W / 4;
  constexpr int PER = (QUADS + kThreads - 1) / kThreads;
  constexpr bool OPS = W == 64;       // operands staged as records (w = 64: 3.39 -> 3.32 ms at NS; w = 32 slower)
  constexpr int GP = W / 4 + 1;       // record groups a staged row
  __shared__ __align__(16) uint16_t vp[OPS ? 1 : 3][OPS ? 8 : 64 * LDP];
  __shared__ __align__(16) uint4 vr[OPS ? 64 * GP * 3 : 1];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = lane & 15, q = lane >> 4;
  const int64_t col0 = (int64_t)blockIdx.x * (64 * CT) + 16 * CT * wv;
  SplitA ma[KC][CT];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc)
#pragma unroll
    for (int j = 0; j < CT; ++j) {
      const int64_t col = col0 + 16 * j + c;
      float x[4];
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int k = 16 * kc + 4 * q + s4;
        x[s4] = (k < w && col < C) ? M[(int64_t)k * C + col] : 0.f;
      }
      ma[kc][j] = split_a(x[0], x[1], x[2], x[3]);
    }
  const int64_t n_tiles = (N + 63) / 64;
  float4 pre[PER];
  auto fetch = [&](int64_t tile) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      const int row = idx / (W / 4), k = 4 * (idx % (W / 4));
      const int64_t r = tile * 64 + row;
      pre[p] = (idx < QUADS && r < N) ? load_v4(v + r * ldv + k, k, w, vec_v) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  if ((int64_t)blockIdx.y < n_tiles) fetch(blockIdx.y);
  for (int64_t tile = blockIdx.y; tile < n_tiles; tile += gridDim.y) {
    __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      if (idx < QUADS) {
        if constexpr (OPS)
          store_operands(&vr[((idx / (W / 4)) * GP + idx % (W / 4)) * 3], pre[p]);
        else
          store_planes(vp[0], vp[1], vp[2], (idx / (W / 4)) * LDP + 4 * (idx % (W / 4)), pre[p]);
      }
    }
    __syncthreads();
    if (tile + gridDim.y < n_tiles) fetch(tile + gridDim.y);
    const int64_t row0 = tile * 64;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      floatx4 acc[CT];
#pragma unroll
      for (int j = 0; j < CT; ++j) acc[j] = kZero4;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        SplitB b;
        if constexpr (OPS) {
          b = load_operands(&vr[((16 * rt + c) * GP + 4 * kc + q) * 3]);
        } else {
          const int at = (16 * rt + c) * LDP + 16 * kc + 4 * q;
          b = split_b_planes(*reinterpret_cast<const uint2*>(&vp[0][at]), *reinterpret_cast<const uint2*>(&vp[1][at]),
                             *reinterpret_cast<const uint2*>(&vp[2][at]));
        }
#pragma unroll
        for (int j = 0; j < CT; ++j) acc[j] = mfma_split(ma[kc][j], b, acc[j]);
      }
      if constexpr (CT == 2 && !OPS) {
        // Lane (c, q) holds row c's columns 4q.. of both 16-column tiles.  Lanes c and c ^ 8
        // trade halves (c < 8 gives its second tile, c >= 8 its first; one DPP rotate by 8
        // within each 16-lane row), so each of the two stores writes eight whole rows of the
        // wave's 32 columns (128 contiguous bytes a row) instead of 64-byte halves of sixteen:
        // 1.44 -> 1.23 ms for w = 32 at 256x512, B = 4.  The 64-real form keeps its stores
        // (3.31 vs 3.35 ms with the trade: its stores then wait for both tiles' longer chains).
        const bool lo = c < 8;
        floatx4 sw;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sw[i] = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(lo ? acc[1][i] : acc[0][i]),
                                                             kDppRowRor8, 0xF, 0xF, false));
        const int64_t col = col0 + 16 * (c >> 3) + 4 * q;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int64_t row = row0 + 16 * rt + 8 * h + (c & 7);
          const floatx4 val = (h == 0) == lo ? acc[h] : sw;
          if (row < N) {
            float* dst = out + row * C;
            if (vec_out && col + 3 < C) {
              *reinterpret_cast<float4*>(dst + col) = make_float4(val[0], val[1], val[2], val[3]);
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i)
                if (col + i < C) dst[col + i] = val[i];
            }
          }
        }
      } else {
        const int64_t row = row0 + 16 * rt + c;
        if (row < N) {
          float* dst = out + row * C;
#pragma unroll
          for (int j = 0; j < CT; ++j) {
            const int64_t col = col0 + 16 * j + 4 * q;
            if (vec_out && col + 3 < C) {
              *reinterpret_cast<float4*>(dst + col) = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i)
                if (col + i < C) dst[col + i] = acc[j][i];
            }
          }
        }
      }
    }
  }
}

// Input gradient: tiles of 64 RT rows, each wave 16 RT rows over the whole
// contraction; a 64-column chunk of dmix is staged as fp32 (each wave splits
// its own rows' A operands), the chunk of M as three bf16 planes split once
// per workgroup; running totals every four chunks.
template <int W>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void node_mix_dinput_split(const float* __restrict__ dmix,
                                                                  const float* __restrict__ M, int64_t N, int w,
                                                                  int64_t C, float* __restrict__ dv, int64_t lddv) {
  constexpr int RT = SplitRT<W>, ROWS = 64 * RT;
  // chunks of KC columns (32 for the widest vectors: fewer staged registers); LDM: a 16-lane 8-byte read
  // covers 32 banks once
  constexpr int KC = W == 128 ? 32 : 64, LDM = KC + 4, JW = W / 16, KS = KC / 16;
  // 64-column chunks of dmix unpadded, 16-byte unit u of row r at u ^ (r mod 16): a 16-byte read's set of
  // 16 lanes (c < 8 of one lane row, c >= 8 of another) then meets 16 distinct bank quads
  constexpr bool SWZ = KC == 64;
  constexpr int LDD = SWZ ? KC : KC + 4;
  constexpr int TOTAL_EVERY = 256 / KC;  // chunks a running sum spans before it joins the total
  constexpr int DQ = ROWS * KC / 4 / kThreads;
  constexpr int MQ = W * KC / 4 / kThreads;
  __shared__ __align__(16) float dt[ROWS * LDD];
  __shared__ __align__(16) uint16_t mp[3][W * LDM];  // M's hi, mid and lo pieces, row k of M at k * LDM
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = lane & 15, q = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * ROWS;
  const int64_t n_chunks = (C + KC - 1) / KC;
  constexpr int CQ = KC / 4;  // 16-byte pieces of a chunk row
  float4 pd[DQ], pm[MQ];
  auto fetch = [&](int64_t ch) {
    const int64_t c0 = ch * KC;
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx / CQ, cq = idx % CQ;
      const int64_t r = row0 + row, col = c0 + 4 * cq;
      pd[p] = (r < N && col < C) ? *reinterpret_cast<const float4*>(dmix + r * C + col)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int p = 0; p < MQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx / CQ, cq = idx % CQ;
      const int64_t col = c0 + 4 * cq;
      pm[p] = (row < w && col < C) ? *reinterpret_cast<const float4*>(M + (int64_t)row * C + col)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  floatx4 acc[RT][JW], tot[RT][JW];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int j = 0; j < JW; ++j) acc[rt][j] = tot[rt][j] = kZero4;
  fetch(0);
  for (int64_t ch = 0; ch < n_chunks; ++ch) {
    __syncthreads();
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      const int u = SWZ ? (idx % CQ) ^ ((idx / CQ) & 15) : idx % CQ;
      *reinterpret_cast<float4*>(&dt[(idx / CQ) * LDD + 4 * u]) = pd[p];
    }
#pragma unroll
    for (int p = 0; p < MQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      store_planes(mp[0], mp[1], mp[2], (idx / CQ) * LDM + 4 * (idx % CQ), pm[p]);
    }
    __syncthreads();
    if (ch + 1 < n_chunks) fetch(ch + 1);
#pragma unroll
    for (int kc = 0; kc < KS; ++kc) {
      SplitA a[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int u = SWZ ? (4 * kc + q) ^ c : 4 * kc + q;
        const float4 x = *reinterpret_cast<const float4*>(&dt[(16 * RT * wv + 16 * rt + c) * LDD + 4 * u]);
        a[rt] = split_a(x.x, x.y, x.z, x.w);
      }
#pragma unroll
      for (int j = 0; j < JW; ++j) {
        const int at = (16 * j + c) * LDM + 16 * kc + 4 * q;
        const SplitB b = split_b_planes(*reinterpret_cast<const uint2*>(&mp[0][at]),
                                        *reinterpret_cast<const uint2*>(&mp[1][at]),
                                        *reinterpret_cast<const uint2*>(&mp[2][at]));
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[rt][j] = mfma_split(a[rt], b, acc[rt][j]);
      }
    }
    if (ch % TOTAL_EVERY == TOTAL_EVERY - 1 || ch + 1 == n_chunks) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < JW; ++j) {
          tot[rt][j] += acc[rt][j];
          acc[rt][j] = kZero4;
        }
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int j = 0; j < JW; ++j) {
      const int col = 16 * j + c;
      if (col >= w) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t r = row0 + 16 * RT * wv + 16 * rt + 4 * q + i;
        if (r < N) dv[r * lddv + col] = tot[rt][j][i];
      }
    }
}

// Weight gradient: workgroup (x, y) owns the whole (w x 16 JT)-column tile
// [16 JT x, 16 JT (x + 1)) over rows [y rps, min(N, (y + 1) rps)); its four
// waves take rows 16 wv .. 16 wv + 15 of each 64-row chunk, a wave's 16 rows
// forming one contraction chunk of split products, each wave accumulating the
// whole tile and writing one partial: 4 S partial matrices.
template <int W, typename V = float, typename DM = float>
__global__ __launch_bounds__(kThreads) void node_mix_dweight_split(const V* __restrict__ v, int64_t ldv,
                                                                   const DM* __restrict__ dmix, int64_t N, int w,
                                                                   int64_t C, int64_t rps, float* __restrict__ partial,
                                                                   int vec_v) {
  constexpr int JT = SplitJT<W>, COLS = 16 * JT;
  // lanes (c, q) read rows 16 wv + 4 q + s: strides with 4 LD = 16 (mod 64) words put a quarter-wave's
  // rows in distinct banks
  constexpr int RC = 64, LDV = W + 4, LDM = COLS + 4, IW = W / 16;
  constexpr int VQ = (RC * W / 4 + kThreads - 1) / kThreads;
  constexpr int CQ = COLS / 4;  // 16-byte pieces of a dmix row
  constexpr int DQ = (RC * CQ + kThreads - 1) / kThreads;
  __shared__ __align__(16) float vt[RC * LDV];
  __shared__ __align__(16) float dt[RC * LDM];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = lane & 15, q = lane >> 4;
  const int64_t c0 = (int64_t)blockIdx.x * COLS;
  const int64_t first = (int64_t)blockIdx.y * rps, last = first + rps < N ? first + rps : N;
  float4 pv[VQ], pd[DQ];
  auto fetch = [&](int64_t r0) {
#pragma unroll
    for (int p = 0; p < VQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx / (W / 4), k = 4 * (idx % (W / 4));
      const int64_t r = r0 + row;
      pv[p] = (idx < RC * W / 4 && r < last) ? load_v4(v + r * ldv + k, k, w, vec_v) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads, row = idx / CQ, cq = idx % CQ;
      const int64_t r = r0 + row, col = c0 + 4 * cq;
      pd[p] = (idx < RC * CQ && r < last && col < C) ? load_dm4(dmix + r * C + col) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  floatx4 acc[IW][JT];
#pragma unroll
  for (int i = 0; i < IW; ++i)
#pragma unroll
    for (int j = 0; j < JT; ++j) acc[i][j] = kZero4;
  if (first < last) fetch(first);
  for (int64_t r0 = first; r0 < last; r0 += RC) {
    __syncthreads();
#pragma unroll
    for (int p = 0; p < VQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      if (idx < RC * W / 4) *reinterpret_cast<float4*>(&vt[(idx / (W / 4)) * LDV + 4 * (idx % (W / 4))]) = pv[p];
    }
#pragma unroll
    for (int p = 0; p < DQ; ++p) {
      const int idx = threadIdx.x + p * kThreads;
      if (idx < RC * CQ) *reinterpret_cast<float4*>(&dt[(idx / CQ) * LDM + 4 * (idx % CQ)]) = pd[p];
    }
    __syncthreads();
    if (r0 + RC < last) fetch(r0 + RC);
    // rows 16 wv + 4 q + s of the chunk are contraction indices 4 q + s
    const int rb = 16 * wv + 4 * q;
    SplitA a[IW];
#pragma unroll
    for (int i = 0; i < IW; ++i)
      a[i] = split_a(vt[rb * LDV + 16 * i + c], vt[(rb + 1) * LDV + 16 * i + c], vt[(rb + 2) * LDV + 16 * i + c],
                     vt[(rb + 3) * LDV + 16 * i + c]);
#pragma unroll
    for (int j = 0; j < JT; ++j) {
      const SplitB b = split_b(dt[rb * LDM + 16 * j + c], dt[(rb + 1) * LDM + 16 * j + c],
                               dt[(rb + 2) * LDM + 16 * j + c], dt[(rb + 3) * LDM + 16 * j + c]);
#pragma unroll
      for (int i = 0; i < IW; ++i) acc[i][j] = mfma_split(a[i], b, acc[i][j]);
    }
  }
  float* out = partial + ((int64_t)blockIdx.y * 4 + wv) * w * C;
#pragma unroll
  for (int i = 0; i < IW; ++i)
#pragma unroll
    for (int j = 0; j < JT; ++j) {
      const int64_t col = c0 + 16 * j + c;
      if (col >= C) continue;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int row = 16 * i + 4 * q + ii;
        if (row < w) out[(int64_t)row * C + col] = acc[i][j][ii];
      }
    }
}

// dM[e] = sum over y = 0, 1, ..., count - 1 of partial[y stride][e], in that order.
__global__ __launch_bounds__(kThreads) void node_mix_reduce_kernel(const float* __restrict__ partial, int64_t n,
                                                                   int64_t count, int64_t stride,
                                                                   float* __restrict__ dM) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= n) return;
  float s = 0.f;
  for (int64_t y = 0; y < count; ++y) s += partial[y * stride * n + e];
  dM[e] = s;
}

// Partial sums over slices of kReduceSlice consecutive partial matrices, each
// in order and written over its slice's first matrix (the one partial no other
// thread reads at e), so a second pass adds kReduceSlice times fewer rows.
constexpr int64_t kReduceSlice = 32;

__global__ __launch_bounds__(kThreads) void node_mix_reduce_slices_kernel(float* __restrict__ partial, int64_t n,
                                                                          int64_t parts) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= n) return;
  const int64_t y0 = (int64_t)blockIdx.y * kReduceSlice;
  const int64_t y1 = y0 + kReduceSlice < parts ? y0 + kReduceSlice : parts;
  float s = 0.f;
  for (int64_t y = y0; y < y1; ++y) s += partial[y * n + e];
  partial[y0 * n + e] = s;
}

// dM = the sum of the `parts` partial matrices of n entries in a fixed order:
// directly for a few, else by slices of kReduceSlice then over the slices.
int launch_reduce(float* partial, int64_t n, int64_t parts, float* dM, hipStream_t stream) {
  const unsigned blocks = (unsigned)((n + kThreads - 1) / kThreads);
  if (parts <= 2 * kReduceSlice) {
    hipLaunchKernelGGL(node_mix_reduce_kernel, dim3(blocks), dim3(kThreads), 0, stream, partial, n, parts, (int64_t)1,
                       dM);
    return check_launch("node_mix_backward_weight (reduce)");
  }
  const int64_t slices = (parts + kReduceSlice - 1) / kReduceSlice;
  hipLaunchKernelGGL(node_mix_reduce_slices_kernel, dim3(blocks, (unsigned)slices), dim3(kThreads), 0, stream, partial,
                     n, parts);
  const int rc = check_launch("node_mix_backward_weight (reduce slices)");
  if (rc != GM_OK) return rc;
  hipLaunchKernelGGL(node_mix_reduce_kernel, dim3(blocks), dim3(kThreads), 0, stream, partial, n, slices,
                     kReduceSlice, dM);
  return check_launch("node_mix_backward_weight (reduce)");
}

int check_shapes(int64_t N, int64_t w, int64_t C) {
  GM_REQUIRE(N >= 0 && C >= 0, "N and C must be non-negative");
  GM_REQUIRE(w >= 1 && w <= 128, "the node vector's width w must be in [1, 128]");
  return GM_OK;
}

int width_class(int64_t w) { return w <= 16 ? 16 : (w <= 32 ? 32 : (w <= 64 ? 64 : 128)); }

// Column tile of the weight gradient's workgroups: 64 columns for vectors up to
// 64 reals; above, 32 for the split kernel and 128 for the fp32 one.
int64_t weight_tile(int64_t w) { return w <= 64 ? 64 : (split_products() ? 32 : 128); }

// Partial matrices a workgroup row writes: four (one a wave) but for the fp32
// kernel of vectors above 64 reals (one).
int64_t weight_partials_per_split(int64_t w) { return (w <= 64 || split_products()) ? 4 : 1; }

// Row groups g of a grid of nx x g workgroups whose rows each workgroup loops
// over in equal shares: about `want` workgroups in whole rounds of the
// `slots` resident ones (g = floor(r slots / nx), r = want / slots rounded,
// at least one), so that no last round runs on a fraction of the chip;
// ceil(want / nx) when the occupancy is unknown or a round holds fewer
// workgroups than there are column tiles.
int64_t round_groups(int64_t nx, int64_t want, int64_t slots) {
  if (nx < 1) nx = 1;
  if (slots < nx) return (want + nx - 1) / nx;
  int64_t r = (want + slots / 2) / slots;
  if (r < 1) r = 1;
  return (r * slots) / nx;
}

// The weight gradient's kernel for vectors of w reals (float vectors; the
// bfloat16 form shares its workspace, so its grid follows this one).
const void* dweight_kernel(int64_t w) {
  const bool sp = split_products();
  switch (width_class(w)) {
    case 16: return sp ? (const void*)node_mix_dweight_split<16> : (const void*)node_mix_dweight_k_kernel<16>;
    case 32: return sp ? (const void*)node_mix_dweight_split<32> : (const void*)node_mix_dweight_k_kernel<32>;
    case 64: return sp ? (const void*)node_mix_dweight_split<64> : (const void*)node_mix_dweight_k_kernel<64>;
    default: return sp ? (const void*)node_mix_dweight_split<128> : (const void*)node_mix_dweight_kernel<128>;
  }
}

// The weight gradient's row splits: about 1024 workgroups in whole rounds, whole 64-row chunks per split.
void weight_splits(int64_t N, int64_t w, int64_t C, int64_t max_splits, int64_t& splits, int64_t& rps) {
  const int64_t tile = weight_tile(w);
  const int64_t nx = (C + tile - 1) / tile > 0 ? (C + tile - 1) / tile : 1;
  const int64_t chunks = (N + 63) / 64;
  int64_t s = round_groups(nx, 1024, resident_blocks(dweight_kernel(w), kThreads));
  if (s > chunks) s = chunks;
  if (s > max_splits) s = max_splits;
  if (s < 1) s = 1;
  rps = ((chunks + s - 1) / s) * 64;
  splits = rps > 0 ? (N + rps - 1) / rps : 1;
  if (splits < 1) splits = 1;
}

int launch_dweight(const float* v, int64_t ldv, const float* dmix, int64_t N, int64_t w, int64_t C, int64_t splits,
                   int64_t rps, float* partial, float* dM, hipStream_t stream) {
  const int64_t tile = weight_tile(w), nx = (C + tile - 1) / tile;
  if (N > 0 && nx > 0) {
    const dim3 grid((unsigned)nx, (unsigned)splits), block(kThreads);
    const int vec = aligned(v, 16) && ldv % 4 == 0;
    const bool sp = split_products();
    switch (width_class(w)) {
      case 16:
        if (sp) hipLaunchKernelGGL(node_mix_dweight_split<16>, grid, block, 0, stream, v, ldv, dmix, N, (int)w, C, rps, partial, vec);
        else hipLaunchKernelGGL(node_mix_dweight_k_kernel<16>, grid, block, 0, stream, v, ldv, dmix, N, (int)w, C, rps, partial, vec);
        break;
      case 32:
        if (sp) hipLaunchKernelGGL(node_mix_dweight_split<32>, grid, block, 0, stream, v, ldv, dmix, N, (int)w, C, rps, partial, vec);
        else hipLaunchKernelGGL(node_mix_dweight_k_kernel<32>, grid, block, 0, stream, v, ldv, dmix, N, (int)w, C, rps, partial, vec);
        break;
      case 64:
        if (sp) hipLaunchKernelGGL(node_mix_dweight_split<64>, grid, block, 0, stream, v, ldv, dmix, N, (int)w, C, rps, partial, vec);
        else hipLaunchKernelGGL(node_mix_dweight_k_kernel<64>, grid, block, 0, stream, v, ldv, dmix, N, (int)w, C, rps, partial, vec);
        break;
      default:
        if (sp) hipLaunchKernelGGL(node_mix_dweight_split<128>, grid, block, 0, stream, v, ldv, dmix, N, (int)w, C, rps, partial, vec);
        else hipLaunchKernelGGL(node_mix_dweight_kernel<128>, grid, block, 0, stream, v, ldv, dmix, N, (int)w, C, rps, partial, vec);
        break;
    }
    const int rc = check_launch("node_mix_backward_weight");
    if (rc != GM_OK) return rc;
  }
  const int64_t n = w * C;
  if (n > 0) {
    const int64_t parts = (N > 0 && C > 0) ? splits * weight_partials_per_split(w) : (int64_t)0;
    return launch_reduce(partial, n, parts, dM, stream);
  }
  return GM_OK;
}

constexpr int64_t kScratchFloats = int64_t(1) << 23;
constexpr int kMaxDevices = 64;

// Each device's address of `scratch`, looked up once with that device current,
// and an event per device that orders the calls sharing that device's array:
// each call's stream waits for the previous call's kernels (on whatever stream
// they ran) before it writes the partials, and the call records the event
// after its reduction.  The mutex is held from the wait to the record, so calls
// from several host threads or streams serialise on the GPU instead of racing.
std::mutex scratch_mutex;
float* scratch_address[kMaxDevices] = {};
hipEvent_t scratch_done[kMaxDevices] = {};

int scratch_on_current_device(int* device_out, float** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(GM_ERR_LAUNCH, std::string("hipGetDevice: ") + hipGetErrorString(err));
  GM_REQUIRE(device >= 0 && device < kMaxDevices, "the current device index is out of the scratch table's range");
  if (scratch_address[device] == nullptr) {
    void* address = nullptr;
    err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (err != hipSuccess || address == nullptr)
      return fail(GM_ERR_LAUNCH, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(err));
    hipEvent_t done = nullptr;
    err = hipEventCreateWithFlags(&done, hipEventDisableTiming);
    if (err != hipSuccess)
      return fail(GM_ERR_LAUNCH, std::string("hipEventCreateWithFlags(scratch): ") + hipGetErrorString(err));
    scratch_done[device] = done;
    scratch_address[device] = static_cast<float*>(address);
  }
  *device_out = device;
  *out = scratch_address[device];
  return GM_OK;
}

}  // namespace
}  // namespace gm

extern "C" int gm_node_mix_forward_f32(const float* v, int64_t ldv, const float* M, int64_t N, int64_t w, int64_t C,
                                       float* out, void* stream) {
  int rc = gm::check_shapes(N, w, C);
  if (rc != GM_OK) return rc;
  if (N == 0 || C == 0) return GM_OK;
  GM_REQUIRE(v && M && out, "v, M and out must be device pointers");
  GM_REQUIRE(ldv >= w, "ldv must be at least w");
  const hipStream_t s = (hipStream_t)stream;
  const int vec_v = gm::aligned(v, 16) && ldv % 4 == 0;
  const int vec_out = gm::aligned(out, 16) && C % 4 == 0;
  const int W = gm::width_class(w);
  const bool sp = gm::split_products();
  const int CT = sp ? (W == 128 ? gm::SplitCT<128> : gm::SplitCT<64>) : (W == 128 ? 2 : 4);
  const int64_t nx = (C + 64 * CT - 1) / (64 * CT), n_tiles = (N + 63) / 64;
  const void* kernel = nullptr;
  switch (W) {
    case 16: kernel = sp ? (const void*)gm::node_mix_forward_split<16> : (const void*)gm::node_mix_forward_kernel<16, 4>; break;
    case 32: kernel = sp ? (const void*)gm::node_mix_forward_split<32> : (const void*)gm::node_mix_forward_kernel<32, 4>; break;
    case 64: kernel = sp ? (const void*)gm::node_mix_forward_split<64> : (const void*)gm::node_mix_forward_kernel<64, 4>; break;
    default: kernel = sp ? (const void*)gm::node_mix_forward_split<128> : (const void*)gm::node_mix_forward_kernel<128, 2>; break;
  }
  int64_t ny = gm::round_groups(nx, 2048, gm::resident_blocks(kernel, gm::kThreads));
  if (ny > n_tiles) ny = n_tiles;
  if (ny > 65535) ny = 65535;
  const dim3 grid((unsigned)nx, (unsigned)ny), block(gm::kThreads);
  if (sp) {
    switch (W) {
      case 16: hipLaunchKernelGGL((gm::node_mix_forward_split<16>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
      case 32: hipLaunchKernelGGL((gm::node_mix_forward_split<32>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
      case 64: hipLaunchKernelGGL((gm::node_mix_forward_split<64>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
      default: hipLaunchKernelGGL((gm::node_mix_forward_split<128>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
    }
    return gm::check_launch("node_mix_forward");
  }
  switch (W) {
    case 16: hipLaunchKernelGGL((gm::node_mix_forward_kernel<16, 4>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
    case 32: hipLaunchKernelGGL((gm::node_mix_forward_kernel<32, 4>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
    case 64: hipLaunchKernelGGL((gm::node_mix_forward_kernel<64, 4>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
    default: hipLaunchKernelGGL((gm::node_mix_forward_kernel<128, 2>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
  }
  return gm::check_launch("node_mix_forward");
}

extern "C" int gm_node_mix_backward_input_f32(const float* dmix, const float* M, int64_t N, int64_t w, int64_t C,
                                              float* dv, int64_t lddv, void* stream) {
  int rc = gm::check_shapes(N, w, C);
  if (rc != GM_OK) return rc;
  if (N == 0) return GM_OK;
  GM_REQUIRE(dv && lddv >= w, "dv must be a device pointer with lddv >= w");
  GM_REQUIRE(C == 0 || (dmix && M), "dmix and M must be device pointers");
  GM_REQUIRE(C % 4 == 0 && gm::aligned(dmix, 16) && gm::aligned(M, 16),
             "dmix and M must be 16-byte aligned with C a multiple of 4");
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((N + 127) / 128)), block(gm::kThreads);
  if (gm::split_products()) {
    const dim3 grid128((unsigned)((N + 64 * gm::SplitRT<128> - 1) / (64 * gm::SplitRT<128>)));
    switch (gm::width_class(w)) {
      case 16: hipLaunchKernelGGL(gm::node_mix_dinput_split<16>, grid, block, 0, s, dmix, M, N, (int)w, C, dv, lddv); break;
      case 32: hipLaunchKernelGGL(gm::node_mix_dinput_split<32>, grid, block, 0, s, dmix, M, N, (int)w, C, dv, lddv); break;
      case 64: hipLaunchKernelGGL(gm::node_mix_dinput_split<64>, grid, block, 0, s, dmix, M, N, (int)w, C, dv, lddv); break;
      default: hipLaunchKernelGGL(gm::node_mix_dinput_split<128>, grid128, block, 0, s, dmix, M, N, (int)w, C, dv, lddv); break;
    }
    return gm::check_launch("node_mix_backward_input");
  }
  switch (gm::width_class(w)) {
    case 16: hipLaunchKernelGGL(gm::node_mix_dinput_kernel<16>, grid, block, 0, s, dmix, M, N, (int)w, C, dv, lddv); break;
    case 32: hipLaunchKernelGGL(gm::node_mix_dinput_kernel<32>, grid, block, 0, s, dmix, M, N, (int)w, C, dv, lddv); break;
    case 64: hipLaunchKernelGGL(gm::node_mix_dinput_kernel<64>, grid, block, 0, s, dmix, M, N, (int)w, C, dv, lddv); break;
    default: hipLaunchKernelGGL(gm::node_mix_dinput_kernel<128>, grid, block, 0, s, dmix, M, N, (int)w, C, dv, lddv); break;
  }
  return gm::check_launch("node_mix_backward_input");
}

extern "C" int64_t gm_node_mix_weight_partials(int64_t N, int64_t w, int64_t C) {
  int64_t splits = 1, rps = 64;
  gm::weight_splits(N, w, C, 1 << 20, splits, rps);
  return splits * gm::weight_partials_per_split(w) * w * C;
}

extern "C" int gm_node_mix_backward_weight_f32(const float* v, int64_t ldv, const float* dmix, int64_t N, int64_t w,
                                               int64_t C, float* partial, float* dM, void* stream) {
  int rc = gm::check_shapes(N, w, C);
  if (rc != GM_OK) return rc;
  if (w * C == 0) return GM_OK;
  GM_REQUIRE(dM && partial, "partial and dM must be device pointers");
  GM_REQUIRE(N == 0 || (v && dmix && ldv >= w), "v (ldv >= w) and dmix must be device pointers");
  GM_REQUIRE(C % 4 == 0 && (N == 0 || gm::aligned(dmix, 16)), "dmix must be 16-byte aligned with C a multiple of 4");
  int64_t splits = 1, rps = 64;
  gm::weight_splits(N, w, C, 1 << 20, splits, rps);
  return gm::launch_dweight(v, ldv, dmix, N, w, C, splits, rps, partial, dM, (hipStream_t)stream);
}

extern "C" int gm_node_mix_backward_weight_noalloc_f32(const float* v, int64_t ldv, const float* dmix, int64_t N,
                                                       int64_t w, int64_t C, float* dM, void* stream) {
  int rc = gm::check_shapes(N, w, C);
  if (rc != GM_OK) return rc;
  if (w * C == 0) return GM_OK;
  GM_REQUIRE(dM, "dM must be a device pointer");
  GM_REQUIRE(N == 0 || (v && dmix && ldv >= w), "v (ldv >= w) and dmix must be device pointers");
  GM_REQUIRE(C % 4 == 0 && (N == 0 || gm::aligned(dmix, 16)), "dmix must be 16-byte aligned with C a multiple of 4");
  const int64_t per_split = gm::weight_partials_per_split(w) * w * C;
  GM_REQUIRE(per_split <= gm::kScratchFloats,
             "w * C is too large for the no-allocation weight gradient: its partials need " +
                 std::to_string(per_split) + " floats a row split, the scratch holds " +
                 std::to_string(gm::kScratchFloats));
  const hipStream_t s = (hipStream_t)stream;
  std::lock_guard<std::mutex> lock(gm::scratch_mutex);
  float* partial = nullptr;
  int device = -1;
  rc = gm::scratch_on_current_device(&device, &partial);
  if (rc != GM_OK) return rc;
  // Under stream capture the ordering is the graph's (an event recorded outside
  // a capture cannot be waited on inside it): replays of the graph and other
  // calls on that GPU must not overlap.
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  hipError_t err = hipStreamIsCapturing(s, &capture);
  if (err != hipSuccess) return gm::fail(GM_ERR_LAUNCH, std::string("hipStreamIsCapturing: ") + hipGetErrorString(err));
  const bool ordered = capture == hipStreamCaptureStatusNone;
  if (ordered) {
    err = hipStreamWaitEvent(s, gm::scratch_done[device], 0);
    if (err != hipSuccess) return gm::fail(GM_ERR_LAUNCH, std::string("hipStreamWaitEvent: ") + hipGetErrorString(err));
  }
  // as many row splits as the scratch holds (every partial is written in full: nothing to clear)
  int64_t splits = 1, rps = 64;
  gm::weight_splits(N, w, C, gm::kScratchFloats / per_split, splits, rps);
  rc = gm::launch_dweight(v, ldv, dmix, N, w, C, splits, rps, partial, dM, s);
  if (rc != GM_OK || !ordered) return rc;
  err = hipEventRecord(gm::scratch_done[device], s);
  if (err != hipSuccess) return gm::fail(GM_ERR_LAUNCH, std::string("hipEventRecord: ") + hipGetErrorString(err));
  return GM_OK;
}

// bfloat16 node vectors (the rows of a bfloat16 field): the split kernels widen
// them exactly while staging, so the products and outputs are the float32
// entry points' on the widened values.  Vectors up to 64 reals.
extern "C" int gm_node_mix_forward_bf16(const uint16_t* v, int64_t ldv, const float* M, int64_t N, int64_t w,
                                        int64_t C, float* out, void* stream) {
  int rc = gm::check_shapes(N, w, C);
  if (rc != GM_OK) return rc;
  GM_REQUIRE(w <= 64, "bfloat16 node vectors at most 64 reals wide");
  if (N == 0 || C == 0) return GM_OK;
  GM_REQUIRE(v && M && out, "v, M and out must be device pointers");
  GM_REQUIRE(ldv >= w, "ldv must be at least w");
  const hipStream_t s = (hipStream_t)stream;
  const int vec_v = gm::aligned(v, 8) && ldv % 4 == 0;
  const int vec_out = gm::aligned(out, 16) && C % 4 == 0;
  const int W = gm::width_class(w);
  const int64_t nx = (C + 127) / 128, n_tiles = (N + 63) / 64;
  const void* kernel = W == 16 ? (const void*)gm::node_mix_forward_split<16, uint16_t>
                       : W == 32 ? (const void*)gm::node_mix_forward_split<32, uint16_t>
                                 : (const void*)gm::node_mix_forward_split<64, uint16_t>;
  int64_t ny = gm::round_groups(nx, 2048, gm::resident_blocks(kernel, gm::kThreads));
  if (ny > n_tiles) ny = n_tiles;
  if (ny > 65535) ny = 65535;
  const dim3 grid((unsigned)nx, (unsigned)ny), block(gm::kThreads);
  switch (W) {
    case 16: hipLaunchKernelGGL((gm::node_mix_forward_split<16, uint16_t>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
    case 32: hipLaunchKernelGGL((gm::node_mix_forward_split<32, uint16_t>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
    default: hipLaunchKernelGGL((gm::node_mix_forward_split<64, uint16_t>), grid, block, 0, s, v, ldv, M, N, (int)w, C, out, vec_v, vec_out); break;
  }
  return gm::check_launch("node_mix_forward (bfloat16 vectors)");
}

namespace gm {
namespace {

// The split weight gradient for node vectors of type V and mix gradients of
// type DM (bfloat16 widened exactly while staged): partials, then the
// fixed-order reduction.
template <typename V, typename DM>
int split_dweight(const V* v, int64_t ldv, const DM* dmix, int64_t N, int64_t w, int64_t C, float* partial, float* dM,
                  hipStream_t s) {
  int64_t splits = 1, rps = 64;
  weight_splits(N, w, C, 1 << 20, splits, rps);
  const int64_t tile = weight_tile(w), nx = (C + tile - 1) / tile;
  if (N > 0 && nx > 0) {
    const dim3 grid((unsigned)nx, (unsigned)splits), block(kThreads);
    const int vec = aligned(v, sizeof(V) == 2 ? 8 : 16) && ldv % 4 == 0;
    switch (width_class(w)) {
      case 16: hipLaunchKernelGGL((node_mix_dweight_split<16, V, DM>), grid, block, 0, s, v, ldv, dmix, N, (int)w, C, rps, partial, vec); break;
      case 32: hipLaunchKernelGGL((node_mix_dweight_split<32, V, DM>), grid, block, 0, s, v, ldv, dmix, N, (int)w, C, rps, partial, vec); break;
      case 64: hipLaunchKernelGGL((node_mix_dweight_split<64, V, DM>), grid, block, 0, s, v, ldv, dmix, N, (int)w, C, rps, partial, vec); break;
      default:
        if constexpr (sizeof(V) == 4)
          hipLaunchKernelGGL((node_mix_dweight_split<128, V, DM>), grid, block, 0, s, v, ldv, dmix, N, (int)w, C, rps, partial, vec);
        break;
    }
    const int rc = check_launch("node_mix_backward_weight");
    if (rc != GM_OK) return rc;
  }
  const int64_t parts = (N > 0 && C > 0) ? splits * weight_partials_per_split(w) : (int64_t)0;
  return launch_reduce(partial, w * C, parts, dM, s);
}

}  // namespace
}  // namespace gm

extern "C" int gm_node_mix_backward_weight_bf16(const uint16_t* v, int64_t ldv, const float* dmix, int64_t N,
                                                int64_t w, int64_t C, float* partial, float* dM, void* stream) {
  int rc = gm::check_shapes(N, w, C);
  if (rc != GM_OK) return rc;
  GM_REQUIRE(w <= 64, "bfloat16 node vectors at most 64 reals wide");
  if (w * C == 0) return GM_OK;
  GM_REQUIRE(dM && partial, "partial and dM must be device pointers");
  GM_REQUIRE(N == 0 || (v && dmix && ldv >= w), "v (ldv >= w) and dmix must be device pointers");
  GM_REQUIRE(C % 4 == 0 && (N == 0 || gm::aligned(dmix, 16)), "dmix must be 16-byte aligned with C a multiple of 4");
  return gm::split_dweight(v, ldv, dmix, N, w, C, partial, dM, (hipStream_t)stream);
}

extern "C" int gm_node_mix_backward_weight_bf16_bf16(const uint16_t* v, int64_t ldv, const uint16_t* dmix, int64_t N,
                                                     int64_t w, int64_t C, float* partial, float* dM, void* stream) {
  int rc = gm::check_shapes(N, w, C);
  if (rc != GM_OK) return rc;
  GM_REQUIRE(w <= 64, "bfloat16 node vectors at most 64 reals wide");
  GM_REQUIRE(gm::split_products(), "bfloat16 mix gradients need the split products (GM_SPLIT_PRODUCTS unset or 1)");
  if (w * C == 0) return GM_OK;
  GM_REQUIRE(dM && partial, "partial and dM must be device pointers");
  GM_REQUIRE(N == 0 || (v && dmix && ldv >= w), "v (ldv >= w) and dmix must be device pointers");
  GM_REQUIRE(C % 4 == 0 && (N == 0 || gm::aligned(dmix, 8)), "dmix must be 8-byte aligned with C a multiple of 4");
  return gm::split_dweight(v, ldv, dmix, N, w, C, partial, dM, (hipStream_t)stream);
}

extern "C" int gm_node_mix_backward_weight_f32_bf16(const float* v, int64_t ldv, const uint16_t* dmix, int64_t N,
                                                    int64_t w, int64_t C, float* partial, float* dM, void* stream) {
  int rc = gm::check_shapes(N, w, C);
  if (rc != GM_OK) return rc;
  GM_REQUIRE(gm::split_products(), "bfloat16 mix gradients need the split products (GM_SPLIT_PRODUCTS unset or 1)");
  if (w * C == 0) return GM_OK;
  GM_REQUIRE(dM && partial, "partial and dM must be device pointers");
  GM_REQUIRE(N == 0 || (v && dmix && ldv >= w), "v (ldv >= w) and dmix must be device pointers");
  GM_REQUIRE(C % 4 == 0 && (N == 0 || gm::aligned(dmix, 8)), "dmix must be 8-byte aligned with C a multiple of 4");
  return gm::split_dweight(v, ldv, dmix, N, w, C, partial, dM, (hipStream_t)stream);
}
