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
// Forward: one thread per edge for every head, the basis computed once from
// rho, the heads' parameters as uniform operands.  Backward: a fixed grid whose threads
// stride over the edges, per head accumulating their (T x B + T) gradient
// terms in registers (recomputing the basis and pre-activation), then one
// fixed-order reduction per workgroup into a partial row; a second kernel
// sums the partial rows in order.  No atomics: the parameter gradients are
// deterministic.
#include <hip/hip_runtime.h>

#include "common.hpp"

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
  float* partial;       // (n_blocks, H, T * B + T) backward
  int64_t n_edges;
  int H, T, B;
  float inv_width;      // 1 / sigma
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

template <int B>
__device__ __forceinline__ void basis_of(float r, ConstPtr centers, float inv_width, float* b) {
  const float s = r * r;
#pragma unroll
  for (int k = 0; k < B; ++k) {
    const float z = (s - centers[k]) * inv_width;
    b[k] = fast_exp(-0.5f * z * z);
  }
}

// One thread per edge for every head: the basis once, then each head's
// Linear + SiLU with its parameters read as uniform (scalar) operands.
template <int T, int B>
__global__ __launch_bounds__(kTrunkThreads) void trunk_forward_kernel(TrunkArgs a) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= a.n_edges) return;
  const ConstPtr weight = as_const(a.weight), bias = as_const(a.bias);
  float b[B];
  basis_of<B>(a.rho[e], as_const(a.centers), a.inv_width, b);
  for (int hh = 0; hh < a.H; ++hh) {
    const ConstPtr W = weight + hh * T * B;
    float out[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float p = bias ? bias[hh * T + t] : 0.f;
#pragma unroll
      for (int k = 0; k < B; ++k) p = fmaf(W[t * B + k], b[k], p);
      out[t] = p * sigmoid_of(p);
    }
    float* dst = a.h + ((int64_t)hh * a.n_edges + e) * T;
#pragma unroll
    for (int t = 0; t < T; t += 4) *reinterpret_cast<float4*>(dst + t) = make_float4(out[t], out[t + 1], out[t + 2], out[t + 3]);
  }
}

// A fixed grid whose threads stride over the edges; per head and per half of
// its features, each thread accumulates its gradient terms in registers
// (recomputing the basis and pre-activation, the next edge's loads issued
// before this edge's arithmetic), then one fixed-order reduction per
// workgroup into a partial row.
template <int T, int B>
__global__ __launch_bounds__(kTrunkThreads) void trunk_backward_kernel(TrunkArgs a) {
  constexpr int P = T * B + T, TH = T / 2, PH = TH * B + TH;
  __shared__ float red[kTrunkThreads / 64][PH];  // per-wave sums
  const ConstPtr weight = as_const(a.weight), bias = as_const(a.bias), centers = as_const(a.centers);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Waves 0-1 take features 0..TH-1 and waves 2-3 features TH..T-1 of the same edges in the
  // same pass, so the second half of each dh row is read while its line is still in L2
  // (one pass per head; the features' half is wave-uniform, so the weights stay scalar operands).
  constexpr int kEdgeThreads = kTrunkThreads / 2;
  const int t0 = (wave >> 1) * TH;
  const int64_t stride = (int64_t)gridDim.x * kEdgeThreads;
  const int64_t first = (int64_t)blockIdx.x * kEdgeThreads + (threadIdx.x & (kEdgeThreads - 1));
  for (int hh = 0; hh < a.H; ++hh) {
    const ConstPtr W = weight + hh * T * B;
    float acc[PH];
#pragma unroll
    for (int i = 0; i < PH; ++i) acc[i] = 0.f;
    const float* dh = a.dh + (int64_t)hh * a.n_edges * T + t0;
    float4 g[TH / 4];
    float r = 0.f;
    if (first < a.n_edges) {
      r = a.rho[first];
#pragma unroll
      for (int u = 0; u < TH / 4; ++u) g[u] = *reinterpret_cast<const float4*>(dh + first * T + 4 * u);
    }
    // each thread's edges e = first, first + stride, ... in order
    for (int64_t e = first; e < a.n_edges; e += stride) {
      const float rc = r;
      float gv[TH];
#pragma unroll
      for (int u = 0; u < TH / 4; ++u) {
        gv[4 * u] = g[u].x;
        gv[4 * u + 1] = g[u].y;
        gv[4 * u + 2] = g[u].z;
        gv[4 * u + 3] = g[u].w;
      }
      const int64_t en = e + stride;
      if (en < a.n_edges) {
        r = a.rho[en];
#pragma unroll
        for (int u = 0; u < TH / 4; ++u) g[u] = *reinterpret_cast<const float4*>(dh + en * T + 4 * u);
      }
      float b[B];
      basis_of<B>(rc, centers, a.inv_width, b);
#pragma unroll
      for (int t = 0; t < TH; ++t) {
        float p = bias ? bias[hh * T + t0 + t] : 0.f;
#pragma unroll
        for (int k = 0; k < B; ++k) p = fmaf(W[(t0 + t) * B + k], b[k], p);
        const float sg = sigmoid_of(p);
        const float dp = gv[t] * sg * (1.f + p * (1.f - sg));  // dh * d silu / d pre
#pragma unroll
        for (int k = 0; k < B; ++k) acc[t * B + k] = fmaf(dp, b[k], acc[t * B + k]);
        acc[TH * B + t] += dp;
      }
    }
    // the block's sum in a fixed order: a butterfly per wave, then the half's two waves in order
#pragma unroll
    for (int i = 0; i < PH; ++i) {
      float v = acc[i];
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      if (lane == 0) red[wave][i] = v;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 2 * PH; i += blockDim.x) {
      const int half = i / PH, j = i % PH;
      const float sum = red[2 * half][j] + red[2 * half + 1][j];
      // weights of features half * TH .. half * TH + TH - 1, then their biases
      const int slot = j < TH * B ? half * TH * B + j : T * B + half * TH + (j - TH * B);
      a.partial[((int64_t)blockIdx.x * a.H + hh) * P + slot] = sum;
    }
    __syncthreads();
  }
}

// out[h][i] = sum over blocks of partial[block][h][i], blocks in order.
__global__ __launch_bounds__(256) void trunk_reduce_kernel(const float* partial, int64_t n_blocks, int HP, float* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= HP) return;
  float s = 0.f;
  for (int64_t b = 0; b < n_blocks; ++b) s += partial[b * HP + i];
  out[i] = s;
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

constexpr int64_t kTrunkBackwardBlocks = 2048;  // the backward's fixed grid (threads stride over the edges)

int64_t backward_blocks(int64_t n_edges) {
  const int64_t need = (n_edges + kTrunkThreads / 2 - 1) / (kTrunkThreads / 2);  // 128 edges per block pass
  return need < kTrunkBackwardBlocks ? (need > 0 ? need : 1) : kTrunkBackwardBlocks;
}

template <int B>
void launch(bool forward, const TrunkArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)(forward ? (a.n_edges + kTrunkThreads - 1) / kTrunkThreads : backward_blocks(a.n_edges))),
      block(kTrunkThreads);
  if (forward)
    hipLaunchKernelGGL((trunk_forward_kernel<16, B>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((trunk_backward_kernel<16, B>), grid, block, 0, stream, a);
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

extern "C" int64_t gm_radial_trunk_partials(int64_t n_edges) { return gm::backward_blocks(n_edges); }

extern "C" int gm_radial_trunk_forward_f32(const float* rho, const float* weight, const float* bias,
                                           const float* centers, int64_t n_edges, int64_t H, int64_t T, int64_t B,
                                           double width, float* h, void* stream) {
  gm::TrunkArgs a;
  const int status = gm::prepare(a, rho, weight, bias, centers, n_edges, H, T, B, width);
  if (status != GM_OK) return status;
  if (n_edges == 0) return GM_OK;
  GM_REQUIRE(h && gm::aligned(h, 16), "h must be a 16-byte aligned device pointer");
  a.h = h;
  gm::launch_any(true, a, (hipStream_t)stream);
  return gm::check_launch("radial_trunk_forward");
}

extern "C" int gm_radial_trunk_backward_f32(const float* dh, const float* rho, const float* weight, const float* bias,
                                            const float* centers, int64_t n_edges, int64_t H, int64_t T, int64_t B,
                                            double width, float* partial, float* dparams, void* stream) {
  gm::TrunkArgs a;
  const int status = gm::prepare(a, rho, weight, bias, centers, n_edges, H, T, B, width);
  if (status != GM_OK) return status;
  GM_REQUIRE(dparams, "dparams must be a device pointer");
  const int HP = (int)(H * (T * B + T));
  if (n_edges == 0) {
    hipLaunchKernelGGL(gm::trunk_reduce_kernel, dim3((HP + 255) / 256), dim3(256), 0, (hipStream_t)stream, partial,
                       (int64_t)0, HP, dparams);
    return gm::check_launch("radial_trunk_backward (empty)");
  }
  GM_REQUIRE(dh && gm::aligned(dh, 16) && partial, "dh (16-byte aligned) and partial must be device pointers");
  a.dh = dh;
  a.partial = partial;
  gm::launch_any(false, a, (hipStream_t)stream);
  int rc = gm::check_launch("radial_trunk_backward");
  if (rc != GM_OK) return rc;
  hipLaunchKernelGGL(gm::trunk_reduce_kernel, dim3((HP + 255) / 256), dim3(256), 0, (hipStream_t)stream, partial,
                     gm_radial_trunk_partials(n_edges), HP, dparams);
  return gm::check_launch("radial_trunk_backward (reduce)");
}
