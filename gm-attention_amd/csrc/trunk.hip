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
// rho, the heads' parameters in LDS.  Backward: a fixed grid whose threads
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

__device__ __forceinline__ float silu_of(float x) { return x / (1.f + expf(-x)); }

template <int T, int B>
__device__ __forceinline__ void basis_of(float r, const float* centers, float inv_width, float* b) {
  const float s = r * r;
#pragma unroll
  for (int k = 0; k < B; ++k) {
    const float z = (s - centers[k]) * inv_width;
    b[k] = expf(-0.5f * z * z);
  }
}

template <int T, int B>
__global__ __launch_bounds__(kTrunkThreads) void trunk_forward_kernel(TrunkArgs a) {
  __shared__ float w[8][T * B + T];
  __shared__ float cen[B];
  for (int i = threadIdx.x; i < a.H * (T * B + T); i += blockDim.x) {
    const int hh = i / (T * B + T), k = i % (T * B + T);
    w[hh][k] = k < T * B ? a.weight[hh * T * B + k] : (a.bias ? a.bias[hh * T + (k - T * B)] : 0.f);
  }
  if (threadIdx.x < B) cen[threadIdx.x] = a.centers[threadIdx.x];
  __syncthreads();
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= a.n_edges) return;
  float b[B];
  basis_of<T, B>(a.rho[e], cen, a.inv_width, b);
  for (int hh = 0; hh < a.H; ++hh) {
    float out[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float p = w[hh][T * B + t];
#pragma unroll
      for (int k = 0; k < B; ++k) p += w[hh][t * B + k] * b[k];
      out[t] = silu_of(p);
    }
    float* dst = a.h + ((int64_t)hh * a.n_edges + e) * T;
#pragma unroll
    for (int t = 0; t < T; t += 4) *reinterpret_cast<float4*>(dst + t) = make_float4(out[t], out[t + 1], out[t + 2], out[t + 3]);
  }
}

template <int T, int B>
__global__ __launch_bounds__(kTrunkThreads) void trunk_backward_kernel(TrunkArgs a) {
  constexpr int P = T * B + T;
  __shared__ float w[8][P];
  __shared__ float cen[B];
  __shared__ float red[kTrunkThreads / 64][P];  // per-wave sums
  for (int i = threadIdx.x; i < a.H * P; i += blockDim.x) {
    const int hh = i / P, k = i % P;
    w[hh][k] = k < T * B ? a.weight[hh * T * B + k] : (a.bias ? a.bias[hh * T + (k - T * B)] : 0.f);
  }
  if (threadIdx.x < B) cen[threadIdx.x] = a.centers[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int hh = 0; hh < a.H; ++hh) {
    float acc[P];
#pragma unroll
    for (int i = 0; i < P; ++i) acc[i] = 0.f;
    // each thread's edges e = tid, tid + stride, ... in order
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < a.n_edges; e += stride) {
      float b[B];
      basis_of<T, B>(a.rho[e], cen, a.inv_width, b);
      const float* g = a.dh + ((int64_t)hh * a.n_edges + e) * T;
#pragma unroll
      for (int t4 = 0; t4 < T; t4 += 4) {
        const float4 v = *reinterpret_cast<const float4*>(g + t4);
        const float gv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int t = t4 + u;
          float p = w[hh][T * B + t];
#pragma unroll
          for (int k = 0; k < B; ++k) p += w[hh][t * B + k] * b[k];
          const float sg = 1.f / (1.f + expf(-p));
          const float dp = gv[u] * sg * (1.f + p * (1.f - sg));  // dh * d silu / d pre
#pragma unroll
          for (int k = 0; k < B; ++k) acc[t * B + k] += dp * b[k];
          acc[T * B + t] += dp;
        }
      }
    }
    // the block's sum in a fixed order: a butterfly per wave, then the waves in order
#pragma unroll
    for (int i = 0; i < P; ++i) {
      float v = acc[i];
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      if (lane == 0) red[wave][i] = v;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < P; i += blockDim.x) {
      float sum = 0.f;
      for (int wv = 0; wv < kTrunkThreads / 64; ++wv) sum += red[wv][i];
      a.partial[((int64_t)blockIdx.x * a.H + hh) * P + i] = sum;
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
  const int64_t need = (n_edges + kTrunkThreads - 1) / kTrunkThreads;
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
