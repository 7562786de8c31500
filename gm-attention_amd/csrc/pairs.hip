// The steerable kernel's pair terms, fused per term, for CDNA4 (gfx950).
//
// One term of the per-edge readout (the general, not factored, kernel):
//
//   out(e) += post(e) s(e) f( sum_a M_ba(e) uu_a(e) ),   uu = pre(e) u~(e),
//   M_ba(e) = sum_t W_{ba,t} h_t(e) + bias_ba,
//
// with u~ = u, conj(u) or a real u promoted; f the identity or Re; the rows of
// W in (b, a) order, a complex entry as the row pair (re, im).  (The
// reference's math contract: nn/fused/pairs.h:1-22, 180-330.)
//
// Mapping: one lane per edge, 256-lane workgroups.  The term's weights and
// biases are the same for every lane, so they are read at wave-uniform
// addresses (the scalar path) and enter the FMAs as scalar operands; the
// edge's trunk row, input row and its gradient live in registers (loops over
// the trunk and the input side are unrolled to the 16-wide caps with uniform
// guards).  Backward: per edge the coefficient gradient gm = gq conj(uu_a) is
// written coefficient-major (consecutive lanes, consecutive addresses), the
// trunk gradient W^T gm and the input gradient M^H gq accumulate in registers
// in the same pass over the weights, and each edge's rows of grad_u and
// grad_hidden are updated once.  Terms run one launch each, in stream order,
// so the accumulations into out / grad_u / grad_hidden never race.
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace gm {
namespace {

constexpr int kPairsMaxMult = 16;
constexpr int kPairsMaxTrunk = 16;

template <typename T>
struct PairsArgs {
  int64_t n_edges;
  int a, b, trunk, flags;
  const T* hidden;  // (E, trunk)
  const T* u;       // (E, a) real or (E, a, 2) complex
  const T* pre;     // (E, 2) or null
  const T* post;    // (E, 2) or null
  const T* scale;   // (E) or null
  T* out;           // (E, b) real or (E, b, 2), accumulated
  const T* grad_out;
  T* grad_u;
  T* grad_hidden;
  T* grad_k;  // (width, >= E): row r at r * grad_k_stride
  int64_t grad_k_stride;
};

template <typename T>
__device__ __forceinline__ void load_edge(const PairsArgs<T>& p, int64_t e, T (&h)[kPairsMaxTrunk],
                                          T (&ur)[kPairsMaxMult], T (&ui)[kPairsMaxMult]) {
  const T* hr = p.hidden + e * p.trunk;
#pragma unroll
  for (int k = 0; k < kPairsMaxTrunk; ++k) h[k] = k < p.trunk ? hr[k] : T(0);
  T pr = T(1), pi = T(0);
  if (p.pre) {
    pr = p.pre[2 * e];
    pi = p.pre[2 * e + 1];
  }
  const bool real_u = p.flags & GM_PAIRS_U_REAL;
  const bool conj_u = p.flags & GM_PAIRS_CONJ_U;
#pragma unroll
  for (int a = 0; a < kPairsMaxMult; ++a) {
    T vr = T(0), vi = T(0);
    if (a < p.a) {
      if (real_u) {
        vr = p.u[e * p.a + a];
      } else {
        vr = p.u[2 * (e * p.a + a)];
        vi = p.u[2 * (e * p.a + a) + 1];
        if (conj_u) vi = -vi;
      }
    }
    ur[a] = pr * vr - pi * vi;
    ui[a] = pr * vi + pi * vr;
  }
}

// The entry M_idx at this edge: the weight rows at uniform addresses.
template <typename T, bool CM>
__device__ __forceinline__ void entry(const T* __restrict__ W, const T* __restrict__ bias, int trunk, int idx,
                                      const T (&h)[kPairsMaxTrunk], T& mr, T& mi) {
  if constexpr (CM) {
    const T* wr = W + (int64_t)(2 * idx) * trunk;
    const T* wi = wr + trunk;
    mr = bias ? bias[2 * idx] : T(0);
    mi = bias ? bias[2 * idx + 1] : T(0);
#pragma unroll
    for (int k = 0; k < kPairsMaxTrunk; ++k) {
      if (k < trunk) {
        mr += wr[k] * h[k];
        mi += wi[k] * h[k];
      }
    }
  } else {
    const T* w = W + (int64_t)idx * trunk;
    mr = bias ? bias[idx] : T(0);
    mi = T(0);
#pragma unroll
    for (int k = 0; k < kPairsMaxTrunk; ++k) {
      if (k < trunk) mr += w[k] * h[k];
    }
  }
}

template <typename T, bool CM>
__global__ __launch_bounds__(256) void pairs_forward_kernel(PairsArgs<T> p, const T* __restrict__ W,
                                                            const T* __restrict__ bias) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= p.n_edges) return;
  T h[kPairsMaxTrunk], ur[kPairsMaxMult], ui[kPairsMaxMult];
  load_edge(p, e, h, ur, ui);
  const T s = p.scale ? p.scale[e] : T(1);
  T qr_post = s, qi_post = T(0);  // post(e) s(e)
  if (p.post) {
    qr_post = p.post[2 * e] * s;
    qi_post = p.post[2 * e + 1] * s;
  }
  const bool out_real = p.flags & GM_PAIRS_OUT_REAL;
  for (int bi = 0; bi < p.b; ++bi) {
    T qr[2] = {T(0), T(0)}, qi[2] = {T(0), T(0)};  // two partial sums break the FMA chain
#pragma unroll
    for (int a = 0; a < kPairsMaxMult; ++a) {
      if (a < p.a) {
        T mr, mi;
        entry<T, CM>(W, bias, p.trunk, bi * p.a + a, h, mr, mi);
        qr[a & 1] += mr * ur[a] - mi * ui[a];
        qi[a & 1] += mr * ui[a] + mi * ur[a];
      }
    }
    const T r = qr[0] + qr[1], i = qi[0] + qi[1];
    const int64_t o = e * p.b + bi;
    if (out_real) {
      p.out[o] += r * s;
    } else {
      p.out[2 * o] += qr_post * r - qi_post * i;
      p.out[2 * o + 1] += qr_post * i + qi_post * r;
    }
  }
}

template <typename T, bool CM>
__global__ __launch_bounds__(256) void pairs_backward_kernel(PairsArgs<T> p, const T* __restrict__ W,
                                                             const T* __restrict__ bias) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= p.n_edges) return;
  T h[kPairsMaxTrunk], ur[kPairsMaxMult], ui[kPairsMaxMult];
  load_edge(p, e, h, ur, ui);
  const T s = p.scale ? p.scale[e] : T(1);
  T pr = s, pi = T(0);
  if (p.post) {
    pr = p.post[2 * e] * s;
    pi = p.post[2 * e + 1] * s;
  }
  const bool out_real = p.flags & GM_PAIRS_OUT_REAL;
  T gur[kPairsMaxMult], gui[kPairsMaxMult], gh[kPairsMaxTrunk];
#pragma unroll
  for (int a = 0; a < kPairsMaxMult; ++a) gur[a] = gui[a] = T(0);
#pragma unroll
  for (int k = 0; k < kPairsMaxTrunk; ++k) gh[k] = T(0);
  T* gk = p.grad_k + e;
  const int64_t stride = p.grad_k_stride;
  for (int bi = 0; bi < p.b; ++bi) {
    const int64_t o = e * p.b + bi;
    T gqr, gqi;  // dL/dq for q = M uu
    if (out_real) {
      gqr = p.grad_out[o] * s;
      gqi = T(0);
    } else {
      const T gr = p.grad_out[2 * o], gi = p.grad_out[2 * o + 1];
      gqr = pr * gr + pi * gi;  // conj(post s) g
      gqi = pr * gi - pi * gr;
    }
#pragma unroll
    for (int a = 0; a < kPairsMaxMult; ++a) {
      if (a < p.a) {
        const int idx = bi * p.a + a;
        const T gmr = gqr * ur[a] + gqi * ui[a];  // gm = gq conj(uu_a)
        const T gmi = gqi * ur[a] - gqr * ui[a];
        T mr, mi;
        if constexpr (CM) {
          const T* wr = W + (int64_t)(2 * idx) * p.trunk;
          const T* wi = wr + p.trunk;
          mr = bias ? bias[2 * idx] : T(0);
          mi = bias ? bias[2 * idx + 1] : T(0);
#pragma unroll
          for (int k = 0; k < kPairsMaxTrunk; ++k) {
            if (k < p.trunk) {
              mr += wr[k] * h[k];
              mi += wi[k] * h[k];
              gh[k] += wr[k] * gmr + wi[k] * gmi;
            }
          }
          gk[(int64_t)(2 * idx) * stride] = gmr;
          gk[(int64_t)(2 * idx + 1) * stride] = gmi;
        } else {
          const T* w = W + (int64_t)idx * p.trunk;
          mr = bias ? bias[idx] : T(0);
          mi = T(0);
#pragma unroll
          for (int k = 0; k < kPairsMaxTrunk; ++k) {
            if (k < p.trunk) {
              mr += w[k] * h[k];
              gh[k] += w[k] * gmr;
            }
          }
          gk[(int64_t)idx * stride] = gmr;
        }
        gur[a] += mr * gqr + mi * gqi;  // conj(M) gq
        gui[a] += mr * gqi - mi * gqr;
      }
    }
  }
  // through uu = pre u~, then u~ = conj(u) or a real u promoted
  T cr = T(1), ci = T(0);
  if (p.pre) {
    cr = p.pre[2 * e];
    ci = -p.pre[2 * e + 1];
  }
  const bool real_u = p.flags & GM_PAIRS_U_REAL;
  const bool conj_u = p.flags & GM_PAIRS_CONJ_U;
#pragma unroll
  for (int a = 0; a < kPairsMaxMult; ++a) {
    if (a < p.a) {
      const T gr = cr * gur[a] - ci * gui[a];
      T gi = cr * gui[a] + ci * gur[a];
      if (real_u) {
        p.grad_u[e * p.a + a] += gr;
      } else {
        if (conj_u) gi = -gi;
        p.grad_u[2 * (e * p.a + a)] += gr;
        p.grad_u[2 * (e * p.a + a) + 1] += gi;
      }
    }
  }
  T* ghr = p.grad_hidden + e * p.trunk;
#pragma unroll
  for (int k = 0; k < kPairsMaxTrunk; ++k) {
    if (k < p.trunk) ghr[k] += gh[k];
  }
}

template <typename T>
int prepare(PairsArgs<T>& p, const T* hidden, const T* weight, const T* u, const T* pre, const T* post,
            const T* scale, int64_t n_edges, int64_t a, int64_t b, int64_t trunk, int64_t flags) {
  p = PairsArgs<T>{};
  GM_REQUIRE(a >= 1 && a <= kPairsMaxMult && b >= 1 && b <= kPairsMaxMult, "block dimensions must be in 1..16");
  GM_REQUIRE(trunk >= 1 && trunk <= kPairsMaxTrunk, "trunk width must be in 1..16");
  GM_REQUIRE(n_edges >= 0 && n_edges < (int64_t(1) << 31) * 256, "n_edges out of range");
  GM_REQUIRE((flags & ~int64_t(GM_PAIRS_MATRIX_COMPLEX | GM_PAIRS_U_REAL | GM_PAIRS_CONJ_U | GM_PAIRS_OUT_REAL)) == 0,
             "unknown flag bits");
  if (n_edges > 0) GM_REQUIRE(hidden && weight && u, "hidden, weight and u must be device pointers");
  p.n_edges = n_edges;
  p.a = (int)a;
  p.b = (int)b;
  p.trunk = (int)trunk;
  p.flags = (int)flags;
  p.hidden = hidden;
  p.u = u;
  p.pre = pre;
  p.post = post;
  p.scale = scale;
  return GM_OK;
}

template <typename T>
int pairs_forward(const T* hidden, const T* weight, const T* bias, const T* u, const T* pre, const T* post,
                  const T* scale, T* out, int64_t n_edges, int64_t a, int64_t b, int64_t trunk, int64_t flags,
                  hipStream_t stream) {
  PairsArgs<T> p;
  const int status = prepare(p, hidden, weight, u, pre, post, scale, n_edges, a, b, trunk, flags);
  if (status != GM_OK) return status;
  if (n_edges == 0) return GM_OK;
  GM_REQUIRE(out, "out must be a device pointer");
  p.out = out;
  const dim3 grid((unsigned)((n_edges + 255) / 256));
  if (flags & GM_PAIRS_MATRIX_COMPLEX)
    hipLaunchKernelGGL((pairs_forward_kernel<T, true>), grid, dim3(256), 0, stream, p, weight, bias);
  else
    hipLaunchKernelGGL((pairs_forward_kernel<T, false>), grid, dim3(256), 0, stream, p, weight, bias);
  return check_launch("pairs_forward");
}

template <typename T>
int pairs_backward(const T* hidden, const T* weight, const T* bias, const T* u, const T* pre, const T* post,
                   const T* scale, const T* grad_out, T* grad_u, T* grad_hidden, T* grad_k, int64_t grad_k_stride,
                   int64_t n_edges, int64_t a, int64_t b, int64_t trunk, int64_t flags, hipStream_t stream) {
  PairsArgs<T> p;
  const int status = prepare(p, hidden, weight, u, pre, post, scale, n_edges, a, b, trunk, flags);
  if (status != GM_OK) return status;
  if (n_edges == 0) return GM_OK;
  GM_REQUIRE(grad_out && grad_u && grad_hidden && grad_k, "the gradients must be device pointers");
  GM_REQUIRE(grad_k_stride >= n_edges, "grad_k's row stride must cover every edge");
  p.grad_out = grad_out;
  p.grad_u = grad_u;
  p.grad_hidden = grad_hidden;
  p.grad_k = grad_k;
  p.grad_k_stride = grad_k_stride;
  const dim3 grid((unsigned)((n_edges + 255) / 256));
  if (flags & GM_PAIRS_MATRIX_COMPLEX)
    hipLaunchKernelGGL((pairs_backward_kernel<T, true>), grid, dim3(256), 0, stream, p, weight, bias);
  else
    hipLaunchKernelGGL((pairs_backward_kernel<T, false>), grid, dim3(256), 0, stream, p, weight, bias);
  return check_launch("pairs_backward");
}

}  // namespace
}  // namespace gm

#define GM_PAIRS_ENTRY(SUF, T)                                                                                     \
  extern "C" int gm_pairs_forward_##SUF(const T* hidden, const T* weight, const T* bias, const T* u, const T* pre, \
                                        const T* post, const T* scale, T* out, int64_t n_edges, int64_t a,        \
                                        int64_t b, int64_t trunk, int64_t flags, void* stream) {                 \
    return gm::pairs_forward<T>(hidden, weight, bias, u, pre, post, scale, out, n_edges, a, b, trunk, flags,      \
                                (hipStream_t)stream);                                                              \
  }                                                                                                                \
  extern "C" int gm_pairs_backward_##SUF(const T* hidden, const T* weight, const T* bias, const T* u,             \
                                         const T* pre, const T* post, const T* scale, const T* grad_out,          \
                                         T* grad_u, T* grad_hidden, T* grad_k, int64_t grad_k_stride,             \
                                         int64_t n_edges, int64_t a, int64_t b, int64_t trunk, int64_t flags,     \
                                         void* stream) {                                                           \
    return gm::pairs_backward<T>(hidden, weight, bias, u, pre, post, scale, grad_out, grad_u, grad_hidden,        \
                                 grad_k, grad_k_stride, n_edges, a, b, trunk, flags, (hipStream_t)stream);         \
  }

GM_PAIRS_ENTRY(f32, float)
GM_PAIRS_ENTRY(f64, double)
