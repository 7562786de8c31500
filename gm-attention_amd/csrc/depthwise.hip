// The depthwise steerable convolution over CSR neighbour lists, forward and
// backward, for CDNA4 (gfx950).
//
//   out_i = sum_{e=(i<-j)} w_e m_e,  per copy (unit) of the field:
//     scalar copy a:          m = rc[e, a] v_j,a
//     complex copy a of n:    z = tau_n(e) v_j,a,  m = A z + rho_e^{2n} e^{2 i n phi_e} B conj(z)
//   with A = cc[e, coff + 2a], B = cc[e, coff + 2 a_n + 2a] (complex pairs).
// (The reference's math contract, fused/attention.h:4-39, 167-232, 265-287.)
//
// Forward: one wavefront per target node, lanes over the field's copies (a
// lane holds up to NU copies), a serial walk over the neighbourhood: per edge
// the wave reads the edge's coefficient row (contiguous), the source's value
// row (contiguous) and the edge's phases and weight (broadcast).
// Backward: one wavefront per SOURCE node over the edges grouped by source:
// each edge's coefficient gradients are its own rows (written once), and the
// source's value gradient sum_e conj(tau) dz_e accumulates in registers, so
// no atomics are needed and the result is deterministic.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "layout.hpp"

namespace gm {
namespace {

constexpr int kMaxUnitsPerLane = 8;  // 8 * 64 = 512 copies >= any D <= 512

template <typename T>
struct ConvArgs {
  const T* v;
  const T* rc;  // (n_edges, A0)
  const T* cc;  // (n_edges, W)
  const T* transport;
  const T* angular;
  const T* rho;
  const T* weights;
  const int64_t* row_ptr;
  const int64_t* source;
  const T* g;
  T* out;
  T* dv;
  T* drc;
  T* dcc;
  const int64_t* src_ptr;
  const int64_t* src_order;
  const int64_t* target;
  int64_t n_nodes;
  int D, orders, A0, W, units;
  AttnLayout L;
};

// One copy of the field as a lane sees it.
struct Unit {
  int n;     // frequency (0: scalar)
  int col;   // first flat column (the real part for a pair)
  int ca;    // rc column (scalar) or A's column in cc (complex)
  int cb;    // B's column in cc (complex)
  bool live;
};

template <typename T>
__device__ __forceinline__ Unit unit_of(const ConvArgs<T>& a, int u) {
  Unit out{0, 0, 0, 0, false};
  if (u >= a.units) return out;
  int first = 0;
  for (int f = 0; f < a.L.F; ++f) {
    const int an = a.L.a[f];
    if (u < first + an) {
      const int c = u - first;
      out.n = a.L.n[f];
      out.live = true;
      if (out.n == 0) {
        out.col = a.L.off[f] + c;
        out.ca = c;  // the reference indexes rc by copy: rc[e * A0 + a]
      } else {
        out.col = a.L.off[f] + 2 * c;
        out.ca = a.L.coff[f] + 2 * c;
        out.cb = a.L.coff[f] + 2 * an + 2 * c;
      }
      return out;
    }
    first += an;
  }
  return out;
}

template <typename T>
__device__ __forceinline__ T radial_power(T rho, int n) {  // (r / c)^{2n} by repeated multiplication
  T s = T(1);
  for (int i = 0; i < 2 * n; ++i) s *= rho;
  return s;
}

template <typename T, int NU>
__global__ __launch_bounds__(256) void conv_forward_kernel(ConvArgs<T> a) {
  const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x & 63;
  const int64_t i = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (i >= a.n_nodes) return;
  Unit un[NU];
  T accr[NU], acci[NU];
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    un[k] = unit_of(a, lane + kWave * k);
    accr[k] = T(0);
    acci[k] = T(0);
  }
  const int64_t e0 = a.row_ptr[i], e1 = a.row_ptr[i + 1];
  for (int64_t e = e0; e < e1; ++e) {
    const int64_t j = a.source[e];
    const T w_e = a.weights[e];
    const T rho = a.rho[e];
    const T* vj = a.v + j * a.D;
    const T* tr = a.transport + e * a.orders * 2;
    const T* an = a.angular + e * a.orders * 2;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      if (!un[k].live) continue;
      if (un[k].n == 0) {
        accr[k] += w_e * (a.rc[e * a.A0 + un[k].ca] * vj[un[k].col]);
      } else {
        const int n = un[k].n;
        const T tc = tr[2 * n], ts = tr[2 * n + 1];
        const T v0 = vj[un[k].col], v1 = vj[un[k].col + 1];
        const T zr = tc * v0 - ts * v1, zi = tc * v1 + ts * v0;  // z = tau v
        const T* crow = a.cc + e * a.W;
        const T Ar = crow[un[k].ca], Ai = crow[un[k].ca + 1];
        const T Br = crow[un[k].cb], Bi = crow[un[k].cb + 1];
        const T p = radial_power(rho, n);
        const T wr = p * an[4 * n], wi = p * an[4 * n + 1];  // w = (r/c)^{2n} e^{2 i n phi}
        const T bzr = Br * zr + Bi * zi, bzi = Bi * zr - Br * zi;  // B conj(z)
        const T mr = (Ar * zr - Ai * zi) + (wr * bzr - wi * bzi);
        const T mi = (Ar * zi + Ai * zr) + (wr * bzi + wi * bzr);
        accr[k] += w_e * mr;
        acci[k] += w_e * mi;
      }
    }
  }
  T* oi = a.out + i * a.D;
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    if (!un[k].live) continue;
    oi[un[k].col] = accr[k];
    if (un[k].n != 0) oi[un[k].col + 1] = acci[k];
  }
}

template <typename T, int NU>
__global__ __launch_bounds__(256) void conv_backward_kernel(ConvArgs<T> a) {
  const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x & 63;
  const int64_t j = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (j >= a.n_nodes) return;
  Unit un[NU];
  T vr[NU], vi[NU], dvr[NU], dvi[NU];
  const T* vj = a.v + j * a.D;
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    un[k] = unit_of(a, lane + kWave * k);
    vr[k] = un[k].live ? vj[un[k].col] : T(0);
    vi[k] = (un[k].live && un[k].n != 0) ? vj[un[k].col + 1] : T(0);
    dvr[k] = T(0);
    dvi[k] = T(0);
  }
  const int64_t g0 = a.src_ptr[j], g1 = a.src_ptr[j + 1];
  for (int64_t g = g0; g < g1; ++g) {
    const int64_t e = a.src_order[g];
    const int64_t t = a.target[e];
    const T w_e = a.weights[e];
    const T rho = a.rho[e];
    const T* gt = a.g + t * a.D;
    const T* tr = a.transport + e * a.orders * 2;
    const T* an = a.angular + e * a.orders * 2;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      if (!un[k].live) continue;
      if (un[k].n == 0) {
        const int64_t ri = e * a.A0 + un[k].ca;
        const T dm = w_e * gt[un[k].col];
        a.drc[ri] = dm * vr[k];
        dvr[k] += dm * a.rc[ri];
      } else {
        const int n = un[k].n;
        const T tc = tr[2 * n], ts = tr[2 * n + 1];
        const T zr = tc * vr[k] - ts * vi[k], zi = tc * vi[k] + ts * vr[k];
        const T* crow = a.cc + e * a.W;
        T* drow = a.dcc + e * a.W;
        const T Ar = crow[un[k].ca], Ai = crow[un[k].ca + 1];
        const T Br = crow[un[k].cb], Bi = crow[un[k].cb + 1];
        const T p = radial_power(rho, n);
        const T wr = p * an[4 * n], wi = p * an[4 * n + 1];
        const T dmr = w_e * gt[un[k].col], dmi = w_e * gt[un[k].col + 1];
        // dA = dm conj(z); dB = (dm conj(w)) z
        drow[un[k].ca] = dmr * zr + dmi * zi;
        drow[un[k].ca + 1] = dmi * zr - dmr * zi;
        const T xr = dmr * wr + dmi * wi, xi = dmi * wr - dmr * wi;
        drow[un[k].cb] = xr * zr - xi * zi;
        drow[un[k].cb + 1] = xr * zi + xi * zr;
        // dz = conj(A) dm + w (B conj(dm))
        const T bdr = Br * dmr + Bi * dmi, bdi = Bi * dmr - Br * dmi;
        const T dzr = (Ar * dmr + Ai * dmi) + (wr * bdr - wi * bdi);
        const T dzi = (Ar * dmi - Ai * dmr) + (wr * bdi + wi * bdr);
        // dv += conj(tau) dz
        dvr[k] += tc * dzr + ts * dzi;
        dvi[k] += tc * dzi - ts * dzr;
      }
    }
  }
  T* dvj = a.dv + j * a.D;
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    if (!un[k].live) continue;
    dvj[un[k].col] = dvr[k];
    if (un[k].n != 0) dvj[un[k].col + 1] = dvi[k];
  }
}

template <typename T>
int prepare(ConvArgs<T>& a, const T* v, const T* rc, const T* cc, const T* transport, const T* angular,
            const T* rho, const T* weights, const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
            int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t A0, int64_t W) {
  a = ConvArgs<T>{};
  GM_REQUIRE(n_nodes >= 0 && n_edges >= 0 && A0 >= 0 && W >= 0, "sizes must be non-negative");
  GM_REQUIRE(n_nodes < (int64_t(1) << 31) * kWavesPerBlock, "too many nodes for one launch");
  int rc_status = parse_attention_layout(desc, F, 1, D, orders, a.L);
  if (rc_status != GM_OK) return rc_status;
  // The depthwise layout covers the flat width exactly once (the outputs are written per copy).
  int covered = 0, units = 0;
  for (int f = 0; f < a.L.F; ++f) {
    covered += a.L.a[f] * a.L.dim[f];
    units += a.L.a[f];
    GM_REQUIRE(2 * a.L.n[f] < orders, "the angular table must hold order 2n for every frequency n");
    if (a.L.n[f] == 0) {
      GM_REQUIRE(a.L.a[f] <= A0, "rc narrower than the scalar copies");
    } else {
      GM_REQUIRE(a.L.coff[f] + 4 * a.L.a[f] <= W, "cc narrower than the descriptor's coefficient columns");
    }
  }
  GM_REQUIRE(covered == D, "the descriptor rows must tile the flat width D");
  if (n_nodes > 0) GM_REQUIRE(v && row_ptr, "v and row_ptr must be device pointers");
  if (n_edges > 0) {
    GM_REQUIRE(transport && angular && rho && weights && source, "the per-edge tables must be device pointers");
    GM_REQUIRE((A0 == 0 || rc) && (W == 0 || cc), "the coefficients must be device pointers");
  }
  a.v = v;
  a.rc = rc;
  a.cc = cc;
  a.transport = transport;
  a.angular = angular;
  a.rho = rho;
  a.weights = weights;
  a.row_ptr = row_ptr;
  a.source = source;
  a.n_nodes = n_nodes;
  a.D = (int)D;
  a.orders = (int)orders;
  a.A0 = (int)A0;
  a.W = (int)W;
  a.units = units;
  return GM_OK;
}

template <typename T, int NU>
void launch_n(bool forward, const ConvArgs<T>& a, hipStream_t stream) {
  const dim3 grid((unsigned)blocks_for(a.n_nodes));
  if (forward)
    hipLaunchKernelGGL((conv_forward_kernel<T, NU>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((conv_backward_kernel<T, NU>), grid, dim3(256), 0, stream, a);
}

template <typename T>
void launch(bool forward, const ConvArgs<T>& a, hipStream_t stream) {
  const int nu = (a.units + kWave - 1) / kWave;
  switch (nu <= 1 ? 1 : nu) {
    case 1: launch_n<T, 1>(forward, a, stream); break;
    case 2: launch_n<T, 2>(forward, a, stream); break;
    case 3: launch_n<T, 3>(forward, a, stream); break;
    case 4: launch_n<T, 4>(forward, a, stream); break;
    case 5: launch_n<T, 5>(forward, a, stream); break;
    case 6: launch_n<T, 6>(forward, a, stream); break;
    case 7: launch_n<T, 7>(forward, a, stream); break;
    default: launch_n<T, kMaxUnitsPerLane>(forward, a, stream); break;
  }
}

template <typename T>
int conv_forward(const T* v, const T* rc, const T* cc, const T* transport, const T* angular, const T* rho,
                 const T* weights, const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
                 int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t A0, int64_t W, T* out,
                 hipStream_t stream) {
  ConvArgs<T> a;
  const int status = prepare(a, v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, n_nodes, n_edges,
                             D, orders, F, A0, W);
  if (status != GM_OK) return status;
  if (n_nodes == 0) return GM_OK;
  GM_REQUIRE(out, "out must be a device pointer");
  a.out = out;
  launch(true, a, stream);
  return check_launch("conv_forward");
}

template <typename T>
int conv_backward(const T* g, const T* v, const T* rc, const T* cc, const T* transport, const T* angular,
                  const T* rho, const T* weights, const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
                  int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t A0, int64_t W,
                  const int64_t* src_ptr, const int64_t* src_order, const int64_t* target, T* dv, T* drc, T* dcc,
                  hipStream_t stream) {
  ConvArgs<T> a;
  const int status = prepare(a, v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, n_nodes, n_edges,
                             D, orders, F, A0, W);
  if (status != GM_OK) return status;
  if (n_nodes == 0) return GM_OK;
  GM_REQUIRE(g && dv && src_ptr, "g, dv and src_ptr must be device pointers");
  if (n_edges > 0) {
    GM_REQUIRE(src_order && target, "src_order and target must be device pointers");
    GM_REQUIRE((A0 == 0 || drc) && (W == 0 || dcc), "drc and dcc must be device pointers");
  }
  a.g = g;
  a.dv = dv;
  a.drc = drc;
  a.dcc = dcc;
  a.src_ptr = src_ptr;
  a.src_order = src_order;
  a.target = target;
  launch(false, a, stream);
  return check_launch("conv_backward");
}

}  // namespace
}  // namespace gm

extern "C" int gm_conv_forward_f32(const float* v, const float* rc, const float* cc, const float* transport,
                                   const float* angular, const float* rho, const float* weights, const int64_t* desc,
                                   const int64_t* row_ptr, const int64_t* source, int64_t n_nodes, int64_t n_edges,
                                   int64_t D, int64_t orders, int64_t F, int64_t A0, int64_t W, float* out,
                                   void* stream) {
  return gm::conv_forward<float>(v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, n_nodes, n_edges,
                                 D, orders, F, A0, W, out, (hipStream_t)stream);
}

extern "C" int gm_conv_forward_f64(const double* v, const double* rc, const double* cc, const double* transport,
                                   const double* angular, const double* rho, const double* weights,
                                   const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
                                   int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F,
                                   int64_t A0, int64_t W, double* out, void* stream) {
  return gm::conv_forward<double>(v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, n_nodes,
                                  n_edges, D, orders, F, A0, W, out, (hipStream_t)stream);
}

extern "C" int gm_conv_backward_f32(const float* g, const float* v, const float* rc, const float* cc,
                                    const float* transport, const float* angular, const float* rho,
                                    const float* weights, const int64_t* desc, const int64_t* row_ptr,
                                    const int64_t* source, int64_t n_nodes, int64_t n_edges, int64_t D,
                                    int64_t orders, int64_t F, int64_t A0, int64_t W, const int64_t* src_ptr,
                                    const int64_t* src_order, const int64_t* target, float* dv, float* drc,
                                    float* dcc, void* stream) {
  return gm::conv_backward<float>(g, v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, n_nodes,
                                  n_edges, D, orders, F, A0, W, src_ptr, src_order, target, dv, drc, dcc,
                                  (hipStream_t)stream);
}

extern "C" int gm_conv_backward_f64(const double* g, const double* v, const double* rc, const double* cc,
                                    const double* transport, const double* angular, const double* rho,
                                    const double* weights, const int64_t* desc, const int64_t* row_ptr,
                                    const int64_t* source, int64_t n_nodes, int64_t n_edges, int64_t D,
                                    int64_t orders, int64_t F, int64_t A0, int64_t W, const int64_t* src_ptr,
                                    const int64_t* src_order, const int64_t* target, double* dv, double* drc,
                                    double* dcc, void* stream) {
  return gm::conv_backward<double>(g, v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, n_nodes,
                                   n_edges, D, orders, F, A0, W, src_ptr, src_order, target, dv, drc, dcc,
                                   (hipStream_t)stream);
}
