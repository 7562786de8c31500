// The transformer block's pointwise operators on the flat node layout:
// the merged equivariant layer normalization and the scalar-gated
// nonlinearity, forward and backward, for float, double and bfloat16 fields
// (bfloat16 in and out, float arithmetic; parameters in float, or double for
// double fields).
//
// Layer normalization (nn/normalization.py:22-190 in the reference): at a
// node, with frequency 0 in the first a0 entries and frequency n's copies as
// (re, im) pairs at [off_n, off_n + 2 m_n),
//   mu = mean x0;  v0 = mean (x0 - mu)^2;  vn = (1 / 2 m_n) sum |x_n|^2;
//   d = sqrt(mean over present frequencies of v + eps);
//   y = gamma * (x - mu [frequency 0 only]) / d + beta [frequency 0 only].
// gamma arrives expanded to the flat width (one value per coordinate).
// One wavefront per node; the backward keeps dgamma / dbeta partial sums per
// wavefront across the nodes it visits and reduces the rows in a fixed order.
//
// Gated nonlinearity (nn/nonlinearities.py:51-166): y0 = SiLU(h0), and each
// copy a of frequency n scaled by act(pre[n, a]), act = SiLU or 2 sigmoid,
// pre the gate pre-activations (affine in h0, a library GEMM upstream).
#include <algorithm>

#include "common.hpp"

namespace gm {
namespace {

constexpr int kPwMaxFreq = 8;        // nonzero frequencies of one field type
constexpr int kPwMaxChunks = 16;     // flat width up to 64 * 16 = 1024
constexpr int kPwWaves = 4;          // wavefronts (nodes) per workgroup
constexpr int kPwThreads = kWave * kPwWaves;
constexpr int kPwReduceThreads = 256;

// bfloat16 as raw 16-bit storage: widening is a shift; narrowing rounds to nearest even.
struct bf16 {
  uint16_t bits;
};

__device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
__device__ __forceinline__ double load(const double* p, int64_t i) { return p[i]; }
__device__ __forceinline__ float load(const bf16* p, int64_t i) {
  return __uint_as_float(static_cast<uint32_t>(p[i].bits) << 16);
}
__device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
__device__ __forceinline__ void store(double* p, int64_t i, double v) { p[i] = v; }
__device__ __forceinline__ void store(bf16* p, int64_t i, float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    p[i].bits = static_cast<uint16_t>((u >> 16) | 0x40);  // quiet NaN
    return;
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  p[i].bits = static_cast<uint16_t>(u >> 16);
}

template <typename T>
struct AccOf {
  using type = float;
};
template <>
struct AccOf<double> {
  using type = double;
};

template <typename A>
__device__ __forceinline__ A wave_sum(A v) {
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

template <typename A>
__device__ __forceinline__ A sigmoid(A x) {
  return A(1) / (A(1) + exp(-x));
}

struct PwLayout {
  int64_t n_nodes;
  int D;       // flat width
  int a0;      // frequency-0 entries (0 when absent)
  int nf;      // nonzero frequencies
  int off[kPwMaxFreq];
  int mult[kPwMaxFreq];
};

// Which statistic entry k of the flat row feeds: 0 for frequency 0, 1 + f for the f-th nonzero frequency.
__device__ __forceinline__ int slot_of(const PwLayout& L, int k) {
  if (k < L.a0) return 0;
  int s = 1;
  for (int f = 0; f < L.nf; ++f)
    if (k >= L.off[f] && k < L.off[f] + 2 * L.mult[f]) s = 1 + f;
  return s;
}

template <typename T, typename A>
struct NormArgs {
  PwLayout L;
  const T* x;
  const A* gamma;  // (D): per-coordinate gains
  const A* beta;   // (a0) or null
  T* y;
  A* mean;         // (n_nodes)
  A* inv_d;        // (n_nodes)
  double eps;
  // backward
  const T* gy;
  T* dx;
  A* partial;      // (n_waves, D + a0): dgamma then dbeta
};

// Per-node statistics of the values a lane holds (entries lane + 64 j, j < CH).
template <int CH, typename A>
__device__ __forceinline__ void node_stats(const PwLayout& L, const A* v, int lane, A& mu, A& inv_d, double eps) {
  A s0 = 0;
  for (int j = 0; j < CH; ++j) {
    const int k = lane + kWave * j;
    if (k < L.a0) s0 += v[j];
  }
  mu = L.a0 > 0 ? wave_sum(s0) / A(L.a0) : A(0);
  A acc[1 + kPwMaxFreq];
  for (int s = 0; s <= L.nf; ++s) acc[s] = 0;
  for (int j = 0; j < CH; ++j) {
    const int k = lane + kWave * j;
    if (k < L.D) {
      const int s = slot_of(L, k);
      const A c = s == 0 ? v[j] - mu : v[j];
      for (int t = 0; t <= L.nf; ++t)
        if (t == s) acc[t] += c * c;
    }
  }
  A total = 0;
  int present = 0;
  if (L.a0 > 0) {
    total += wave_sum(acc[0]) / A(L.a0);
    ++present;
  }
  for (int f = 0; f < L.nf; ++f) {
    total += wave_sum(acc[1 + f]) / A(2 * L.mult[f]);
    ++present;
  }
  inv_d = A(1) / sqrt(total / A(present) + A(eps));
}

// CH: 64-entry chunks per row (the flat width rounded up to a power of two).
template <typename T, int CH>
__global__ __launch_bounds__(kPwThreads) void layer_norm_forward_kernel(NormArgs<T, typename AccOf<T>::type> a) {
  using A = typename AccOf<T>::type;
  const int lane = threadIdx.x % kWave;
  const int64_t node = (int64_t)blockIdx.x * kPwWaves + threadIdx.x / kWave;
  if (node >= a.L.n_nodes) return;
  const int64_t row = node * a.L.D;
  A v[CH];
  for (int j = 0; j < CH; ++j) {
    const int k = lane + kWave * j;
    v[j] = k < a.L.D ? A(load(a.x, row + k)) : A(0);
  }
  A mu, inv_d;
  node_stats<CH>(a.L, v, lane, mu, inv_d, a.eps);
  for (int j = 0; j < CH; ++j) {
    const int k = lane + kWave * j;
    if (k < a.L.D) {
      const bool scalar = k < a.L.a0;
      A out = a.gamma[k] * ((scalar ? v[j] - mu : v[j]) * inv_d);
      if (scalar && a.beta) out += a.beta[k];
      store(a.y, row + k, out);
    }
  }
  if (lane == 0) {
    a.mean[node] = mu;
    a.inv_d[node] = inv_d;
  }
}

// Persistent wavefronts: wave w visits nodes w, w + W, ...; dx per node, and
// its dgamma / dbeta partial row over the nodes it visited.
template <typename T, int CH>
__global__ __launch_bounds__(kPwThreads) void layer_norm_backward_kernel(NormArgs<T, typename AccOf<T>::type> a) {
  using A = typename AccOf<T>::type;
  const int lane = threadIdx.x % kWave;
  const int64_t wave = (int64_t)blockIdx.x * kPwWaves + threadIdx.x / kWave;
  const int64_t n_waves = (int64_t)gridDim.x * kPwWaves;
  const int present = (a.L.a0 > 0 ? 1 : 0) + a.L.nf;
  A dgamma[CH], dbeta[CH], w[CH];
  for (int j = 0; j < CH; ++j) {
    dgamma[j] = dbeta[j] = 0;
    const int k = lane + kWave * j;
    // d(mean v)/d x_k = w_k x'_k / present with w = 2 / a0 (frequency 0) or 1 / m_n
    A wk = 0;
    if (k < a.L.D) {
      const int s = slot_of(a.L, k);
      wk = s == 0 ? A(2) / A(a.L.a0) : A(1) / A(a.L.mult[s - 1]);
    }
    w[j] = wk / A(2 * present);
  }
  for (int64_t node = wave; node < a.L.n_nodes; node += n_waves) {
    const int64_t row = node * a.L.D;
    const A mu = a.mean[node], inv_d = a.inv_d[node];
    A xhat[CH], gh[CH], gy[CH];
    A p = 0, g0 = 0;
    for (int j = 0; j < CH; ++j) {
      const int k = lane + kWave * j;
      xhat[j] = gh[j] = gy[j] = 0;
      if (k < a.L.D) {
        const bool scalar = k < a.L.a0;
        const A x = A(load(a.x, row + k));
        xhat[j] = (scalar ? x - mu : x) * inv_d;
        gy[j] = A(load(a.gy, row + k));
        gh[j] = gy[j] * a.gamma[k];
        p += gh[j] * xhat[j];
        if (scalar) g0 += gh[j];
      }
    }
    p = wave_sum(p);
    g0 = a.L.a0 > 0 ? wave_sum(g0) / A(a.L.a0) : A(0);
    for (int j = 0; j < CH; ++j) {
      const int k = lane + kWave * j;
      if (k < a.L.D) {
        const bool scalar = k < a.L.a0;
        store(a.dx, row + k, inv_d * (gh[j] - (scalar ? g0 : A(0)) - p * xhat[j] * w[j]));
        dgamma[j] += gy[j] * xhat[j];
        if (scalar) dbeta[j] += gy[j];
      }
    }
  }
  A* out = a.partial + wave * (a.L.D + a.L.a0);
  for (int j = 0; j < CH; ++j) {
    const int k = lane + kWave * j;
    if (k < a.L.D) out[k] = dgamma[j];
    if (k < a.L.a0) out[a.L.D + k] = dbeta[j];
  }
}

// dparams[c] = sum over rows r of partial[r, c], rows in increasing order per
// thread, then a fixed tree over the workgroup.
template <typename A>
__global__ __launch_bounds__(kPwReduceThreads) void pw_reduce_kernel(const A* __restrict__ partial, int64_t rows,
                                                                     int cols, A* __restrict__ out) {
  __shared__ A buf[kPwReduceThreads];
  const int c = blockIdx.x;
  A s = 0;
  for (int64_t r = threadIdx.x; r < rows; r += kPwReduceThreads) s += partial[r * cols + c];
  buf[threadIdx.x] = s;
  __syncthreads();
  for (int step = kPwReduceThreads / 2; step > 0; step >>= 1) {
    if (threadIdx.x < step) buf[threadIdx.x] += buf[threadIdx.x + step];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[c] = buf[0];
}

template <typename T>
struct GateArgs {
  PwLayout L;     // the hidden field's layout
  int G;          // gate width: sum of the nonzero frequencies' multiplicities
  int goff[kPwMaxFreq];
  int double_sigmoid;
  const T* h;     // (n_nodes, D)
  const T* pre;   // (n_nodes, G)
  T* y;
  const T* gy;
  T* dh;
  T* dpre;
};

template <typename A>
__device__ __forceinline__ void gate_of(A pre, int double_sigmoid, A& g, A& dg) {
  const A s = sigmoid(pre);
  if (double_sigmoid) {
    g = A(2) * s;
    dg = A(2) * s * (A(1) - s);
  } else {
    g = pre * s;
    dg = s * (A(1) + pre * (A(1) - s));
  }
}

// One thread per (node, unit): units 0..a0-1 are the scalar channels, then one per gated copy.
template <typename T, bool kBackward>
__global__ __launch_bounds__(256) void gate_kernel(GateArgs<T> a) {
  using A = typename AccOf<T>::type;
  const int units = a.L.a0 + a.G;
  const int64_t total = a.L.n_nodes * units;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += stride) {
    const int64_t node = t / units;
    const int u = (int)(t - node * units);
    const int64_t row = node * a.L.D;
    if (u < a.L.a0) {
      const A h = A(load(a.h, row + u));
      A g, dg;
      gate_of(h, 0, g, dg);  // SiLU and its derivative
      if (kBackward)
        store(a.dh, row + u, A(load(a.gy, row + u)) * dg);
      else
        store(a.y, row + u, g);
      continue;
    }
    const int c = u - a.L.a0;
    int f = 0;
    for (int q = 1; q < a.L.nf; ++q)
      if (c >= a.goff[q]) f = q;
    const int copy = c - a.goff[f];
    const int64_t k = row + a.L.off[f] + 2 * copy;
    const A pre = A(load(a.pre, node * a.G + c));
    A g, dg;
    gate_of(pre, a.double_sigmoid, g, dg);
    const A h0 = A(load(a.h, k)), h1 = A(load(a.h, k + 1));
    if (kBackward) {
      const A gy0 = A(load(a.gy, k)), gy1 = A(load(a.gy, k + 1));
      store(a.dh, k, gy0 * g);
      store(a.dh, k + 1, gy1 * g);
      store(a.dpre, node * a.G + c, dg * (gy0 * h0 + gy1 * h1));
    } else {
      store(a.y, k, g * h0);
      store(a.y, k + 1, g * h1);
    }
  }
}

int fill_layout(PwLayout& L, int64_t n_nodes, int64_t D, int64_t a0, int64_t nf, const int64_t* offsets,
                const int64_t* mults) {
  GM_REQUIRE(n_nodes >= 0, "n_nodes must be non-negative");
  GM_REQUIRE(D >= 1 && D <= kWave * kPwMaxChunks, "the flat width must lie in 1..1024");
  GM_REQUIRE(nf >= 0 && nf <= kPwMaxFreq, "at most 8 nonzero frequencies");
  GM_REQUIRE(a0 >= 0 && a0 <= D, "a0 must lie in 0..D");
  GM_REQUIRE(a0 > 0 || nf > 0, "the field must have at least one frequency");
  GM_REQUIRE(nf == 0 || (offsets && mults), "offsets and multiplicities (host arrays) are required");
  L.n_nodes = n_nodes;
  L.D = (int)D;
  L.a0 = (int)a0;
  L.nf = (int)nf;
  int64_t next = a0;
  for (int f = 0; f < nf; ++f) {
    GM_REQUIRE(mults[f] >= 1 && offsets[f] == next, "frequency blocks must follow frequency 0 contiguously");
    L.off[f] = (int)offsets[f];
    L.mult[f] = (int)mults[f];
    next += 2 * mults[f];
  }
  GM_REQUIRE(next == D, "the frequency blocks must fill the flat width");
  return GM_OK;
}

int64_t norm_blocks(int64_t n_nodes) { return std::max<int64_t>(1, std::min<int64_t>((n_nodes + 3) / 4, 1024)); }

// Launch KERNEL<T, CH> with CH the flat width's 64-entry chunks rounded up to a power of two.
#define GM_PW_DISPATCH_CH(KERNEL, T, D, GRID, STREAM, ARGS)                                     \
  do {                                                                                          \
    const int64_t chunks_ = ((D) + kWave - 1) / kWave;                                          \
    if (chunks_ <= 1)                                                                           \
      hipLaunchKernelGGL((KERNEL<T, 1>), GRID, dim3(kPwThreads), 0, STREAM, ARGS);              \
    else if (chunks_ <= 2)                                                                      \
      hipLaunchKernelGGL((KERNEL<T, 2>), GRID, dim3(kPwThreads), 0, STREAM, ARGS);              \
    else if (chunks_ <= 4)                                                                      \
      hipLaunchKernelGGL((KERNEL<T, 4>), GRID, dim3(kPwThreads), 0, STREAM, ARGS);              \
    else if (chunks_ <= 8)                                                                      \
      hipLaunchKernelGGL((KERNEL<T, 8>), GRID, dim3(kPwThreads), 0, STREAM, ARGS);              \
    else                                                                                        \
      hipLaunchKernelGGL((KERNEL<T, 16>), GRID, dim3(kPwThreads), 0, STREAM, ARGS);             \
  } while (0)

template <typename T>
int norm_forward(const T* x, const typename AccOf<T>::type* gamma, const typename AccOf<T>::type* beta,
                 int64_t n_nodes, int64_t D, int64_t a0, int64_t nf, const int64_t* offsets, const int64_t* mults,
                 double eps, T* y, typename AccOf<T>::type* mean, typename AccOf<T>::type* inv_d, void* stream) {
  NormArgs<T, typename AccOf<T>::type> a{};
  const int status = fill_layout(a.L, n_nodes, D, a0, nf, offsets, mults);
  if (status != GM_OK) return status;
  GM_REQUIRE(eps > 0, "eps must be positive");
  if (n_nodes == 0) return GM_OK;
  GM_REQUIRE(x && gamma && y && mean && inv_d, "x, gamma, y, mean and inv_d must be device pointers");
  a.x = x;
  a.gamma = gamma;
  a.beta = a0 > 0 ? beta : nullptr;
  a.y = y;
  a.mean = mean;
  a.inv_d = inv_d;
  a.eps = eps;
  GM_PW_DISPATCH_CH(layer_norm_forward_kernel, T, D, dim3((unsigned)((n_nodes + kPwWaves - 1) / kPwWaves)),
                    (hipStream_t)stream, a);
  return check_launch("layer_norm_forward");
}

template <typename T>
int norm_backward(const T* gy, const T* x, const typename AccOf<T>::type* gamma,
                  const typename AccOf<T>::type* mean, const typename AccOf<T>::type* inv_d, int64_t n_nodes,
                  int64_t D, int64_t a0, int64_t nf, const int64_t* offsets, const int64_t* mults, T* dx,
                  typename AccOf<T>::type* partial, typename AccOf<T>::type* dparams, void* stream) {
  using A = typename AccOf<T>::type;
  NormArgs<T, A> a{};
  const int status = fill_layout(a.L, n_nodes, D, a0, nf, offsets, mults);
  if (status != GM_OK) return status;
  GM_REQUIRE(partial && dparams, "partial and dparams must be device pointers");
  if (n_nodes > 0) GM_REQUIRE(gy && x && gamma && mean && inv_d && dx, "gy, x, gamma, mean, inv_d and dx must be device pointers");
  a.gy = gy;
  a.x = x;
  a.gamma = gamma;
  a.mean = const_cast<A*>(mean);  // read only in the backward
  a.inv_d = const_cast<A*>(inv_d);
  a.dx = dx;
  a.partial = partial;
  const int64_t blocks = norm_blocks(n_nodes);
  const hipStream_t s = (hipStream_t)stream;
  GM_PW_DISPATCH_CH(layer_norm_backward_kernel, T, D, dim3((unsigned)blocks), s, a);
  int rc = check_launch("layer_norm_backward");
  if (rc != GM_OK) return rc;
  hipLaunchKernelGGL(pw_reduce_kernel<A>, dim3((unsigned)(D + a0)), dim3(kPwReduceThreads), 0, s,
                     (const A*)partial, blocks * kPwWaves, (int)(D + a0), dparams);
  return check_launch("layer_norm_backward (reduce)");
}

template <typename T>
int gate(bool backward, const T* h, const T* pre, const T* gy, int64_t n_nodes, int64_t D, int64_t a0, int64_t nf,
         const int64_t* offsets, const int64_t* mults, int64_t double_sigmoid, T* y, T* dh, T* dpre, void* stream) {
  GateArgs<T> a{};
  const int status = fill_layout(a.L, n_nodes, D, a0, nf, offsets, mults);
  if (status != GM_OK) return status;
  GM_REQUIRE(a0 > 0, "the gated nonlinearity needs frequency-0 channels");
  int g = 0;
  for (int f = 0; f < nf; ++f) {
    a.goff[f] = g;
    g += (int)mults[f];
  }
  a.G = g;
  a.double_sigmoid = double_sigmoid ? 1 : 0;
  if (n_nodes == 0) return GM_OK;
  GM_REQUIRE(h && (pre || g == 0), "h and pre must be device pointers");
  if (backward)
    GM_REQUIRE(gy && dh && (dpre || g == 0), "gy, dh and dpre must be device pointers");
  else
    GM_REQUIRE(y, "y must be a device pointer");
  a.h = h;
  a.pre = pre;
  a.y = y;
  a.gy = gy;
  a.dh = dh;
  a.dpre = dpre;
  const int64_t total = n_nodes * (a0 + g);
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((total + 255) / 256, 16384));
  const hipStream_t s = (hipStream_t)stream;
  if (backward)
    hipLaunchKernelGGL((gate_kernel<T, true>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((gate_kernel<T, false>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch(backward ? "gate_backward" : "gate_forward");
}

}  // namespace
}  // namespace gm

extern "C" int64_t gm_layer_norm_partial_rows(int64_t n_nodes) { return gm::norm_blocks(n_nodes) * gm::kPwWaves; }

// X: the element type in the C signature (uint16_t for bfloat16), T: the kernels' element type.
#define GM_NORM_ENTRY(SFX, X, T, A)                                                                                 \
  extern "C" int gm_layer_norm_forward_##SFX(const X* x, const A* gamma, const A* beta, int64_t n_nodes, int64_t D, \
                                             int64_t a0, int64_t nf, const int64_t* offsets, const int64_t* mults, \
                                             double eps, X* y, A* mean, A* inv_d, void* stream) {                   \
    return gm::norm_forward<T>(reinterpret_cast<const T*>(x), gamma, beta, n_nodes, D, a0, nf, offsets, mults,    \
                               eps, reinterpret_cast<T*>(y), mean, inv_d, stream);                                  \
  }                                                                                                                \
  extern "C" int gm_layer_norm_backward_##SFX(const X* gy, const X* x, const A* gamma, const A* mean,              \
                                              const A* inv_d, int64_t n_nodes, int64_t D, int64_t a0, int64_t nf,   \
                                              const int64_t* offsets, const int64_t* mults, X* dx, A* partial,      \
                                              A* dparams, void* stream) {                                           \
    return gm::norm_backward<T>(reinterpret_cast<const T*>(gy), reinterpret_cast<const T*>(x), gamma, mean, inv_d, \
                                n_nodes, D, a0, nf, offsets, mults, reinterpret_cast<T*>(dx), partial, dparams,     \
                                stream);                                                                            \
  }                                                                                                                \
  extern "C" int gm_gate_forward_##SFX(const X* h, const X* pre, int64_t n_nodes, int64_t D, int64_t a0,           \
                                       int64_t nf, const int64_t* offsets, const int64_t* mults,                   \
                                       int64_t double_sigmoid, X* y, void* stream) {                                \
    return gm::gate<T>(false, reinterpret_cast<const T*>(h), reinterpret_cast<const T*>(pre), nullptr, n_nodes, D, \
                       a0, nf, offsets, mults, double_sigmoid, reinterpret_cast<T*>(y), nullptr, nullptr, stream);  \
  }                                                                                                                \
  extern "C" int gm_gate_backward_##SFX(const X* gy, const X* h, const X* pre, int64_t n_nodes, int64_t D,         \
                                        int64_t a0, int64_t nf, const int64_t* offsets, const int64_t* mults,       \
                                        int64_t double_sigmoid, X* dh, X* dpre, void* stream) {                     \
    return gm::gate<T>(true, reinterpret_cast<const T*>(h), reinterpret_cast<const T*>(pre),                       \
                       reinterpret_cast<const T*>(gy), n_nodes, D, a0, nf, offsets, mults, double_sigmoid, nullptr, \
                       reinterpret_cast<T*>(dh), reinterpret_cast<T*>(dpre), stream);                               \
  }

GM_NORM_ENTRY(f32, float, float, float)
GM_NORM_ENTRY(f64, double, double, double)
GM_NORM_ENTRY(bf16, uint16_t, gm::bf16, float)
