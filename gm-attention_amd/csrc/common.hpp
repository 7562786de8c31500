// Shared device and host helpers of libgmhip.so (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <string>

#include "gm_hip.h"

namespace gm {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;  // 256-thread workgroups: one node per wavefront

// ---- error reporting (runtime.hip) ----
void set_error(const std::string& message);
int fail(int code, const std::string& message);  // set_error + return code
int check_launch(const char* what);               // hipGetLastError after a launch

// ---- launch geometry (runtime.hip) ----
// Workgroups of `kernel` (`threads` threads, `lds` bytes of dynamic LDS)
// resident on the current device at once, CUs x workgroups per CU; 0 when the
// runtime cannot say (no device).  Cached per device and kernel.
int64_t resident_blocks(const void* kernel, int threads, size_t lds = 0);
// The workgroups of a grid whose workgroups share the work evenly: about
// `want`, in whole rounds of `slots` resident ones (r slots, r = want / slots
// rounded, at least one), so that no last round runs on a fraction of the
// chip; `want` itself when the occupancy is unknown.
inline int64_t whole_rounds(int64_t want, int64_t slots) {
  if (slots <= 0) return want;
  int64_t r = (want + slots / 2) / slots;
  return (r < 1 ? 1 : r) * slots;
}

#define GM_REQUIRE(cond, message)                                   \
  do {                                                              \
    if (!(cond)) return ::gm::fail(GM_ERR_ARGUMENT, (message));     \
  } while (0)

// ---- device helpers ----

template <typename T>
__device__ __forceinline__ T neg_inf() {
  return -static_cast<T>(INFINITY);
}

// Blocks are dispatched round-robin over the eight XCDs, each with its own L2.
// Remap so XCD x runs a contiguous range of logical blocks: neighbouring nodes
// (which share most of their neighbours' rows) then share one L2.
__host__ __device__ __forceinline__ int64_t xcd_block(int64_t b, int64_t nb) {
  const int64_t q = nb >> 3, r = nb & 7, x = b & 7;
  return x * q + (x < r ? x : r) + (b >> 3);
}

// The same XCD assignment in chunks of logical blocks dealt round-robin
// (XCD x runs chunks x, x + 8, ...; the last partial round keeps its order):
// every XCD then runs work from every latitude band.  Contiguous ranges are
// even only when each XCD's range holds a pole and an equator alike (B = 4 on
// eight XCDs); with two samples a range is a quarter of a sample and the
// polar quarters carry about five times the edges of the equatorial ones.
// Chunks are 32 blocks from 256 blocks up, nb / 32 (at least 1) below, so a
// small launch is still dealt in whole rounds.
__host__ __device__ __forceinline__ int64_t xcd_spread_block(int64_t b, int64_t nb) {
  const int64_t chunk = nb >= 256 ? 32 : (nb >= 64 ? nb >> 5 : 1);
  const int64_t full = nb / (8 * chunk) * (8 * chunk);
  if (b >= full) return b;
  const int64_t x = b & 7, i = b >> 3;
  return ((i / chunk) * 8 + x) * chunk + (i % chunk);
}

// xcd_block while its contiguous ranges hold about equal work (every range's
// CSR entries within a quarter of an eighth of the total), else
// xcd_spread_block.  `ptr` holds the CSR offsets of the n_items items the
// blocks own, `per` items a block; every block reads the same nine offsets
// and reaches the same choice.
__host__ __device__ __forceinline__ int64_t xcd_balanced_block(int64_t b, int64_t nb, const int64_t* ptr,
                                                               int64_t n_items, int per) {
  const int64_t q = nb >> 3, r = nb & 7;
  const int64_t first = ptr[0], total = ptr[n_items] - first;
  int64_t worst = 0, prev = first;
  for (int x = 1; x <= 8; ++x) {
    int64_t item = (x * q + (x < r ? x : r)) * per;
    if (item > n_items) item = n_items;
    const int64_t e = ptr[item];
    worst = e - prev > worst ? e - prev : worst;
    prev = e;
  }
  return 32 * worst > 5 * total ? xcd_spread_block(b, nb) : xcd_block(b, nb);
}

// Four consecutive elements (16 B for float, 32 B for double), aligned.
template <typename T>
struct Quad {
  T v[4];
};

__device__ __forceinline__ Quad<float> ld4(const float* p) {
  const float4 x = *reinterpret_cast<const float4*>(p);
  return {{x.x, x.y, x.z, x.w}};
}
__device__ __forceinline__ Quad<double> ld4(const double* p) {
  const double2 x = reinterpret_cast<const double2*>(p)[0];
  const double2 y = reinterpret_cast<const double2*>(p)[1];
  return {{x.x, x.y, y.x, y.y}};
}
__device__ __forceinline__ void st4(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st4(double* p, const double* v) {
  reinterpret_cast<double2*>(p)[0] = make_double2(v[0], v[1]);
  reinterpret_cast<double2*>(p)[1] = make_double2(v[2], v[3]);
}

__device__ __forceinline__ float gm_exp(float x) { return expf(x); }
__device__ __forceinline__ double gm_exp(double x) { return exp(x); }

// Sum over the lanes of one group g = lane % G (G a power of two dividing 64):
// a butterfly over the lane bits above log2(G); every lane gets its group's total.
template <typename T>
__device__ __forceinline__ T group_sum_pow2(T v, int G) {
  for (int off = G; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Sum over lanes h, h + G, ..., h + (S - 1) G for any G (S = 64 / G, floor):
// a tree into slot 0, then broadcast from lane h.  Lanes at or past S * G
// contribute nothing and receive their group's total all the same.
template <typename T>
__device__ __forceinline__ T group_sum(T v, int lane, int G, int S) {
  const int s = lane / G, h = lane % G;
  if (s >= S) v = T(0);
  for (int step = 1; step < S; step <<= 1) {
    const int from = lane + step * G;
    const T o = __shfl(v, from < kWave ? from : lane, kWave);
    if ((s % (2 * step)) == 0 && s + step < S) v += o;
  }
  return __shfl(v, h, kWave);
}

// Online softmax state (running maximum m and sum l of exp(x - m)).
template <typename T>
__device__ __forceinline__ void online_add(T& m, T& l, T x) {
  if (x == neg_inf<T>()) return;
  if (x > m) {
    l = (m == neg_inf<T>() ? T(0) : l * gm_exp(m - x)) + T(1);
    m = x;
  } else {
    l += gm_exp(x - m);
  }
}

template <typename T>
__device__ __forceinline__ void online_merge(T& m, T& l, T mo, T lo) {
  const T mn = m > mo ? m : mo;
  if (mn == neg_inf<T>()) return;
  const T a = (m == neg_inf<T>()) ? T(0) : l * gm_exp(m - mn);
  const T b = (mo == neg_inf<T>()) ? T(0) : lo * gm_exp(mo - mn);
  m = mn;
  l = a + b;
}

// Merge the online states of lanes h, h + G, ... (any G, S = 64 / G).
template <typename T>
__device__ __forceinline__ void group_online(T& m, T& l, int lane, int G, int S) {
  const int s = lane / G, h = lane % G;
  if (s >= S) {
    m = neg_inf<T>();
    l = T(0);
  }
  for (int step = 1; step < S; step <<= 1) {
    const int from = lane + step * G;
    const T mo = __shfl(m, from < kWave ? from : lane, kWave);
    const T lo = __shfl(l, from < kWave ? from : lane, kWave);
    if ((s % (2 * step)) == 0 && s + step < S) online_merge(m, l, mo, lo);
  }
  m = __shfl(m, h, kWave);
  l = __shfl(l, h, kWave);
}

inline bool aligned(const void* p, size_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

inline int64_t blocks_for(int64_t items) { return (items + kWavesPerBlock - 1) / kWavesPerBlock; }

}  // namespace gm
