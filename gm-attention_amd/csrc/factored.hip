// The factored steerable kernel over source-grouped edges, forward (the
// per-edge rows), the weighted per-target aggregate of the rows, and the
// backward (from the rows' gradient, or from the targets' gradient through
// the target index), for CDNA4 (gfx950).
//
// Per edge e = (i <- j), with h~ = (1, h(e)) and the source's mixes Z(j)
// (K x C: the complex blocks' (wc, 2) pairs then the real block's wr reals):
//   u_b(e)   = sum_t h~_t Z_t,b(j)                    (each block's combination)
//   row(e)   = per output group, sum_b F_b(e) u_b(e)   (F_b = e^{i a phi} e^{i s gamma} (r/c)^p;
//                                                     rows onto frequency 0 take the real part)
//   out(i)   = sum_{e -> i} w_e row(e)
// and from an edge's output gradient G (scaled by w_e in the aggregated form)
// the packed row W(e) = G conj(F_b) per block, dh_t(e) = <W(e), Z_t(j)> for
// t >= 1, dZ_t(j) = sum_{e <- j} h~_t(e) W(e), dw_e = <g(i), row(e)>.
// (The math contract of the reference's fused/factored.h:1-50.)
//
// Mapping: one wave64 workgroup per source group.  The source's Z(j) is
// staged once in LDS, column-major with K padded to a multiple of four, so
// one column's K mixes are 16-byte broadcast reads.  Lanes take the group's
// edges 64 at a time.  The backward parks each edge's W(e) and h~(e) in LDS
// and then lets every lane own whole packed columns of dZ(j), accumulated in
// registers over all of the group's edges and written once: no atomics, and
// a fixed summation order.
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "common.hpp"

namespace gm {
namespace {

struct Block {
  int kind, zoff, bm, ang, tr, power, ooff, take_real;
};

template <typename T>
struct FactArgs {
  const T* h;          // (n_edges, K - 1)
  const T* zc;         // (n_nodes, K, wc, 2)
  const T* zr;         // (n_nodes, K, wr)
  const T* angular;    // (n_edges, n_f, 2)
  const T* transport;  // (n_edges, n_f, 2)
  const T* rho;        // (n_edges,)
  const int64_t* order;
  const int64_t* group_ptr;
  const int64_t* group_source;
  T* out;  // rows (n_edges, d_out)
  // backward
  const T* g;             // (n_edges, d_out) or (n_targets, d_out) with `target`
  const int64_t* target;  // aggregated form or null
  const T* weights;       // aggregated form or null
  const T* rows;          // aggregated form or null
  T* dh;
  T* dzc;
  T* dzr;
  T* dweights;
  int64_t n_groups;
  int K, wc, wr, C, KP, CP, n_f, n_blocks, d_out;
  int tile;  // backward: edges per LDS tile (a power of two <= 64)
  Block desc[GM_FACT_MAX_BLOCKS];
};

template <typename T>
__device__ __forceinline__ void block_factor(const FactArgs<T>& a, int64_t e, const Block& d, T rho, T& fr, T& fi) {
  fr = T(1);
  fi = T(0);
  if (d.ang != 0) {
    const int o = d.ang < 0 ? -d.ang : d.ang;
    const T* p = a.angular + (e * a.n_f + o) * 2;
    fr = p[0];
    fi = d.ang < 0 ? -p[1] : p[1];
  }
  if (d.tr != 0) {
    const int o = d.tr < 0 ? -d.tr : d.tr;
    const T* p = a.transport + (e * a.n_f + o) * 2;
    const T pr = p[0], pi = d.tr < 0 ? -p[1] : p[1];
    const T nr = fr * pr - fi * pi, ni = fr * pi + fi * pr;
    fr = nr;
    fi = ni;
  }
  T s = T(1);
  for (int i = 0; i < d.power; ++i) s *= rho;
  fr *= s;
  fi *= s;
}

// Z(j) into LDS as Zt[c * KP + t] (t >= K padded with zeros).
template <typename T>
__device__ __forceinline__ void stage_mixes(const FactArgs<T>& a, int64_t j, T* Zt, int lane) {
  const int wc2 = 2 * a.wc;
  const T* zc = a.zc + j * (int64_t)a.K * wc2;
  const T* zr = a.zr + j * (int64_t)a.K * a.wr;
  for (int idx = lane; idx < a.KP * a.C; idx += kWave) {
    const int t = idx / a.C, c = idx - t * a.C;
    T v = T(0);
    if (t < a.K) v = c < wc2 ? zc[t * wc2 + c] : zr[t * a.wr + (c - wc2)];
    Zt[c * a.KP + t] = v;
  }
}

template <typename T, int KMAX>
__device__ __forceinline__ void load_features(const FactArgs<T>& a, int64_t e, T* hh) {
  const T* he = a.h + e * (a.K - 1);
  hh[0] = T(1);
#pragma unroll
  for (int t = 1; t < KMAX; ++t) hh[t] = t < a.K ? he[t - 1] : T(0);
}

// sum_t hh[t] Zt[col][t] over t < KMAX (the padding is zero).
template <typename T, int KMAX>
__device__ __forceinline__ T combine(const T* hh, const T* zcol) {
  T s = T(0);
#pragma unroll
  for (int t = 0; t < KMAX; ++t) s += hh[t] * zcol[t];
  return s;
}

// ------------------------------------------------------------------ forward

template <typename T, int KMAX, int BM>
__global__ __launch_bounds__(64) void factored_forward_kernel(FactArgs<T> a) {
  extern __shared__ __align__(16) unsigned char smem[];
  T* Zt = reinterpret_cast<T*>(smem);
  const int lane = threadIdx.x;
  const int64_t gi = xcd_block(blockIdx.x, gridDim.x);
  const int64_t j = a.group_source[gi];
  const int64_t g0 = a.group_ptr[gi], g1 = a.group_ptr[gi + 1];
  stage_mixes(a, j, Zt, lane);
  __syncthreads();
  const int wc2 = 2 * a.wc;
  for (int64_t g = g0 + lane; g < g1; g += kWave) {
    const int64_t e = a.order[g];
    T hh[KMAX];
    load_features<T, KMAX>(a, e, hh);
    const T rho = a.rho[e];
    T* row = a.out + e * a.d_out;
    T acc[2 * BM];
#pragma unroll
    for (int u = 0; u < 2 * BM; ++u) acc[u] = T(0);
    int open = -1, open_bm = 0;
    bool open_scalar = false;
    for (int b = 0; b < a.n_blocks; ++b) {
      const Block d = a.desc[b];
      if (d.ooff != open) {
        if (open >= 0) {
#pragma unroll
          for (int u = 0; u < BM; ++u)
            if (u < open_bm) {
              if (open_scalar) {
                row[open + u] = acc[2 * u];
              } else {
                row[open + 2 * u] = acc[2 * u];
                row[open + 2 * u + 1] = acc[2 * u + 1];
              }
            }
        }
#pragma unroll
        for (int u = 0; u < 2 * BM; ++u) acc[u] = T(0);
        open = d.ooff;
        open_bm = d.bm;
        open_scalar = d.kind == 0 || d.take_real;
      }
      if (d.kind == 0) {
#pragma unroll
        for (int u = 0; u < BM; ++u)
          if (u < d.bm) acc[2 * u] += combine<T, KMAX>(hh, Zt + (wc2 + d.zoff + u) * a.KP);
        continue;
      }
      T fr, fi;
      block_factor(a, e, d, rho, fr, fi);
#pragma unroll
      for (int u = 0; u < BM; ++u)
        if (u < d.bm) {
          const int col = 2 * (d.zoff + u);
          const T ur = combine<T, KMAX>(hh, Zt + col * a.KP);
          const T ui = combine<T, KMAX>(hh, Zt + (col + 1) * a.KP);
          acc[2 * u] += fr * ur - fi * ui;
          if (!d.take_real) acc[2 * u + 1] += fr * ui + fi * ur;
        }
    }
    if (open >= 0) {
#pragma unroll
      for (int u = 0; u < BM; ++u)
        if (u < open_bm) {
          if (open_scalar) {
            row[open + u] = acc[2 * u];
          } else {
            row[open + 2 * u] = acc[2 * u];
            row[open + 2 * u + 1] = acc[2 * u + 1];
          }
        }
    }
  }
}

// ---------------------------------------------------------------- aggregate

template <typename T>
struct AggArgs {
  const T* rows;
  const T* weights;
  const int64_t* row_ptr;
  T* out;
  int64_t n_targets;
  int d_out, S;  // S edge slots of d_out lanes each (S = 1: lanes stride the columns)
};

template <typename T>
__global__ __launch_bounds__(256) void aggregate_kernel(AggArgs<T> a) {
  const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x & 63;
  const int64_t i = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (i >= a.n_targets) return;
  const int64_t e0 = a.row_ptr[i], e1 = a.row_ptr[i + 1];
  T* o = a.out + i * a.d_out;
  if (a.S == 1) {
    for (int c = lane; c < a.d_out; c += kWave) {
      T s = T(0);
      for (int64_t e = e0; e < e1; ++e) s += a.weights[e] * a.rows[e * a.d_out + c];
      o[c] = s;
    }
    return;
  }
  const int c = lane % a.d_out, slot = lane / a.d_out;
  T s = T(0);
  if (slot < a.S)
    for (int64_t e = e0 + slot; e < e1; e += a.S) s += a.weights[e] * a.rows[e * a.d_out + c];
  s = group_sum(s, lane, a.d_out, a.S);
  if (slot == 0) o[c] = s;
}

// ----------------------------------------------------------------- backward

template <typename T, int KMAX, int NQ>
__global__ __launch_bounds__(64) void factored_backward_kernel(FactArgs<T> a) {
  extern __shared__ __align__(16) unsigned char smem[];
  T* Zt = reinterpret_cast<T*>(smem);  // C * KP
  T* Wt = Zt + a.C * a.KP;             // tile * CP: the tile's packed W rows
  T* Ht = Wt + a.tile * a.CP;          // tile * KP: the tile's h~ rows
  const int lane = threadIdx.x;
  const int64_t gi = xcd_block(blockIdx.x, gridDim.x);
  const int64_t j = a.group_source[gi];
  const int64_t g0 = a.group_ptr[gi], g1 = a.group_ptr[gi + 1];
  stage_mixes(a, j, Zt, lane);
  const int wc2 = 2 * a.wc;
  T acc[NQ][KMAX];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int t = 0; t < KMAX; ++t) acc[q][t] = T(0);
  __syncthreads();

  for (int64_t base = g0; base < g1; base += a.tile) {
    const int n = (int)((g1 - base) < a.tile ? (g1 - base) : a.tile);
    T* w = Wt + lane * a.CP;
    T* hrow = Ht + lane * a.KP;
    if (lane < n) {
      const int64_t e = a.order[base + lane];
      T hh[KMAX];
      load_features<T, KMAX>(a, e, hh);
#pragma unroll
      for (int t = 0; t < KMAX; ++t) hrow[t] = hh[t];
      for (int t = KMAX; t < a.KP; ++t) hrow[t] = T(0);
      const T scale = a.weights ? a.weights[e] : T(1);
      const T* grow = a.target ? a.g + a.target[e] * a.d_out : a.g + e * a.d_out;
      if (a.dweights) {
        const T* r = a.rows + e * a.d_out;
        T s = T(0);
        for (int c = 0; c < a.d_out; ++c) s += grow[c] * r[c];
        a.dweights[e] = s;
      }
      const T rho = a.rho[e];
      for (int b = 0; b < a.n_blocks; ++b) {
        const Block d = a.desc[b];
        if (d.kind == 0) {
          for (int u = 0; u < d.bm; ++u) w[wc2 + d.zoff + u] = scale * grow[d.ooff + u];
          continue;
        }
        T fr, fi;
        block_factor(a, e, d, rho, fr, fi);
        for (int u = 0; u < d.bm; ++u) {
          const T gr = scale * (d.take_real ? grow[d.ooff + u] : grow[d.ooff + 2 * u]);
          const T gim = d.take_real ? T(0) : scale * grow[d.ooff + 2 * u + 1];
          w[2 * (d.zoff + u)] = gr * fr + gim * fi;  // W = G conj(F)
          w[2 * (d.zoff + u) + 1] = gim * fr - gr * fi;
        }
      }
      // dh_t = <W, Z_t> for t >= 1 (the constant feature has no gradient)
      T dht[KMAX];
#pragma unroll
      for (int t = 0; t < KMAX; ++t) dht[t] = T(0);
      for (int c = 0; c < a.C; ++c) {
        const T wc = w[c];
        const T* z = Zt + c * a.KP;
#pragma unroll
        for (int t = 1; t < KMAX; ++t) dht[t] += wc * z[t];
      }
      T* dh = a.dh + e * (a.K - 1);
#pragma unroll
      for (int t = 1; t < KMAX; ++t)
        if (t < a.K) dh[t - 1] = dht[t];
    }
    __syncthreads();
    // dZ_t(j)[c] += sum over the tile's edges of h~_t W_c, lanes over columns
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = lane + kWave * q;
      if (c < a.C) {
        for (int ee = 0; ee < n; ++ee) {
          const T wv = Wt[ee * a.CP + c];
          const T* hr = Ht + ee * a.KP;
#pragma unroll
          for (int t = 0; t < KMAX; ++t) acc[q][t] += hr[t] * wv;
        }
      }
    }
    __syncthreads();
  }
  T* dzc = a.dzc + j * (int64_t)a.K * wc2;
  T* dzr = a.dzr + j * (int64_t)a.K * a.wr;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c = lane + kWave * q;
    if (c < a.C) {
#pragma unroll
      for (int t = 0; t < KMAX; ++t)
        if (t < a.K) {
          if (c < wc2)
            dzc[t * wc2 + c] = acc[q][t];
          else
            dzr[t * a.wr + (c - wc2)] = acc[q][t];
        }
    }
  }
}

// ------------------------------------------------------------------- launch

template <typename T>
int prepare(FactArgs<T>& a, const T* h, const T* zc, const T* zr, const T* angular, const T* transport, const T* rho,
            const int32_t* desc, const int64_t* order, const int64_t* group_ptr, const int64_t* group_source,
            int64_t n_nodes, int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f,
            int64_t n_blocks, int64_t d_out) {
  a = FactArgs<T>{};
  GM_REQUIRE(n_nodes >= 0 && n_edges >= 0 && n_groups >= 0, "sizes must be non-negative");
  GM_REQUIRE(K >= 1 && K <= GM_FACT_MAX_K, "k must be in [1, 20] (the trunk width + 1)");
  GM_REQUIRE(wc >= 0 && wr >= 0 && 2 * wc + wr >= 1 && 2 * wc + wr <= GM_FACT_MAX_C, "2 wc + wr must be in [1, 320]");
  GM_REQUIRE(d_out >= 1 && d_out <= GM_FACT_MAX_OUT, "d_out must be in [1, 128]");
  GM_REQUIRE(n_f >= 1, "the phase tables need at least one order");
  GM_REQUIRE(desc != nullptr, "desc must be a host pointer to (n_blocks, 8) int32");
  GM_REQUIRE(n_blocks >= 1 && n_blocks <= GM_FACT_MAX_BLOCKS, "between 1 and 64 blocks");
  GM_REQUIRE(n_groups <= n_edges && n_groups <= n_nodes, "more source groups than edges or nodes");
  a.K = (int)K;
  a.wc = (int)wc;
  a.wr = (int)wr;
  a.C = (int)(2 * wc + wr);
  // Every kernel instance reads t < KMAX <= 20 mixes per column (zeros past K),
  // so the column stride is 20 whatever K is: no read leaves its column.
  a.KP = GM_FACT_MAX_K;
  a.CP = a.C | 1;  // odd row stride: the lanes' W rows fall in distinct LDS banks
  a.n_f = (int)n_f;
  a.n_blocks = (int)n_blocks;
  a.d_out = (int)d_out;
  a.n_groups = n_groups;
  // Every packed column belongs to exactly one block, and the blocks sharing
  // an output slot are consecutive, alike in width and kind of output.
  int covered_c = 0, covered_r = 0, open = -1;
  bool seen_real = false;
  std::string why;
  for (int b = 0; b < n_blocks; ++b) {
    const int32_t* r = desc + b * GM_FACT_DESC;
    Block d{r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]};
    GM_REQUIRE(d.kind == 0 || d.kind == 1, "a block's kind must be 0 (real) or 1 (complex)");
    GM_REQUIRE(d.bm >= 1 && d.bm <= GM_FACT_MAX_BM, "a block's multiplicity must be in [1, 32]");
    GM_REQUIRE(d.power >= 0 && d.power <= 64, "a block's radial power must be in [0, 64]");
    GM_REQUIRE(std::abs(d.ang) < n_f && std::abs(d.tr) < n_f, "a block's harmonic order exceeds the phase tables");
    const bool scalar = d.kind == 0 || d.take_real;
    GM_REQUIRE(d.ooff >= 0 && d.ooff + (scalar ? d.bm : 2 * d.bm) <= d_out, "a block's output runs past d_out");
    if (d.kind == 0) {
      GM_REQUIRE(!seen_real && d.zoff == 0 && d.bm == wr, "the real block must be one block covering zr");
      seen_real = true;
      covered_r = d.bm;
    } else {
      GM_REQUIRE(d.zoff == covered_c, "the complex blocks must pack zc contiguously in descriptor order");
      covered_c += d.bm;
    }
    if (d.ooff != open) {
      for (int p = 0; p < b; ++p) GM_REQUIRE(desc[p * GM_FACT_DESC + 6] != d.ooff, "blocks sharing an output must be consecutive");
      open = d.ooff;
    } else {
      const int32_t* prev = desc + (b - 1) * GM_FACT_DESC;
      const bool prev_scalar = prev[0] == 0 || prev[7] != 0;
      GM_REQUIRE(prev[2] == d.bm && prev_scalar == scalar, "blocks sharing an output must share its width and kind");
    }
    a.desc[b] = d;
  }
  GM_REQUIRE(covered_c == wc && covered_r == wr, "the blocks must cover zc and zr exactly");
  a.h = h;
  a.zc = zc;
  a.zr = zr;
  a.angular = angular;
  a.transport = transport;
  a.rho = rho;
  a.order = order;
  a.group_ptr = group_ptr;
  a.group_source = group_source;
  if (n_edges > 0) {
    GM_REQUIRE((K == 1 || h) && rho && angular && transport, "the per-edge tables must be device pointers");
    GM_REQUIRE(order && group_ptr && group_source, "order, group_ptr and group_source must be device pointers");
    GM_REQUIRE((wc == 0 || zc) && (wr == 0 || zr), "zc and zr must be device pointers");
  }
  return GM_OK;
}

constexpr size_t kLdsBudget = 64 * 1024;  // per wave64 workgroup

template <typename T>
size_t lds_forward(const FactArgs<T>& a) {
  return sizeof(T) * (size_t)a.C * a.KP;
}

template <typename T>
size_t lds_backward(const FactArgs<T>& a) {
  return sizeof(T) * ((size_t)a.C * a.KP + (size_t)a.tile * (a.CP + a.KP));
}

template <typename T, int KMAX>
void launch_forward_k(const FactArgs<T>& a, int bm, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_groups), block(64);
  const size_t lds = lds_forward(a);
  if (bm <= 4)
    hipLaunchKernelGGL((factored_forward_kernel<T, KMAX, 4>), grid, block, lds, stream, a);
  else if (bm <= 8)
    hipLaunchKernelGGL((factored_forward_kernel<T, KMAX, 8>), grid, block, lds, stream, a);
  else if (bm <= 16)
    hipLaunchKernelGGL((factored_forward_kernel<T, KMAX, 16>), grid, block, lds, stream, a);
  else
    hipLaunchKernelGGL((factored_forward_kernel<T, KMAX, 32>), grid, block, lds, stream, a);
}

template <typename T, int KMAX>
void launch_backward_k(const FactArgs<T>& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_groups), block(64);
  const size_t lds = lds_backward(a);
  switch ((a.C + kWave - 1) / kWave) {
    case 1: hipLaunchKernelGGL((factored_backward_kernel<T, KMAX, 1>), grid, block, lds, stream, a); break;
    case 2: hipLaunchKernelGGL((factored_backward_kernel<T, KMAX, 2>), grid, block, lds, stream, a); break;
    case 3: hipLaunchKernelGGL((factored_backward_kernel<T, KMAX, 3>), grid, block, lds, stream, a); break;
    case 4: hipLaunchKernelGGL((factored_backward_kernel<T, KMAX, 4>), grid, block, lds, stream, a); break;
    default: hipLaunchKernelGGL((factored_backward_kernel<T, KMAX, 5>), grid, block, lds, stream, a); break;
  }
}

template <typename T>
int factored_forward(const T* h, const T* zc, const T* zr, const T* angular, const T* transport, const T* rho,
                     const int32_t* desc, const int64_t* order, const int64_t* group_ptr, const int64_t* group_source,
                     int64_t n_nodes, int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr,
                     int64_t n_f, int64_t n_blocks, int64_t d_out, int64_t max_bm, T* out, hipStream_t stream) {
  FactArgs<T> a;
  const int status = prepare(a, h, zc, zr, angular, transport, rho, desc, order, group_ptr, group_source, n_nodes,
                             n_edges, n_groups, K, wc, wr, n_f, n_blocks, d_out);
  if (status != GM_OK) return status;
  GM_REQUIRE(max_bm >= 1 && max_bm <= GM_FACT_MAX_BM, "max_bm must be in [1, 32]");
  int widest = 1;
  for (int b = 0; b < a.n_blocks; ++b) widest = a.desc[b].bm > widest ? a.desc[b].bm : widest;
  GM_REQUIRE(widest <= max_bm, "a block's multiplicity exceeds max_bm");
  if (n_edges == 0 || n_groups == 0) return GM_OK;
  GM_REQUIRE(out, "out must be a device pointer");
  GM_REQUIRE(lds_forward(a) <= kLdsBudget, "the staged mixes exceed 64 KiB");
  a.out = out;
  if (a.K == 17)
    launch_forward_k<T, 17>(a, widest, stream);
  else
    launch_forward_k<T, GM_FACT_MAX_K>(a, widest, stream);
  return check_launch("factored_forward");
}

template <typename T>
int factored_aggregate(const T* rows, const T* weights, const int64_t* row_ptr, int64_t n_targets, int64_t n_edges,
                       int64_t d_out, T* out, hipStream_t stream) {
  GM_REQUIRE(n_targets >= 0 && n_edges >= 0, "sizes must be non-negative");
  GM_REQUIRE(d_out >= 1 && d_out <= GM_FACT_MAX_OUT, "d_out must be in [1, 128]");
  GM_REQUIRE(n_targets < (int64_t(1) << 31) * kWavesPerBlock, "too many targets for one launch");
  if (n_targets == 0) return GM_OK;
  GM_REQUIRE(row_ptr && out && (n_edges == 0 || (rows && weights)), "rows, weights, row_ptr and out must be device pointers");
  AggArgs<T> a{rows, weights, row_ptr, out, n_targets, (int)d_out, d_out <= 32 ? (int)(kWave / d_out) : 1};
  hipLaunchKernelGGL(aggregate_kernel<T>, dim3((unsigned)blocks_for(n_targets)), dim3(256), 0, stream, a);
  return check_launch("factored_aggregate");
}

template <typename T>
int factored_backward(const T* g, const int64_t* target, const T* weights, const T* rows, const T* h, const T* zc,
                      const T* zr, const T* angular, const T* transport, const T* rho, const int32_t* desc,
                      const int64_t* order, const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes,
                      int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f,
                      int64_t n_blocks, int64_t d_out, T* dh, T* dzc, T* dzr, T* dweights, hipStream_t stream) {
  FactArgs<T> a;
  const int status = prepare(a, h, zc, zr, angular, transport, rho, desc, order, group_ptr, group_source, n_nodes,
                             n_edges, n_groups, K, wc, wr, n_f, n_blocks, d_out);
  if (status != GM_OK) return status;
  const bool aggregated = target != nullptr;
  if (n_edges == 0 || n_groups == 0) return GM_OK;
  GM_REQUIRE(g && (K == 1 || dh) && (wc == 0 || dzc) && (wr == 0 || dzr), "g, dh, dzc and dzr must be device pointers");
  if (aggregated) GM_REQUIRE(weights && rows && dweights, "the aggregated form needs weights, rows and dweights");
  a.tile = kWave;
  while (a.tile > 1 && lds_backward(a) > kLdsBudget) a.tile >>= 1;
  GM_REQUIRE(lds_backward(a) <= kLdsBudget, "the backward's LDS tile exceeds 64 KiB");
  a.g = g;
  a.target = target;
  a.weights = aggregated ? weights : nullptr;
  a.rows = aggregated ? rows : nullptr;
  a.dweights = aggregated ? dweights : nullptr;
  a.dh = dh;
  a.dzc = dzc;
  a.dzr = dzr;
  if (a.K == 17)
    launch_backward_k<T, 17>(a, stream);
  else
    launch_backward_k<T, GM_FACT_MAX_K>(a, stream);
  return check_launch("factored_backward");
}

}  // namespace
}  // namespace gm

#define GM_FACT_EXPORTS(T, S)                                                                                          \
  extern "C" int gm_factored_forward_##S(const T* h, const T* zc, const T* zr, const T* angular, const T* transport,   \
                                         const T* rho, const int32_t* desc, const int64_t* order,                     \
                                         const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes,      \
                                         int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr,        \
                                         int64_t n_f, int64_t n_blocks, int64_t d_out, int64_t max_bm, T* out,        \
                                         void* stream) {                                                              \
    return gm::factored_forward<T>(h, zc, zr, angular, transport, rho, desc, order, group_ptr, group_source, n_nodes, \
                                   n_edges, n_groups, K, wc, wr, n_f, n_blocks, d_out, max_bm, out,                   \
                                   (hipStream_t)stream);                                                              \
  }                                                                                                                   \
  extern "C" int gm_factored_aggregate_##S(const T* rows, const T* weights, const int64_t* row_ptr,                   \
                                           int64_t n_targets, int64_t n_edges, int64_t d_out, T* out, void* stream) { \
    return gm::factored_aggregate<T>(rows, weights, row_ptr, n_targets, n_edges, d_out, out, (hipStream_t)stream);    \
  }                                                                                                                   \
  extern "C" int gm_factored_backward_##S(                                                                            \
      const T* g, const int64_t* target, const T* weights, const T* rows, const T* h, const T* zc, const T* zr,       \
      const T* angular, const T* transport, const T* rho, const int32_t* desc, const int64_t* order,                  \
      const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes, int64_t n_edges, int64_t n_groups,      \
      int64_t K, int64_t wc, int64_t wr, int64_t n_f, int64_t n_blocks, int64_t d_out, T* dh, T* dzc, T* dzr,         \
      T* dweights, void* stream) {                                                                                    \
    return gm::factored_backward<T>(g, target, weights, rows, h, zc, zr, angular, transport, rho, desc, order,        \
                                    group_ptr, group_source, n_nodes, n_edges, n_groups, K, wc, wr, n_f, n_blocks,    \
                                    d_out, dh, dzc, dzr, dweights, (hipStream_t)stream);                              \
  }

GM_FACT_EXPORTS(float, f32)
GM_FACT_EXPORTS(double, f64)
