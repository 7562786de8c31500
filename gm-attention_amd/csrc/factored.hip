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

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "split.hpp"

namespace gm {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

struct Block {
  int16_t kind, zoff, bm, ang, tr, power, ooff, take_real;
};

// One run of the packed mix columns [c0, c0 + width) of every node: column
// c of node j at mix t sits at z[j * node_stride + t * t_stride + (c - c0)]
// (and its gradient at the same place of dz).  The reference's zc
// (n_nodes, K, wc, 2) and zr (n_nodes, K, wr) are the two-run case.
template <typename T>
struct ZSeg {
  const T* z;
  T* dz;
  int64_t node_stride;
  int t_stride, c0, width;
};

template <typename T>
struct FactArgs {
  const T* h;          // (n_edges, K - 1)
  ZSeg<T> seg[GM_FACT_MAX_SEG];
  int n_seg;
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
  T* dweights;
  int accumulate;  // grouped backward: add dh and dweights into the outputs instead of writing them
  int64_t n_groups;
  int K, wc, wr, C, KP, CP, n_f, n_blocks, d_out;
  int64_t g_ld;  // grouped backward: floats between consecutive rows of g (d_out unless a strided view)
  int tile;  // backward: edges per LDS tile (a power of two <= 64)
  int real_ooff;  // the real block's output offset (when wr > 0)
  Block desc[GM_FACT_MAX_BLOCKS];
  uint8_t cmap[GM_FACT_MAX_C / 2];  // complex column -> its block
  // MFMA path tables (C <= 128): per packed column, block | g index of the
  // real part << 8 | of the imaginary part (0xFF: none) << 16 | kind << 24
  // (0 real block, 1 real part, 2 imaginary part); per output slot the
  // V columns it sums, in descriptor order (optr offsets into olist).
  uint32_t colinfo[128];
  uint8_t optr[GM_FACT_MAX_OUT + 1];
  uint8_t olist[128];
  // source-grouped streams (row g is the edge order[g]): the phase pairs
  // (angular orders 0..pa-1, then transport orders 0..pt-1, 16 floats a row),
  // r / cutoff and the edge's target
  const float* phase_g;
  const float* rho_g;
  const int64_t* target_g;
  const int64_t* group_order;  // the groups in launch order (largest first), or null
  const float* zw_g;           // (n_edges, 4): r e^{i phi}, e^{i gamma} in grouping order, or null
  int pa, pt;
  // lane-owned output kernels: per-slot words, slot column -> packed column
  // (0xFF padding), the backward's live dh k-steps (bit 4 nt + r), the LDS
  // stride of a G row
  uint32_t slot[16];
  uint8_t slotcol[128];
  uint32_t colslot32[32];  // packed column -> slot column, four bytes a word
  uint32_t kmask;
  int n_slots, gstride;
  // mixes staged by direct-to-LDS loads (lane-owned backward): the runs
  // merged into blocks contiguous in memory (a block's rows t = 0 .. 16 are
  // `zq_w` floats apart, the row a block's width), staged per node in LDS from
  // row zq_t0 on, block b at float zq_loff[b]; per slot column where its rows
  // sit (the padding columns at a zero word past the blocks, width 0)
  const float* zq_base[GM_FACT_MAX_SEG];
  int64_t zq_ns[GM_FACT_MAX_SEG];
  int zq_w[GM_FACT_MAX_SEG], zq_loff[GM_FACT_MAX_SEG];
  int n_zq, zq_t0, zq_words;  // blocks, first staged row, LDS floats in all
  uint32_t zq_slot[128];       // per slot column: its row zq_t0's float in the area | block width << 16
  // the value kernel's radial trunk evaluated in the lane kernels from rho_g
  // (h_t = SiLU(W1 b + b1) over the Gaussian basis b_k = exp(-((rho^2 - c_k)
  // inv_width)^2 / 2)) instead of reading h; trunk_w null: h is read
  const float* trunk_w;  // (16, trunk_nb)
  const float* trunk_b;  // (16,) or null
  float trunk_c[8];
  float trunk_inv_width;
  int trunk_nb;
  // lane-owned kernels with compiled-in slots: h, the rows and dh are
  // bfloat16 (the pointers above then address 2-byte elements)
  int b16;
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

template <typename T>
__device__ __forceinline__ int seg_of(const FactArgs<T>& a, int c) {
  int s = 0;
  while (s + 1 < a.n_seg && c >= a.seg[s + 1].c0) ++s;
  return s;
}

// Z_t(j) at packed column c (zero past K or C).
template <typename T>
__device__ __forceinline__ T zget(const FactArgs<T>& a, int64_t j, int t, int c) {
  if (t >= a.K || c >= a.C) return T(0);
  const ZSeg<T>& g = a.seg[seg_of(a, c)];
  return g.z[j * g.node_stride + (int64_t)t * g.t_stride + (c - g.c0)];
}

template <typename T>
__device__ __forceinline__ void zput(const FactArgs<T>& a, int64_t j, int t, int c, T v) {
  const ZSeg<T>& g = a.seg[seg_of(a, c)];
  g.dz[j * g.node_stride + (int64_t)t * g.t_stride + (c - g.c0)] = v;
}

// Z(j) into LDS as Zt[c * KP + t] (t >= K padded with zeros).
template <typename T>
__device__ __forceinline__ void stage_mixes(const FactArgs<T>& a, int64_t j, T* Zt, int lane) {
  for (int idx = lane; idx < a.KP * a.C; idx += kWave) {
    const int t = idx / a.C, c = idx - t * a.C;
    Zt[c * a.KP + t] = zget(a, j, t, c);
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
  const int64_t* inv;  // null: edge e's row is rows[e]; else rows[inv[e]] (rows kept in another order)
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
      for (int64_t e = e0; e < e1; ++e) s += a.weights[e] * a.rows[(a.inv ? a.inv[e] : e) * a.d_out + c];
      o[c] = s;
    }
    return;
  }
  const int c = lane % a.d_out, slot = lane / a.d_out;
  T s = T(0);
  if (slot < a.S)
    for (int64_t e = e0 + slot; e < e1; e += a.S) s += a.weights[e] * a.rows[(a.inv ? a.inv[e] : e) * a.d_out + c];
  s = group_sum(s, lane, a.d_out, a.S);
  if (slot == 0) o[c] = s;
}

// Every head's aggregate in one pass: out[i, h, :] = sum_{e -> i} alpha[e, h]
// rows[h, inv[e], :] (rows kept per head in the grouping's order).  One wave
// per target: with d_out a multiple of four, lane l < H d_out / 4 owns the
// four outputs 4 l .. 4 l + 3 (one 16-byte row piece a load), else lane l
// owns the outputs l, l + 64, l + 128.  The edges go in CSR order, kAggStep a
// step with their loads in flight together, so every sum has a fixed order.
struct AggHeadsArgs {
  const float* rows;   // (H, n_rows, d_out)
  const float* alpha;  // (n_edges, H / split): row heads h and h' share a column when h / split == h' / split
  const int64_t* inv;
  const int64_t* row_ptr;
  float* out;  // (n_targets, H, d_out)
  int64_t n_targets, n_rows;
  int H, d_out, split;
};

constexpr int kAggStep = 4;  // edges a step: 55 VGPRs, eight waves a SIMD (eight a step: five waves, 10.4 vs 9.0 ms at NS)

// One wave per target, lane l owning the 16-byte pieces l, l + 64, ...,
// l + 64 (P - 1) of the target's H d_out outputs (piece o: row head o / q4,
// columns 4 (o % q4) ..).  The rows are read in the CSR's edge order, so the
// sums are each head's sums in that order.  The target is wave-uniform, so the
// row indices are scalar loads; with Ha <= 16 weight columns the weights of EW
// edges (64 / Ha rounded down to whole steps) come in one vector load (lane
// u Ha + h: edge u, column h) and reach the lanes that use them by lane
// shuffles, so an edge costs its row pieces' vector load alone.

// B16: the rows are bfloat16 (four to an 8-byte piece, widened exactly), the
// sums float32.
template <int P, bool B16 = false>
__global__ __launch_bounds__(256) void aggregate_heads_vec_kernel(AggHeadsArgs a) {
  const int64_t i = xcd_balanced_block(blockIdx.x, gridDim.x, a.row_ptr, a.n_targets, kWavesPerBlock) * kWavesPerBlock +
                    __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= a.n_targets) return;
  const int q4 = a.d_out / 4, W4 = a.H * q4, Ha = a.H / a.split;
  bool live[P];
  int ha[P];
  int64_t base[P];  // element offsets of the lane's pieces in row 0
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int o = lane + 64 * p;
    live[p] = o < W4;
    const int hh = live[p] ? o / q4 : 0, c4 = live[p] ? o - hh * q4 : 0;
    ha[p] = hh / a.split;
    base[p] = (int64_t)hh * a.n_rows * a.d_out + 4 * c4;
  }
  auto piece = [&](int p, int64_t row) -> floatx4 {
    if constexpr (B16) {
      const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(a.rows) + base[p] +
                                                      row * a.d_out);
      return floatx4{bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y)};
    } else {
      return *reinterpret_cast<const floatx4*>(a.rows + base[p] + row * a.d_out);
    }
  };
  const int64_t e0 = a.row_ptr[i], e1 = a.row_ptr[i + 1];
  floatx4 s[P];
#pragma unroll
  for (int p = 0; p < P; ++p) s[p] = floatx4{0.f, 0.f, 0.f, 0.f};
  // the weights of edges eb .. eb + EW - 1: lane u Ha + h holds edge eb + u's column h
  const int EW = Ha <= 16 ? kWave / Ha / kAggStep * kAggStep : 0;
  auto load_w = [&](int64_t eb) {
    const int64_t k = eb * Ha + lane;
    return lane < EW * Ha && k < e1 * Ha ? a.alpha[k] : 0.f;
  };
  float wb = EW ? load_w(e0) : 0.f;
  int in_batch = 0;  // the step's first edge within its weight batch
  // the next batch's row indices are requested behind this batch's rows, so each
  // batch waits for one round trip rather than an index load and then the rows
  int64_t r[kAggStep];
#pragma unroll
  for (int u = 0; u < kAggStep; ++u) r[u] = e0 + u < e1 ? a.inv[e0 + u] : 0;
  for (int64_t e = e0; e < e1; e += kAggStep) {
    float w[kAggStep][P];
    floatx4 v[kAggStep][P];
#pragma unroll
    for (int u = 0; u < kAggStep; ++u)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const bool in = live[p] && e + u < e1;
        if (EW) {
          w[u][p] = __shfl(wb, (in_batch + u) * Ha + ha[p], kWave);
          if (!in) w[u][p] = 0.f;
        } else {
          w[u][p] = in ? a.alpha[(e + u) * Ha + ha[p]] : 0.f;
        }
        v[u][p] = in ? piece(p, r[u]) : floatx4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int u = 0; u < kAggStep; ++u) {
      const int64_t n = e + kAggStep + u;
      r[u] = n < e1 ? a.inv[n] : 0;
    }
    in_batch += kAggStep;
    if (in_batch == EW) {
      in_batch = 0;
      wb = load_w(e + kAggStep);
    }
#pragma unroll
    for (int u = 0; u < kAggStep; ++u)
#pragma unroll
      for (int p = 0; p < P; ++p) s[p] += w[u][p] * v[u][p];
  }
  float* o = a.out + i * (int64_t)a.H * a.d_out;
#pragma unroll
  for (int p = 0; p < P; ++p)
    if (live[p]) *reinterpret_cast<floatx4*>(o + 4 * (lane + 64 * p)) = s[p];
}

// Any d_out: lane l owns outputs l, l + 64, ... (at most kAggScalar of them).
constexpr int kAggScalar = 16;

__global__ __launch_bounds__(256) void aggregate_heads_kernel(AggHeadsArgs a) {
  const int64_t i = xcd_block(blockIdx.x, gridDim.x) * kWavesPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= a.n_targets) return;
  const int W = a.H * a.d_out, Ha = a.H / a.split;
  const int64_t e0 = a.row_ptr[i], e1 = a.row_ptr[i + 1];
  float* o = a.out + i * W;
  for (int k0 = 0; k0 < kAggScalar; k0 += 4) {
    if (64 * k0 >= W) break;
    int hh[4], cc[4];
    bool live[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = lane + 64 * (k0 + k);
      live[k] = c < W;
      hh[k] = live[k] ? c / a.d_out : 0;
      cc[k] = live[k] ? c - hh[k] * a.d_out : 0;
    }
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t e = e0; e < e1; e += 4) {
      float w[4][4], v[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool in = e + u < e1;
        const int64_t r = in ? a.inv[e + u] : 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          w[u][k] = in && live[k] ? a.alpha[(e + u) * Ha + hh[k] / a.split] : 0.f;
          v[u][k] = in && live[k] ? a.rows[((int64_t)hh[k] * a.n_rows + r) * a.d_out + cc[k]] : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) s[k] += w[u][k] * v[u][k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (live[k]) o[lane + 64 * (k0 + k)] = s[k];
  }
}

// dst_t[h, g] = src[perm[g], h] (a row gather and a transpose), and its
// inverse dst[perm[g], h] = src_t[h, g]: one thread per row g, whole rows
// moved as 16-byte pieces where the width allows (W4 = width / 4 pieces).
// Each XCD runs a contiguous range of the blocks: the rows of neighbouring
// sources share the cache lines they gather from (or scatter into), and those
// lines then meet in one L2 instead of being fetched (or written back in
// pieces) by several.
template <int W4>
__global__ __launch_bounds__(256) void gather_transpose_kernel(const float* src, const int64_t* perm, int64_t n,
                                                               int width, float* dst_t) {
  const int64_t g = xcd_block(blockIdx.x, gridDim.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  const float* row = src + perm[g] * width;
  if constexpr (W4 > 0) {
#pragma unroll
    for (int u = 0; u < W4; ++u) {
      const floatx4 v = *reinterpret_cast<const floatx4*>(row + 4 * u);
#pragma unroll
      for (int k = 0; k < 4; ++k) dst_t[(4 * u + k) * n + g] = v[k];
    }
  } else {
    for (int h = 0; h < width; ++h) dst_t[h * n + g] = row[h];
  }
}

template <int W4>
__global__ __launch_bounds__(256) void scatter_transpose_kernel(const float* src_t, const int64_t* perm, int64_t n,
                                                                int width, float* dst) {
  const int64_t g = xcd_block(blockIdx.x, gridDim.x) * blockDim.x + threadIdx.x;
  if (g >= n) return;
  float* row = dst + perm[g] * width;
  if constexpr (W4 > 0) {
#pragma unroll
    for (int u = 0; u < W4; ++u) {
      floatx4 v;
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = src_t[(4 * u + k) * n + g];
      *reinterpret_cast<floatx4*>(row + 4 * u) = v;
    }
  } else {
    for (int h = 0; h < width; ++h) row[h] = src_t[h * n + g];
  }
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
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c = lane + kWave * q;
    if (c < a.C) {
#pragma unroll
      for (int t = 0; t < KMAX; ++t)
        if (t < a.K) zput(a, j, t, c, acc[q][t]);
    }
  }
}

// -------------------------------------------------------- MFMA (fp32, K <= 17)
//
// With h~ = (1, h) and T = K - 1 <= 16 trunk features, every source group's
// products are 16-deep matrix products on v_mfma_f32_16x16x4f32 (lane l
// supplies A[l % 16][l / 16] and B[l / 16][l % 16] and holds
// D[4 (l / 16) + r][l % 16]), 16 edges at a time:
//   forward   P^T (C x 16 edges) = Z_{1..16}^T (C x 16) H^T (16 x 16 edges), plus Z_0;
//   backward  dh (16 edges x 16)  = W (16 edges x C) Z_{1..16}^T (C x 16),
//             dZ_{1..16} (16 x C) += H^T (16 x 16 edges) W (16 edges x C),
//             dZ_0 (C)           += the column sums of W.
// The k index of the forward's product runs over the trunk features as
// t - 1 = 4 (l / 16) + s, so a lane's slice of h(e) is one 16-byte load.
// The source's Z(j) lives in registers for the whole group; the tile's edge
// phases, factors, gradient rows and W go through LDS; every output slot sums
// its blocks in descriptor order (host-built lists), so results do not
// depend on scheduling.


constexpr int kMT = 16;  // edges per MFMA tile
constexpr int kHsStride = 20;  // floats per edge row of the backward's h tile in LDS: 16 features + 4 (no bank shared by a read's lanes)

// The MFMA kernels run one wave per workgroup, and a wave's LDS operations
// execute in order, so handing LDS data between its lanes needs only a
// compiler-level ordering point: a wavefront-scope release/acquire pair (no
// wait on outstanding global loads or stores, which __syncthreads' workgroup
// fences would add).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}



// The tile's edge ids (zero past n) into eid, the edges' rho and phase rows
// (angular then transport, 4 n_f floats) into LDS, and then every block's
// factor F[e][b] from them.
// Z(j) into LDS as Zs[t * ZP + c] for t < 17 (zero past K and past C).  Lane
// l owns the elements l, l + 64, ... of the 17 x CV block: it issues every
// load first (a fixed, unrolled count), so they are all in flight at once,
// and then writes them; its run is a short uniform-bound search.
template <int NT>
__device__ __forceinline__ void stage_z(const FactArgs<float>& a, int64_t j, float* Zs, int lane) {
  constexpr int CV = 16 * NT, ZP = CV + 4, PER = (17 * CV + kWave - 1) / kWave;
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int idx = lane + kWave * i;
    const int t = idx / CV, c = idx - t * CV;
    v[i] = 0.f;
    if (t < a.K && c < a.C) {
      int r = 0;
#pragma unroll
      for (int k = 1; k < GM_FACT_MAX_SEG; ++k)
        if (k < a.n_seg && c >= a.seg[k].c0) r = k;
      const ZSeg<float>& g = a.seg[r];
      v[i] = g.z[j * g.node_stride + (int64_t)t * g.t_stride + (c - g.c0)];
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int idx = lane + kWave * i;
    const int t = idx / CV, c = idx - t * CV;
    if (t < 17) Zs[t * ZP + c] = v[i];
  }
}

// dZ(j) from LDS Ds[t * zp + c] to the runs' gradient arrays.
__device__ __forceinline__ void store_dz(const FactArgs<float>& a, int64_t j, const float* Ds, int zp, int lane) {
  for (int r = 0; r < a.n_seg; ++r) {
    const ZSeg<float>& g = a.seg[r];
    float* dst = g.dz + j * g.node_stride;
    for (int t = 0; t < a.K; ++t)
      for (int c = lane; c < g.width; c += kWave) dst[(int64_t)t * g.t_stride + c] = Ds[t * zp + g.c0 + c];
  }
}

// The descriptor rows into LDS (a lane-indexed table; kernel arguments read
// with a per-lane index would be fetched from memory each time).
__device__ __forceinline__ void stage_desc(const FactArgs<float>& a, Block* Ds, int lane) {
  for (int b = lane; b < a.n_blocks; b += kWave) Ds[b] = a.desc[b];
}

__device__ __forceinline__ void stage_edges(const FactArgs<float>& a, int64_t base, int n, int64_t* eid, int lane) {
  if (lane < kMT) eid[lane] = lane < n ? a.order[base + lane] : 0;
}

__device__ __forceinline__ void stage_phases(const FactArgs<float>& a, const int64_t* eid, int n, float* Ph, float* Rh,
                                             int m, int q) {
  const int w = 4 * a.n_f, half = 2 * a.n_f;
  for (int e = q; e < kMT; e += 4) {
    const int64_t ee = eid[e];
    for (int k = m; k < w; k += kMT) {
      float v = 0.f;
      if (e < n) v = k < half ? a.angular[ee * half + k] : a.transport[ee * half + (k - half)];
      Ph[e * w + k] = v;
    }
  }
  if (q == 0) Rh[m] = m < n ? a.rho[eid[m]] : 0.f;
}

__device__ __forceinline__ void stage_factors(const FactArgs<float>& a, const Block* Bd, const float* Ph,
                                              const float* Rh, float* Ft, int lane) {
  const int nb = a.n_blocks, w = 4 * a.n_f, half = 2 * a.n_f;
  for (int idx = lane; idx < kMT * nb; idx += kWave) {
    const int e = idx & (kMT - 1), b = idx >> 4;
    const Block d = Bd[b];
    const float* ph = Ph + e * w;
    float fr = 1.f, fi = 0.f;
    if (d.ang != 0) {
      const int o = d.ang < 0 ? -d.ang : d.ang;
      fr = ph[2 * o];
      fi = d.ang < 0 ? -ph[2 * o + 1] : ph[2 * o + 1];
    }
    if (d.tr != 0) {
      const int o = d.tr < 0 ? -d.tr : d.tr;
      const float pr = ph[half + 2 * o], pi = d.tr < 0 ? -ph[half + 2 * o + 1] : ph[half + 2 * o + 1];
      const float nr = fr * pr - fi * pi, ni = fr * pi + fi * pr;
      fr = nr;
      fi = ni;
    }
    float sc = 1.f;
    for (int i = 0; i < d.power; ++i) sc *= Rh[e];
    Ft[2 * (e * nb + b)] = fr * sc;
    Ft[2 * (e * nb + b) + 1] = fi * sc;
  }
}

template <int NT>
__global__ __launch_bounds__(64) void factored_forward_mfma(FactArgs<float> a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nb = a.n_blocks, CV = 16 * NT, VP = CV + 1, wc2 = 2 * a.wc, d_out = a.d_out;
  constexpr int ZP = 16 * NT + 4;
  int64_t* eid = reinterpret_cast<int64_t*>(smem);  // [kMT]
  Block* Bd = reinterpret_cast<Block*>(eid + kMT);  // [nb]
  float* Rh = reinterpret_cast<float*>(Bd + GM_FACT_MAX_BLOCKS);  // [kMT]
  float* Ph = Rh + kMT;                             // [kMT][4 n_f]
  float* Ft = Ph + kMT * 4 * a.n_f;                 // [kMT][nb][2]
  float* Vt = Ft + kMT * nb * 2;                    // [kMT][VP]
  float* Zs = Vt + kMT * VP;                        // [17][ZP]
  uint8_t* optr = reinterpret_cast<uint8_t*>(Zs + 17 * ZP);  // [d_out + 1]
  uint8_t* olist = optr + GM_FACT_MAX_OUT + 1;                // [optr[d_out]]
  const int lane = threadIdx.x, m = lane & 15, q = lane >> 4;
  for (int i = lane; i <= d_out; i += kWave) optr[i] = a.optr[i];
  for (int i = lane; i < a.optr[d_out]; i += kWave) olist[i] = a.olist[i];
  stage_desc(a, Bd, lane);
  const int64_t gi = xcd_block(blockIdx.x, gridDim.x);
  const int64_t j = a.group_source[gi];
  const int64_t g0 = a.group_ptr[gi], g1 = a.group_ptr[gi + 1];
  stage_z<NT>(a, j, Zs, lane);
  wave_sync();
  float za[NT][4], z0[NT][4];
  int vb[NT][2];  // the block of each complex column pair this lane holds (-1: real block or padding)
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      za[nt][s] = Zs[(1 + 4 * q + s) * ZP + 16 * nt + m];
      z0[nt][s] = Zs[16 * nt + 4 * q + s];
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int c = 16 * nt + 4 * q + 2 * p;
      vb[nt][p] = c < wc2 ? (int)a.cmap[c >> 1] : -1;
    }
  }
  for (int64_t base = g0; base < g1; base += kMT) {
    const int n = (int)((g1 - base) < kMT ? (g1 - base) : kMT);
    stage_edges(a, base, n, eid, lane);
    wave_sync();
    floatx4 hv = floatx4{0.f, 0.f, 0.f, 0.f};  // h(e = m)[t - 1 = 4 q + s]
    if (m < n) {
      const float* he = a.h + eid[m] * (a.K - 1);
      if (a.K == 17) {
        hv = *reinterpret_cast<const floatx4*>(he + 4 * q);
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) hv[s] = 4 * q + s + 1 < a.K ? he[4 * q + s] : 0.f;
      }
    }
    stage_phases(a, eid, n, Ph, Rh, m, q);
    floatx4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt] = mfma16(za[nt][s], hv[s], acc[nt]);
    wave_sync();
    stage_factors(a, Bd, Ph, Rh, Ft, lane);
    wave_sync();
    // V = F (P + Z_0) on the complex columns, P + Z_0 on the real block's
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int c = 16 * nt + 4 * q + 2 * p;
        const float ur = acc[nt][2 * p] + z0[nt][2 * p], ui = acc[nt][2 * p + 1] + z0[nt][2 * p + 1];
        float vr = ur, vi = ui;
        if (vb[nt][p] >= 0) {
          const float* f = Ft + 2 * (m * nb + vb[nt][p]);
          vr = f[0] * ur - f[1] * ui;
          vi = f[0] * ui + f[1] * ur;
        }
        Vt[m * VP + c] = vr;
        Vt[m * VP + c + 1] = vi;
      }
    wave_sync();
    for (int e = q; e < n; e += 4) {
      const float* v = Vt + e * VP;
      float* row = a.out + eid[e] * d_out;
      for (int o = m; o < d_out; o += kMT) {
        float sum = 0.f;
        for (int k = optr[o]; k < optr[o + 1]; ++k) sum += v[olist[k]];
        row[o] = sum;
      }
    }
    wave_sync();
  }
}

template <int NT>
__global__ __launch_bounds__(64) void factored_backward_mfma(FactArgs<float> a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nb = a.n_blocks, CV = 16 * NT, WP = CV + 1, wc2 = 2 * a.wc, d_out = a.d_out;
  constexpr int ZP = 16 * NT + 4;
  int64_t* eid = reinterpret_cast<int64_t*>(smem);  // [kMT]
  Block* Bd = reinterpret_cast<Block*>(eid + kMT);  // [nb]
  float* Rh = reinterpret_cast<float*>(Bd + GM_FACT_MAX_BLOCKS);  // [kMT]
  float* St = Rh + kMT;                             // [kMT] the edges' weights
  float* Ph = St + kMT;                             // [kMT][4 n_f]
  float* Ft = Ph + kMT * 4 * a.n_f;                 // [kMT][nb][2]
  float* Gt = Ft + kMT * nb * 2;                    // [kMT][d_out] the edges' output gradients (unscaled)
  float* Wt = Gt + kMT * d_out;                     // [kMT][WP]
  float* Ht = Wt + kMT * WP;                        // [kMT][16]
  float* Zs = Ht + kMT * 16;                        // [17][ZP] Z(j), then dZ(j)
  const int lane = threadIdx.x, m = lane & 15, q = lane >> 4;
  stage_desc(a, Bd, lane);
  const int64_t gi = xcd_block(blockIdx.x, gridDim.x);
  const int64_t j = a.group_source[gi];
  const int64_t g0 = a.group_ptr[gi], g1 = a.group_ptr[gi + 1];
  stage_z<NT>(a, j, Zs, lane);
  wave_sync();
  float zb[4 * NT];  // B operand of dh: Z[t = 1 + m][c = q + 4 s]
#pragma unroll
  for (int s = 0; s < 4 * NT; ++s) zb[s] = Zs[(1 + m) * ZP + q + 4 * s];
  uint32_t ci[NT];  // this lane's columns c = 16 nt + m: block | gre << 8 | gim << 16 | kind << 24
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) ci[nt] = 16 * nt + m < a.C ? a.colinfo[16 * nt + m] : 0xFFFFFFFFu;
  floatx4 dz[NT];
  float dz0[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    dz[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    dz0[nt] = 0.f;
  }
  for (int64_t base = g0; base < g1; base += kMT) {
    const int n = (int)((g1 - base) < kMT ? (g1 - base) : kMT);
    stage_edges(a, base, n, eid, lane);
    if (lane < kMT) St[lane] = (lane < n && a.weights) ? a.weights[a.order[base + lane]] : 1.f;
    wave_sync();
    for (int e = q; e < kMT; e += 4) {
      const float* grow = e < n ? (a.target ? a.g + a.target[eid[e]] * d_out : a.g + eid[e] * d_out) : nullptr;
      for (int o = m; o < d_out; o += kMT) Gt[e * d_out + o] = grow ? grow[o] : 0.f;
    }
    {
      const int e = lane >> 2, part = lane & 3;  // one 16-byte slice of one edge's h
      floatx4 hv = floatx4{0.f, 0.f, 0.f, 0.f};
      if (e < n) {
        const float* he = a.h + eid[e] * (a.K - 1);
        if (a.K == 17) {
          hv = *reinterpret_cast<const floatx4*>(he + 4 * part);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) hv[s] = 4 * part + s + 1 < a.K ? he[4 * part + s] : 0.f;
        }
      }
      *reinterpret_cast<floatx4*>(Ht + e * 16 + 4 * part) = hv;
    }
    stage_phases(a, eid, n, Ph, Rh, m, q);
    wave_sync();
    stage_factors(a, Bd, Ph, Rh, Ft, lane);
    wave_sync();
    if (a.dweights && lane < n) {
      const float* r = a.rows + eid[lane] * d_out;
      const float* gr = Gt + lane * d_out;
      float sum = 0.f;
      for (int o = 0; o < d_out; ++o) sum += gr[o] * r[o];
      a.dweights[eid[lane]] = sum;
    }
    // W[e = q + 4 i][c = 16 nt + m] = w_e G conj(F) (complex) or w_e G (real block)
    float w[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint32_t info = ci[nt];
      const int b = info & 0xFF, gre = (info >> 8) & 0xFF, gim = (info >> 16) & 0xFF, kind = info >> 24;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = q + 4 * i;
        float v = 0.f;
        if (info != 0xFFFFFFFFu) {
          const float* gr = Gt + e * d_out;
          const float g_re = gr[gre], g_im = gim == 0xFF ? 0.f : gr[gim];
          if (kind == 0) {
            v = g_re;
          } else {
            const float* f = Ft + 2 * (e * nb + b);
            v = kind == 1 ? g_re * f[0] + g_im * f[1] : g_im * f[0] - g_re * f[1];
          }
          v *= St[e];
        }
        w[nt][i] = v;
        Wt[e * WP + 16 * nt + m] = v;
      }
    }
    wave_sync();
    // dh (16 edges x 16 t) = W Z^T: lane holds dh[e = 4 q + r][t = 1 + m]
    floatx4 dh = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4 * NT; ++s) dh = mfma16(Wt[m * WP + q + 4 * s], zb[s], dh);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = 4 * q + r;
      if (e < n && m + 1 < a.K) a.dh[eid[e] * (a.K - 1) + m] = dh[r];
    }
    // dZ_{1..16} += H^T W (W straight from this lane's registers); dZ_0 += column sums
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dz[nt] = mfma16(Ht[(q + 4 * i) * 16 + m], w[nt][i], dz[nt]);
        dz0[nt] += w[nt][i];
      }
    wave_sync();
  }
  // dZ(j) through LDS (Zs is free again) to the runs' gradient arrays
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    dz0[nt] += __shfl_xor(dz0[nt], 16, kWave);
    dz0[nt] += __shfl_xor(dz0[nt], 32, kWave);
    const int c = 16 * nt + m;
#pragma unroll
    for (int r = 0; r < 4; ++r) Zs[(1 + 4 * q + r) * ZP + c] = dz[nt][r];
    if (q == 0) Zs[c] = dz0[nt];
  }
  wave_sync();
  store_dz(a, j, Zs, ZP, lane);
}

// ------------------------------------------------ MFMA over source-grouped streams
//
// The same products as above with every per-edge stream already in source
// order (row g of h, the phases, rho, the rows, dh and dweights is the g-th
// edge of the grouping): a tile's loads are contiguous and their addresses
// are known before the tile starts, so the next tile's loads are issued
// while the current one computes.  Only the backward's target gradient
// rows are gathered (through target_g).

constexpr int kPhaseRow = 16;  // floats per grouped phase row (8 pairs)

__device__ __forceinline__ void factors_grouped(const FactArgs<float>& a, const Block* Bd, const float* Ph,
                                                const float* Rh, float* Ft, int lane) {
  const int nb = a.n_blocks;
  for (int idx = lane; idx < kMT * nb; idx += kWave) {
    const int e = idx & (kMT - 1), b = idx >> 4;
    const Block d = Bd[b];
    const float* ph = Ph + e * kPhaseRow;
    float fr = 1.f, fi = 0.f;
    if (d.ang != 0) {
      const int o = d.ang < 0 ? -d.ang : d.ang;
      fr = ph[2 * o];
      fi = d.ang < 0 ? -ph[2 * o + 1] : ph[2 * o + 1];
    }
    if (d.tr != 0) {
      const int o = a.pa + (d.tr < 0 ? -d.tr : d.tr);
      const float pr = ph[2 * o], pi = d.tr < 0 ? -ph[2 * o + 1] : ph[2 * o + 1];
      const float nr = fr * pr - fi * pi, ni = fr * pi + fi * pr;
      fr = nr;
      fi = ni;
    }
    float sc = 1.f;
    for (int i = 0; i < d.power; ++i) sc *= Rh[e];
    Ft[2 * (e * nb + b)] = fr * sc;
    Ft[2 * (e * nb + b) + 1] = fi * sc;
  }
}

struct TileIn {
  floatx4 h;    // this lane's slice of h: forward h(g = base + m)[4 q .. 4 q + 3]; backward h(base + l / 4)[4 (l % 4) ..]
  floatx4 ph;   // phase row of edge base + l / 4, floats 4 (l % 4) .. + 3
  float rho;    // rho of edge base + l (l < 16)
  float w;      // backward: the weight of edge base + l
  int64_t tgt;  // backward: the target of edge base + l
};

template <bool BACKWARD>
__device__ __forceinline__ TileIn load_tile(const FactArgs<float>& a, int64_t base, int n, int lane) {
  const int m = lane & 15, q = lane >> 4, e4 = lane >> 2, part = lane & 3;
  TileIn t;
  t.h = floatx4{0.f, 0.f, 0.f, 0.f};
  t.ph = floatx4{0.f, 0.f, 0.f, 0.f};
  t.rho = 0.f;
  t.w = 0.f;
  t.tgt = 0;
  if (!BACKWARD) {
    if (m < n) t.h = *reinterpret_cast<const floatx4*>(a.h + (base + m) * 16 + 4 * q);
  } else {
    if (e4 < n) t.h = *reinterpret_cast<const floatx4*>(a.h + (base + e4) * 16 + 4 * part);
  }
  if (e4 < n) t.ph = *reinterpret_cast<const floatx4*>(a.phase_g + (base + e4) * kPhaseRow + 4 * part);
  if (lane < n) {
    t.rho = a.rho_g[base + lane];
    if (BACKWARD) {
      t.w = a.weights[base + lane];
      t.tgt = a.target_g[base + lane];
    }
  }
  return t;
}

template <int NT>
__global__ __launch_bounds__(64) void factored_forward_grouped(FactArgs<float> a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nb = a.n_blocks, CV = 16 * NT, VP = CV + 1, wc2 = 2 * a.wc, d_out = a.d_out;
  Block* Bd = reinterpret_cast<Block*>(smem);                      // [nb]
  float* Ph = reinterpret_cast<float*>(Bd + GM_FACT_MAX_BLOCKS);   // [kMT][kPhaseRow]
  float* Rh = Ph + kMT * kPhaseRow;                                // [kMT]
  float* Ft = Rh + kMT;                                            // [kMT][nb][2]
  float* Vt = Ft + kMT * nb * 2;                                   // [kMT][VP]
  uint8_t* optr = reinterpret_cast<uint8_t*>(Vt + kMT * VP);       // [d_out + 1]
  uint8_t* olist = optr + GM_FACT_MAX_OUT + 1;
  const int lane = threadIdx.x, m = lane & 15, q = lane >> 4;
  for (int i = lane; i <= d_out; i += kWave) optr[i] = a.optr[i];
  for (int i = lane; i < a.optr[d_out]; i += kWave) olist[i] = a.olist[i];
  stage_desc(a, Bd, lane);
  const int64_t gi = a.group_order ? a.group_order[blockIdx.x] : xcd_spread_block(blockIdx.x, gridDim.x);
  if (gi < 0 || gi >= a.n_groups) return;  // a malformed order names no group
  const int64_t j = a.group_source[gi];
  const int64_t g0 = a.group_ptr[gi], g1 = a.group_ptr[gi + 1];
  float za[NT][4], z0[NT][4];
  int vb[NT][2];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      za[nt][s] = zget(a, j, 1 + 4 * q + s, 16 * nt + m);
      z0[nt][s] = zget(a, j, 0, 16 * nt + 4 * q + s);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int c = 16 * nt + 4 * q + 2 * p;
      vb[nt][p] = c < wc2 ? (int)a.cmap[c >> 1] : -1;
    }
  }
  TileIn next = load_tile<false>(a, g0, (int)((g1 - g0) < kMT ? (g1 - g0) : kMT), lane);
  for (int64_t base = g0; base < g1; base += kMT) {
    const int n = (int)((g1 - base) < kMT ? (g1 - base) : kMT);
    const TileIn cur = next;
    if (base + kMT < g1) {
      const int64_t nb2 = base + kMT;
      next = load_tile<false>(a, nb2, (int)((g1 - nb2) < kMT ? (g1 - nb2) : kMT), lane);
    }
    *reinterpret_cast<floatx4*>(Ph + 4 * lane) = cur.ph;
    if (lane < kMT) Rh[lane] = cur.rho;
    floatx4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt] = mfma16(za[nt][s], cur.h[s], acc[nt]);
    wave_sync();
    factors_grouped(a, Bd, Ph, Rh, Ft, lane);
    wave_sync();
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int c = 16 * nt + 4 * q + 2 * p;
        const float ur = acc[nt][2 * p] + z0[nt][2 * p], ui = acc[nt][2 * p + 1] + z0[nt][2 * p + 1];
        float vr = ur, vi = ui;
        if (vb[nt][p] >= 0) {
          const float* f = Ft + 2 * (m * nb + vb[nt][p]);
          vr = f[0] * ur - f[1] * ui;
          vi = f[0] * ui + f[1] * ur;
        }
        Vt[m * VP + c] = vr;
        Vt[m * VP + c + 1] = vi;
      }
    wave_sync();
    for (int e = q; e < n; e += 4) {
      const float* v = Vt + e * VP;
      float* row = a.out + (base + e) * d_out;
      for (int o = m; o < d_out; o += kMT) {
        float sum = 0.f;
        for (int k = optr[o]; k < optr[o + 1]; ++k) sum += v[olist[k]];
        row[o] = sum;
      }
    }
    wave_sync();
  }
}

template <int NT>
__global__ __launch_bounds__(64) void factored_backward_grouped(FactArgs<float> a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nb = a.n_blocks, CV = 16 * NT, WP = CV + 1, wc2 = 2 * a.wc, d_out = a.d_out;
  int64_t* Tg = reinterpret_cast<int64_t*>(smem);                  // [kMT] targets
  Block* Bd = reinterpret_cast<Block*>(Tg + kMT);                  // [nb]
  float* Ph = reinterpret_cast<float*>(Bd + GM_FACT_MAX_BLOCKS);   // [kMT][kPhaseRow]
  float* Rh = Ph + kMT * kPhaseRow;                                // [kMT]
  float* St = Rh + kMT;                                            // [kMT]
  float* Ft = St + kMT;                                            // [kMT][nb][2]
  float* Gt = Ft + kMT * nb * 2;                                   // [kMT][d_out]
  float* Wt = Gt + kMT * d_out;                                    // [kMT][WP]
  float* Ht = Wt + kMT * WP;                                       // [kMT][16]
  const int lane = threadIdx.x, m = lane & 15, q = lane >> 4;
  stage_desc(a, Bd, lane);
  const int64_t gi = a.group_order ? a.group_order[blockIdx.x] : xcd_spread_block(blockIdx.x, gridDim.x);
  if (gi < 0 || gi >= a.n_groups) return;  // a malformed order names no group
  const int64_t j = a.group_source[gi];
  const int64_t g0 = a.group_ptr[gi], g1 = a.group_ptr[gi + 1];
  float zb[4 * NT];
#pragma unroll
  for (int s = 0; s < 4 * NT; ++s) zb[s] = zget(a, j, 1 + m, q + 4 * s);
  uint32_t ci[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) ci[nt] = 16 * nt + m < a.C ? a.colinfo[16 * nt + m] : 0xFFFFFFFFu;
  floatx4 dz[NT];
  float dz0[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    dz[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    dz0[nt] = 0.f;
  }
  TileIn next = load_tile<true>(a, g0, (int)((g1 - g0) < kMT ? (g1 - g0) : kMT), lane);
  for (int64_t base = g0; base < g1; base += kMT) {
    const int n = (int)((g1 - base) < kMT ? (g1 - base) : kMT);
    const TileIn cur = next;
    if (base + kMT < g1) {
      const int64_t nb2 = base + kMT;
      next = load_tile<true>(a, nb2, (int)((g1 - nb2) < kMT ? (g1 - nb2) : kMT), lane);
    }
    *reinterpret_cast<floatx4*>(Ph + 4 * lane) = cur.ph;
    *reinterpret_cast<floatx4*>(Ht + 4 * lane) = cur.h;  // Ht[e = l / 4][4 (l % 4) ..]
    if (lane < kMT) {
      Rh[lane] = cur.rho;
      St[lane] = cur.w;
      Tg[lane] = cur.tgt;
    }
    wave_sync();
    for (int e = q; e < kMT; e += 4) {
      const float* grow = e < n ? a.g + Tg[e] * a.g_ld : nullptr;
      for (int o = m; o < d_out; o += kMT) Gt[e * d_out + o] = grow ? grow[o] : 0.f;
    }
    factors_grouped(a, Bd, Ph, Rh, Ft, lane);
    wave_sync();
    if (lane < n) {
      const float* r = a.rows + (base + lane) * d_out;
      const float* gr = Gt + lane * d_out;
      float sum = 0.f;
      for (int o = 0; o < d_out; ++o) sum += gr[o] * r[o];
      a.dweights[base + lane] = a.accumulate ? a.dweights[base + lane] + sum : sum;
    }
    float w[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint32_t info = ci[nt];
      const int b = info & 0xFF, gre = (info >> 8) & 0xFF, gim = (info >> 16) & 0xFF, kind = info >> 24;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = q + 4 * i;
        float v = 0.f;
        if (info != 0xFFFFFFFFu) {
          const float* gr = Gt + e * d_out;
          const float g_re = gr[gre], g_im = gim == 0xFF ? 0.f : gr[gim];
          if (kind == 0) {
            v = g_re;
          } else {
            const float* f = Ft + 2 * (e * nb + b);
            v = kind == 1 ? g_re * f[0] + g_im * f[1] : g_im * f[0] - g_re * f[1];
          }
          v *= St[e];
        }
        w[nt][i] = v;
        Wt[e * WP + 16 * nt + m] = v;
      }
    }
    wave_sync();
    floatx4 dh = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4 * NT; ++s) dh = mfma16(Wt[m * WP + q + 4 * s], zb[s], dh);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = 4 * q + r;
      if (e < n && m + 1 < a.K) a.dh[(base + e) * 16 + m] = a.accumulate ? a.dh[(base + e) * 16 + m] + dh[r] : dh[r];
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dz[nt] = mfma16(Ht[(q + 4 * i) * 16 + m], w[nt][i], dz[nt]);
        dz0[nt] += w[nt][i];
      }
    wave_sync();
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    dz0[nt] += __shfl_xor(dz0[nt], 16, kWave);
    dz0[nt] += __shfl_xor(dz0[nt], 32, kWave);
    const int c = 16 * nt + m;
    if (c >= a.C) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 1 + 4 * q + r;
      if (t < a.K) zput(a, j, t, c, dz[nt][r]);
    }
    if (q == 0) zput(a, j, 0, c, dz0[nt]);
  }
}

// ------------------------------------------------------------ lane-owned outputs
//
// Plans whose blocks come in multiplicities of four, with radial power equal
// to the angular order (F_b = (r e^{i phi})^a e^{i s gamma}: every plan the
// steerable kernel builds), run on kernels where the four lanes sharing an
// edge split every block by copy: lane q owns the copies k = q (mod 4).
// A lane's slots are its (block, copy) pairs, ordered so that the blocks
// summed into one output follow each other; slot s sits in MFMA column tile
// s / 2 at register pair s % 2.  The forward then sums its own slots into its
// own outputs in registers (no LDS pass over the row), and the backward forms
// W in the same slots, takes dh straight from them on MFMA and transposes W
// once through LDS for dZ.  Per-slot words:
//   bits 0-6 the output base (+ q for scalar outputs, + 2 q for complex),
//   7 active, 8 the real block (factor 1), 9 scalar output, 10 last slot of
//   its output, 11-13 the angular entry, 14 its conjugate, 15-17 the
//   transport entry, 18 its conjugate.
// The words are compile-time constants for the plans the steerable kernel
// builds with four copies per frequency and head (then the phases stay in
// registers and every slot's code is fixed), kernel arguments otherwise.
//
// Every per-edge stream of a group is read and written through a buffer
// resource bounded to the group: the lanes past the group's last edge load
// zeros and their stores are dropped, so the tile loop has no branches and
// the wait for the prefetched tile never waits on the tile's own stores.
// Z(j) comes in (and dZ(j) goes out) through LDS in slot-column order, run by
// run, with coalesced row reads.
constexpr int kMaxSlots = 16;
constexpr int kPhStride = 18;  // floats per LDS phase row: 16 + 2 puts the 16 rows' 8-byte reads in distinct banks
constexpr int kWtStride = 20;  // floats per LDS W column (16 edges + 4): 16-byte aligned four-edge reads

enum : uint32_t {
  kSlotActive = 1u << 7,
  kSlotReal = 1u << 8,
  kSlotScalar = 1u << 9,
  kSlotFlush = 1u << 10,
  kSlotAConj = 1u << 14,
  kSlotTConj = 1u << 18,
};

__host__ __device__ constexpr int slot_ob(uint32_t w) { return (int)(w & 0x7F); }
__host__ __device__ constexpr int slot_ai(uint32_t w) { return (int)((w >> 11) & 7); }
__host__ __device__ constexpr int slot_ti(uint32_t w) { return (int)((w >> 15) & 7); }

// Compile-time slot words: PA angular entries in the phase row, DOUT floats a row.
template <int PA, int DOUT, uint32_t... W>
struct StaticSlots {
  static constexpr bool kStatic = true;
  static constexpr int kSlots = (int)sizeof...(W);
  static constexpr int kPa = PA;
  static constexpr int kDout = DOUT;
  __host__ __device__ static constexpr uint32_t word(int s) {
    constexpr uint32_t w[] = {W..., 0u};
    return s >= 0 && s < kSlots ? w[s] : 0u;
  }
  // one past the highest angular and transport orders the slots use
  __host__ __device__ static constexpr int angular_orders() {
    int n = 1;
    for (int s = 0; s < kSlots; ++s)
      if (!(word(s) & kSlotReal) && slot_ai(word(s)) + 1 > n) n = slot_ai(word(s)) + 1;
    return n;
  }
  __host__ __device__ static constexpr int transport_orders() {
    int n = 1;
    for (int s = 0; s < kSlots; ++s)
      if (!(word(s) & kSlotReal) && slot_ti(word(s)) - PA + 1 > n) n = slot_ti(word(s)) - PA + 1;
    return n;
  }
};
struct RuntimeSlots {
  static constexpr bool kStatic = false;
  static constexpr int kSlots = kMaxSlots;
  static constexpr int kPa = 0;
  static constexpr int kDout = 0;
  __host__ __device__ static constexpr uint32_t word(int) { return 0u; }
  __host__ __device__ static constexpr int angular_orders() { return 1; }
  __host__ __device__ static constexpr int transport_orders() { return 1; }
};
// frequencies 0..2, four copies each: 13 slots (one real, two onto frequency
// 0 taking the real part, five onto each of frequencies 1 and 2)
using SlotsF2 = StaticSlots<5, 20, 0x28380u, 0x70a80u, 0x79680u, 0x28884u, 0x30084u, 0x71084u, 0x3c884u, 0x79c84u,
                            0x2908cu, 0x3088cu, 0x7188cu, 0x3808cu, 0x7a48cu>;
// frequencies 0..1, four copies each: 5 slots
using SlotsF1 = StaticSlots<3, 12, 0x18380u, 0x60e80u, 0x18884u, 0x20084u, 0x61484u>;
// scalar input onto frequencies 0..2, sixteen copies each (a restriction from
// scalar channels cut into shares of sixteen copies): 12 slots
using SlotsS16 = StaticSlots<3, 80, 0x18780u, 0x18784u, 0x18788u, 0x1878cu, 0x18c90u, 0x18c98u, 0x18ca0u, 0x18ca8u,
                             0x194b0u, 0x194b8u, 0x194c0u, 0x194c8u>;


template <class P>
__device__ __forceinline__ uint32_t slot_word(const FactArgs<float>& a, int s) {
  if constexpr (P::kStatic)
    return P::word(s);
  else
    return a.slot[s];
}

// The first slot of slot s's output (its G and row values are loaded there).
template <class P>
__device__ __forceinline__ constexpr int group_start(int s) {
  int b = s;
  while (b > 0 && !(P::word(b - 1) & kSlotFlush)) --b;
  return b;
}

// A (byte-addressed) buffer resource over n_bytes from p: reads past the end
// return zero, writes past it are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span(const void* p, int64_t n_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)n_bytes, 0x00020000);
}
__device__ __forceinline__ float bload1(__amdgpu_buffer_rsrc_t r, int off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ float2 bload2(__amdgpu_buffer_rsrc_t r, int off) {
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  const u2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}
__device__ __forceinline__ int64_t bload_i64(__amdgpu_buffer_rsrc_t r, int off) {
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  const u2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  return (int64_t)(((uint64_t)v[1] << 32) | v[0]);
}
__device__ __forceinline__ floatx4 bload4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ void bstore1(float v, __amdgpu_buffer_rsrc_t r, int off) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
}
__device__ __forceinline__ void bstore2(float x, float y, __amdgpu_buffer_rsrc_t r, int off) {
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(u2{__float_as_uint(x), __float_as_uint(y)}, r, off, 0, 0);
}
__device__ __forceinline__ void bstore4(floatx4 v, __amdgpu_buffer_rsrc_t r, int off) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, off, 0, 0);
}
constexpr int kDrop = 0x7FFFFFF0;  // a byte offset past every group's span: the access is dropped

// Per-edge streams (trunk features h and their gradients dh, output rows) by
// element index: float32, or with B16 bfloat16 (rounded to nearest even on
// store, widened exactly on load) at half the bytes.  Arithmetic is float32
// either way.
template <bool B16>
__device__ __forceinline__ int64_t stream_bytes(int64_t n) {
  return n * (B16 ? 2 : 4);
}
template <bool B16>
__device__ __forceinline__ void sstore1(float v, __amdgpu_buffer_rsrc_t r, int i) {
  if constexpr (B16)
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)(pack_bf16(v, 0.f) & 0xFFFFu), r, 2 * i, 0, 0);
  else
    bstore1(v, r, 4 * i);
}
template <bool B16>
__device__ __forceinline__ void sstore2(float x, float y, __amdgpu_buffer_rsrc_t r, int i) {
  if constexpr (B16)
    __builtin_amdgcn_raw_buffer_store_b32(pack_bf16(x, y), r, 2 * i, 0, 0);
  else
    bstore2(x, y, r, 4 * i);
}
template <bool B16>
__device__ __forceinline__ void sstore4(floatx4 v, __amdgpu_buffer_rsrc_t r, int i) {
  if constexpr (B16) {
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(u2{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])}, r, 2 * i, 0, 0);
  } else {
    bstore4(v, r, 4 * i);
  }
}
template <bool B16>
__device__ __forceinline__ float sload1(__amdgpu_buffer_rsrc_t r, int i) {
  if constexpr (B16)
    return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, 2 * i, 0, 0) << 16);
  else
    return bload1(r, 4 * i);
}
template <bool B16>
__device__ __forceinline__ float2 sload2(__amdgpu_buffer_rsrc_t r, int i) {
  if constexpr (B16) {
    const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(r, 2 * i, 0, 0);
    return make_float2(bf16_lo(v), bf16_hi(v));
  } else {
    return bload2(r, 4 * i);
  }
}
// A lane's four trunk features: with bfloat16 streams kept packed (the two
// words as the bit patterns of h[0] and h[1]) until hwiden turns them into
// floats where they are used, so two tiles in flight hold half the registers.
template <bool B16>
__device__ __forceinline__ floatx4 hload(__amdgpu_buffer_rsrc_t r, int i) {
  if constexpr (B16) {
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    const u2 v = __builtin_amdgcn_raw_buffer_load_b64(r, 2 * i, 0, 0);
    return floatx4{__uint_as_float(v[0]), __uint_as_float(v[1]), 0.f, 0.f};
  } else {
    return bload4(r, 4 * i);
  }
}
template <bool B16>
__device__ __forceinline__ floatx4 hwiden(const floatx4& h) {
  if constexpr (B16) {
    const uint32_t a = __float_as_uint(h[0]), b = __float_as_uint(h[1]);
    return floatx4{bf16_lo(a), bf16_hi(a), bf16_lo(b), bf16_hi(b)};
  } else {
    return h;
  }
}
template <bool B16>
__device__ __forceinline__ floatx4 sload4(__amdgpu_buffer_rsrc_t r, int i) {
  if constexpr (B16) {
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    const u2 v = __builtin_amdgcn_raw_buffer_load_b64(r, 2 * i, 0, 0);
    return floatx4{bf16_lo(v[0]), bf16_hi(v[0]), bf16_lo(v[1]), bf16_hi(v[1])};
  } else {
    return bload4(r, 4 * i);
  }
}

// SlotsF2 by Horner's rule.  With z = r e^{i phi}, w = e^{i gamma} and
// p = z conj(w), the thirteen factors are
//   output 0 (real part): 1, p, p^2                      (slots 0, 1, 2)
//   output 1: z, w, z p, conj(z) w^2, z p^2               (slots 3 .. 7)
//   output 2: z^2, z w, z^2 p, w^2, z^2 p^2               (slots 8 .. 12)
// so each output is a leading power times a quadratic in p plus two single
// terms: 75 operations a tile instead of a product per slot.
template <class P>
constexpr bool kHorner = std::is_same<P, SlotsF2>::value;

struct F2Powers {
  float pr, pi;    // p = z conj(w)
  float z2r, z2i;  // z^2
  float w2r, w2i;  // w^2
  float zwr, zwi;  // z w
  float cr, ci;    // conj(z) w^2
};

__device__ __forceinline__ F2Powers f2_powers(const floatx4& zw) {
  const float zr = zw[0], zi = zw[1], wr = zw[2], wi = zw[3];
  F2Powers f;
  f.pr = zr * wr + zi * wi;
  f.pi = zi * wr - zr * wi;
  f.z2r = zr * zr - zi * zi;
  f.z2i = 2.f * (zr * zi);
  f.w2r = wr * wr - wi * wi;
  f.w2i = 2.f * (wr * wi);
  f.zwr = zr * wr - zi * wi;
  f.zwi = zr * wi + zi * wr;
  f.cr = zr * f.w2r + zi * f.w2i;
  f.ci = zr * f.w2i - zi * f.w2r;
  return f;
}

// x y + c (complex)
__device__ __forceinline__ void cmac(float xr, float xi, float yr, float yi, float cr, float ci, float& r, float& i) {
  r = fmaf(xr, yr, fmaf(-xi, yi, cr));
  i = fmaf(xr, yi, fmaf(xi, yr, ci));
}

// conj(x) y
__device__ __forceinline__ void cjmul(float xr, float xi, float yr, float yi, float& r, float& i) {
  r = fmaf(xr, yr, xi * yi);
  i = fmaf(xr, yi, -(xi * yr));
}

// Forward: edge m's three outputs from u (slot s at acc[s / 2][2 (s % 2)], +1 imaginary), stored.
template <bool B16>
__device__ __forceinline__ void f2_forward_outputs(const floatx4 (&acc)[7], const floatx4& zw,
                                                   __amdgpu_buffer_rsrc_t out_r, int row, int q) {
  const F2Powers f = f2_powers(zw);
#define GM_U(s) acc[(s) >> 1][2 * ((s)&1)], acc[(s) >> 1][2 * ((s)&1) + 1]
  float tr, ti, vr, vi;
  // output 0: Re(u0) + Re(p (u1 + p u2))
  cmac(f.pr, f.pi, GM_U(2), GM_U(1), tr, ti);
  sstore1<B16>(fmaf(f.pr, tr, fmaf(-f.pi, ti, acc[0][0])), out_r, row + q);
  // output 1: z (u3 + p (u5 + p u7)) + w u4 + conj(z) w^2 u6
  const float zr = zw[0], zi = zw[1], wr = zw[2], wi = zw[3];
  cmac(f.pr, f.pi, GM_U(7), GM_U(5), tr, ti);
  cmac(f.pr, f.pi, tr, ti, GM_U(3), tr, ti);
  vr = 0.f;
  vi = 0.f;
  cmac(f.cr, f.ci, GM_U(6), vr, vi, vr, vi);
  cmac(wr, wi, GM_U(4), vr, vi, vr, vi);
  cmac(zr, zi, tr, ti, vr, vi, vr, vi);
  sstore2<B16>(vr, vi, out_r, row + 4 + 2 * q);
  // output 2: z^2 (u8 + p (u10 + p u12)) + z w u9 + w^2 u11
  cmac(f.pr, f.pi, GM_U(12), GM_U(10), tr, ti);
  cmac(f.pr, f.pi, tr, ti, GM_U(8), tr, ti);
  vr = 0.f;
  vi = 0.f;
  cmac(f.w2r, f.w2i, GM_U(11), vr, vi, vr, vi);
  cmac(f.zwr, f.zwi, GM_U(9), vr, vi, vr, vi);
  cmac(f.z2r, f.z2i, tr, ti, vr, vi, vr, vi);
  sstore2<B16>(vr, vi, out_r, row + 12 + 2 * q);
#undef GM_U
}

// Backward: W = conj(F) (w G) per slot for edge m, G_k = (gr[k], gi[k]) the
// weighted gradient of output k (gi[0] unused: output 0 takes the real part).
__device__ __forceinline__ void f2_backward_weights(const floatx4& zw, const float (&gr)[3], const float (&gi)[3],
                                                    float (&wv)[7][4]) {
  const F2Powers f = f2_powers(zw);
  const float zr = zw[0], zi = zw[1], wr = zw[2], wi = zw[3];
#define GM_W(s) wv[(s) >> 1][2 * ((s)&1)], wv[(s) >> 1][2 * ((s)&1) + 1]
  // output 0: 1, p, p^2 applied to a real gradient
  wv[0][0] = gr[0];
  wv[0][1] = 0.f;
  wv[0][2] = f.pr * gr[0];
  wv[0][3] = -(f.pi * gr[0]);
  cjmul(f.pr, f.pi, wv[0][2], wv[0][3], GM_W(2));
  // output 1: z, w, z p, conj(z) w^2, z p^2
  cjmul(zr, zi, gr[1], gi[1], GM_W(3));
  cjmul(f.pr, f.pi, wv[1][2], wv[1][3], GM_W(5));
  cjmul(f.pr, f.pi, wv[2][2], wv[2][3], GM_W(7));
  cjmul(wr, wi, gr[1], gi[1], GM_W(4));
  cjmul(f.cr, f.ci, gr[1], gi[1], GM_W(6));
  // output 2: z^2, z w, z^2 p, w^2, z^2 p^2
  cjmul(f.z2r, f.z2i, gr[2], gi[2], GM_W(8));
  cjmul(f.pr, f.pi, wv[4][0], wv[4][1], GM_W(10));
  cjmul(f.pr, f.pi, wv[5][0], wv[5][1], GM_W(12));
  cjmul(f.zwr, f.zwi, gr[2], gi[2], GM_W(9));
  cjmul(f.w2r, f.w2i, gr[2], gi[2], GM_W(11));
  wv[6][2] = 0.f;  // slot 13 is empty
  wv[6][3] = 0.f;
#undef GM_W
}

// Z(j) into LDS in slot-column order, Zs[t * ZS + sc] for t < 17, zero in the
// padding columns, in two steps so that a kernel can put its first tiles'
// loads into the same memory round trip.  z_issue: when every run is at most
// one wave wide, lane c requests column c of every run (all 17 rows of all
// runs in flight together, each row coalesced across the lanes).  z_commit:
// the padding cleared and the values written to their slot columns; wider
// runs (and every run when Batch is false) are staged there run by run.
struct ZStage {
  float v[GM_FACT_MAX_SEG][17];
  bool narrow;
};

template <bool Batch>
__device__ __forceinline__ void z_issue(const FactArgs<float>& a, int64_t j, int lane, ZStage& st) {
  st.narrow = Batch;
  if (!Batch) return;  // runs staged one by one: fewer registers held
  for (int r = 0; r < a.n_seg; ++r) st.narrow = st.narrow && a.seg[r].width <= kWave;
  if (!st.narrow) return;
#pragma unroll
  for (int r = 0; r < GM_FACT_MAX_SEG; ++r) {
    if (r < a.n_seg && lane < a.seg[r].width) {
      const ZSeg<float>& g = a.seg[r];
      // the node's 17 mix rows of this run through one buffer: row t at byte t * ts * 4 (a scalar offset)
      const int ts = g.t_stride;
      const auto zr = span(g.z + j * g.node_stride, ((int64_t)16 * ts + g.width) * 4);
#pragma unroll
      for (int t = 0; t < 17; ++t)
        st.v[r][t] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(zr, lane * 4, t * ts * 4, 0));
    }
  }
}

template <int ZS>
__device__ __forceinline__ void z_commit(const FactArgs<float>& a, int64_t j, float* Zs, const uint8_t* colslot,
                                         int lane, const ZStage& st) {
  for (int i = lane; i < 17 * ZS / 4; i += kWave) reinterpret_cast<floatx4*>(Zs)[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  wave_sync();
  if (st.narrow) {
#pragma unroll
    for (int r = 0; r < GM_FACT_MAX_SEG; ++r) {
      if (r < a.n_seg && lane < a.seg[r].width) {
        const int sc = colslot[a.seg[r].c0 + lane];
#pragma unroll
        for (int t = 0; t < 17; ++t) Zs[t * ZS + sc] = st.v[r][t];
      }
    }
  } else {
    for (int r = 0; r < a.n_seg; ++r) {
      const ZSeg<float>& g = a.seg[r];
      const int ts = g.t_stride;
      const auto zr = span(g.z + j * g.node_stride, ((int64_t)16 * ts + g.width) * 4);
      for (int c = lane; c < g.width; c += kWave) {
        const int sc = colslot[g.c0 + c];
        float v[17];
#pragma unroll
        for (int t = 0; t < 17; ++t)
          v[t] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(zr, c * 4, t * ts * 4, 0));
#pragma unroll
        for (int t = 0; t < 17; ++t) Zs[t * ZS + sc] = v[t];
      }
    }
  }
  wave_sync();
}

// dZ(j) out of LDS (slot-column order) into the runs' gradient arrays.
template <int ZS>
__device__ __forceinline__ void flush_dz_slots(const FactArgs<float>& a, int64_t j, const float* Zs,
                                               const uint8_t* colslot, int lane) {
  for (int r = 0; r < a.n_seg; ++r) {
    const ZSeg<float>& g = a.seg[r];
    const int ts = g.t_stride;
    const auto dzr = span(g.dz + j * g.node_stride, ((int64_t)16 * ts + g.width) * 4);
    for (int c = lane; c < g.width; c += kWave) {
      const int sc = colslot[g.c0 + c];
      float v[17];
#pragma unroll
      for (int t = 0; t < 17; ++t) v[t] = Zs[t * ZS + sc];
#pragma unroll
      for (int t = 0; t < 17; ++t)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[t]), dzr, c * 4, t * ts * 4, 0);
    }
  }
}

// The rows of packed column -> slot column, into LDS (128 bytes).
__device__ __forceinline__ void stage_colslot(const FactArgs<float>& a, uint8_t* colslot, int lane) {
  if (lane < 32) reinterpret_cast<uint32_t*>(colslot)[lane] = a.colslot32[lane];
}

// The lane's edge's phase registers.  Fixed slots: zw = (r e^{i phi},
// e^{i gamma}), from which every factor is a product of powers; runtime
// slots: chunk q of the edge's phase row (staged to LDS).
template <class P>
struct PhaseRegs {
  floatx4 ph;
};

// Powers z^o (o < angular orders) of z = r e^{i phi} and w^o of w = e^{i gamma}
// (o < transport orders), by squaring and one multiplication per odd power.
template <class P>
struct Powers {
  static constexpr int NA = P::kStatic ? P::angular_orders() : 1;
  static constexpr int NW = P::kStatic ? P::transport_orders() : 1;
  float zr[NA], zi[NA], wr[NW], wi[NW];
};

__device__ __forceinline__ void cmul(float ar, float ai, float br, float bi, float& cr, float& ci) {
  cr = ar * br - ai * bi;
  ci = ar * bi + ai * br;
}

template <class P>
__device__ __forceinline__ Powers<P> powers(const floatx4& zw) {
  Powers<P> p;
  p.zr[0] = 1.f;
  p.zi[0] = 0.f;
#pragma unroll
  for (int o = 1; o < Powers<P>::NA; ++o) {
    if (o == 1) {
      p.zr[1] = zw[0];
      p.zi[1] = zw[1];
    } else if (o % 2 == 0) {
      cmul(p.zr[o / 2], p.zi[o / 2], p.zr[o / 2], p.zi[o / 2], p.zr[o], p.zi[o]);
    } else {
      cmul(p.zr[o - 1], p.zi[o - 1], zw[0], zw[1], p.zr[o], p.zi[o]);
    }
  }
  p.wr[0] = 1.f;
  p.wi[0] = 0.f;
#pragma unroll
  for (int o = 1; o < Powers<P>::NW; ++o) {
    if (o == 1) {
      p.wr[1] = zw[2];
      p.wi[1] = zw[3];
    } else if (o % 2 == 0) {
      cmul(p.wr[o / 2], p.wi[o / 2], p.wr[o / 2], p.wi[o / 2], p.wr[o], p.wi[o]);
    } else {
      cmul(p.wr[o - 1], p.wi[o - 1], zw[2], zw[3], p.wr[o], p.wi[o]);
    }
  }
  return p;
}

// Slot s's factor z^a w^t (conjugates as the word says) for compile-time slots.
template <class P>
__device__ __forceinline__ void static_factor(const Powers<P>& p, int s, float& fr, float& fi) {
  const uint32_t w = P::word(s);
  const int ai = slot_ai(w), to = slot_ti(w) - P::kPa;
  const float ar = p.zr[ai], aim = (w & kSlotAConj) ? -p.zi[ai] : p.zi[ai];
  const float tr = p.wr[to], tim = (w & kSlotTConj) ? -p.wi[to] : p.wi[to];
  if (ai == 0) {
    fr = tr;
    fi = tim;
  } else if (to == 0) {
    fr = ar;
    fi = aim;
  } else {
    cmul(ar, aim, tr, tim, fr, fi);
  }
}

// Runtime slot words: the tile's phase rows in LDS (lane (m, q) writes chunk q
// of edge m, the angular entries scaled by rho^o), then per-slot reads.
__device__ __forceinline__ void stage_phases_lanes(const FactArgs<float>& a, float* Ph, floatx4 chunk, float rho,
                                                   int m, int q) {
  const int o = 2 * q;
  const float r2 = rho * rho;
  float p = 1.f;
  for (int i = 0; i < q; ++i) p *= r2;
  const float s0 = o < a.pa ? p : 1.f, s1 = o + 1 < a.pa ? p * rho : 1.f;
  float* dst = Ph + m * kPhStride + 2 * o;
  *reinterpret_cast<float2*>(dst) = make_float2(chunk[0] * s0, chunk[1] * s0);
  *reinterpret_cast<float2*>(dst + 2) = make_float2(chunk[2] * s1, chunk[3] * s1);
}

__device__ __forceinline__ void runtime_factor(const float* prow, uint32_t w, float& fr, float& fi) {
  const float2 A = *reinterpret_cast<const float2*>(prow + 2 * slot_ai(w));
  const float2 T = *reinterpret_cast<const float2*>(prow + 2 * slot_ti(w));
  const float ai = (w & kSlotAConj) ? -A.y : A.y, ti = (w & kSlotTConj) ? -T.y : T.y;
  fr = A.x * T.x - ai * ti;
  fi = A.x * ti + ai * T.x;
}

// Whether the dh k-step (nt, r) reads any real column (else it is skipped).
template <class P>
__device__ __forceinline__ bool kstep_live(const FactArgs<float>& a, int nt, int r) {
  const int s = 2 * nt + (r >> 1);
  const uint32_t w = slot_word<P>(a, s);
  return (w & kSlotActive) && !((w & kSlotReal) && (r & 1));
}

// The fused trunk as one 16 x 16 matrix product per tile: pre (16 features x
// 16 edges) = b1 + W1 (16 x 8) B (8 basis functions x 16 edges) in two
// k-steps, so lane (m, q) supplies W1[m][4 s + q] and the basis function
// 4 s + q of edge m (two exponentials) and holds the pre-activations of
// features 4 q .. 4 q + 3 of edge m -- the layout the kernels use for h.
struct TrunkLane {
  float wa[2];   // W1[m][4 s + q], s = 0, 1 (zero past the basis)
  floatx4 b1;    // b1[4 q .. 4 q + 3]
};

__device__ __forceinline__ TrunkLane trunk_lane(const FactArgs<float>& a, int m, int q) {
  TrunkLane t;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int k = 4 * s + q;
    t.wa[s] = k < a.trunk_nb ? a.trunk_w[m * a.trunk_nb + k] : 0.f;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) t.b1[r] = a.trunk_b ? a.trunk_b[4 * q + r] : 0.f;
  return t;
}

// h of features 4 q .. 4 q + 3 of edge m (rho its distance / cutoff); the
// pre-activations into pre.  Basis exp(-((rho^2 - c_k) / width)^2 / 2) and
// SiLU on the hardware exponential and reciprocal, as the trunk kernel.
__device__ __forceinline__ floatx4 trunk_features(const FactArgs<float>& a, const TrunkLane& t, int q, float rho,
                                                  floatx4& pre) {
  const float s2 = rho * rho;
  pre = t.b1;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int k = 4 * s + q;
    const float z = (s2 - (k < 8 ? a.trunk_c[k] : 0.f)) * a.trunk_inv_width;
    const float b = k < a.trunk_nb ? __builtin_amdgcn_exp2f(-0.5f * z * z * 1.44269504088896340736f) : 0.f;
    pre = mfma16(t.wa[s], b, pre);
  }
  floatx4 h;
#pragma unroll
  for (int r = 0; r < 4; ++r) h[r] = pre[r] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-pre[r] * 1.44269504088896340736f));
  return h;
}

template <class P>
struct FwdTile {
  floatx4 h;        // h(edge m)[4 q .. 4 q + 3]
  PhaseRegs<P> ph;  // fixed slots: edge m's zw; runtime: chunk q of its phase row
  float rho;        // runtime slots or the fused trunk: rho of edge m
};

// ph_r spans the zw rows (fixed slots) or the phase rows (runtime slots).
template <class P, bool B16 = false>
__device__ __forceinline__ FwdTile<P> load_fwd(__amdgpu_buffer_rsrc_t h_r, __amdgpu_buffer_rsrc_t ph_r,
                                               __amdgpu_buffer_rsrc_t rho_r, int tb, int m, int q, bool fused) {
  FwdTile<P> t;
  const int e = tb + m;
  if (fused) {
    t.h = floatx4{0.f, 0.f, 0.f, 0.f};
  } else {
    t.h = hload<B16>(h_r, e * 16 + 4 * q);
  }
  if constexpr (P::kStatic) {
    t.ph.ph = bload4(ph_r, e * 16);
    t.rho = fused ? bload1(rho_r, e * 4) : 0.f;
  } else {
    t.ph.ph = bload4(ph_r, (e * kPhaseRow + 4 * q) * 4);
    t.rho = bload1(rho_r, e * 4);
  }
  return t;
}

// Edge m's outputs from u (slot s at acc[s / 2][2 (s % 2)], +1 imaginary):
// V = F u per slot, summed over each output's slots and stored.
template <int NT, class P, bool B16 = false>
__device__ __forceinline__ void forward_outputs(const FactArgs<float>& a, const FwdTile<P>& cur,
                                                const floatx4 (&acc)[NT], float* Ph, __amdgpu_buffer_rsrc_t out_r,
                                                int d_out, int tb, int m, int q) {
  if constexpr (kHorner<P>) {
    f2_forward_outputs<B16>(acc, cur.ph.ph, out_r, (tb + m) * d_out, q);
    return;
  }
  Powers<P> pw;
  if constexpr (P::kStatic) {
    pw = powers<P>(cur.ph.ph);
  } else {
    stage_phases_lanes(a, Ph, cur.ph.ph, cur.rho, m, q);
    wave_sync();
  }
  // V = F u per slot, summed over each output's slots and stored
  const int row = (tb + m) * d_out;
  float sr = 0.f, si = 0.f;
#pragma unroll
  for (int s = 0; s < 2 * NT; ++s) {
    const uint32_t w = slot_word<P>(a, s);
    const float ur = acc[s >> 1][2 * (s & 1)], ui = acc[s >> 1][2 * (s & 1) + 1];
    if (P::kStatic && (w & kSlotReal)) {
      sr += ur;
    } else {
      float fr, fi;
      if constexpr (P::kStatic)
        static_factor<P>(pw, s, fr, fi);
      else
        runtime_factor(Ph + m * kPhStride, w, fr, fi);
      sr += fr * ur - fi * ui;
      si += fr * ui + fi * ur;
    }
    if (w & kSlotFlush) {
      if (w & kSlotScalar)
        sstore1<B16>(sr, out_r, row + slot_ob(w) + q);
      else
        sstore2<B16>(sr, si, out_r, row + slot_ob(w) + 2 * q);
      sr = 0.f;
      si = 0.f;
    }
  }
  if constexpr (!P::kStatic) wave_sync();
}

// One forward tile: 16 edges from tb, the rows stored through out_r.
template <int NT, class P, bool B16 = false>
__device__ __forceinline__ void forward_tile(const FactArgs<float>& a, const FwdTile<P>& cur, const float (&za)[NT][4],
                                             const floatx4 (&z0)[NT], float* Ph, __amdgpu_buffer_rsrc_t out_r,
                                             int d_out, int tb, int m, int q, const TrunkLane& tl, bool fused) {
  // h(edge m)[4 q .. 4 q + 3]: read, or the trunk's features evaluated here
  floatx4 pre;
  const floatx4 h = fused ? trunk_features(a, tl, q, cur.rho, pre) : hwiden<B16>(cur.h);
  // u(e) = Z0 + sum_t h_t Z_t: lane (m, q) ends with edge m's slot columns 16 nt + 4 q + r
  floatx4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = z0[nt];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = mfma16(za[nt][s], h[s], acc[nt]);
  forward_outputs<NT, P, B16>(a, cur, acc, Ph, out_r, d_out, tb, m, q);
}

// forward_tile with the product on the bf16 matrix cores (fixed slots, trunk
// features read): Z's pieces for the lane's features 4 q .. 4 q + 3 at columns
// 16 nt + m are held for the group, h's are split per tile.
// Z's row 0 (the bias feature) is read from the LDS copy per tile.
// With B16 the features are bfloat16 values, their own single piece: the
// three piece products of Z's pieces hi, mid and lo with h in two
// instructions.
template <int NT, class P, bool B16 = false>
__device__ __forceinline__ void forward_tile_split(const FactArgs<float>& a, const FwdTile<P>& cur,
                                                   const SplitA (&zs)[NT], const float* Zs, float* Ph,
                                                   __amdgpu_buffer_rsrc_t out_r, int d_out, int tb, int m, int q) {
  floatx4 acc[NT];
  if constexpr (B16) {
    const uint32_t h01 = __float_as_uint(cur.h[0]), h23 = __float_as_uint(cur.h[1]);  // the packed features
    const u32x4 hh{h01, h23, h01, h23}, zh{0u, 0u, h01, h23};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      floatx4 c = mfma_bf16(zs[nt].hl, zh, *reinterpret_cast<const floatx4*>(Zs + 16 * nt + 4 * q));  // lo h
      acc[nt] = mfma_bf16(zs[nt].hm, hh, c);                                                          // hi h + mid h
    }
  } else {
    const SplitB hb = split_b(cur.h[0], cur.h[1], cur.h[2], cur.h[3]);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      acc[nt] = mfma_split(zs[nt], hb, *reinterpret_cast<const floatx4*>(Zs + 16 * nt + 4 * q));
  }
  forward_outputs<NT, P, B16>(a, cur, acc, Ph, out_r, d_out, tb, m, q);
}

// SPLIT (fixed slots, trunk features read): the product on the bf16 matrix
// cores in fp32 accuracy.  B16 (fixed slots, trunk features read): h read and
// the rows stored in bfloat16.
template <int NT, class P, bool FUSED, bool SPLIT, bool B16 = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(P::kStatic ? (FUSED || SPLIT ? 3 : 4) : 1))) void
factored_forward_lanes(FactArgs<float> a) {
  static_assert(!SPLIT || (P::kStatic && !FUSED), "the split product serves fixed slots with trunk features read");
  static_assert(!B16 || (P::kStatic && !FUSED), "bfloat16 streams serve fixed slots with trunk features read");
  constexpr int ZS = 16 * NT + 4;
  __shared__ __align__(16) float Zs[17 * ZS];
  __shared__ __align__(16) float Ph[P::kStatic ? 4 : kMT * kPhStride];
  __shared__ __align__(16) uint8_t colslot[128];
  const int lane = threadIdx.x, m = lane & 15, q = lane >> 4;
  const int d_out = P::kStatic ? P::kDout : a.d_out;
  const int64_t gi = a.group_order ? a.group_order[blockIdx.x] : xcd_spread_block(blockIdx.x, gridDim.x);
  if (gi < 0 || gi >= a.n_groups) return;  // a malformed order names no group
  const int64_t j = a.group_source[gi];
  const int64_t g0 = a.group_ptr[gi];
  const int ng = (int)(a.group_ptr[gi + 1] - g0);
  constexpr bool fused = FUSED;
  // h and the rows: float32, or bfloat16 (B16) at half the bytes
  const char* h_b = reinterpret_cast<const char*>(a.h);
  char* out_b = reinterpret_cast<char*>(a.out);
  const auto h_r = span(fused ? nullptr : h_b + stream_bytes<B16>(g0 * 16), fused ? 0 : stream_bytes<B16>((int64_t)ng * 16));
  const auto ph_r = P::kStatic ? span(a.zw_g + g0 * 4, (int64_t)ng * 16)
                               : span(a.phase_g + g0 * kPhaseRow, (int64_t)ng * kPhaseRow * 4);
  const auto rho_r = span(a.rho_g + g0, (int64_t)ng * 4);
  const auto out_r = span(out_b + stream_bytes<B16>(g0 * d_out), stream_bytes<B16>((int64_t)ng * d_out));
  // two tiles in flight: each buffer is refilled right after its tile's
  // stores, so waiting for a tile never waits for the previous tile's stores.
  // The first two are requested with the node's mixes (one round trip).
  FwdTile<P> ta = load_fwd<P, B16>(h_r, ph_r, rho_r, 0, m, q, fused);
  FwdTile<P> tbf = load_fwd<P, B16>(h_r, ph_r, rho_r, kMT, m, q, fused);
  stage_colslot(a, colslot, lane);
  ZStage zst;
  z_issue<P::kStatic>(a, j, lane, zst);
  wave_sync();
  z_commit<ZS>(a, j, Zs, colslot, lane, zst);
  float za[SPLIT ? 1 : NT][4];
  SplitA zs[SPLIT ? NT : 1];
  floatx4 z0[SPLIT ? 1 : NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float zt[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) zt[s] = Zs[(1 + 4 * q + s) * ZS + 16 * nt + m];
    if constexpr (SPLIT) {
      zs[nt] = split_a(zt[0], zt[1], zt[2], zt[3]);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) za[nt][s] = zt[s];
      z0[nt] = *reinterpret_cast<const floatx4*>(Zs + 16 * nt + 4 * q);
    }
  }
  TrunkLane tl{};
  if (fused) tl = trunk_lane(a, m, q);
  for (int tb = 0;;) {
    if constexpr (SPLIT)
      forward_tile_split<NT, P, B16>(a, ta, zs, Zs, Ph, out_r, d_out, tb, m, q);
    else
      forward_tile<NT, P, B16>(a, ta, za, z0, Ph, out_r, d_out, tb, m, q, tl, fused);
    ta = load_fwd<P, B16>(h_r, ph_r, rho_r, tb + 2 * kMT, m, q, fused);
    tb += kMT;
    if (tb >= ng) break;
    if constexpr (SPLIT)
      forward_tile_split<NT, P, B16>(a, tbf, zs, Zs, Ph, out_r, d_out, tb, m, q);
    else
      forward_tile<NT, P, B16>(a, tbf, za, z0, Ph, out_r, d_out, tb, m, q, tl, fused);
    tbf = load_fwd<P, B16>(h_r, ph_r, rho_r, tb + 2 * kMT, m, q, fused);
    tb += kMT;
    if (tb >= ng) break;
  }
}

template <class P>
struct BwdTile {
  floatx4 h;        // h(edge m)[4 q .. 4 q + 3] (read; zero under the fused trunk)
  PhaseRegs<P> ph;  // as in the forward
  float rho, w;     // edge m (rho: runtime slots or the fused trunk)
  int64_t tgt;      // runtime slots: the target of edge m
  floatx4 dh_old;   // accumulating: dh(edge m)[4 q .. 4 q + 3] already in the output
  float dw_old;     // accumulating: dweights(edge m) already in the output
};

template <class P, bool B16 = false>
__device__ __forceinline__ BwdTile<P> load_bwd(__amdgpu_buffer_rsrc_t h_r, __amdgpu_buffer_rsrc_t ph_r,
                                               __amdgpu_buffer_rsrc_t rho_r, __amdgpu_buffer_rsrc_t w_r,
                                               __amdgpu_buffer_rsrc_t t_r, int tb, int m, int q, bool fused,
                                               __amdgpu_buffer_rsrc_t dh_r, __amdgpu_buffer_rsrc_t dw_r, bool acc) {
  BwdTile<P> t;
  const int e = tb + m;
  t.h = fused ? floatx4{0.f, 0.f, 0.f, 0.f} : hload<B16>(h_r, e * 16 + 4 * q);
  if constexpr (P::kStatic) {
    t.ph.ph = bload4(ph_r, e * 16);
    t.tgt = 0;
    t.rho = fused ? bload1(rho_r, e * 4) : 0.f;
  } else {
    t.ph.ph = bload4(ph_r, (e * kPhaseRow + 4 * q) * 4);
    t.tgt = bload_i64(t_r, e * 8);
    t.rho = bload1(rho_r, e * 4);
  }
  t.w = bload1(w_r, e * 4);
  if (acc) {
    t.dh_old = sload4<B16>(dh_r, e * 16 + 4 * q);
    t.dw_old = bload1(dw_r, e * 4);
  } else {
    t.dh_old = floatx4{0.f, 0.f, 0.f, 0.f};
    t.dw_old = 0.f;
  }
  return t;
}

// Static slots: the target gradient's and the row's values of the lane's
// outputs (per output group, loaded at its first slot) for edge m.
template <int NT>
struct OutVals {
  float gr[2 * NT], gi[2 * NT], rr[2 * NT], ri[2 * NT];
};

template <int NT, class P, bool B16 = false>
__device__ __forceinline__ void load_outs(OutVals<NT>& v, const float* grow, __amdgpu_buffer_rsrc_t rows_r, int row,
                                          int q) {
#pragma unroll
  for (int s = 0; s < 2 * NT; ++s) {
    const uint32_t w = P::word(s);
    if (!(w & kSlotActive) || group_start<P>(s) != s) continue;
    if (w & kSlotScalar) {
      const int o = slot_ob(w) + q;
      v.gr[s] = grow[o];
      v.gi[s] = 0.f;
      v.rr[s] = sload1<B16>(rows_r, row + o);
      v.ri[s] = 0.f;
    } else {
      const int o = slot_ob(w) + 2 * q;
      const float2 gv = *reinterpret_cast<const float2*>(grow + o);
      const float2 rv = sload2<B16>(rows_r, row + o);
      v.gr[s] = gv.x;
      v.gi[s] = gv.y;
      v.rr[s] = rv.x;
      v.ri[s] = rv.y;
    }
  }
}

struct BwdSpans {
  __amdgpu_buffer_rsrc_t h, ph, rho, w, t, rows, dh, dw;
};

// One backward tile: 16 edges from tb; dh and dweights stored, dZ
// accumulated in registers.
template <int NT, class P, class O, bool B16 = false>
__device__ __forceinline__ void backward_tile(const FactArgs<float>& a, const BwdTile<P>& cur, const O& outs,
                                              const floatx4 (&zb)[NT], floatx4 (&dz)[NT], float (&dz0)[NT], float* Sh,
                                              float* Ph, float* Gt, int64_t* Tg, float* Hs, const BwdSpans& sp,
                                              int d_out, int ng, int tb, int m, int q, const TrunkLane& tl,
                                              bool fused) {
  const int row = (tb + m) * d_out;
  // edge m's features 4 q .. 4 q + 3 (read as one 16-byte piece, or the fused trunk's),
  // handed to the dZ operand's layout (feature m of edges 4 q + i) through Hs with the
  // W transpose below
  floatx4 pre;
  const floatx4 hf = fused ? trunk_features(a, tl, q, cur.rho, pre) : hwiden<B16>(cur.h);
  *reinterpret_cast<floatx4*>(Hs + m * kHsStride + 4 * q) = hf;
  float wv[NT][4];
  float dwp = 0.f;  // this lane's share of dweights(edge m)
  if constexpr (kHorner<P>) {
    // the weighted gradient values w G of the three outputs (first slots 0, 3, 8)
    float gr[3], gi[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int s = k == 0 ? 0 : (k == 1 ? 3 : 8);
      dwp += outs.gr[s] * outs.rr[s] + outs.gi[s] * outs.ri[s];
      gr[k] = cur.w * outs.gr[s];
      gi[k] = cur.w * outs.gi[s];
    }
    f2_backward_weights(cur.ph.ph, gr, gi, wv);
  } else if constexpr (P::kStatic) {
    const Powers<P> pw = powers<P>(cur.ph.ph);
    // the edge's weighted gradient values w G, once per output group
    float wgr[2 * NT], wgi[2 * NT];
#pragma unroll
    for (int s = 0; s < 2 * NT; ++s) {
      const uint32_t w = P::word(s);
      if ((w & kSlotActive) && group_start<P>(s) == s) {
        dwp += outs.gr[s] * outs.rr[s] + outs.gi[s] * outs.ri[s];
        wgr[s] = cur.w * outs.gr[s];
        wgi[s] = cur.w * outs.gi[s];
      }
    }
#pragma unroll
    for (int s = 0; s < 2 * NT; ++s) {
      const uint32_t w = P::word(s);
      const int b = group_start<P>(s);
      if (!(w & kSlotActive)) {
        wv[s >> 1][2 * (s & 1)] = 0.f;
        wv[s >> 1][2 * (s & 1) + 1] = 0.f;
      } else if (w & kSlotReal) {
        wv[s >> 1][2 * (s & 1)] = wgr[b];
        wv[s >> 1][2 * (s & 1) + 1] = 0.f;
      } else {
        float fr, fi;
        static_factor<P>(pw, s, fr, fi);
        const float gr = wgr[b], gim = (w & kSlotScalar) ? 0.f : wgi[b];
        wv[s >> 1][2 * (s & 1)] = fr * gr + fi * gim;
        wv[s >> 1][2 * (s & 1) + 1] = fr * gim - fi * gr;
      }
    }
  } else {
    // the targets' gradient rows through LDS (zero for absent edges and past d_out)
    const int GS = a.gstride;
    stage_phases_lanes(a, Ph, cur.ph.ph, cur.rho, m, q);
    if (q == 0) Tg[m] = cur.tgt;
    wave_sync();
    for (int e = q; e < kMT; e += 4) {
      const float* grow = tb + e < ng ? a.g + Tg[e] * a.g_ld : nullptr;
      for (int o = m; o < GS; o += kMT) Gt[e * GS + o] = grow && o < d_out ? grow[o] : 0.f;
    }
    wave_sync();
    for (int o = q; o < d_out; o += 4) dwp += Gt[m * GS + o] * sload1<B16>(sp.rows, row + o);
    const float* prow = Ph + m * kPhStride;
    const float* gq1 = Gt + m * GS + q;
    const float* gq2 = Gt + m * GS + 2 * q;
#pragma unroll
    for (int s = 0; s < 2 * NT; ++s) {
      const uint32_t w = a.slot[s];
      float fr, fi;
      runtime_factor(prow, w, fr, fi);
      const float* gp = ((w & kSlotScalar) ? gq1 : gq2) + slot_ob(w);
      const float gr = gp[0], gim = (w & kSlotScalar) ? 0.f : gp[1];
      wv[s >> 1][2 * (s & 1)] = cur.w * (fr * gr + fi * gim);
      wv[s >> 1][2 * (s & 1) + 1] = cur.w * (fr * gim - fi * gr);
    }
  }
  // dweights = <g(target), row>: the four lanes' shares of edge m
  dwp += __shfl_xor(dwp, 16, kWave);
  dwp += __shfl_xor(dwp, 32, kWave);
  bstore1(dwp + cur.dw_old, sp.dw, q == 0 ? (tb + m) * 4 : kDrop);
  // dh(e)_t = sum_c W(e)_c Z_t,c: lane (m, q) ends with edge m's features 4 q .. 4 q + 3
  floatx4 dh = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (kstep_live<P>(a, nt, r)) dh = mfma16(zb[nt][r], wv[nt][r], dh);
  sstore4<B16>(dh + cur.dh_old, sp.dh, (tb + m) * 16 + 4 * q);
  // W through LDS, column-major, for dZ's edge-major operand
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) Sh[(16 * nt + 4 * q + r) * kWtStride + m] = wv[nt][r];
  wave_sync();
  floatx4 hb;
#pragma unroll
  for (int i = 0; i < 4; ++i) hb[i] = Hs[(4 * q + i) * kHsStride + m];
  // dZ_t,c += sum_e h_t(e) W(e)_c over edges 4 q' + i; the t = 0 column sums W
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const floatx4 wt = *reinterpret_cast<const floatx4*>(Sh + (16 * nt + m) * kWtStride + 4 * q);
#pragma unroll
    for (int i = 0; i < 4; ++i) dz[nt] = mfma16(hb[i], wt[i], dz[nt]);
    dz0[nt] += (wt[0] + wt[1]) + (wt[2] + wt[3]);
  }
  wave_sync();
}

// --------------------------------------------------- mixes by direct-to-LDS loads
//
// The lane-owned backward's mixes Z(j), rows t = 1 .. 16 (the only rows it
// reads: dh pairs W with Z_{1..16}, and dZ's row 0 is W's column sum), staged
// by direct-to-LDS buffer loads instead of a load and an LDS write per run,
// row and lane.  The mix runs are merged into the blocks they form in memory
// (each head's rows of one input frequency: (17, width) contiguous per node),
// so a node's mixes are a few 16-byte-per-lane loads; they land in the area
// the W transposes use later, in block layout, and each lane reads its dh
// operands Z_{1+m}(slot columns 16 nt + 4 q + r) through a per-slot-column
// table (block row offset | block width << 16) staged with them.

#ifndef GM_FACT_STREAM_WORDS
#define GM_FACT_STREAM_WORDS (17 * 128 + 4 * 4 + 4)
#endif

// s_waitcnt immediates (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8).  The compiler inserts no wait for the LDS writes of a
// direct-to-LDS load, so its readers wait explicitly.
constexpr unsigned kWaitVm0 = 0x0F70;  // vmcnt(0)

// Node j's mixes, rows zq_t0 .. 16 of every block, into Zq by direct-to-LDS
// loads (lane i of a load writes its 16 bytes at the load's LDS base + 16 i).
__device__ __forceinline__ void z_stream(const FactArgs<float>& a, int64_t j, float* Zq, int lane) {
  const int rows = 17 - a.zq_t0;
  for (int b = 0; b < a.n_zq; ++b) {
    const int n = rows * a.zq_w[b];  // floats of the block's rows
    const auto r = span(a.zq_base[b] + j * a.zq_ns[b] + (int64_t)a.zq_t0 * a.zq_w[b], (int64_t)n * 4);
    for (int u = 0; 256 * u < n; ++u)
      if (64 * u + lane < (n + 3) / 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, Zq + a.zq_loff[b] + 256 * u, 16, (64 * u + lane) * 16, 0, 0, 0);
  }
}

// ACC: dh and dweights added into the outputs (a later share of a head).
// ZDMA (compiled-in slots, trunk read): the mixes by direct-to-LDS loads (z_stream).
// B16 (compiled-in slots, trunk read): h, the rows and dh in bfloat16.
template <int NT, class P, bool FUSED, bool ACC, bool ZDMA = false, bool B16 = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(P::kStatic ? (FUSED || P::kDout > 40 ? 2 : 3) : 1))) void
factored_backward_lanes(FactArgs<float> a) {
  static_assert(!ZDMA || (P::kStatic && !FUSED), "the staged-mix form serves fixed slots with trunk features read");
  static_assert(!B16 || (P::kStatic && !FUSED), "bfloat16 streams serve fixed slots with trunk features read");
  constexpr int ZS = 16 * NT + 4;
  constexpr int kZWords = 17 * ZS, kWWords = 16 * NT * kWtStride;
  __shared__ __align__(16) float Sh[kZWords > kWWords ? kZWords : kWWords];  // Z in, then W's transpose, then dZ out
  __shared__ __align__(16) float Ph[P::kStatic ? 4 : kMT * kPhStride];
  __shared__ __align__(16) float Gt[P::kStatic ? 4 : kMT * (GM_FACT_MAX_OUT + 4)];
  __shared__ __align__(16) uint8_t colslot[128];
  __shared__ int64_t Tg[P::kStatic ? 1 : kMT];
  __shared__ __align__(16) float Hs[kMT * kHsStride];  // the tile's trunk features, edge-major
  __shared__ __align__(16) uint32_t zsl[ZDMA ? 16 * NT : 1];  // ZDMA: where each slot column's rows sit
  const int lane = threadIdx.x, m = lane & 15, q = lane >> 4;
  const int d_out = P::kStatic ? P::kDout : a.d_out;
  const int64_t gi = a.group_order ? a.group_order[blockIdx.x] : xcd_spread_block(blockIdx.x, gridDim.x);
  if (gi < 0 || gi >= a.n_groups) return;  // a malformed order names no group
  const int64_t j = a.group_source[gi];
  const int64_t g0 = a.group_ptr[gi];
  const int ng = (int)(a.group_ptr[gi + 1] - g0);
  constexpr bool fused = FUSED;
  BwdSpans sp;
  // h, the rows and dh: float32, or bfloat16 (B16) at half the bytes
  const char* h_b = reinterpret_cast<const char*>(a.h);
  const char* rows_b = reinterpret_cast<const char*>(a.rows);
  char* dh_b = reinterpret_cast<char*>(a.dh);
  sp.h = span(fused ? nullptr : h_b + stream_bytes<B16>(g0 * 16), fused ? 0 : stream_bytes<B16>((int64_t)ng * 16));
  sp.ph = P::kStatic ? span(a.zw_g + g0 * 4, (int64_t)ng * 16)
                     : span(a.phase_g + g0 * kPhaseRow, (int64_t)ng * kPhaseRow * 4);
  sp.rho = span(a.rho_g + g0, (int64_t)ng * 4);
  sp.w = span(a.weights + g0, (int64_t)ng * 4);
  sp.t = span(a.target_g + g0, (int64_t)ng * 8);
  sp.rows = span(rows_b + stream_bytes<B16>(g0 * d_out), stream_bytes<B16>((int64_t)ng * d_out));
  sp.dh = span(dh_b + stream_bytes<B16>(g0 * 16), stream_bytes<B16>((int64_t)ng * 16));
  sp.dw = span(a.dweights + g0, (int64_t)ng * 4);
  constexpr bool acc = ACC;
  // Two tiles in flight (buffers A and B, each refilled right after its
  // tile's stores); with static slots the targets run three tiles ahead and
  // the targets' gradient values and row values two, so no load is waited
  // for within the tile after the one that issued it.
  // The first tiles' streams and targets are requested with the node's mixes
  // (one round trip), then the targets' gradient values.
  BwdTile<P> ta = load_bwd<P, B16>(sp.h, sp.ph, sp.rho, sp.w, sp.t, 0, m, q, fused, sp.dh, sp.dw, acc);
  BwdTile<P> tbf = load_bwd<P, B16>(sp.h, sp.ph, sp.rho, sp.w, sp.t, kMT, m, q, fused, sp.dh, sp.dw, acc);
  int64_t t0 = 0, t1 = 0;
  if constexpr (P::kStatic) {
    t0 = bload_i64(sp.t, m * 8);
    t1 = bload_i64(sp.t, (kMT + m) * 8);
  }
  stage_colslot(a, colslot, lane);
  ZStage zst;
  if constexpr (ZDMA) {
    z_stream(a, j, Sh, lane);
    for (int i = lane; i < 16 * NT; i += kWave) zsl[i] = a.zq_slot[i];
    if (lane == 0) Sh[a.zq_words] = 0.f;
  } else {
    z_issue<P::kStatic>(a, j, lane, zst);
  }
  OutVals<P::kStatic ? NT : 1> oa, ob;
  int64_t tn = 0;  // static slots: the targets of the tile two ahead of the current one
  if constexpr (P::kStatic) {
    load_outs<NT, P, B16>(oa, a.g + t0 * a.g_ld, sp.rows, m * d_out, q);
    load_outs<NT, P, B16>(ob, a.g + t1 * a.g_ld, sp.rows, (kMT + m) * d_out, q);
    tn = bload_i64(sp.t, (2 * kMT + m) * 8);
  }
  // Z_t(j) for t = 1 + m at the lane's slot columns 16 nt + 4 q + r
  floatx4 zb[NT];
  if constexpr (ZDMA) {
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // the direct-to-LDS loads have landed (the compiler does not track them)
    wave_sync();
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint4 w = *reinterpret_cast<const uint4*>(zsl + 16 * nt + 4 * q);
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) zb[nt][r] = Sh[(ws[r] & 0xFFFFu) + m * (ws[r] >> 16)];
    }
  } else {
    wave_sync();
    z_commit<ZS>(a, j, Sh, colslot, lane, zst);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) zb[nt] = *reinterpret_cast<const floatx4*>(Sh + (1 + m) * ZS + 16 * nt + 4 * q);
  }
  wave_sync();
  floatx4 dz[NT];
  float dz0[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    dz[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    dz0[nt] = 0.f;
  }
  TrunkLane tl{};
  if (fused) tl = trunk_lane(a, m, q);
  for (int tb = 0;;) {
    backward_tile<NT, P, decltype(oa), B16>(a, ta, oa, zb, dz, dz0, Sh, Ph, Gt, Tg, Hs, sp, d_out, ng, tb, m, q, tl,
                                            fused);
    if constexpr (P::kStatic) {
      load_outs<NT, P, B16>(oa, a.g + tn * a.g_ld, sp.rows, (tb + 2 * kMT + m) * d_out, q);
      tn = bload_i64(sp.t, (tb + 3 * kMT + m) * 8);
    }
    ta = load_bwd<P, B16>(sp.h, sp.ph, sp.rho, sp.w, sp.t, tb + 2 * kMT, m, q, fused, sp.dh, sp.dw, acc);
    tb += kMT;
    if (tb >= ng) break;
    backward_tile<NT, P, decltype(ob), B16>(a, tbf, ob, zb, dz, dz0, Sh, Ph, Gt, Tg, Hs, sp, d_out, ng, tb, m, q, tl,
                                            fused);
    if constexpr (P::kStatic) {
      load_outs<NT, P, B16>(ob, a.g + tn * a.g_ld, sp.rows, (tb + 2 * kMT + m) * d_out, q);
      tn = bload_i64(sp.t, (tb + 3 * kMT + m) * 8);
    }
    tbf = load_bwd<P, B16>(sp.h, sp.ph, sp.rho, sp.w, sp.t, tb + 2 * kMT, m, q, fused, sp.dh, sp.dw, acc);
    tb += kMT;
    if (tb >= ng) break;
  }
  // dZ(j) into LDS in slot-column order, then out by runs
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    dz0[nt] += __shfl_xor(dz0[nt], 16, kWave);
    dz0[nt] += __shfl_xor(dz0[nt], 32, kWave);
#pragma unroll
    for (int i = 0; i < 4; ++i) Sh[(1 + 4 * q + i) * ZS + 16 * nt + m] = dz[nt][i];
    if (q == 0) Sh[16 * nt + m] = dz0[nt];
  }
  wave_sync();
  flush_dz_slots<ZS>(a, j, Sh, colslot, lane);
}

// ------------------------------------------------------------------- launch

// The mix runs of a call: the caller's (pointer, node stride, mix stride,
// width) runs, in packed-column order.
template <typename T>
struct Runs {
  const T* const* z;
  T* const* dz;  // null in the forward
  const int64_t* node_stride;
  const int64_t* t_stride;
  const int64_t* width;
  int64_t n;
};

template <typename T>
int prepare(FactArgs<T>& a, const T* h, const Runs<T>& runs, const T* angular, const T* transport, const T* rho,
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
  a.g_ld = d_out;
  a.n_groups = n_groups;
  // Every packed column belongs to exactly one block, and the blocks sharing
  // an output slot are consecutive, alike in width and kind of output.
  int covered_c = 0, covered_r = 0, open = -1;
  bool seen_real = false;
  bool taken[GM_FACT_MAX_C / 2] = {};
  std::string why;
  for (int b = 0; b < n_blocks; ++b) {
    const int32_t* r = desc + b * GM_FACT_DESC;
    for (int k = 0; k < GM_FACT_DESC; ++k) GM_REQUIRE(r[k] >= -32768 && r[k] <= 32767, "descriptor entries must fit 16 bits");
    Block d{(int16_t)r[0], (int16_t)r[1], (int16_t)r[2], (int16_t)r[3], (int16_t)r[4], (int16_t)r[5], (int16_t)r[6],
            (int16_t)r[7]};
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
      a.real_ooff = d.ooff;
    } else {
      GM_REQUIRE(d.zoff >= 0 && d.zoff + d.bm <= wc, "a complex block's columns run past wc");
      for (int u = 0; u < d.bm; ++u) {
        GM_REQUIRE(!taken[d.zoff + u], "two complex blocks share a packed column");
        taken[d.zoff + u] = true;
        a.cmap[d.zoff + u] = (uint8_t)b;
      }
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
  if (a.C <= 128) {
    // the MFMA path's tables: what each packed column reads of an edge's
    // output gradient, and which V columns each output slot sums
    int real_block = -1;
    for (int b = 0; b < n_blocks; ++b)
      if (a.desc[b].kind == 0) real_block = b;
    for (int c = 0; c < a.C; ++c) {
      uint32_t blk, gre, gim = 0xFF, kind;
      if (c < 2 * wc) {
        blk = a.cmap[c >> 1];
        const Block& d = a.desc[blk];
        const int jj = (c >> 1) - d.zoff;
        if (d.take_real) {
          gre = d.ooff + jj;
        } else {
          gre = d.ooff + 2 * jj;
          gim = d.ooff + 2 * jj + 1;
        }
        kind = (c & 1) ? 2 : 1;
      } else {
        blk = (uint32_t)real_block;
        gre = a.real_ooff + (c - 2 * wc);
        kind = 0;
      }
      a.colinfo[c] = blk | (gre << 8) | (gim << 16) | (kind << 24);
    }
    int count = 0;
    for (int o = 0; o < d_out; ++o) {
      a.optr[o] = (uint8_t)count;
      for (int b = 0; b < n_blocks; ++b) {
        const Block& d = a.desc[b];
        const bool scalar = d.kind == 0 || d.take_real;
        const int k = o - d.ooff;
        if (k < 0 || k >= (scalar ? d.bm : 2 * d.bm)) continue;
        const int col = d.kind == 0 ? 2 * wc + d.zoff + k : d.take_real ? 2 * (d.zoff + k) : 2 * (d.zoff + (k >> 1)) + (k & 1);
        GM_REQUIRE(count < 128, "more than 128 output terms");
        a.olist[count++] = (uint8_t)col;
      }
    }
    a.optr[d_out] = (uint8_t)count;
  }
  // the mix runs: in packed-column order, tiling [0, C), none straddling the
  // complex / real boundary at 2 wc
  GM_REQUIRE(runs.n >= 1 && runs.n <= GM_FACT_MAX_SEG, "between 1 and 4 mix runs");
  a.n_seg = (int)runs.n;
  int c0 = 0;
  for (int r = 0; r < a.n_seg; ++r) {
    const int64_t w = runs.width[r];
    GM_REQUIRE(w >= 1 && c0 + w <= a.C, "the mix runs must tile the packed columns");
    GM_REQUIRE(!(c0 < 2 * wc && c0 + w > 2 * wc), "a mix run straddles the complex and real columns");
    GM_REQUIRE(runs.node_stride[r] >= 0 && runs.t_stride[r] >= 0, "mix strides must be non-negative");
    GM_REQUIRE(runs.t_stride[r] <= (int64_t(1) << 30), "mix stride too large");
    a.seg[r] = ZSeg<T>{runs.z[r], runs.dz ? runs.dz[r] : nullptr, runs.node_stride[r], (int)runs.t_stride[r], c0,
                       (int)w};
    if (n_edges > 0) GM_REQUIRE(runs.z[r] != nullptr, "every mix run must be a device pointer");
    c0 += (int)w;
  }
  GM_REQUIRE(c0 == a.C, "the mix runs must tile the packed columns");
  a.h = h;
  a.angular = angular;
  a.transport = transport;
  a.rho = rho;
  a.order = order;
  a.group_ptr = group_ptr;
  a.group_source = group_source;
  if (n_edges > 0) {
    GM_REQUIRE((K == 1 || h) && rho && angular && transport, "the per-edge tables must be device pointers");
    GM_REQUIRE(order && group_ptr && group_source, "order, group_ptr and group_source must be device pointers");
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

// The MFMA kernels serve fp32 plans with at most 16 trunk features and 128
// packed columns (GM_FACTORED_MFMA=0 selects the vector kernels instead).
bool mfma_eligible(const FactArgs<float>& a) {
  static const bool off = [] {
    const char* v = std::getenv("GM_FACTORED_MFMA");
    return v != nullptr && v[0] == '0';
  }();
  return !off && a.K <= 17 && a.C <= 128 && aligned(a.h, 16);
}
template <typename T>
bool mfma_eligible(const FactArgs<T>&) {
  return false;
}

size_t lds_forward_mfma(const FactArgs<float>& a, int NT) {
  return sizeof(int64_t) * kMT + sizeof(Block) * GM_FACT_MAX_BLOCKS +
         sizeof(float) * (size_t)(kMT + kMT * 4 * a.n_f + kMT * a.n_blocks * 2 + kMT * (16 * NT + 1) +
                                  17 * (16 * NT + 4)) +
         (GM_FACT_MAX_OUT + 1) + 128;
}

size_t lds_backward_mfma(const FactArgs<float>& a, int NT) {
  return sizeof(int64_t) * kMT + sizeof(Block) * GM_FACT_MAX_BLOCKS +
         sizeof(float) * (size_t)(2 * kMT + kMT * 4 * a.n_f + kMT * a.n_blocks * 2 + kMT * a.d_out +
                                  kMT * (16 * NT + 1) + kMT * 16 + 17 * (16 * NT + 4));
}

template <int NT>
void launch_mfma_nt(bool forward, const FactArgs<float>& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_groups), block(64);
  if (forward)
    hipLaunchKernelGGL(factored_forward_mfma<NT>, grid, block, lds_forward_mfma(a, NT), stream, a);
  else
    hipLaunchKernelGGL(factored_backward_mfma<NT>, grid, block, lds_backward_mfma(a, NT), stream, a);
}

void launch_mfma(bool forward, const FactArgs<float>& a, hipStream_t stream) {
  switch ((a.C + 15) / 16) {
    case 1: launch_mfma_nt<1>(forward, a, stream); break;
    case 2: launch_mfma_nt<2>(forward, a, stream); break;
    case 3: launch_mfma_nt<3>(forward, a, stream); break;
    case 4: launch_mfma_nt<4>(forward, a, stream); break;
    case 5: launch_mfma_nt<5>(forward, a, stream); break;
    case 6: launch_mfma_nt<6>(forward, a, stream); break;
    case 7: launch_mfma_nt<7>(forward, a, stream); break;
    default: launch_mfma_nt<8>(forward, a, stream); break;
  }
}
template <typename T>
void launch_mfma(bool, const FactArgs<T>&, hipStream_t) {}

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
int factored_forward(const T* h, const Runs<T>& runs, const T* angular, const T* transport, const T* rho,
                     const int32_t* desc, const int64_t* order, const int64_t* group_ptr, const int64_t* group_source,
                     int64_t n_nodes, int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr,
                     int64_t n_f, int64_t n_blocks, int64_t d_out, int64_t max_bm, T* out, hipStream_t stream) {
  FactArgs<T> a;
  const int status = prepare(a, h, runs, angular, transport, rho, desc, order, group_ptr, group_source, n_nodes,
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
  if (mfma_eligible(a)) {
    launch_mfma(true, a, stream);
    return check_launch("factored_forward (mfma)");
  }
  if (a.K == 17)
    launch_forward_k<T, 17>(a, widest, stream);
  else
    launch_forward_k<T, GM_FACT_MAX_K>(a, widest, stream);
  return check_launch("factored_forward");
}

template <typename T>
int factored_aggregate(const T* rows, const T* weights, const int64_t* row_ptr, int64_t n_targets, int64_t n_edges,
                       int64_t d_out, T* out, hipStream_t stream, const int64_t* inv = nullptr) {
  GM_REQUIRE(n_targets >= 0 && n_edges >= 0, "sizes must be non-negative");
  GM_REQUIRE(d_out >= 1 && d_out <= GM_FACT_MAX_OUT, "d_out must be in [1, 128]");
  GM_REQUIRE(n_targets < (int64_t(1) << 31) * kWavesPerBlock, "too many targets for one launch");
  if (n_targets == 0) return GM_OK;
  GM_REQUIRE(row_ptr && out && (n_edges == 0 || (rows && weights)), "rows, weights, row_ptr and out must be device pointers");
  AggArgs<T> a{rows, weights, row_ptr, out, inv, n_targets, (int)d_out, d_out <= 32 ? (int)(kWave / d_out) : 1};
  hipLaunchKernelGGL(aggregate_kernel<T>, dim3((unsigned)blocks_for(n_targets)), dim3(256), 0, stream, a);
  return check_launch("factored_aggregate");
}

template <typename T>
int factored_backward(const T* g, const int64_t* target, const T* weights, const T* rows, const T* h,
                      const Runs<T>& runs, const T* angular, const T* transport, const T* rho, const int32_t* desc,
                      const int64_t* order, const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes,
                      int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f,
                      int64_t n_blocks, int64_t d_out, T* dh, T* dweights, hipStream_t stream) {
  FactArgs<T> a;
  const int status = prepare(a, h, runs, angular, transport, rho, desc, order, group_ptr, group_source, n_nodes,
                             n_edges, n_groups, K, wc, wr, n_f, n_blocks, d_out);
  if (status != GM_OK) return status;
  const bool aggregated = target != nullptr;
  if (n_edges == 0 || n_groups == 0) return GM_OK;
  GM_REQUIRE(g && (K == 1 || dh) && runs.dz, "g, dh and the mix gradients must be device pointers");
  for (int r = 0; r < a.n_seg; ++r) GM_REQUIRE(a.seg[r].dz != nullptr, "every mix gradient run must be a device pointer");
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
  if (mfma_eligible(a)) {
    launch_mfma(false, a, stream);
    return check_launch("factored_backward (mfma)");
  }
  if (a.K == 17)
    launch_backward_k<T, 17>(a, stream);
  else
    launch_backward_k<T, GM_FACT_MAX_K>(a, stream);
  return check_launch("factored_backward");
}

}  // namespace
}  // namespace gm

namespace gm {
namespace {

size_t lds_forward_grouped(const FactArgs<float>& a, int NT) {
  return sizeof(Block) * GM_FACT_MAX_BLOCKS +
         sizeof(float) * (size_t)(kMT * kPhaseRow + kMT + kMT * a.n_blocks * 2 + kMT * (16 * NT + 1)) +
         (GM_FACT_MAX_OUT + 1) + 128;
}

size_t lds_backward_grouped(const FactArgs<float>& a, int NT) {
  return sizeof(int64_t) * kMT + sizeof(Block) * GM_FACT_MAX_BLOCKS +
         sizeof(float) * (size_t)(kMT * kPhaseRow + 2 * kMT + kMT * a.n_blocks * 2 + kMT * a.d_out +
                                  kMT * (16 * NT + 1) + kMT * 16);
}

template <int NT>
void launch_grouped_nt(bool forward, const FactArgs<float>& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_groups), block(64);
  if (forward)
    hipLaunchKernelGGL(factored_forward_grouped<NT>, grid, block, lds_forward_grouped(a, NT), stream, a);
  else
    hipLaunchKernelGGL(factored_backward_grouped<NT>, grid, block, lds_backward_grouped(a, NT), stream, a);
}

// The staged mixes' blocks (FactArgs::zq_*) from row t0 on, for an LDS area of
// `capacity` floats: the runs merged where one continues another in memory
// with the same strides, each block's rows contiguous (its t stride its width)
// and 16-byte aligned at every node (the direct-to-LDS loads move 16 bytes a
// lane), and the per-slot-column table of where each column's rows sit.
// False when the runs do not form such blocks or the rows exceed the area.
bool prepare_zq(FactArgs<float>& a, int t0, int capacity) {
  a.n_zq = 0;
  a.zq_t0 = t0;
  int order[GM_FACT_MAX_SEG];
  for (int r = 0; r < a.n_seg; ++r) order[r] = r;
  std::sort(order, order + a.n_seg, [&](int x, int y) { return a.seg[x].z < a.seg[y].z; });
  int blk_of[GM_FACT_MAX_SEG], off_in[GM_FACT_MAX_SEG];
  int64_t ts[GM_FACT_MAX_SEG];
  for (int i = 0; i < a.n_seg; ++i) {
    const ZSeg<float>& g = a.seg[order[i]];
    const int b = a.n_zq - 1;
    if (b >= 0 && g.z == a.zq_base[b] + a.zq_w[b] && g.node_stride == a.zq_ns[b] && g.t_stride == ts[b]) {
      blk_of[order[i]] = b;
      off_in[order[i]] = a.zq_w[b];
      a.zq_w[b] += g.width;
    } else {
      a.zq_base[a.n_zq] = g.z;
      a.zq_ns[a.n_zq] = g.node_stride;
      ts[a.n_zq] = g.t_stride;
      a.zq_w[a.n_zq] = g.width;
      blk_of[order[i]] = a.n_zq;
      off_in[order[i]] = 0;
      ++a.n_zq;
    }
  }
  int words = 0;
  for (int b = 0; b < a.n_zq; ++b) {
    if (ts[b] != a.zq_w[b]) return false;  // a block's rows are not contiguous
    if (!aligned(a.zq_base[b], 16) || a.zq_ns[b] % 4 != 0 || ((int64_t)t0 * a.zq_w[b]) % 4 != 0) return false;
    a.zq_loff[b] = words;
    words += ((17 - t0) * a.zq_w[b] + 3) / 4 * 4;
  }
  if (words + 1 > capacity) return false;
  a.zq_words = words;
  for (int sc = 0; sc < 128; ++sc) a.zq_slot[sc] = (uint32_t)words;  // padding: the zero word, width 0
  for (int r = 0; r < a.n_seg; ++r)
    for (int c = 0; c < a.seg[r].width; ++c) {
      const int p = a.seg[r].c0 + c, b = blk_of[r];
      for (int sc = 0; sc < 128; ++sc)
        if (a.slotcol[sc] == p) a.zq_slot[sc] = (uint32_t)(a.zq_loff[b] + off_in[r] + c) | (uint32_t)a.zq_w[b] << 16;
    }
  return true;
}

// GM_FACTORED_ZDMA=0: the lane-owned backward stages its mixes by register loads and LDS writes
// (read at every launch, as GM_FACTORED_STATIC is).
inline bool zdma_backward() {
  const char* v = std::getenv("GM_FACTORED_ZDMA");
  return v == nullptr || v[0] != '0';
}

// The lane-owned kernels over bfloat16 streams (compiled-in slots, trunk features read).
template <int NT, class P>
void launch_lanes_b16(bool forward, const FactArgs<float>& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_groups), block(64);
  if (forward) {
    if (split_products())
      hipLaunchKernelGGL((factored_forward_lanes<NT, P, false, true, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((factored_forward_lanes<NT, P, false, false, true>), grid, block, 0, stream, a);
    return;
  }
  constexpr int area = 17 * (16 * NT + 4) > 16 * NT * kWtStride ? 17 * (16 * NT + 4) : 16 * NT * kWtStride;
  FactArgs<float> za = a;
  if (zdma_backward() && prepare_zq(za, 1, area)) {
    if (a.accumulate)
      hipLaunchKernelGGL((factored_backward_lanes<NT, P, false, true, true, true>), grid, block, 0, stream, za);
    else
      hipLaunchKernelGGL((factored_backward_lanes<NT, P, false, false, true, true>), grid, block, 0, stream, za);
  } else if (a.accumulate) {
    hipLaunchKernelGGL((factored_backward_lanes<NT, P, false, true, false, true>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((factored_backward_lanes<NT, P, false, false, false, true>), grid, block, 0, stream, a);
  }
}

template <int NT, class P = RuntimeSlots>
void launch_lanes_nt(bool forward, const FactArgs<float>& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_groups), block(64);
  const bool fused = a.trunk_w != nullptr;  // the trunk evaluated in the kernels: their own instantiation
  if constexpr (P::kStatic) {
    if (a.b16) return launch_lanes_b16<NT, P>(forward, a, stream);
  }
  if (forward) {
    if (fused)
      hipLaunchKernelGGL((factored_forward_lanes<NT, P, true, false>), grid, block, 0, stream, a);
    else if (P::kStatic && split_products())
      hipLaunchKernelGGL((factored_forward_lanes<NT, P, false, P::kStatic>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((factored_forward_lanes<NT, P, false, false>), grid, block, 0, stream, a);
  } else {
    if constexpr (P::kStatic) {
      // the mixes by direct-to-LDS loads into the W-transpose area (16 rows of every block)
      constexpr int area = 17 * (16 * NT + 4) > 16 * NT * kWtStride ? 17 * (16 * NT + 4) : 16 * NT * kWtStride;
      FactArgs<float> za = a;
      if (!fused && zdma_backward() && prepare_zq(za, 1, area)) {
        if (a.accumulate)
          hipLaunchKernelGGL((factored_backward_lanes<NT, P, false, true, true>), grid, block, 0, stream, za);
        else
          hipLaunchKernelGGL((factored_backward_lanes<NT, P, false, false, true>), grid, block, 0, stream, za);
        return;
      }
    }
    if (fused)
      hipLaunchKernelGGL((factored_backward_lanes<NT, P, true, false>), grid, block, 0, stream, a);
    else if (a.accumulate)
      hipLaunchKernelGGL((factored_backward_lanes<NT, P, false, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((factored_backward_lanes<NT, P, false, false>), grid, block, 0, stream, a);
  }
}

// Whether a plan's runtime slot words are P's compile-time ones.
template <class P>
bool matches(const FactArgs<float>& a) {
  if (a.n_slots != P::kSlots || a.d_out != P::kDout || a.pa != P::kPa) return false;
  for (int s = 0; s < a.n_slots; ++s)
    if (a.slot[s] != P::word(s)) return false;
  return true;
}

// Whether a plan's lane slots are one of the compiled-in tables
// (GM_FACTORED_STATIC=0 declines them, read at every launch).
bool fixed_table(const FactArgs<float>& a) {
  const char* env = std::getenv("GM_FACTORED_STATIC");
  return (env == nullptr || env[0] != '0') && a.n_slots > 0 &&
         (matches<SlotsF2>(a) || matches<SlotsF1>(a) || matches<SlotsS16>(a));
}

// Whether the compiled-in slot kernels serve a prepared call (they read the zw rows).
bool fixed_slots(const FactArgs<float>& a) { return a.zw_g != nullptr && fixed_table(a); }

void launch_grouped(bool forward, const FactArgs<float>& a, hipStream_t stream) {
  if (a.n_slots > 0) {
    const char* env = std::getenv("GM_FACTORED_STATIC");
    const bool fixed = (env == nullptr || env[0] != '0') && a.zw_g != nullptr;
    if (fixed && matches<SlotsF2>(a)) return launch_lanes_nt<(SlotsF2::kSlots + 1) / 2, SlotsF2>(forward, a, stream);
    if (fixed && matches<SlotsF1>(a)) return launch_lanes_nt<(SlotsF1::kSlots + 1) / 2, SlotsF1>(forward, a, stream);
    if (fixed && matches<SlotsS16>(a)) return launch_lanes_nt<(SlotsS16::kSlots + 1) / 2, SlotsS16>(forward, a, stream);
    switch ((a.n_slots + 1) / 2) {
      case 1: launch_lanes_nt<1>(forward, a, stream); return;
      case 2: launch_lanes_nt<2>(forward, a, stream); return;
      case 3: launch_lanes_nt<3>(forward, a, stream); return;
      case 4: launch_lanes_nt<4>(forward, a, stream); return;
      case 5: launch_lanes_nt<5>(forward, a, stream); return;
      case 6: launch_lanes_nt<6>(forward, a, stream); return;
      case 7: launch_lanes_nt<7>(forward, a, stream); return;
      default: launch_lanes_nt<8>(forward, a, stream); return;
    }
  }
  switch ((a.C + 15) / 16) {
    case 1: launch_grouped_nt<1>(forward, a, stream); break;
    case 2: launch_grouped_nt<2>(forward, a, stream); break;
    case 3: launch_grouped_nt<3>(forward, a, stream); break;
    case 4: launch_grouped_nt<4>(forward, a, stream); break;
    case 5: launch_grouped_nt<5>(forward, a, stream); break;
    case 6: launch_grouped_nt<6>(forward, a, stream); break;
    case 7: launch_grouped_nt<7>(forward, a, stream); break;
    default: launch_grouped_nt<8>(forward, a, stream); break;
  }
}

// The lane-owned slot tables of a grouped plan, or n_slots = 0 when the plan
// does not fit them (GM_FACTORED_LANES=0 declines every plan): blocks in
// multiplicities of four, radial power equal to the angular order, complex
// outputs at even offsets of an even-width row, at most 16 slots.
void prepare_lanes(FactArgs<float>& a) {
  const char* env = std::getenv("GM_FACTORED_LANES");
  const bool off = env != nullptr && env[0] == '0';
  a.n_slots = 0;
  if (off || a.K != 17 || a.d_out % 2 != 0 || a.pa + a.pt > 8) return;
  uint32_t slot[kMaxSlots] = {};
  uint8_t slotcol[128];
  for (int i = 0; i < 128; ++i) slotcol[i] = 0xFF;
  int n = 0;
  for (int b = 0; b < a.n_blocks;) {
    int e = b + 1;  // the output group: blocks b .. e - 1 share an output offset (consecutive, alike)
    while (e < a.n_blocks && a.desc[e].ooff == a.desc[b].ooff) ++e;
    const Block& d0 = a.desc[b];
    const bool scalar = d0.kind == 0 || d0.take_real;
    if (d0.bm % 4 != 0 || (!scalar && d0.ooff % 2 != 0)) return;
    for (int u = 0; u < d0.bm / 4; ++u)
      for (int k = b; k < e; ++k) {
        const Block& d = a.desc[k];
        if (n >= kMaxSlots) return;
        uint32_t w = kSlotActive | (scalar ? kSlotScalar : 0u) | (uint32_t)(scalar ? d.ooff + 4 * u : d.ooff + 8 * u);
        if (d.kind == 0) {
          w |= kSlotReal | (uint32_t)a.pa << 15;  // angular entry 0 and transport entry pa: both e^{i 0} = 1
        } else {
          const int aa = std::abs(d.ang), ta = std::abs(d.tr);
          if (d.power != aa) return;
          w |= (uint32_t)aa << 11 | (d.ang < 0 ? kSlotAConj : 0u) | (uint32_t)(a.pa + ta) << 15 |
               (d.tr < 0 ? kSlotTConj : 0u);
        }
        if (k == e - 1) w |= kSlotFlush;
        slot[n] = w;
        for (int q = 0; q < 4; ++q) {
          const int sc = 16 * (n / 2) + 4 * q + 2 * (n % 2);
          if (d.kind == 0) {
            slotcol[sc] = (uint8_t)(2 * a.wc + d.zoff + 4 * u + q);
          } else {
            const int cc = d.zoff + 4 * u + q;
            slotcol[sc] = (uint8_t)(2 * cc);
            slotcol[sc + 1] = (uint8_t)(2 * cc + 1);
          }
        }
        ++n;
      }
    b = e;
  }
  if (n == 0) return;
  uint32_t kmask = 0;
  for (int nt = 0; nt < (n + 1) / 2; ++nt)
    for (int r = 0; r < 4; ++r)
      for (int q = 0; q < 4; ++q)
        if (slotcol[16 * nt + 4 * q + r] != 0xFF) kmask |= 1u << (4 * nt + r);
  int gs = a.d_out + 1;
  while (gs % 4 != 2) ++gs;  // G rows 2 (mod 4) floats apart: the 16 rows' reads fall in distinct banks
  for (int i = 0; i < kMaxSlots; ++i) a.slot[i] = slot[i];
  for (int i = 0; i < 128; ++i) a.slotcol[i] = slotcol[i];
  a.kmask = kmask;
  uint8_t colslot[128];
  for (int i = 0; i < 128; ++i) colslot[i] = 0;
  for (int sc = 0; sc < 128; ++sc)
    if (slotcol[sc] != 0xFF) colslot[slotcol[sc]] = (uint8_t)sc;
  for (int i = 0; i < 32; ++i)
    a.colslot32[i] = (uint32_t)colslot[4 * i] | (uint32_t)colslot[4 * i + 1] << 8 | (uint32_t)colslot[4 * i + 2] << 16 |
                     (uint32_t)colslot[4 * i + 3] << 24;
  a.gstride = gs;
  a.n_slots = n;
}

// The grouped path's extra checks: fp32, 16 trunk features, at most 128
// packed columns, both phase tables within one 8-pair row, 16-byte rows.
// The fused trunk's parameters: W1 (16, nb) and b1 (16) device pointers, the
// basis centres (host, nb) and width; trunk_w null leaves h to be read.
struct TrunkParams {
  const float* w;
  const float* b;
  const float* centers;
  int64_t nb;
  double width;
};

int prepare_grouped(FactArgs<float>& a, const float* h, const Runs<float>& runs, const float* phase_g,
                    const float* rho_g, const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source,
                    int64_t n_nodes, int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa,
                    int64_t pt, int64_t n_blocks, int64_t d_out, const TrunkParams& trunk) {
  GM_REQUIRE(pa >= 1 && pt >= 1 && pa + pt <= kPhaseRow / 2, "the grouped phase rows hold at most 8 pairs");
  const bool fused = trunk.w != nullptr;
  // under the fused trunk h is never read: rho_g stands in for prepare's pointer check
  const int status = prepare(a, fused ? rho_g : h, runs, phase_g, phase_g, rho_g, desc, group_ptr /* order unused */,
                             group_ptr, group_source, n_nodes, n_edges, n_groups, K, wc, wr, pa > pt ? pa : pt,
                             n_blocks, d_out);
  if (status != GM_OK) return status;
  a.trunk_w = nullptr;
  a.trunk_b = nullptr;
  a.trunk_nb = 0;
  if (fused) {
    a.h = nullptr;
    GM_REQUIRE(trunk.nb >= 1 && trunk.nb <= 8, "the fused trunk takes 1 to 8 basis functions");
    GM_REQUIRE(trunk.width > 0.0 && trunk.centers != nullptr, "the fused trunk needs its basis centres and width");
    a.trunk_w = trunk.w;
    a.trunk_b = trunk.b;
    a.trunk_nb = (int)trunk.nb;
    a.trunk_inv_width = (float)(1.0 / trunk.width);
    for (int k = 0; k < 8; ++k) a.trunk_c[k] = k < trunk.nb ? trunk.centers[k] : 0.f;
  }
  GM_REQUIRE(K == 17, "the grouped kernels take 16 trunk features (K = 17)");
  GM_REQUIRE(a.C <= 128, "the grouped kernels take at most 128 packed columns");
  for (int b = 0; b < a.n_blocks; ++b) {
    const Block& d = a.desc[b];
    GM_REQUIRE(std::abs(d.ang) < pa && std::abs(d.tr) < pt, "a block's harmonic order exceeds the grouped phase rows");
  }
  if (n_edges > 0) GM_REQUIRE((fused || (h && aligned(h, 16))) && phase_g && aligned(phase_g, 16) && rho_g,
                              "h and the phase rows must be 16-byte aligned device pointers");
  a.phase_g = phase_g;
  a.rho_g = rho_g;
  a.pa = (int)pa;
  a.pt = (int)pt;
  prepare_lanes(a);
  if (fused && n_edges > 0) {
    GM_REQUIRE(a.n_slots > 0, "the fused trunk runs in the lane-owned kernels only; this plan takes the generic ones");
    GM_REQUIRE(trunk.w != nullptr, "trunk_w must be a device pointer");
  }
  return GM_OK;
}

// The reference's zc / zr as two mix runs (an empty one dropped).
template <typename T>
struct TwoRuns {
  const T* z[2];
  T* dz[2];
  int64_t node_stride[2], t_stride[2], width[2];
  int64_t n = 0;
  TwoRuns(const T* zc, const T* zr, T* dzc, T* dzr, int64_t K, int64_t wc, int64_t wr) {
    if (wc > 0) add(zc, dzc, K * 2 * wc, 2 * wc, 2 * wc);
    if (wr > 0) add(zr, dzr, K * wr, wr, wr);
  }
  void add(const T* p, T* dp, int64_t ns, int64_t ts, int64_t w) {
    z[n] = p;
    dz[n] = dp;
    node_stride[n] = ns;
    t_stride[n] = ts;
    width[n] = w;
    ++n;
  }
  Runs<T> runs(bool backward) const { return Runs<T>{z, backward ? dz : nullptr, node_stride, t_stride, width, n}; }
};

}  // namespace
}  // namespace gm

#define GM_FACT_EXPORTS(T, S)                                                                                          \
  extern "C" int gm_factored_forward_##S(const T* h, const T* zc, const T* zr, const T* angular, const T* transport,   \
                                         const T* rho, const int32_t* desc, const int64_t* order,                     \
                                         const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes,      \
                                         int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr,        \
                                         int64_t n_f, int64_t n_blocks, int64_t d_out, int64_t max_bm, T* out,        \
                                         void* stream) {                                                              \
    const gm::TwoRuns<T> two(zc, zr, nullptr, nullptr, K, wc, wr);                                                    \
    return gm::factored_forward<T>(h, two.runs(false), angular, transport, rho, desc, order, group_ptr, group_source, \
                                   n_nodes, n_edges, n_groups, K, wc, wr, n_f, n_blocks, d_out, max_bm, out,          \
                                   (hipStream_t)stream);                                                              \
  }                                                                                                                   \
  extern "C" int gm_factored_forward_seg_##S(                                                                         \
      const T* h, const T* const* z, const int64_t* node_stride, const int64_t* t_stride, const int64_t* width,       \
      int64_t n_runs, const T* angular, const T* transport, const T* rho, const int32_t* desc, const int64_t* order,  \
      const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes, int64_t n_edges, int64_t n_groups,      \
      int64_t K, int64_t wc, int64_t wr, int64_t n_f, int64_t n_blocks, int64_t d_out, int64_t max_bm, T* out,        \
      void* stream) {                                                                                                 \
    GM_REQUIRE(z && node_stride && t_stride && width, "the mix runs must be host arrays");                           \
    const gm::Runs<T> runs{z, nullptr, node_stride, t_stride, width, n_runs};                                         \
    return gm::factored_forward<T>(h, runs, angular, transport, rho, desc, order, group_ptr, group_source, n_nodes,   \
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
    const gm::TwoRuns<T> two(zc, zr, dzc, dzr, K, wc, wr);                                                            \
    return gm::factored_backward<T>(g, target, weights, rows, h, two.runs(true), angular, transport, rho, desc,       \
                                    order, group_ptr, group_source, n_nodes, n_edges, n_groups, K, wc, wr, n_f,       \
                                    n_blocks, d_out, dh, dweights, (hipStream_t)stream);                              \
  }                                                                                                                   \
  extern "C" int gm_factored_backward_seg_##S(                                                                        \
      const T* g, const int64_t* target, const T* weights, const T* rows, const T* h, const T* const* z,             \
      T* const* dz, const int64_t* node_stride, const int64_t* t_stride, const int64_t* width, int64_t n_runs,        \
      const T* angular, const T* transport, const T* rho, const int32_t* desc, const int64_t* order,                  \
      const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes, int64_t n_edges, int64_t n_groups,      \
      int64_t K, int64_t wc, int64_t wr, int64_t n_f, int64_t n_blocks, int64_t d_out, T* dh, T* dweights,            \
      void* stream) {                                                                                                 \
    GM_REQUIRE(z && dz && node_stride && t_stride && width, "the mix runs must be host arrays");                     \
    const gm::Runs<T> runs{z, dz, node_stride, t_stride, width, n_runs};                                              \
    return gm::factored_backward<T>(g, target, weights, rows, h, runs, angular, transport, rho, desc, order,          \
                                    group_ptr, group_source, n_nodes, n_edges, n_groups, K, wc, wr, n_f, n_blocks,    \
                                    d_out, dh, dweights, (hipStream_t)stream);                                        \
  }

GM_FACT_EXPORTS(float, f32)
GM_FACT_EXPORTS(double, f64)

namespace gm {
namespace {

// The grouped forward; b16: h_g and rows_g hold bfloat16 (compiled-in lane slots only).
int forward_grouped(bool b16, const float* h_g, const float* const* z, const int64_t* node_stride,
                    const int64_t* t_stride, const int64_t* width, int64_t n_runs, const float* phase_g,
                    const float* rho_g, const float* zw_g, const int32_t* desc, const int64_t* group_ptr,
                    const int64_t* group_source, const int64_t* group_order, int64_t n_nodes, int64_t n_edges,
                    int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt, int64_t n_blocks,
                    int64_t d_out, const float* trunk_w, const float* trunk_b, const float* trunk_centers,
                    int64_t trunk_nb, double trunk_width, float* rows_g, void* stream) {
  GM_REQUIRE(z && node_stride && t_stride && width, "the mix runs must be host arrays");
  GM_REQUIRE(!(b16 && trunk_w), "bfloat16 streams read the trunk features (no fused trunk)");
  const gm::Runs<float> runs{z, nullptr, node_stride, t_stride, width, n_runs};
  gm::FactArgs<float> a;
  const gm::TrunkParams trunk{trunk_w, trunk_b, trunk_centers, trunk_nb, trunk_width};
  const int status = gm::prepare_grouped(a, h_g, runs, phase_g, rho_g, desc, group_ptr, group_source, n_nodes, n_edges,
                                         n_groups, K, wc, wr, pa, pt, n_blocks, d_out, trunk);
  if (status != GM_OK) return status;
  if (n_edges == 0 || n_groups == 0) return GM_OK;
  GM_REQUIRE(rows_g, "rows must be a device pointer");
  a.out = rows_g;
  a.group_order = group_order;
  GM_REQUIRE(zw_g == nullptr || gm::aligned(zw_g, 16), "zw_g must be a 16-byte aligned device pointer (or null)");
  a.zw_g = zw_g;
  a.b16 = b16;
  if (b16) GM_REQUIRE(fixed_slots(a), "bfloat16 streams take plans with compiled-in lane slots (gm_factored_lanes_fixed)");
  gm::launch_grouped(true, a, (hipStream_t)stream);
  return gm::check_launch("factored_forward_grouped");
}

// The grouped backward; b16: rows_g, h_g and dh_g hold bfloat16 (compiled-in lane slots only).
int backward_grouped(bool b16, const float* g, int64_t g_ld, const int64_t* target_g, const float* weights_g,
                     const float* rows_g, const float* h_g, const float* const* z, float* const* dz,
                     const int64_t* node_stride, const int64_t* t_stride, const int64_t* width, int64_t n_runs,
                     const float* phase_g, const float* rho_g, const float* zw_g, const int32_t* desc,
                     const int64_t* group_ptr, const int64_t* group_source, const int64_t* group_order, int64_t n_nodes,
                     int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt,
                     int64_t n_blocks, int64_t d_out, const float* trunk_w, const float* trunk_b,
                     const float* trunk_centers, int64_t trunk_nb, double trunk_width, int64_t accumulate, float* dh_g,
                     float* dweights_g, void* stream) {
  GM_REQUIRE(z && dz && node_stride && t_stride && width, "the mix runs must be host arrays");
  GM_REQUIRE(!(b16 && trunk_w), "bfloat16 streams read the trunk features (no fused trunk)");
  GM_REQUIRE(g_ld >= d_out, "g_ld must be at least d_out");
  GM_REQUIRE(g_ld == d_out || (g_ld % 2 == 0 && gm::aligned(g, 8)),
             "strided gradient rows need an even row stride and 8-byte aligned rows");
  const gm::Runs<float> runs{z, dz, node_stride, t_stride, width, n_runs};
  gm::FactArgs<float> a;
  const gm::TrunkParams trunk{trunk_w, trunk_b, trunk_centers, trunk_nb, trunk_width};
  const int status = gm::prepare_grouped(a, h_g, runs, phase_g, rho_g, desc, group_ptr, group_source, n_nodes, n_edges,
                                         n_groups, K, wc, wr, pa, pt, n_blocks, d_out, trunk);
  if (status != GM_OK) return status;
  if (n_edges == 0 || n_groups == 0) return GM_OK;
  GM_REQUIRE(g && target_g && weights_g && rows_g && dh_g && dweights_g,
             "g, target_g, weights_g, rows_g, dh_g and dweights_g must be device pointers");
  for (int r = 0; r < a.n_seg; ++r) GM_REQUIRE(a.seg[r].dz != nullptr, "every mix gradient run must be a device pointer");
  a.g = g;
  a.g_ld = g_ld;
  a.group_order = group_order;
  GM_REQUIRE(zw_g == nullptr || gm::aligned(zw_g, 16), "zw_g must be a 16-byte aligned device pointer (or null)");
  a.zw_g = zw_g;
  a.target_g = target_g;
  a.weights = weights_g;
  a.rows = rows_g;
  a.dh = dh_g;
  a.dweights = dweights_g;
  a.accumulate = accumulate != 0;
  GM_REQUIRE(!(a.accumulate && trunk_w), "the fused trunk's backward writes dh_g and dweights_g (no accumulate)");
  a.b16 = b16;
  if (b16) GM_REQUIRE(fixed_slots(a), "bfloat16 streams take plans with compiled-in lane slots (gm_factored_lanes_fixed)");
  gm::launch_grouped(false, a, (hipStream_t)stream);
  return gm::check_launch("factored_backward_grouped");
}

}  // namespace
}  // namespace gm

extern "C" int gm_factored_forward_grouped_f32(
    const float* h_g, const float* const* z, const int64_t* node_stride, const int64_t* t_stride,
    const int64_t* width, int64_t n_runs, const float* phase_g, const float* rho_g, const float* zw_g,
    const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source, const int64_t* group_order,
    int64_t n_nodes, int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt,
    int64_t n_blocks, int64_t d_out, const float* trunk_w, const float* trunk_b, const float* trunk_centers,
    int64_t trunk_nb, double trunk_width, float* rows_g, void* stream) {
  return gm::forward_grouped(false, h_g, z, node_stride, t_stride, width, n_runs, phase_g, rho_g, zw_g, desc,
                             group_ptr, group_source, group_order, n_nodes, n_edges, n_groups, K, wc, wr, pa, pt,
                             n_blocks, d_out, trunk_w, trunk_b, trunk_centers, trunk_nb, trunk_width, rows_g, stream);
}

extern "C" int gm_factored_forward_grouped_bf16(
    const uint16_t* h_g, const float* const* z, const int64_t* node_stride, const int64_t* t_stride,
    const int64_t* width, int64_t n_runs, const float* phase_g, const float* rho_g, const float* zw_g,
    const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source, const int64_t* group_order,
    int64_t n_nodes, int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt,
    int64_t n_blocks, int64_t d_out, uint16_t* rows_g, void* stream) {
  return gm::forward_grouped(true, reinterpret_cast<const float*>(h_g), z, node_stride, t_stride, width, n_runs,
                             phase_g, rho_g, zw_g, desc, group_ptr, group_source, group_order, n_nodes, n_edges,
                             n_groups, K, wc, wr, pa, pt, n_blocks, d_out, nullptr, nullptr, nullptr, 0, 0.0,
                             reinterpret_cast<float*>(rows_g), stream);
}

extern "C" int gm_factored_backward_grouped_ld_f32(
    const float* g, int64_t g_ld, const int64_t* target_g, const float* weights_g, const float* rows_g,
    const float* h_g, const float* const* z, float* const* dz, const int64_t* node_stride, const int64_t* t_stride,
    const int64_t* width, int64_t n_runs, const float* phase_g, const float* rho_g, const float* zw_g,
    const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source, const int64_t* group_order,
    int64_t n_nodes, int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt,
    int64_t n_blocks, int64_t d_out, const float* trunk_w, const float* trunk_b, const float* trunk_centers,
    int64_t trunk_nb, double trunk_width, int64_t accumulate, float* dh_g, float* dweights_g, void* stream) {
  return gm::backward_grouped(false, g, g_ld, target_g, weights_g, rows_g, h_g, z, dz, node_stride, t_stride, width,
                              n_runs, phase_g, rho_g, zw_g, desc, group_ptr, group_source, group_order, n_nodes,
                              n_edges, n_groups, K, wc, wr, pa, pt, n_blocks, d_out, trunk_w, trunk_b, trunk_centers,
                              trunk_nb, trunk_width, accumulate, dh_g, dweights_g, stream);
}

extern "C" int gm_factored_backward_grouped_ld_bf16(
    const float* g, int64_t g_ld, const int64_t* target_g, const float* weights_g, const uint16_t* rows_g,
    const uint16_t* h_g, const float* const* z, float* const* dz, const int64_t* node_stride, const int64_t* t_stride,
    const int64_t* width, int64_t n_runs, const float* phase_g, const float* rho_g, const float* zw_g,
    const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source, const int64_t* group_order,
    int64_t n_nodes, int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt,
    int64_t n_blocks, int64_t d_out, int64_t accumulate, uint16_t* dh_g, float* dweights_g, void* stream) {
  return gm::backward_grouped(true, g, g_ld, target_g, weights_g, reinterpret_cast<const float*>(rows_g),
                              reinterpret_cast<const float*>(h_g), z, dz, node_stride, t_stride, width, n_runs,
                              phase_g, rho_g, zw_g, desc, group_ptr, group_source, group_order, n_nodes, n_edges,
                              n_groups, K, wc, wr, pa, pt, n_blocks, d_out, nullptr, nullptr, nullptr, 0, 0.0,
                              accumulate, reinterpret_cast<float*>(dh_g), dweights_g, stream);
}

extern "C" int gm_factored_backward_grouped_f32(
    const float* g, const int64_t* target_g, const float* weights_g, const float* rows_g, const float* h_g,
    const float* const* z, float* const* dz, const int64_t* node_stride, const int64_t* t_stride,
    const int64_t* width, int64_t n_runs, const float* phase_g, const float* rho_g, const float* zw_g,
    const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source, const int64_t* group_order,
    int64_t n_nodes, int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt,
    int64_t n_blocks, int64_t d_out, const float* trunk_w, const float* trunk_b, const float* trunk_centers,
    int64_t trunk_nb, double trunk_width, int64_t accumulate, float* dh_g, float* dweights_g, void* stream) {
  return gm_factored_backward_grouped_ld_f32(g, d_out, target_g, weights_g, rows_g, h_g, z, dz, node_stride, t_stride,
                                             width, n_runs, phase_g, rho_g, zw_g, desc, group_ptr, group_source,
                                             group_order, n_nodes, n_edges, n_groups, K, wc, wr, pa, pt, n_blocks,
                                             d_out, trunk_w, trunk_b, trunk_centers, trunk_nb, trunk_width, accumulate,
                                             dh_g, dweights_g, stream);
}

extern "C" int gm_factored_aggregate_gather_f32(const float* rows, const int64_t* inv, const float* weights,
                                                const int64_t* row_ptr, int64_t n_targets, int64_t n_edges,
                                                int64_t d_out, float* out, void* stream) {
  GM_REQUIRE(n_edges == 0 || inv, "inv must be a device pointer");
  return gm::factored_aggregate<float>(rows, weights, row_ptr, n_targets, n_edges, d_out, out, (hipStream_t)stream,
                                       inv);
}

namespace gm {
namespace {

// A plan's lane tables; fixed (optional): whether compiled-in slot kernels serve it.
int lane_tables(const int32_t* desc, int64_t n_blocks, int64_t wc, int64_t wr, int64_t d_out, int64_t pa, int64_t pt,
                int32_t* n_slots, uint32_t* slot, uint8_t* slotcol, int32_t* fixed) {
  GM_REQUIRE(n_slots != nullptr, "n_slots must be a host pointer");
  GM_REQUIRE(pa >= 1 && pt >= 1 && pa + pt <= gm::kPhaseRow / 2, "the grouped phase rows hold at most 8 pairs");
  gm::FactArgs<float> a;
  // the two runs of zc / zr (no memory behind them: nothing is read)
  const float* z[2] = {nullptr, nullptr};
  const int64_t zero[2] = {0, 0};
  int64_t width[2] = {2 * wc, wr}, n_runs = 2;
  if (wc == 0 || wr == 0) {
    width[0] = 2 * wc + wr;
    n_runs = 1;
  }
  const gm::Runs<float> runs{z, nullptr, zero, zero, width, n_runs};
  const float* none = nullptr;
  const int status = gm::prepare<float>(a, none, runs, none, none, none, desc, nullptr, nullptr, nullptr, 0, 0, 0, 17,
                                        wc, wr, pa > pt ? pa : pt, n_blocks, d_out);
  if (status != GM_OK) return status;
  for (int b = 0; b < a.n_blocks; ++b)
    GM_REQUIRE(std::abs(a.desc[b].ang) < pa && std::abs(a.desc[b].tr) < pt,
               "a block's harmonic order exceeds the grouped phase rows");
  a.pa = (int)pa;
  a.pt = (int)pt;
  gm::prepare_lanes(a);
  *n_slots = a.n_slots;
  if (slot)
    for (int i = 0; i < gm::kMaxSlots; ++i) slot[i] = a.n_slots ? a.slot[i] : 0u;
  if (slotcol)
    for (int i = 0; i < 128; ++i) slotcol[i] = a.n_slots ? a.slotcol[i] : (uint8_t)0xFF;
  if (fixed) *fixed = gm::fixed_table(a) ? 1 : 0;
  return GM_OK;
}

}  // namespace
}  // namespace gm

extern "C" int gm_factored_lane_tables(const int32_t* desc, int64_t n_blocks, int64_t wc, int64_t wr, int64_t d_out,
                                       int64_t pa, int64_t pt, int32_t* n_slots, uint32_t* slot, uint8_t* slotcol) {
  return gm::lane_tables(desc, n_blocks, wc, wr, d_out, pa, pt, n_slots, slot, slotcol, nullptr);
}

extern "C" int gm_factored_lanes_fixed(const int32_t* desc, int64_t n_blocks, int64_t wc, int64_t wr, int64_t d_out,
                                       int64_t pa, int64_t pt, int32_t* fixed) {
  GM_REQUIRE(fixed != nullptr, "fixed must be a host pointer");
  int32_t n_slots = 0;
  return gm::lane_tables(desc, n_blocks, wc, wr, d_out, pa, pt, &n_slots, nullptr, nullptr, fixed);
}

namespace gm {
namespace {

// rows float32, or bfloat16 (b16: the 16-byte-piece kernels only, as 8-byte pieces)
int aggregate_heads(bool b16, const float* rows, const int64_t* inv, const float* alpha, const int64_t* row_ptr,
                    int64_t n_targets, int64_t n_edges, int64_t H, int64_t d_out, int64_t split, float* out,
                    void* stream) {
  GM_REQUIRE(n_targets >= 0 && n_edges >= 0, "sizes must be non-negative");
  GM_REQUIRE(H >= 1 && d_out >= 1 && H * d_out <= 64 * gm::kAggScalar, "H d_out must be in [1, 1024]");
  GM_REQUIRE(split >= 1 && H % split == 0, "split must divide H");
  GM_REQUIRE(n_targets < (int64_t(1) << 31) * gm::kWavesPerBlock, "too many targets for one launch");
  if (n_targets == 0) return GM_OK;
  GM_REQUIRE(row_ptr && out && (n_edges == 0 || (rows && inv && alpha)),
             "rows, inv, alpha, row_ptr and out must be device pointers");
  const gm::AggHeadsArgs a{rows, alpha, inv, row_ptr, out, n_targets, n_edges, (int)H, (int)d_out, (int)split};
  const dim3 grid((unsigned)gm::blocks_for(n_targets)), block(256);
  const int64_t pieces = d_out % 4 == 0 ? H * d_out / 4 : 0;
  const bool vec = pieces > 0 && pieces <= 64 * 4 && gm::aligned(rows, b16 ? 8 : 16) && gm::aligned(out, 16);
  if (b16) {
    GM_REQUIRE(vec, "bfloat16 rows take d_out a multiple of 4, H d_out <= 1024, 8-byte aligned rows and 16-byte aligned out");
    if (pieces <= 64)
      hipLaunchKernelGGL((gm::aggregate_heads_vec_kernel<1, true>), grid, block, 0, (hipStream_t)stream, a);
    else if (pieces <= 128)
      hipLaunchKernelGGL((gm::aggregate_heads_vec_kernel<2, true>), grid, block, 0, (hipStream_t)stream, a);
    else if (pieces <= 192)
      hipLaunchKernelGGL((gm::aggregate_heads_vec_kernel<3, true>), grid, block, 0, (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL((gm::aggregate_heads_vec_kernel<4, true>), grid, block, 0, (hipStream_t)stream, a);
    return gm::check_launch("factored_aggregate_heads");
  }
  if (vec && pieces <= 64)
    hipLaunchKernelGGL(gm::aggregate_heads_vec_kernel<1>, grid, block, 0, (hipStream_t)stream, a);
  else if (vec && pieces <= 128)
    hipLaunchKernelGGL(gm::aggregate_heads_vec_kernel<2>, grid, block, 0, (hipStream_t)stream, a);
  else if (vec && pieces <= 192)
    hipLaunchKernelGGL(gm::aggregate_heads_vec_kernel<3>, grid, block, 0, (hipStream_t)stream, a);
  else if (vec)
    hipLaunchKernelGGL(gm::aggregate_heads_vec_kernel<4>, grid, block, 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(gm::aggregate_heads_kernel, grid, block, 0, (hipStream_t)stream, a);
  return gm::check_launch("factored_aggregate_heads");
}

}  // namespace
}  // namespace gm

extern "C" int gm_factored_aggregate_heads_f32(const float* rows, const int64_t* inv, const float* alpha,
                                               const int64_t* row_ptr, int64_t n_targets, int64_t n_edges, int64_t H,
                                               int64_t d_out, int64_t split, float* out, void* stream) {
  return gm::aggregate_heads(false, rows, inv, alpha, row_ptr, n_targets, n_edges, H, d_out, split, out, stream);
}

extern "C" int gm_factored_aggregate_heads_bf16(const uint16_t* rows, const int64_t* inv, const float* alpha,
                                                const int64_t* row_ptr, int64_t n_targets, int64_t n_edges, int64_t H,
                                                int64_t d_out, int64_t split, float* out, void* stream) {
  return gm::aggregate_heads(true, reinterpret_cast<const float*>(rows), inv, alpha, row_ptr, n_targets, n_edges, H,
                             d_out, split, out, stream);
}

extern "C" int gm_gather_transpose_f32(const float* src, const int64_t* perm, int64_t n, int64_t width, float* dst_t,
                                       void* stream) {
  GM_REQUIRE(n >= 0 && width >= 1 && width <= 64, "n must be non-negative and width in [1, 64]");
  if (n == 0) return GM_OK;
  GM_REQUIRE(src && perm && dst_t, "src, perm and dst_t must be device pointers");
  GM_REQUIRE(n < (int64_t(1) << 31) * 256, "too many rows for one launch");
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  const bool vec = gm::aligned(src, 16);
  if (vec && width == 8)
    hipLaunchKernelGGL(gm::gather_transpose_kernel<2>, grid, block, 0, (hipStream_t)stream, src, perm, n, (int)width,
                       dst_t);
  else if (vec && width == 4)
    hipLaunchKernelGGL(gm::gather_transpose_kernel<1>, grid, block, 0, (hipStream_t)stream, src, perm, n, (int)width,
                       dst_t);
  else
    hipLaunchKernelGGL(gm::gather_transpose_kernel<0>, grid, block, 0, (hipStream_t)stream, src, perm, n, (int)width,
                       dst_t);
  return gm::check_launch("gather_transpose");
}

extern "C" int gm_scatter_transpose_f32(const float* src_t, const int64_t* perm, int64_t n, int64_t width, float* dst,
                                        void* stream) {
  GM_REQUIRE(n >= 0 && width >= 1 && width <= 64, "n must be non-negative and width in [1, 64]");
  if (n == 0) return GM_OK;
  GM_REQUIRE(src_t && perm && dst, "src_t, perm and dst must be device pointers");
  GM_REQUIRE(n < (int64_t(1) << 31) * 256, "too many rows for one launch");
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  const bool vec = gm::aligned(dst, 16);
  if (vec && width == 8)
    hipLaunchKernelGGL(gm::scatter_transpose_kernel<2>, grid, block, 0, (hipStream_t)stream, src_t, perm, n,
                       (int)width, dst);
  else if (vec && width == 4)
    hipLaunchKernelGGL(gm::scatter_transpose_kernel<1>, grid, block, 0, (hipStream_t)stream, src_t, perm, n,
                       (int)width, dst);
  else
    hipLaunchKernelGGL(gm::scatter_transpose_kernel<0>, grid, block, 0, (hipStream_t)stream, src_t, perm, n,
                       (int)width, dst);
  return gm::check_launch("scatter_transpose");
}
