// Scores and neighbourhood softmax over CSR neighbour lists, forward and
// backward, for CDNA4 (gfx950).
//
// Per edge e = (i <- j) and head h:
//   s[e,h]  = scale * sum_n Re< q_i,n,h , tau_n(e) k_j,n,h > + bias[e]
//   alpha   = softmax of s over i's edges with inside[e] != 0 (others 0)
// and, from d alpha, ds = scale * alpha * (d alpha - sum_e alpha d alpha),
// dq_i = sum_e ds tau k_j, dk_j = sum_{e: source j} ds conj(tau) q_i.
// (The math contract of the reference's fused/attention.h:4-39, 145-165,
// 236-247, 295-348.)
//
// Mapping: one wavefront per target node; its 64 lanes are (edge slot s,
// head h) with S = 64 / H slots, so a lane scores its head on every S-th edge
// of the neighbourhood, holding its head's query columns in registers, and
// the 8 lanes of one edge read that edge's key row as contiguous 16-byte
// pieces.  The forward takes the eager softmax's steps (the scores and their
// maximum, the sum of exponentials, the quotients), each reduced across the
// slots of a head with lane shuffles; a lane's first scores stay in registers
// (alpha written once), scores past them park in alpha and are read back.
// The backward is two passes: per target (the adjoint's per-head total, ds,
// and dq) and per source over the edges grouped by source (dk), so no atomics
// are used and the result is deterministic; ds is written to its edge's place
// in the source grouping and the per-source pass reads ds, the targets and the
// transport rows as streams.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "layout.hpp"

namespace gm {
namespace {

template <typename T>
struct SmArgs {
  const T* q;
  const T* k;
  const uint16_t* qb;  // bfloat16 rows (the bf16 entry points; T = float): read in place of q and k
  const uint16_t* kb;
  const T* transport;  // (n_edges, orders, 2)
  const T* bias;
  const uint8_t* inside;
  const int64_t* row_ptr;
  const int64_t* source;
  const T* alpha_in;  // backward: the forward's alpha
  const T* dalpha;
  T* alpha;
  T* ds;  // (n_edges, H) workspace
  T* dq;
  T* dk;
  const int64_t* src_ptr;
  const int64_t* src_order;
  const int32_t* target_s;  // each edge's target, in the source grouping's order
  const int32_t* inv;       // each edge's place in the source grouping
  const T* transport_s;     // the transport rows in the source grouping's order
  int64_t n_nodes;
  int D, orders, H, S, hshift;  // hshift = log2(H) on the fast path
  T scale;
  AttnLayout L;
  Chunks C;
};

// ---------------------------------------------------------------- fast path
// Every head segment is whole chunks of four reals; H in {1, 2, 4, 8, 16}.

template <typename T>
__device__ __forceinline__ T chunk_dot(const T* q4, const Quad<T>& k, int n, const T* tr) {
  if (n == 0) return q4[0] * k.v[0] + q4[1] * k.v[1] + q4[2] * k.v[2] + q4[3] * k.v[3];
  const T c = tr[2 * n], s = tr[2 * n + 1];
  // tau k = (c k0 - s k1, c k1 + s k0) per pair, dotted with q's pair.
  T acc = q4[0] * (c * k.v[0] - s * k.v[1]) + q4[1] * (c * k.v[1] + s * k.v[0]);
  acc += q4[2] * (c * k.v[2] - s * k.v[3]) + q4[3] * (c * k.v[3] + s * k.v[2]);
  return acc;
}

// The edges of one lane go in steps of kSmStep edges, each step's row gathers
// issued together after the next step's ids were requested.  One edge a step
// measured fastest at NS (backward 8.0 -> 7.4 ms against two or four a step):
// the kernels are bound by L2 gathers of the rows, and fewer registers buy
// more waves a SIMD than a wider step buys gathers in flight.
constexpr int kSmStep = 1;

template <typename T>
__device__ __forceinline__ T chunk_dot_pair(const T* q4, const Quad<T>& k, int n, T c, T s) {
  if (n == 0) return q4[0] * k.v[0] + q4[1] * k.v[1] + q4[2] * k.v[2] + q4[3] * k.v[3];
  T acc = q4[0] * (c * k.v[0] - s * k.v[1]) + q4[1] * (c * k.v[1] + s * k.v[0]);
  acc += q4[2] * (c * k.v[2] - s * k.v[3]) + q4[3] * (c * k.v[3] + s * k.v[2]);
  return acc;
}

// Chunk c's frequency: compile-time when the plan's orders are packed in ORD
// (four bits a chunk, ORD != 0), else the descriptor's.
template <uint32_t ORD>
__device__ __forceinline__ int chunk_order(const Chunks& C, int c) {
  if constexpr (ORD != 0)
    return (int)((ORD >> (4 * c)) & 15u);
  else
    return C.order[c];
}

constexpr int max_order_of(uint32_t ord) {
  int m = 0;
  for (int c = 0; c < 8; ++c)
    if ((int)((ord >> (4 * c)) & 15u) > m) m = (int)((ord >> (4 * c)) & 15u);
  return m;
}

__device__ __forceinline__ void ld_pair(const float* p, float& x, float& y) {
  const float2 v = *reinterpret_cast<const float2*>(p);
  x = v.x;
  y = v.y;
}
__device__ __forceinline__ void ld_pair(const double* p, double& x, double& y) {
  const double2 v = *reinterpret_cast<const double2*>(p);
  x = v.x;
  y = v.y;
}

// The transport (cos, sin) each chunk of one edge reads.  With compile-time
// orders every order's pair is one 8-byte (16-byte) load and order 0 loads
// nothing; otherwise one pair per chunk from the descriptor.
template <typename T, int NCH, uint32_t ORD>
__device__ __forceinline__ void transport_pairs(const Chunks& C, const T* tr, T (&tc)[NCH], T (&ts)[NCH]) {
  if constexpr (ORD != 0) {
    constexpr int MO = max_order_of(ORD);
    T cs[MO + 1], sn[MO + 1];
    cs[0] = T(1);
    sn[0] = T(0);
#pragma unroll
    for (int o = 1; o <= MO; ++o) ld_pair(tr + 2 * o, cs[o], sn[o]);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      tc[c] = cs[chunk_order<ORD>(C, c)];
      ts[c] = sn[chunk_order<ORD>(C, c)];
    }
  } else {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      tc[c] = tr[2 * C.order[c]];
      ts[c] = tr[2 * C.order[c] + 1];
    }
  }
}

// The chunk orders of heads with four copies of frequencies 0, 1 and 2 (one
// scalar chunk, two chunks each of frequencies 1 and 2), compiled in.
constexpr uint32_t kOrders012 = 0x22110u;

// Scores a lane keeps in registers: rows of up to S * kSmRegs edges (128 at
// eight heads) are normalised from registers, so alpha is written once; the
// edges past that park their raw score in alpha and are read back for the sum
// and for the quotient.
constexpr int kSmRegs = 16;
// Parked scores a lane reads back per batch (their loads in flight together).
constexpr int kSmTail = 8;
// Steps of the batched per-source pass whose rows are requested together.
constexpr int kSrcPair = 2;
constexpr bool kSmPrefetch = true;  // next step's source ids requested before this step's rows are used
// Edges a lane of the per-target backward keeps alpha and dalpha of in registers (a multiple of 4).
constexpr int kSmBwdRegs = 8;

// One step's gathers for kSmStep edges of a lane: the chunks of the gathered
// (key or query) rows and the transport pairs.
template <typename T, int NCH>
struct Gather {
  Quad<T> row[kSmStep][NCH];
  T tc[kSmStep][NCH], ts[kSmStep][NCH];
};

// A row's four reals at p as the element type (bfloat16 rows widened exactly).
template <typename T>
__device__ __forceinline__ Quad<T> row4(const T* p) {
  return ld4(p);
}
template <typename T>
__device__ __forceinline__ Quad<T> row4(const uint16_t* p) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  return {{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u), __uint_as_float(v.y << 16),
           __uint_as_float(v.y & 0xFFFF0000u)}};
}

// The query (KEY false) or key rows: the element type's, or bfloat16 under B16.
template <typename T, bool B16, bool KEY>
__device__ __forceinline__ auto rows_of(const SmArgs<T>& a) {
  if constexpr (B16)
    return KEY ? a.kb : a.qb;
  else
    return KEY ? a.k : a.q;
}

template <typename T, int NCH, uint32_t ORD, typename R>
__device__ __forceinline__ void gather(const SmArgs<T>& a, Gather<T, NCH>& g, const R* rows,
                                       const int64_t (&node)[kSmStep], const T* transport,
                                       const int64_t (&te)[kSmStep], int h) {
#pragma unroll
  for (int u = 0; u < kSmStep; ++u) {
    const R* r = rows + node[u] * a.D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) g.row[u][c] = row4<T>(r + a.C.base[c] + h * a.C.stride[c]);
    transport_pairs<T, NCH, ORD>(a.C, transport + te[u] * a.orders * 2, g.tc[u], g.ts[u]);
  }
}

// The same from the lane's chunk offsets, computed once per wave (one 64-bit
// add per chunk and edge).
template <typename T, int NCH, uint32_t ORD, typename R>
__device__ __forceinline__ void gather_at(const SmArgs<T>& a, Gather<T, NCH>& g, const R* rows,
                                          const int64_t (&node)[kSmStep], const T* transport,
                                          const int64_t (&te)[kSmStep], const int64_t (&off)[NCH]) {
#pragma unroll
  for (int u = 0; u < kSmStep; ++u) {
    const R* r = rows + node[u] * a.D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) g.row[u][c] = row4<T>(r + off[c]);
    transport_pairs<T, NCH, ORD>(a.C, transport + te[u] * a.orders * 2, g.tc[u], g.ts[u]);
  }
}

// Re< q, tau k > summed over a head's chunks.  With compile-time orders the
// chunks of one order share their rotation: per order the two sums
// A = sum q.k and B = sum (q1 k0 - q0 k1) over the pairs, then c A + s B
// (tau k = (c k0 - s k1, c k1 + s k0) per pair).
template <typename T, int NCH, uint32_t ORD>
__device__ __forceinline__ T score_dot(const Chunks& C, const T (&q)[NCH * 4], const Gather<T, NCH>& g, int u) {
  if constexpr (ORD != 0) {
    constexpr int MO = max_order_of(ORD);
    T A[MO + 1], B[MO + 1], cs[MO + 1], sn[MO + 1];
#pragma unroll
    for (int o = 0; o <= MO; ++o) A[o] = B[o] = cs[o] = sn[o] = T(0);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int o = chunk_order<ORD>(C, c);
      const T* q4 = &q[4 * c];
      const Quad<T>& k = g.row[u][c];
#pragma unroll
      for (int v = 0; v < 4; ++v) A[o] = fma(q4[v], k.v[v], A[o]);
      if (o != 0) {
#pragma unroll
        for (int v = 0; v < 4; v += 2) B[o] = fma(-q4[v], k.v[v + 1], fma(q4[v + 1], k.v[v], B[o]));
        cs[o] = g.tc[u][c];
        sn[o] = g.ts[u][c];
      }
    }
    T acc = A[0];
#pragma unroll
    for (int o = 1; o <= MO; ++o) acc += cs[o] * A[o] + sn[o] * B[o];
    return acc;
  } else {
    T acc = T(0);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      acc += chunk_dot_pair(&q[4 * c], g.row[u][c], chunk_order<ORD>(C, c), g.tc[u][c], g.ts[u][c]);
    return acc;
  }
}

// Forward, in the eager softmax's own steps: the scores and their maximum,
// the sum of exp(s - max), the quotients.  The lane's edges are e0 + s + r S;
// every step requests the next step's source ids before it waits for its own
// rows, so a step costs one memory round trip.  A lane's first R scores stay
// in registers; later ones park in alpha and are read back for the sum and
// for the quotient (their exponential taken again: cheaper than a store).
template <typename T, int NCH, uint32_t ORD, bool B16>
__global__ __launch_bounds__(256) void softmax_forward_fast(SmArgs<T> a) {
  constexpr int U = kSmStep, R = kSmRegs;
  const int64_t blk = xcd_balanced_block(blockIdx.x, gridDim.x, a.row_ptr, a.n_nodes, kWavesPerBlock);
  const int lane = threadIdx.x & 63;
  const int64_t i = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (i >= a.n_nodes) return;
  const int H = a.H, S = a.S;
  const int h = lane & (H - 1), s = lane >> a.hshift;
  const int64_t e0 = a.row_ptr[i], e1 = a.row_ptr[i + 1];

  int64_t off[NCH];
  T q[NCH * 4];
  const auto qi = rows_of<T, B16, false>(a) + i * a.D;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    off[c] = a.C.base[c] + h * a.C.stride[c];
    const Quad<T> x = row4<T>(qi + off[c]);
#pragma unroll
    for (int u = 0; u < 4; ++u) q[4 * c + u] = x.v[u];
  }
  int64_t jn[U];
  if constexpr (kSmPrefetch) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t e = e0 + s + (int64_t)u * S;
      jn[u] = e < e1 ? a.source[e] : 0;
    }
  }
  // one step from eb: scores of the live edges into lw (dead ones -inf)
  auto step = [&](int64_t eb, T (&lw)[U]) {
    int64_t jc[U], te[U];
    bool live[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t e = eb + (int64_t)u * S;
      live[u] = e < e1;
      te[u] = live[u] ? e : eb;
      jc[u] = kSmPrefetch ? jn[u] : a.source[te[u]];
    }
    if constexpr (kSmPrefetch) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t e = eb + (int64_t)(U + u) * S;
        jn[u] = e < e1 ? a.source[e] : 0;
      }
    }
    Gather<T, NCH> g;
    gather_at<T, NCH, ORD>(a, g, rows_of<T, B16, true>(a), jc, a.transport, te, off);
    T bias[U];
    uint8_t in[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      bias[u] = a.bias[te[u]];
      in[u] = a.inside[te[u]];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const T acc = score_dot<T, NCH, ORD>(a.C, q, g, u);
      lw[u] = (live[u] && in[u]) ? a.scale * acc + bias[u] : neg_inf<T>();  // outside the window: excluded
    }
  };
  T sc[R > 0 ? R : 1];
  T m = neg_inf<T>();
#pragma unroll
  for (int t = 0; t < R / U; ++t) {
    const int64_t eb = e0 + s + (int64_t)t * U * S;
    if (eb >= e1) break;
    T lw[U];
    step(eb, lw);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      sc[t * U + u] = lw[u];
      m = lw[u] > m ? lw[u] : m;
    }
  }
  const int64_t tail = e0 + s + (int64_t)R * S;
  for (int64_t eb = tail; eb < e1; eb += (int64_t)U * S) {
    T lw[U];
    step(eb, lw);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t e = eb + (int64_t)u * S;
      if (e < e1) a.alpha[e * H + h] = lw[u];
      m = lw[u] > m ? lw[u] : m;
    }
  }
  for (int o = H; o < kWave; o <<= 1) {
    const T mo = __shfl_xor(m, o, kWave);
    m = mo > m ? mo : m;
  }
  // an excluded edge is exp(-inf) = 0; a row with none inside has max -inf and
  // gives NaN, as the eager division 0 / 0 does
  T l = T(0);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (e0 + s + (int64_t)r * S < e1) {
      sc[r] = gm_exp(sc[r] - m);
      l += sc[r];
    }
  }
  // the parked scores, kSmTail a batch with their loads in flight together, summed in edge order
  constexpr int TU = kSmTail;
  for (int64_t eb = tail; eb < e1; eb += (int64_t)TU * S) {
    T v[TU];
#pragma unroll
    for (int u = 0; u < TU; ++u) {
      const int64_t e = eb + (int64_t)u * S;
      v[u] = e < e1 ? a.alpha[e * H + h] : T(0);
    }
#pragma unroll
    for (int u = 0; u < TU; ++u)
      if (eb + (int64_t)u * S < e1) l += gm_exp(v[u] - m);
  }
  l = group_sum_pow2(l, H);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t e = e0 + s + (int64_t)r * S;
    if (e < e1) a.alpha[e * H + h] = sc[r] / l;
  }
  for (int64_t eb = tail; eb < e1; eb += (int64_t)TU * S) {
    T v[TU];
#pragma unroll
    for (int u = 0; u < TU; ++u) {
      const int64_t e = eb + (int64_t)u * S;
      v[u] = e < e1 ? a.alpha[e * H + h] : T(0);
    }
#pragma unroll
    for (int u = 0; u < TU; ++u) {
      const int64_t e = eb + (int64_t)u * S;
      if (e < e1) a.alpha[e * H + h] = gm_exp(v[u] - m) / l;
    }
  }
}

// The forward for compiled-in chunk orders, with each edge's own entries
// (source id, bias and window flag, transport pairs) read once per 64 edges:
// lane l loads edge base + l's entries (one batch ahead) and every step takes
// its edge's from lane t S + s by a lane shuffle.  The 8 lanes of an edge
// would otherwise load the same entries on every step; the texture data path
// that returns loads is the kernels' bound, and it counts wave instructions,
// not bytes.  Same arithmetic and order of operations as softmax_forward_fast.
template <int MO>
struct EdgeBatch {
  int64_t src;        // source id
  float bm;           // bias, or -inf outside the window and past the row
  float tr[2 * MO];   // (cos, sin) of orders 1 .. MO
};

// A 64-bit value of lane `from` (two 32-bit shuffles).
__device__ __forceinline__ int64_t shfl64(int64_t v, int from) {
  const int lo = __shfl((int)(uint32_t)v, from, kWave), hi = __shfl((int)(v >> 32), from, kWave);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

template <typename T, int NCH, uint32_t ORD, bool B16, int S>
__global__ __launch_bounds__(256) void softmax_forward_batched(SmArgs<T> a) {
  static_assert(ORD != 0 && std::is_same<T, float>::value, "compiled-in orders, float arithmetic");
  constexpr int R = kSmRegs, MO = max_order_of(ORD), SB = kWave / S;  // steps a batch
  static_assert(R % SB == 0, "whole batches in registers");
  const int64_t blk = xcd_balanced_block(blockIdx.x, gridDim.x, a.row_ptr, a.n_nodes, kWavesPerBlock);
  const int lane = threadIdx.x & 63;
  const int64_t i = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (i >= a.n_nodes) return;
  const int H = kWave / S;
  const int h = lane & (H - 1), s = lane / H;

  int64_t off[NCH];
  float q[NCH * 4];
  int64_t e1 = 0;  // the current target's row end (the lambdas below read it)
  auto load_q = [&](int64_t it) {
    const auto qi = rows_of<T, B16, false>(a) + it * a.D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      off[c] = a.C.base[c] + h * a.C.stride[c];
      const Quad<float> x = row4<float>(qi + off[c]);
#pragma unroll
      for (int u = 0; u < 4; ++u) q[4 * c + u] = x.v[u];
    }
  };
  auto load_batch = [&](int64_t base, EdgeBatch<MO>& b) {
    const int64_t e = base + lane;
    if (e < e1) {
      b.src = a.source[e];
      b.bm = a.inside[e] ? a.bias[e] : neg_inf<float>();
      const float* tr = a.transport + e * a.orders * 2;
#pragma unroll
      for (int o = 1; o <= MO; ++o) ld_pair(tr + 2 * o, b.tr[2 * o - 2], b.tr[2 * o - 1]);
    } else {
      b.src = 0;
      b.bm = neg_inf<float>();
#pragma unroll
      for (int o = 0; o < 2 * MO; ++o) b.tr[o] = 0.f;
    }
  };
  const auto krows = rows_of<T, B16, true>(a);
  // score of step t of batch b (edge base + t S + s; -inf when excluded or past the row)
  auto score = [&](const EdgeBatch<MO>& b, int t) {
    const int from = t * S + s;
    const int64_t j = shfl64(b.src, from);
    Gather<float, NCH> g;
    const auto r = krows + j * a.D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) g.row[0][c] = row4<float>(r + off[c]);
    const float bm = __shfl(b.bm, from, kWave);
    float cs[MO + 1], sn[MO + 1];
    cs[0] = 1.f;
    sn[0] = 0.f;
#pragma unroll
    for (int o = 1; o <= MO; ++o) {
      cs[o] = __shfl(b.tr[2 * o - 2], from, kWave);
      sn[o] = __shfl(b.tr[2 * o - 1], from, kWave);
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      g.tc[0][c] = cs[chunk_order<ORD>(a.C, c)];
      g.ts[0][c] = sn[chunk_order<ORD>(a.C, c)];
    }
    const float acc = score_dot<float, NCH, ORD>(a.C, q, g, 0);
    return bm == neg_inf<float>() ? neg_inf<float>() : a.scale * acc + bm;
  };
  // park the scores of the batches from `first` in alpha; the lane's maximum
  auto park = [&](int64_t first, float m) {
    EdgeBatch<MO> cur, nxt;
    if (first < e1) load_batch(first, cur);
    for (int64_t base = first; base < e1; base += kWave) {
      if (base + kWave < e1) load_batch(base + kWave, nxt);
#pragma unroll
      for (int t = 0; t < SB; ++t) {
        if (base + t * S >= e1) break;
        const float lw = score(cur, t);
        const int64_t e = base + t * S + s;
        if (e < e1) a.alpha[e * H + h] = lw;
        m = lw > m ? lw : m;
      }
      cur = nxt;
    }
    return m;
  };
  // the parked scores of those batches: the lane's sum of exp(s - m), in edge order, each batch's
  // loads in flight together (one round trip a batch)
  auto parked_sum = [&](int64_t first, float m) {
    float l = 0.f;
    for (int64_t eb = first + s; eb < e1; eb += kWave) {
      float v[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int64_t e = eb + (int64_t)u * S;
        v[u] = e < e1 ? a.alpha[e * H + h] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < SB; ++u)
        if (eb + (int64_t)u * S < e1) l += gm_exp(v[u] - m);
    }
    return l;
  };
  auto parked_quotients = [&](int64_t first, float m, float l) {
    for (int64_t eb = first + s; eb < e1; eb += kWave) {
      float v[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int64_t e = eb + (int64_t)u * S;
        v[u] = e < e1 ? a.alpha[e * H + h] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int64_t e = eb + (int64_t)u * S;
        if (e < e1) a.alpha[e * H + h] = gm_exp(v[u] - m) / l;
      }
    }
  };
  auto wave_max = [&](float m) {
    for (int o = H; o < kWave; o <<= 1) {
      const float mo = __shfl_xor(m, o, kWave);
      m = mo > m ? mo : m;
    }
    return m;
  };

  const int64_t e0 = a.row_ptr[i];
  e1 = a.row_ptr[i + 1];
  load_q(i);
  // a lane's first R scores stay in registers, later ones park in alpha
  EdgeBatch<MO> cur, nxt;
  load_batch(e0, cur);
  float sc[R];
  float m = neg_inf<float>();
#pragma unroll
  for (int bi = 0; bi < R / SB; ++bi) {
    const int64_t base = e0 + (int64_t)bi * kWave;
    if (base >= e1) break;
    if (base + kWave < e1) load_batch(base + kWave, nxt);
#pragma unroll
    for (int t = 0; t < SB; ++t) {
      const float lw = base + t * S < e1 ? score(cur, t) : neg_inf<float>();
      sc[bi * SB + t] = lw;
      m = lw > m ? lw : m;
    }
    cur = nxt;
  }
  const int64_t tail = e0 + (int64_t)R * S;
  m = wave_max(park(tail, m));
  float l = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (e0 + s + (int64_t)r * S < e1) {
      sc[r] = gm_exp(sc[r] - m);
      l += sc[r];
    }
  }
  l += parked_sum(tail, m);
  l = group_sum_pow2(l, H);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t e = e0 + s + (int64_t)r * S;
    if (e < e1) a.alpha[e * H + h] = sc[r] / l;
  }
  parked_quotients(tail, m, l);
}

// Backward per target: the adjoint's per-head total, ds, and dq.  ds goes to
// its edge's place in the source grouping (inv), so the per-source pass reads
// it as one stream.  A lane's first RB edges keep their alpha and dalpha in
// registers from the totals pass (rows up to RB * S edges, 64 at eight heads,
// read them once); later edges read them again in the main loop.
template <typename T, int NCH, uint32_t ORD, bool B16>
__global__ __launch_bounds__(256) void softmax_backward_target_fast(SmArgs<T> a) {
  static_assert(kSmStep == 1, "one edge a step");
  constexpr int RB = kSmBwdRegs;
  const int64_t blk = xcd_balanced_block(blockIdx.x, gridDim.x, a.row_ptr, a.n_nodes, kWavesPerBlock);
  const int lane = threadIdx.x & 63;
  const int64_t i = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (i >= a.n_nodes) return;
  const int H = a.H, S = a.S;
  const int h = lane & (H - 1), s = lane >> a.hshift;
  const int64_t e0 = a.row_ptr[i], e1 = a.row_ptr[i + 1];

  T ar[RB], dr[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int64_t f = e0 + s + (int64_t)r * S;
    ar[r] = f < e1 ? a.alpha_in[f * H + h] : T(0);
    dr[r] = f < e1 ? a.dalpha[f * H + h] : T(0);
  }
  T total = T(0);
#pragma unroll
  for (int r = 0; r < RB; r += 4)
    total += (ar[r] * dr[r] + ar[r + 1] * dr[r + 1]) + (ar[r + 2] * dr[r + 2] + ar[r + 3] * dr[r + 3]);
  for (int64_t e = e0 + s + (int64_t)RB * S; e < e1; e += 8 * S) {
    T p[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t f = e + (int64_t)u * S;
      p[u] = f < e1 ? a.alpha_in[f * H + h] * a.dalpha[f * H + h] : T(0);
    }
    total += (p[0] + p[1]) + (p[2] + p[3]);
    total += (p[4] + p[5]) + (p[6] + p[7]);
  }
  total = group_sum_pow2(total, H);

  int64_t jn = 0;
  int32_t pn = 0;
  T an = T(0), dn = T(0);
  auto fetch = [&](int64_t e, bool values) {
    const bool live = e < e1;
    jn = live ? a.source[e] : 0;
    pn = live ? a.inv[e] : 0;
    if (values) {
      an = live ? a.alpha_in[e * H + h] : T(0);
      dn = live ? a.dalpha[e * H + h] : T(0);
    }
  };
  T acc[NCH * 4];
#pragma unroll
  for (int u = 0; u < NCH * 4; ++u) acc[u] = T(0);
  // edge e of this lane (its gathers run whether or not it is live, on a clamped index), its source j
  // and grouping place pc: ds and dq's terms
  auto edge = [&](int64_t e, bool live, int64_t j, int32_t pc, T al, T da) {
    int64_t jc[1] = {j}, te[1] = {live ? e : e0};
    Gather<T, NCH> g;
    gather<T, NCH, ORD>(a, g, rows_of<T, B16, true>(a), jc, a.transport, te, h);
    if (!live) return;
    const T ds = a.scale * al * (da - total);
    a.ds[(int64_t)pc * H + h] = ds;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const Quad<T>& k = g.row[0][c];
      if (chunk_order<ORD>(a.C, c) == 0) {
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[4 * c + v] += ds * k.v[v];
      } else {
        const T cr = g.tc[0][c], ci = g.ts[0][c];
        acc[4 * c + 0] += ds * (cr * k.v[0] - ci * k.v[1]);
        acc[4 * c + 1] += ds * (cr * k.v[1] + ci * k.v[0]);
        acc[4 * c + 2] += ds * (cr * k.v[2] - ci * k.v[3]);
        acc[4 * c + 3] += ds * (cr * k.v[3] + ci * k.v[2]);
      }
    }
  };
  fetch(e0 + s, false);
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    if (e0 + (int64_t)r * S >= e1) break;  // the whole row is done (wave-uniform)
    const int64_t e = e0 + s + (int64_t)r * S;
    const int64_t jc = jn;
    const int32_t pc = pn;
    fetch(e + S, r + 1 == RB);  // the next step's ids (and, past the registers, its values)
    edge(e, e < e1, jc, pc, ar[r], dr[r]);
  }
  for (int64_t e = e0 + s + (int64_t)RB * S; e < e1; e += S) {
    const int64_t jc = jn;
    const int32_t pc = pn;
    const T al = an, da = dn;
    fetch(e + S, true);
    edge(e, true, jc, pc, al, da);
  }
#pragma unroll
  for (int u = 0; u < NCH * 4; ++u) acc[u] = group_sum_pow2(acc[u], H);
  if (s == 0) {
    T* dqi = a.dq + i * a.D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) st4(dqi + a.C.base[c] + h * a.C.stride[c], &acc[4 * c]);
  }
}

// Backward per source over the edges grouped by source: ds, the targets and
// the transport rows are streams in that order (ds written there by the
// per-target pass), the query rows are gathered.
template <typename T, int NCH, uint32_t ORD, bool B16>
__global__ __launch_bounds__(256) void softmax_backward_source_fast(SmArgs<T> a) {
  constexpr int U = kSmStep;
  const int64_t blk = xcd_balanced_block(blockIdx.x, gridDim.x, a.src_ptr, a.n_nodes, kWavesPerBlock);
  const int lane = threadIdx.x & 63;
  const int64_t j = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (j >= a.n_nodes) return;
  const int H = a.H, S = a.S;
  const int h = lane & (H - 1), s = lane >> a.hshift;
  const int64_t g0 = a.src_ptr[j], g1 = a.src_ptr[j + 1];

  int64_t tn[U];
  T dn[U];
  auto fetch = [&](int64_t gb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t g = gb + (int64_t)u * S;
      const bool live = g < g1;
      tn[u] = live ? a.target_s[g] : 0;
      dn[u] = live ? a.ds[g * H + h] : T(0);
    }
  };
  T acc[NCH * 4];
#pragma unroll
  for (int u = 0; u < NCH * 4; ++u) acc[u] = T(0);
  fetch(g0 + s);
  for (int64_t gb = g0 + s; gb < g1; gb += (int64_t)U * S) {
    int64_t tc[U], te[U];
    T dsu[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t g = gb + (int64_t)u * S;
      te[u] = g < g1 ? g : gb;
      tc[u] = tn[u];
      dsu[u] = dn[u];
    }
    fetch(gb + (int64_t)U * S);
    Gather<T, NCH> gq;
    gather<T, NCH, ORD>(a, gq, rows_of<T, B16, false>(a), tc, a.transport_s, te, h);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (gb + (int64_t)u * S >= g1) break;
      const T ds = dsu[u];
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const Quad<T>& qq = gq.row[u][c];
        if (chunk_order<ORD>(a.C, c) == 0) {
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[4 * c + v] += ds * qq.v[v];
        } else {
          const T cr = gq.tc[u][c], ci = gq.ts[u][c];
          // conj(tau) q = (c q0 + s q1, c q1 - s q0)
          acc[4 * c + 0] += ds * (cr * qq.v[0] + ci * qq.v[1]);
          acc[4 * c + 1] += ds * (cr * qq.v[1] - ci * qq.v[0]);
          acc[4 * c + 2] += ds * (cr * qq.v[2] + ci * qq.v[3]);
          acc[4 * c + 3] += ds * (cr * qq.v[3] - ci * qq.v[2]);
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < NCH * 4; ++u) acc[u] = group_sum_pow2(acc[u], H);
  if (s == 0) {
    T* dkj = a.dk + j * a.D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) st4(dkj + a.C.base[c] + h * a.C.stride[c], &acc[4 * c]);
  }
}

// The per-source backward pass for compiled-in orders with each edge's own
// entries (target id, transport pairs) read once per 64 edges and shared by
// lane shuffles, as the batched forward; same edges in the same order and the
// same arithmetic as softmax_backward_source_fast.  (The per-target pass in
// this form, its source ids, grouping places and transport batched, measured
// slower than softmax_backward_target_fast at NS: 4.80 vs 4.65 ms.)
template <int MO>
struct IdBatch {
  int id;
  float tr[2 * MO];
};

template <int MO, typename IdT>
__device__ __forceinline__ void load_ids(IdBatch<MO>& b, int64_t e, int64_t end, const IdT* ids,
                                         const float* transport, int orders) {
  if (e < end) {
    b.id = (int)ids[e];
    const float* tr = transport + e * orders * 2;
#pragma unroll
    for (int o = 1; o <= MO; ++o) ld_pair(tr + 2 * o, b.tr[2 * o - 2], b.tr[2 * o - 1]);
  } else {
    b.id = 0;
#pragma unroll
    for (int o = 0; o < 2 * MO; ++o) b.tr[o] = 0.f;
  }
}

// Step t's shared entries: the id and (cos, sin) of orders 0 .. MO from lane `from`.
template <int MO>
__device__ __forceinline__ int take_ids(const IdBatch<MO>& b, int from, float (&cs)[MO + 1], float (&sn)[MO + 1]) {
  cs[0] = 1.f;
  sn[0] = 0.f;
#pragma unroll
  for (int o = 1; o <= MO; ++o) {
    cs[o] = __shfl(b.tr[2 * o - 2], from, kWave);
    sn[o] = __shfl(b.tr[2 * o - 1], from, kWave);
  }
  return __shfl(b.id, from, kWave);
}

template <typename T, int NCH, uint32_t ORD, bool B16, int S>
__global__ __launch_bounds__(256) void softmax_backward_source_batched(SmArgs<T> a) {
  static_assert(ORD != 0 && std::is_same<T, float>::value, "compiled-in orders, float arithmetic");
  constexpr int MO = max_order_of(ORD), SB = kWave / S;
  const int64_t blk = xcd_balanced_block(blockIdx.x, gridDim.x, a.src_ptr, a.n_nodes, kWavesPerBlock);
  const int lane = threadIdx.x & 63;
  const int64_t j = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (j >= a.n_nodes) return;
  const int H = kWave / S;
  const int h = lane & (H - 1), s = lane / H;
  const int64_t g0 = a.src_ptr[j], g1 = a.src_ptr[j + 1];

  int64_t off[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) off[c] = a.C.base[c] + h * a.C.stride[c];
  const auto qrows = rows_of<T, B16, false>(a);
  float acc[NCH * 4];
#pragma unroll
  for (int u = 0; u < NCH * 4; ++u) acc[u] = 0.f;
  IdBatch<MO> cur, nxt;
  load_ids<MO>(cur, g0 + lane, g1, a.target_s, a.transport_s, a.orders);
  for (int64_t base = g0; base < g1; base += kWave) {
    if (base + kWave < g1)
      load_ids<MO>(nxt, base + kWave + lane, g1, a.target_s, a.transport_s, a.orders);
    // two steps' rows and ds requested before either is used: two round trips in flight a wave
#pragma unroll
    for (int t = 0; t < SB; t += kSrcPair) {
      if (base + t * S >= g1) break;
      Quad<float> qq[kSrcPair][NCH];
      float cs[kSrcPair][MO + 1], sn[kSrcPair][MO + 1], ds[kSrcPair];
      bool live[kSrcPair];
#pragma unroll
      for (int u = 0; u < kSrcPair; ++u) {
        const int from = (t + u) * S + s;
        const int64_t g = base + from;
        live[u] = t + u < SB && g < g1;
        const int ti = take_ids<MO>(cur, t + u < SB ? from : s, cs[u], sn[u]);
        ds[u] = live[u] ? a.ds[g * H + h] : 0.f;
        const auto r = qrows + (int64_t)ti * a.D;
#pragma unroll
        for (int c = 0; c < NCH; ++c) qq[u][c] = row4<float>(r + off[c]);
      }
#pragma unroll
      for (int u = 0; u < kSrcPair; ++u) {
        if (!live[u]) continue;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          const int o = chunk_order<ORD>(a.C, c);
          if (o == 0) {
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[4 * c + v] += ds[u] * qq[u][c].v[v];
          } else {
            const float cr = cs[u][o], ci = sn[u][o];
            // conj(tau) q = (c q0 + s q1, c q1 - s q0)
            acc[4 * c + 0] += ds[u] * (cr * qq[u][c].v[0] + ci * qq[u][c].v[1]);
            acc[4 * c + 1] += ds[u] * (cr * qq[u][c].v[1] - ci * qq[u][c].v[0]);
            acc[4 * c + 2] += ds[u] * (cr * qq[u][c].v[2] + ci * qq[u][c].v[3]);
            acc[4 * c + 3] += ds[u] * (cr * qq[u][c].v[3] - ci * qq[u][c].v[2]);
          }
        }
      }
    }
    cur = nxt;
  }
#pragma unroll
  for (int u = 0; u < NCH * 4; ++u) acc[u] = group_sum_pow2(acc[u], H);
  if (s == 0) {
    float* dkj = a.dk + j * a.D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) st4(dkj + off[c], &acc[4 * c]);
  }
}

// ------------------------------------------------------------- generic path
// Any descriptor within the bounds: lanes (slot, head) for the scores, lanes
// over flat columns with a serial edge walk for dq and dk.

template <typename T>
__device__ T generic_score(const SmArgs<T>& a, const T* qi, const T* kj, const T* tr, int h) {
  T acc = T(0);
  for (int f = 0; f < a.L.F; ++f) {
    const int n = a.L.n[f], an = a.L.a[f], off = a.L.off[f];
    if (n == 0) {
      const int base = off + h * an;
      for (int u = 0; u < an; ++u) acc += qi[base + u] * kj[base + u];
    } else {
      const T c = tr[2 * n], s = tr[2 * n + 1];
      const int base = off + 2 * h * an;
      for (int u = 0; u < an; ++u) {
        const T k0 = kj[base + 2 * u], k1 = kj[base + 2 * u + 1];
        acc += qi[base + 2 * u] * (c * k0 - s * k1) + qi[base + 2 * u + 1] * (c * k1 + s * k0);
      }
    }
  }
  return acc;
}

// Where flat column c sits: its frequency, head and pair part (-1 when no row holds it).
struct Col {
  int n, h, part, pair;  // pair: the column of the pair's real part
};

template <typename T>
__device__ Col locate(const SmArgs<T>& a, int c) {
  for (int f = 0; f < a.L.F; ++f) {
    const int dim = a.L.dim[f], width = a.H * a.L.a[f] * dim, off = a.L.off[f];
    if (c >= off && c < off + width) {
      const int local = c - off, copy = local / dim;
      return {a.L.n[f], copy / a.L.a[f], local % dim, c - local % dim};
    }
  }
  return {0, -1, 0, c};
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_forward_generic(SmArgs<T> a) {
  const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x & 63;
  const int64_t i = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (i >= a.n_nodes) return;
  const int H = a.H, S = a.S;
  const int h = lane % H, s = lane / H;
  const int64_t e0 = a.row_ptr[i], e1 = a.row_ptr[i + 1];
  const T* qi = a.q + i * a.D;
  T m = neg_inf<T>(), l = T(0);
  if (s < S) {
    for (int64_t e = e0 + s; e < e1; e += S) {
      const T* tr = a.transport + e * a.orders * 2;
      T lw = a.scale * generic_score(a, qi, a.k + a.source[e] * a.D, tr, h) + a.bias[e];
      if (!a.inside[e]) lw = neg_inf<T>();
      a.alpha[e * H + h] = lw;
      online_add(m, l, lw);
    }
  }
  group_online(m, l, lane, H, S);
  if (s < S) {
    for (int64_t e = e0 + s; e < e1; e += S) a.alpha[e * H + h] = gm_exp(a.alpha[e * H + h] - m) / l;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_backward_target_generic(SmArgs<T> a) {
  const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x & 63;
  const int64_t i = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (i >= a.n_nodes) return;
  const int H = a.H, S = a.S;
  const int h = lane % H, s = lane / H;
  const int64_t e0 = a.row_ptr[i], e1 = a.row_ptr[i + 1];
  T total = T(0);
  if (s < S)
    for (int64_t e = e0 + s; e < e1; e += S) total += a.alpha_in[e * H + h] * a.dalpha[e * H + h];
  total = group_sum(total, lane, H, S);
  T totals[GM_ATTN_MAX_H];
#pragma unroll
  for (int hh = 0; hh < GM_ATTN_MAX_H; ++hh) totals[hh] = __shfl(total, hh < H ? hh : 0, kWave);
  if (s < S)
    for (int64_t e = e0 + s; e < e1; e += S)
      a.ds[e * H + h] = a.scale * a.alpha_in[e * H + h] * (a.dalpha[e * H + h] - total);
  const T* qi = a.q + i * a.D;
  (void)qi;
  for (int c = lane; c < a.D; c += kWave) {
    const Col col = locate(a, c);
    T acc = T(0);
    if (col.h >= 0) {
      const T tot = totals[col.h];
      for (int64_t e = e0; e < e1; ++e) {
        const T ds = a.scale * a.alpha_in[e * H + col.h] * (a.dalpha[e * H + col.h] - tot);
        const T* kj = a.k + a.source[e] * a.D;
        if (col.n == 0) {
          acc += ds * kj[c];
        } else {
          const T* tr = a.transport + e * a.orders * 2;
          const T cr = tr[2 * col.n], ci = tr[2 * col.n + 1];
          const T k0 = kj[col.pair], k1 = kj[col.pair + 1];
          acc += ds * (col.part == 0 ? cr * k0 - ci * k1 : cr * k1 + ci * k0);
        }
      }
    }
    a.dq[i * a.D + c] = acc;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_backward_source_generic(SmArgs<T> a) {
  const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x & 63;
  const int64_t j = blk * kWavesPerBlock + (threadIdx.x >> 6);
  if (j >= a.n_nodes) return;
  const int H = a.H;
  const int64_t g0 = a.src_ptr[j], g1 = a.src_ptr[j + 1];
  for (int c = lane; c < a.D; c += kWave) {
    const Col col = locate(a, c);
    T acc = T(0);
    if (col.h >= 0) {
      for (int64_t g = g0; g < g1; ++g) {
        const int64_t e = a.src_order[g];
        const T ds = a.ds[e * H + col.h];
        const T* qt = a.q + (int64_t)a.target_s[g] * a.D;
        if (col.n == 0) {
          acc += ds * qt[c];
        } else {
          const T* tr = a.transport_s + g * a.orders * 2;
          const T cr = tr[2 * col.n], ci = tr[2 * col.n + 1];
          const T q0 = qt[col.pair], q1 = qt[col.pair + 1];
          acc += ds * (col.part == 0 ? cr * q0 + ci * q1 : cr * q1 - ci * q0);
        }
      }
    }
    a.dk[j * a.D + c] = acc;
  }
}

// ------------------------------------------------------------------ launch

#define GM_FAST_CASES(X) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15) X(16)

enum class Kind { Forward, BackwardTarget, BackwardSource };

// GM_SOFTMAX_BATCHED=0 keeps the per-step entry loads.
inline bool batched_kernels() {
  static const bool on = [] {
    const char* v = std::getenv("GM_SOFTMAX_BATCHED");
    return v == nullptr || v[0] != '0';
  }();
  return on;
}

// The batched forward and per-source kernels for compiled-in orders (float
// arithmetic, S = 64 / H slots of 4 to 32); false when they do not serve the
// call.
template <typename T, int NCH, uint32_t ORD, bool B16, int S>
void launch_batched_s(Kind kind, const SmArgs<T>& a, dim3 grid, hipStream_t stream) {
  switch (kind) {
    case Kind::Forward:
      hipLaunchKernelGGL((softmax_forward_batched<T, NCH, ORD, B16, S>), grid, dim3(256), 0, stream, a);
      break;
    case Kind::BackwardSource:
      hipLaunchKernelGGL((softmax_backward_source_batched<T, NCH, ORD, B16, S>), grid, dim3(256), 0, stream, a);
      break;
    default:
      break;
  }
}

template <typename T, int NCH, uint32_t ORD, bool B16>
bool launch_batched(Kind kind, const SmArgs<T>& a, dim3 grid, hipStream_t stream) {
  if (kind == Kind::BackwardTarget) return false;
  if constexpr (ORD != 0 && std::is_same<T, float>::value) {
    switch (a.S) {
      case 4: launch_batched_s<T, NCH, ORD, B16, 4>(kind, a, grid, stream); return true;
      case 8: launch_batched_s<T, NCH, ORD, B16, 8>(kind, a, grid, stream); return true;
      case 16: launch_batched_s<T, NCH, ORD, B16, 16>(kind, a, grid, stream); return true;
      case 32: launch_batched_s<T, NCH, ORD, B16, 32>(kind, a, grid, stream); return true;
      default: return false;
    }
  }
  return false;
}

template <typename T, int NCH, uint32_t ORD = 0>
void launch_fast_n(Kind kind, const SmArgs<T>& a, dim3 grid, hipStream_t stream) {
  if (batched_kernels() && (a.qb != nullptr ? launch_batched<T, NCH, ORD, true>(kind, a, grid, stream)
                                            : launch_batched<T, NCH, ORD, false>(kind, a, grid, stream)))
    return;
  if (a.qb != nullptr) {
    if constexpr (std::is_same<T, float>::value) {
      switch (kind) {
        case Kind::Forward:
          hipLaunchKernelGGL((softmax_forward_fast<T, NCH, ORD, true>), grid, dim3(256), 0, stream, a);
          break;
        case Kind::BackwardTarget:
          hipLaunchKernelGGL((softmax_backward_target_fast<T, NCH, ORD, true>), grid, dim3(256), 0, stream, a);
          break;
        case Kind::BackwardSource:
          hipLaunchKernelGGL((softmax_backward_source_fast<T, NCH, ORD, true>), grid, dim3(256), 0, stream, a);
          break;
      }
    }
    return;
  }
  switch (kind) {
    case Kind::Forward:
      hipLaunchKernelGGL((softmax_forward_fast<T, NCH, ORD, false>), grid, dim3(256), 0, stream, a);
      break;
    case Kind::BackwardTarget:
      hipLaunchKernelGGL((softmax_backward_target_fast<T, NCH, ORD, false>), grid, dim3(256), 0, stream, a);
      break;
    case Kind::BackwardSource:
      hipLaunchKernelGGL((softmax_backward_source_fast<T, NCH, ORD, false>), grid, dim3(256), 0, stream, a);
      break;
  }
}

// Whether the descriptor's chunk orders are the packed word's.
inline bool orders_are(const Chunks& C, int n, uint32_t ord) {
  if (C.count != n) return false;
  for (int c = 0; c < n; ++c)
    if (C.order[c] != (int)((ord >> (4 * c)) & 15u)) return false;
  return true;
}

template <typename T>
void launch(Kind kind, bool fast, const SmArgs<T>& a, hipStream_t stream) {
  const dim3 grid((unsigned)blocks_for(a.n_nodes));
  if (a.qb != nullptr && !fast) return;  // unreachable: prepare refuses bfloat16 rows off the fast kernels
  if (fast && orders_are(a.C, 5, kOrders012) && a.orders > max_order_of(kOrders012)) {
    launch_fast_n<T, 5, kOrders012>(kind, a, grid, stream);
    return;
  }
  if (fast) {
    switch (a.C.count) {
#define GM_CASE(n) \
  case n:          \
    launch_fast_n<T, n>(kind, a, grid, stream); \
    return;
      GM_FAST_CASES(GM_CASE)
#undef GM_CASE
      default:
        break;
    }
  }
  switch (kind) {
    case Kind::Forward:
      hipLaunchKernelGGL(softmax_forward_generic<T>, grid, dim3(256), 0, stream, a);
      break;
    case Kind::BackwardTarget:
      hipLaunchKernelGGL(softmax_backward_target_generic<T>, grid, dim3(256), 0, stream, a);
      break;
    case Kind::BackwardSource:
      hipLaunchKernelGGL(softmax_backward_source_generic<T>, grid, dim3(256), 0, stream, a);
      break;
  }
}

// q and k are T rows, or bfloat16 rows (qb, kb) with T = float: then only the
// fast kernels serve the call.
template <typename T>
int prepare(SmArgs<T>& a, bool& fast, const T* q, const T* k, const T* transport, const T* bias,
            const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
            int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t H, double scale,
            const uint16_t* qb = nullptr, const uint16_t* kb = nullptr) {
  GM_REQUIRE(n_nodes >= 0 && n_edges >= 0, "sizes must be non-negative");
  GM_REQUIRE(n_nodes < (int64_t(1) << 31) * kWavesPerBlock, "too many nodes for one launch");
  a = SmArgs<T>{};
  const int rc = parse_attention_layout(desc, F, H, D, orders, a.L);
  if (rc != GM_OK) return rc;
  const bool b16 = qb != nullptr || kb != nullptr;
  if (n_nodes > 0) GM_REQUIRE(b16 ? (qb && kb && row_ptr) : (q && k && row_ptr), "q, k and row_ptr must be device pointers");
  if (n_edges > 0) GM_REQUIRE(transport && bias && inside && source, "the per-edge tables must be device pointers");
  a.q = q;
  a.k = k;
  a.qb = qb;
  a.kb = kb;
  a.transport = transport;
  a.bias = bias;
  a.inside = inside;
  a.row_ptr = row_ptr;
  a.source = source;
  a.n_nodes = n_nodes;
  a.D = (int)D;
  a.orders = (int)orders;
  a.H = (int)H;
  a.S = gm::kWave / (int)H;
  a.scale = (T)scale;
  const bool pow2 = (H == 1 || H == 2 || H == 4 || H == 8 || H == 16);
  a.hshift = H == 1 ? 0 : H == 2 ? 1 : H == 4 ? 2 : H == 8 ? 3 : 4;
  fast = pow2 && make_chunks(a.L, a.C) &&
         (b16 ? aligned(qb, 8) && aligned(kb, 8) : aligned(q, 4 * sizeof(T)) && aligned(k, 4 * sizeof(T)));
  if (b16)
    GM_REQUIRE(fast, "bfloat16 rows need heads whose segments are whole chunks of four reals (H a power of two "
                     "up to 16) and 8-byte aligned rows");
  return GM_OK;
}

template <typename T>
int softmax_forward(const T* q, const T* k, const T* transport, const T* bias, const uint8_t* inside,
                    const int64_t* desc, const int64_t* row_ptr, const int64_t* source, int64_t n_nodes,
                    int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t H, double scale, T* alpha,
                    hipStream_t stream, const uint16_t* qb = nullptr, const uint16_t* kb = nullptr) {
  SmArgs<T> a;
  bool fast = false;
  const int rc = prepare(a, fast, q, k, transport, bias, inside, desc, row_ptr, source, n_nodes, n_edges, D, orders,
                         F, H, scale, qb, kb);
  if (rc != GM_OK) return rc;
  if (n_nodes == 0 || n_edges == 0) return GM_OK;
  GM_REQUIRE(alpha, "alpha must be a device pointer");
  a.alpha = alpha;
  launch(Kind::Forward, fast, a, stream);
  return check_launch("softmax_forward");
}

template <typename T>
int softmax_backward(const T* dalpha, const T* q, const T* k, const T* transport, const T* bias, const uint8_t* inside,
                     const int64_t* desc, const int64_t* row_ptr, const int64_t* source, const T* alpha,
                     int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t H, double scale,
                     const int64_t* src_ptr, const int64_t* src_order, const int32_t* target_s, const int32_t* inv,
                     const T* transport_s, T* ds, T* dq, T* dk, hipStream_t stream, const uint16_t* qb = nullptr,
                     const uint16_t* kb = nullptr) {
  SmArgs<T> a;
  bool fast = false;
  const int rc = prepare(a, fast, q, k, transport, bias, inside, desc, row_ptr, source, n_nodes, n_edges, D, orders,
                         F, H, scale, qb, kb);
  if (rc != GM_OK) return rc;
  if (n_nodes == 0) return GM_OK;
  GM_REQUIRE(dq && dk && src_ptr, "dq, dk and src_ptr must be device pointers");
  if (n_edges > 0)
    GM_REQUIRE(dalpha && alpha && src_order && target_s && inv && transport_s && ds,
               "dalpha, alpha, src_order, target_s, inv, transport_s and ds must be device pointers");
  GM_REQUIRE(n_nodes < (int64_t(1) << 31) && n_edges < (int64_t(1) << 31),
             "the source-grouped streams index nodes and edges in 32 bits");
  fast = fast && aligned(dq, 4 * sizeof(T)) && aligned(dk, 4 * sizeof(T));
  if (qb) GM_REQUIRE(fast, "bfloat16 rows need 16-byte aligned dq and dk");
  a.alpha_in = alpha;
  a.dalpha = dalpha;
  a.ds = ds;
  a.dq = dq;
  a.dk = dk;
  a.src_ptr = src_ptr;
  a.src_order = src_order;
  a.target_s = target_s;
  a.inv = inv;
  a.transport_s = transport_s;
  launch(Kind::BackwardTarget, fast, a, stream);
  int status = check_launch("softmax_backward (per target)");
  if (status != GM_OK) return status;
  launch(Kind::BackwardSource, fast, a, stream);
  return check_launch("softmax_backward (per source)");
}

}  // namespace
}  // namespace gm

extern "C" int gm_softmax_forward_f32(const float* q, const float* k, const float* transport, const float* bias,
                                      const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr,
                                      const int64_t* source, int64_t n_nodes, int64_t n_edges, int64_t D,
                                      int64_t orders, int64_t F, int64_t H, double scale, int64_t deg_max,
                                      float* alpha, void* stream) {
  (void)deg_max;
  return gm::softmax_forward<float>(q, k, transport, bias, inside, desc, row_ptr, source, n_nodes, n_edges, D, orders,
                                    F, H, scale, alpha, (hipStream_t)stream);
}

extern "C" int gm_softmax_forward_f64(const double* q, const double* k, const double* transport, const double* bias,
                                      const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr,
                                      const int64_t* source, int64_t n_nodes, int64_t n_edges, int64_t D,
                                      int64_t orders, int64_t F, int64_t H, double scale, int64_t deg_max,
                                      double* alpha, void* stream) {
  (void)deg_max;
  return gm::softmax_forward<double>(q, k, transport, bias, inside, desc, row_ptr, source, n_nodes, n_edges, D,
                                     orders, F, H, scale, alpha, (hipStream_t)stream);
}

extern "C" int gm_softmax_backward_f32(const float* dalpha, const float* q, const float* k, const float* transport,
                                       const float* bias, const uint8_t* inside, const int64_t* desc,
                                       const int64_t* row_ptr, const int64_t* source, const float* alpha,
                                       int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F,
                                       int64_t H, double scale, int64_t deg_max, const int64_t* src_ptr,
                                       const int64_t* src_order, const int32_t* target_s, const int32_t* inv,
                                       const float* transport_s, float* ds, float* dq, float* dk, void* stream) {
  (void)deg_max;
  return gm::softmax_backward<float>(dalpha, q, k, transport, bias, inside, desc, row_ptr, source, alpha, n_nodes,
                                     n_edges, D, orders, F, H, scale, src_ptr, src_order, target_s, inv, transport_s,
                                     ds, dq, dk, (hipStream_t)stream);
}

extern "C" int gm_softmax_backward_f64(const double* dalpha, const double* q, const double* k,
                                       const double* transport, const double* bias, const uint8_t* inside,
                                       const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
                                       const double* alpha, int64_t n_nodes, int64_t n_edges, int64_t D,
                                       int64_t orders, int64_t F, int64_t H, double scale, int64_t deg_max,
                                       const int64_t* src_ptr, const int64_t* src_order, const int32_t* target_s,
                                       const int32_t* inv, const double* transport_s, double* ds, double* dq,
                                       double* dk, void* stream) {
  (void)deg_max;
  return gm::softmax_backward<double>(dalpha, q, k, transport, bias, inside, desc, row_ptr, source, alpha, n_nodes,
                                      n_edges, D, orders, F, H, scale, src_ptr, src_order, target_s, inv,
                                      transport_s, ds, dq, dk, (hipStream_t)stream);
}

extern "C" int gm_softmax_forward_bf16(const uint16_t* q, const uint16_t* k, const float* transport, const float* bias,
                                       const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr,
                                       const int64_t* source, int64_t n_nodes, int64_t n_edges, int64_t D,
                                       int64_t orders, int64_t F, int64_t H, double scale, int64_t deg_max,
                                       float* alpha, void* stream) {
  (void)deg_max;
  return gm::softmax_forward<float>(nullptr, nullptr, transport, bias, inside, desc, row_ptr, source, n_nodes,
                                    n_edges, D, orders, F, H, scale, alpha, (hipStream_t)stream, q, k);
}

extern "C" int gm_softmax_backward_bf16(const float* dalpha, const uint16_t* q, const uint16_t* k,
                                        const float* transport, const float* bias, const uint8_t* inside,
                                        const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
                                        const float* alpha, int64_t n_nodes, int64_t n_edges, int64_t D,
                                        int64_t orders, int64_t F, int64_t H, double scale, int64_t deg_max,
                                        const int64_t* src_ptr, const int64_t* src_order, const int32_t* target_s,
                                        const int32_t* inv, const float* transport_s, float* ds, float* dq,
                                        float* dk, void* stream) {
  (void)deg_max;
  return gm::softmax_backward<float>(dalpha, nullptr, nullptr, transport, bias, inside, desc, row_ptr, source, alpha,
                                     n_nodes, n_edges, D, orders, F, H, scale, src_ptr, src_order, target_s, inv,
                                     transport_s, ds, dq, dk, (hipStream_t)stream, q, k);
}
