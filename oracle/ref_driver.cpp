// A C entry-point driver over the reference's own header-only CPU arithmetic
// (masonfaldet/gm-attention src/gm_attention/nn/fused/attention.h and
// factored.h, included where they lie under /root/reference; nothing of them
// is copied).  Test infrastructure only: it builds oracle/_ref/libgmref.so,
// the compiled reference the Python restatement in oracle/eager.py is pinned
// against (bench.py's CPU baselines time the Python restatement, not this
// library).  The loops below are this
// file's own; they fill the headers' Args structs and call their per-node
// routines in node order, as the reference's attention_cpu.cpp and
// factored_cpu.cpp do (attention_cpu.cpp:197-252, 94-145;
// factored_cpu.cpp:77-219).
#include <cstdint>
#include <cstring>
#include <vector>

#include "attention.h"
#include "factored.h"

namespace {

namespace fa = gm_fused_attention;
namespace ff = gm_factored;

template <typename T>
fa::Args<T> attn_args(int64_t N, int64_t E, int64_t D, int64_t orders, int64_t F, int64_t H, double scale,
                      const int64_t* desc, const int64_t* row_ptr, const int64_t* source) {
  fa::Args<T> a{};
  a.n_nodes = N;
  a.n_edges = E;
  a.H = (int)H;
  a.D = (int)D;
  a.F = (int)F;
  a.orders = (int)orders;
  a.scale = (T)scale;
  a.desc = desc;
  a.row_ptr = row_ptr;
  a.source = source;
  return a;
}

int64_t max_degree(const int64_t* row_ptr, int64_t N) {
  int64_t d = 1;
  for (int64_t i = 0; i < N; ++i) d = std::max(d, row_ptr[i + 1] - row_ptr[i]);
  return d;
}

template <typename T>
void softmax_forward(const T* q, const T* k, const T* transport, const T* bias, const uint8_t* inside,
                     const int64_t* desc, const int64_t* row_ptr, const int64_t* source, int64_t N, int64_t E,
                     int64_t D, int64_t orders, int64_t F, int64_t H, double scale, T* alpha, int64_t first,
                     int64_t last) {
  auto a = attn_args<T>(N, E, D, orders, F, H, scale, desc, row_ptr, source);
  a.q = q;
  a.k = k;
  a.transport = transport;
  a.bias = bias;
  a.inside = inside;
  a.alpha = alpha;
  std::vector<T> scratch((size_t)max_degree(row_ptr, N) * H);
  for (int64_t i = first; i < last; ++i) fa::node_softmax_forward<T>(a, i, scratch.data());
}

template <typename T>
void softmax_backward(const T* dalpha, const T* q, const T* k, const T* transport, const int64_t* desc,
                      const int64_t* row_ptr, const int64_t* source, const T* alpha, int64_t N, int64_t E, int64_t D,
                      int64_t orders, int64_t F, int64_t H, double scale, T* dq, T* dk, int64_t first, int64_t last) {
  auto a = attn_args<T>(N, E, D, orders, F, H, scale, desc, row_ptr, source);
  a.q = q;
  a.k = k;
  a.transport = transport;
  a.alpha = const_cast<T*>(alpha);
  a.dalpha = dalpha;
  a.dq = dq;
  a.dk = dk;
  std::memset(dk, 0, sizeof(T) * N * D);
  std::vector<T> scratch(2 * (size_t)max_degree(row_ptr, N) * H);
  for (int64_t i = first; i < last; ++i) fa::node_softmax_backward<T>(a, i, scratch.data());
}

template <typename T>
fa::Args<T> conv_args(const T* v, const T* rc, const T* cc, const T* transport, const T* angular, const T* rho,
                      const T* weights, const int64_t* desc, const int64_t* row_ptr, const int64_t* source, int64_t N,
                      int64_t E, int64_t D, int64_t orders, int64_t F, int64_t A0, int64_t W) {
  auto a = attn_args<T>(N, E, D, orders, F, 1, 1.0, desc, row_ptr, source);
  a.W = (int)W;
  a.A0 = (int)A0;
  a.v = v;
  a.rc = rc;
  a.cc = cc;
  a.transport = transport;
  a.angular = angular;
  a.rho = rho;
  a.alpha = const_cast<T*>(weights);
  return a;
}

template <typename T>
ff::Args<T> fact_args(const T* h, const T* zc, const T* zr, const T* angular, const T* transport, const T* rho,
                      const int32_t* desc, const int64_t* source, int64_t E, int64_t k, int64_t wc, int64_t wr,
                      int64_t n_f, int64_t n_blocks, int64_t d_out) {
  ff::Args<T> a{};
  a.n_edges = E;
  a.k = (int)k;
  a.wc = (int)wc;
  a.wr = (int)wr;
  a.n_f = (int)n_f;
  a.n_blocks = (int)n_blocks;
  a.d_out = (int)d_out;
  a.h = h;
  a.zc = zc;
  a.zr = zr;
  a.angular = angular;
  a.transport = transport;
  a.rho = rho;
  a.desc = desc;
  a.source = source;
  return a;
}

}  // namespace

#define REF_EXPORTS(T, S)                                                                                          \
  extern "C" void ref_softmax_forward_##S(const T* q, const T* k, const T* transport, const T* bias,              \
                                          const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr,     \
                                          const int64_t* source, int64_t N, int64_t E, int64_t D, int64_t orders, \
                                          int64_t F, int64_t H, double scale, T* alpha, int64_t first,            \
                                          int64_t last) {                                                         \
    softmax_forward<T>(q, k, transport, bias, inside, desc, row_ptr, source, N, E, D, orders, F, H, scale, alpha, \
                       first, last);                                                                              \
  }                                                                                                               \
  extern "C" void ref_softmax_backward_##S(const T* dalpha, const T* q, const T* k, const T* transport,          \
                                           const int64_t* desc, const int64_t* row_ptr, const int64_t* source,    \
                                           const T* alpha, int64_t N, int64_t E, int64_t D, int64_t orders,       \
                                           int64_t F, int64_t H, double scale, T* dq, T* dk, int64_t first,       \
                                           int64_t last) {                                                        \
    softmax_backward<T>(dalpha, q, k, transport, desc, row_ptr, source, alpha, N, E, D, orders, F, H, scale, dq,  \
                        dk, first, last);                                                                         \
  }                                                                                                               \
  extern "C" void ref_conv_forward_##S(const T* v, const T* rc, const T* cc, const T* transport,                 \
                                       const T* angular, const T* rho, const T* weights, const int64_t* desc,     \
                                       const int64_t* row_ptr, const int64_t* source, int64_t N, int64_t E,       \
                                       int64_t D, int64_t orders, int64_t F, int64_t A0, int64_t W, T* out) {     \
    auto a = conv_args<T>(v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, N, E, D, orders, F, \
                          A0, W);                                                                                 \
    a.out = out;                                                                                                  \
    for (int64_t i = 0; i < N; ++i) fa::node_conv_forward<T>(a, i);                                               \
  }                                                                                                               \
  extern "C" void ref_conv_backward_##S(const T* g, const T* v, const T* rc, const T* cc, const T* transport,    \
                                        const T* angular, const T* rho, const T* weights, const int64_t* desc,    \
                                        const int64_t* row_ptr, const int64_t* source, int64_t N, int64_t E,      \
                                        int64_t D, int64_t orders, int64_t F, int64_t A0, int64_t W, T* dv,       \
                                        T* drc, T* dcc) {                                                         \
    auto a = conv_args<T>(v, rc, cc, transport, angular, rho, weights, desc, row_ptr, source, N, E, D, orders, F, \
                          A0, W);                                                                                 \
    a.g = g;                                                                                                      \
    a.dv = dv;                                                                                                    \
    a.drc = drc;                                                                                                  \
    a.dcc = dcc;                                                                                                  \
    std::memset(dv, 0, sizeof(T) * N * D);                                                                        \
    for (int64_t i = 0; i < N; ++i) fa::node_conv_backward<T>(a, i);                                              \
  }                                                                                                               \
  extern "C" void ref_factored_forward_##S(const T* h, const T* zc, const T* zr, const T* angular,               \
                                           const T* transport, const T* rho, const int32_t* desc,                 \
                                           const int64_t* source, int64_t E, int64_t k, int64_t wc, int64_t wr,   \
                                           int64_t n_f, int64_t n_blocks, int64_t d_out, T* out) {                \
    auto a = fact_args<T>(h, zc, zr, angular, transport, rho, desc, source, E, k, wc, wr, n_f, n_blocks, d_out);  \
    a.out = out;                                                                                                  \
    for (int64_t e = 0; e < E; ++e) {                                                                             \
      const int64_t j = source[e];                                                                                \
      ff::edge_message<T, ff::MAX_BM>(a, e, zc + j * k * wc * 2, zr + j * k * wr);                               \
    }                                                                                                             \
  }                                                                                                               \
  extern "C" void ref_factored_aggregate_##S(const T* rows, const T* weights, const int64_t* row_ptr, int64_t N,  \
                                             int64_t d_out, T* out) {                                             \
    for (int64_t i = 0; i < N; ++i) ff::aggregate_node<T>(rows, weights, row_ptr, (int)d_out, i, out);            \
  }                                                                                                               \
  extern "C" void ref_factored_backward_##S(const T* g, const int64_t* target, const T* weights, const T* rows,   \
                                            const T* h, const T* zc, const T* zr, const T* angular,               \
                                            const T* transport, const T* rho, const int32_t* desc,                \
                                            const int64_t* source, int64_t N, int64_t E, int64_t k, int64_t wc,   \
                                            int64_t wr, int64_t n_f, int64_t n_blocks, int64_t d_out, T* dh,      \
                                            T* dzc, T* dzr, T* dweights) {                                        \
    auto a = fact_args<T>(h, zc, zr, angular, transport, rho, desc, source, E, k, wc, wr, n_f, n_blocks, d_out);  \
    a.g = g;                                                                                                      \
    a.target = target;                                                                                            \
    a.weights = weights;                                                                                          \
    a.rows = rows;                                                                                                \
    a.dh = dh;                                                                                                    \
    a.dzc = dzc;                                                                                                  \
    a.dzr = dzr;                                                                                                  \
    a.dweights = dweights;                                                                                        \
    std::memset(dzc, 0, sizeof(T) * N * k * wc * 2);                                                              \
    if (wr) std::memset(dzr, 0, sizeof(T) * N * k * wr);                                                          \
    for (int64_t e = 0; e < E; ++e) {                                                                             \
      const int64_t j = source[e];                                                                                \
      ff::edge_backward<T, ff::MAX_C>(a, e, zc + j * k * wc * 2, zr + j * k * wr, dzc + j * k * wc * 2,           \
                                      dzr + j * k * wr);                                                          \
    }                                                                                                             \
  }

REF_EXPORTS(float, f32)
REF_EXPORTS(double, f64)
