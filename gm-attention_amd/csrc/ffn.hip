// The transformer block's feed-forward as one pass per direction on the bf16
// matrix cores: layer norm -> SO2Linear (D -> Dh) -> scalar gate -> SO2Linear
// (Dh -> D) -> residual, on bfloat16 rows with float32 parameters, statistics
// and accumulation.
//
// Fields: frequencies 0, 1, 2 with A copies each in (flat width D = 5 A:
// A scalars, then A (re, im) pairs per nonzero frequency) and B copies each in
// the hidden field (Dh = 5 B).  The SO2Linear maps are frequency-block
// diagonal, so each frequency's block is its own product:
//   hidden_f = xhat_f M1_f (+ b1 on frequency 0),  y_f = out_f M2_f (+ b2 on 0),
// with M1_f (D_f x Dh_f) and M2_f (Dh_f x D_f) the blocks of the layers' flat
// matrices.  The gate: out_0 = SiLU(hidden_0); per nonzero frequency f and
// copy c, out_f,c = act(pre_f,c) hidden_f,c on both coordinates, with
// pre_f = Wg_f hidden_0 + bg_f (the gate reads the rounded hidden scalars)
// and act = SiLU or 2 sigmoid.  The layer norm pools the frequencies'
// mean-square magnitudes into one denominator and centres frequency 0 only.
//
// One wavefront owns 16 nodes (one row tile of v_mfma_f32_16x16x32_bf16):
// lane (r, g) = (lane % 16, lane / 16) holds node r's flat entries 32 c + 8 g
// .. + 7 of each 32-wide chunk c (the A operand's layout); a product's
// 16 x 16 output tile leaves lane (n, g) with rows 4 g .. 4 g + 3 of column n.
// Hidden values, gates and outputs move between the two layouts through the
// wave's LDS; the weights are read as B operands straight from memory (they
// stay in L2: about 200 KB in bfloat16 for the C4 block).
//
// The backward recomputes the forward from the saved statistics and writes,
// besides dx, the values the weight gradients are products of: xhat
// (bfloat16), hidden_0 (float32), out_f, dhidden_f and dpre (bfloat16), and one
// (dgamma | dbeta) partial row per tile, reduced in a fixed order.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

namespace gm {
namespace {

typedef __bf16 ffn_bf16x8 __attribute__((ext_vector_type(8)));
typedef float ffn_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned ffn_u32x4 __attribute__((ext_vector_type(4)));

struct FfnArgs {
  int64_t N;
  float eps;
  int double_sigmoid;
  const uint16_t* x;       // (N, D) bfloat16
  const float* gamma;      // (D) gains per flat coordinate
  const float* beta;       // (A) or null
  const uint16_t* w1t[3];  // M1_f^T: (Dh_f, D_f) row-major, bfloat16
  const uint16_t* w1n[3];  // M1_f: (D_f, Dh_f)
  const float* b1;         // (B) or null
  const uint16_t* wg;      // (2 B, B): the gates' nn.Linear weights, frequency 1 then 2
  const uint16_t* wgt;     // (B, 2 B): their transpose
  const float* bg;         // (2 B) or null
  const uint16_t* w2t[3];  // M2_f^T: (D_f, Dh_f)
  const uint16_t* w2n[3];  // M2_f: (Dh_f, D_f)
  const float* b2;         // (A) or null
  uint16_t* out;           // (N, D) forward: x + y
  float* mean;             // (N) forward writes, backward reads
  float* inv_d;            // (N)
  // backward
  const uint16_t* dz;      // (N, D) gradient of x + y
  uint16_t* dx;            // (N, D)
  uint16_t* xhat;          // (N, D)
  float* hidden0;          // (N, B) float32 (its values are bfloat16-exact)
  uint16_t* outs[3];       // (N, Dh_f) bfloat16
  uint16_t* dhidden[3];    // (N, Dh_f) bfloat16
  uint16_t* dpre;          // (N, 2 B) bfloat16
  float* partial;          // (tiles, D + A): dgamma, then dbeta
};

// One wavefront per workgroup: handing LDS values between its lanes needs a
// wavefront-scope release/acquire pair around a wave barrier.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

__device__ __forceinline__ ffn_f32x4 mfma(ffn_u32x4 a, ffn_u32x4 b, ffn_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(ffn_bf16x8, a), __builtin_bit_cast(ffn_bf16x8, b),
                                                 c, 0, 0, 0);
}

// Eight consecutive bfloat16 values (16 bytes) of a weight row.
__device__ __forceinline__ ffn_u32x4 frag(const uint16_t* p) { return *reinterpret_cast<const ffn_u32x4*>(p); }

// Eight floats as an operand's eight bfloat16 slots.
__device__ __forceinline__ ffn_u32x4 pack8(const float (&v)[8]) {
  ffn_u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
  return r;
}

__device__ __forceinline__ void unpack8(ffn_u32x4 p, float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(p[i] << 16);
    v[2 * i + 1] = __uint_as_float(p[i] & 0xFFFF0000u);
  }
}

__device__ __forceinline__ float sigm(float x) { return 1.f / (1.f + __expf(-x)); }

__device__ __forceinline__ void act_of(float pre, int double_sigmoid, float& g, float& dg) {
  const float s = sigm(pre);
  if (double_sigmoid) {
    g = 2.f * s;
    dg = 2.f * s * (1.f - s);
  } else {
    g = pre * s;
    dg = s * (1.f + pre * (1.f - s));
  }
}

// Sum over the four lanes of a node (lanes r, r + 16, r + 32, r + 48).
__device__ __forceinline__ float node_sum(float v) {
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

template <int A, int B>
struct Shape {
  static constexpr int D = 5 * A, Dh = 5 * B;
  static constexpr int CH = D / 32;  // 32-wide chunks of a flat row
  static constexpr int C0 = A / 32;  // chunks of frequency 0
  static constexpr int CF = A / 16;  // chunks of a nonzero frequency (2 A reals)
  static constexpr int HS = B + 8;   // LDS row strides: bfloat16 hidden scalars
  static constexpr int OS = 2 * B + 8;  // bfloat16 gated / gradient rows of one frequency
  static constexpr int YS = D + 4;   // float rows of D
  static_assert(A % 32 == 0 && B % 32 == 0, "A and B must be multiples of 32");
  __device__ static constexpr int doff(int f) { return f == 0 ? 0 : (f == 1 ? A : 3 * A); }
};

// The node's statistics and its normalised chunks (the A operands of the
// first product) from its bfloat16 chunks.
template <int A, int B>
__device__ __forceinline__ void normalise(const FfnArgs& p, const ffn_u32x4 (&xr)[Shape<A, B>::CH], int g,
                                          bool use_saved, int64_t node, float& mu, float& inv_d,
                                          ffn_u32x4 (&xh)[Shape<A, B>::CH]) {
  using S = Shape<A, B>;
  float v[S::CH][8];
#pragma unroll
  for (int c = 0; c < S::CH; ++c) unpack8(xr[c], v[c]);
  if (use_saved) {
    mu = p.mean[node];
    inv_d = p.inv_d[node];
  } else {
    float s0 = 0.f;
#pragma unroll
    for (int c = 0; c < S::C0; ++c)
#pragma unroll
      for (int u = 0; u < 8; ++u) s0 += v[c][u];
    mu = node_sum(s0) / float(A);
    float q[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < S::CH; ++c) {
      const int f = c < S::C0 ? 0 : (c < S::C0 + S::CF ? 1 : 2);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float t = f == 0 ? v[c][u] - mu : v[c][u];
        q[f] += t * t;
      }
    }
    const float total = node_sum(q[0]) / float(A) + node_sum(q[1]) / float(2 * A) + node_sum(q[2]) / float(2 * A);
    inv_d = 1.f / sqrtf(total / 3.f + p.eps);
  }
#pragma unroll
  for (int c = 0; c < S::CH; ++c) {
    float h[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = 32 * c + 8 * g + u;
      const bool scalar = c < S::C0;
      const float xn = (scalar ? v[c][u] - mu : v[c][u]) * inv_d;
      h[u] = p.gamma[k] * xn + (scalar && p.beta ? p.beta[k] : 0.f);
    }
    xh[c] = pack8(h);
  }
}

// hidden_0 (16 x B) tiles: bias, then xhat_0 M1_0; each tile handed to `use`
// (tile index, accumulator) as it is made.
template <int A, int B, class F>
__device__ __forceinline__ void hidden0_tiles(const FfnArgs& p, const ffn_u32x4 (&xh)[Shape<A, B>::CH], int r, int g,
                                              F&& use) {
#pragma unroll 1
  for (int t = 0; t < B / 16; ++t) {
    const float b = p.b1 ? p.b1[16 * t + r] : 0.f;
    ffn_f32x4 h0{b, b, b, b};
#pragma unroll
    for (int kc = 0; kc < Shape<A, B>::C0; ++kc)
      h0 = mfma(xh[kc], frag(p.w1t[0] + (16 * t + r) * A + 32 * kc + 8 * g), h0);
    use(t, h0);
  }
}

// The gate pre-activations of nonzero frequency f (16 x B) from the rounded
// hidden scalars in LDS: bias + H0 Wg_f^T.
template <int A, int B>
__device__ __forceinline__ void gate_tile(const FfnArgs& p, const uint16_t* H0, int f, int t, int r, int g,
                                          ffn_f32x4& acc) {
  using S = Shape<A, B>;
  const int row = (f - 1) * B + 16 * t + r;
  const float b = p.bg ? p.bg[row] : 0.f;
  acc = ffn_f32x4{b, b, b, b};
#pragma unroll
  for (int kc = 0; kc < B / 32; ++kc)
    acc = mfma(*reinterpret_cast<const ffn_u32x4*>(H0 + r * S::HS + 32 * kc + 8 * g),
               frag(p.wg + row * B + 32 * kc + 8 * g), acc);
}

template <int A, int B>
__global__ __launch_bounds__(64) void ffn_forward_kernel(FfnArgs p) {
  using S = Shape<A, B>;
  __shared__ __align__(16) uint16_t H0[16 * S::HS];
  __shared__ __align__(16) uint16_t O[16 * S::OS];
  __shared__ __align__(16) float Y[16 * S::YS];
  const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16, node = n0 + r;
  const bool valid = node < p.N;
  ffn_u32x4 xr[S::CH];
#pragma unroll
  for (int c = 0; c < S::CH; ++c)
    xr[c] = valid ? frag(p.x + node * S::D + 32 * c + 8 * g) : ffn_u32x4{0u, 0u, 0u, 0u};
  float mu, inv_d;
  ffn_u32x4 xh[S::CH];
  normalise<A, B>(p, xr, g, false, node, mu, inv_d, xh);
  if (valid && g == 0) {
    p.mean[node] = mu;
    p.inv_d[node] = inv_d;
  }
  // hidden_0, rounded, into LDS; out_0 = SiLU of it feeds y_0
  hidden0_tiles<A, B>(p, xh, r, g, [&](int t, const ffn_f32x4& h0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) H0[(4 * g + i) * S::HS + 16 * t + r] = f32_to_bf16(h0[i]);
  });
  wave_sync();
#pragma unroll 1
  for (int t = 0; t < A / 16; ++t) {
    const float b = p.b2 ? p.b2[16 * t + r] : 0.f;
    ffn_f32x4 acc{b, b, b, b};
#pragma unroll
    for (int kc = 0; kc < B / 32; ++kc) {
      float v[8];
      unpack8(*reinterpret_cast<const ffn_u32x4*>(H0 + r * S::HS + 32 * kc + 8 * g), v);
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = v[u] * sigm(v[u]);
      acc = mfma(pack8(v), frag(p.w2t[0] + (16 * t + r) * B + 32 * kc + 8 * g), acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) Y[(4 * g + i) * S::YS + 16 * t + r] = acc[i];
  }
#pragma unroll 1
  for (int f = 1; f <= 2; ++f) {
    // gate tile tg (copies 16 tg + n) serves hidden tiles 2 tg and 2 tg + 1
    // (columns 32 tg + 16 half + n, copy 16 tg + 8 half + n / 2, held by lane
    // 8 half + n / 2 of the same row group): hidden_f gated, rounded, into LDS
    const int c0 = S::C0 + (f - 1) * S::CF;
#pragma unroll 1
    for (int tg = 0; tg < B / 16; ++tg) {
      ffn_f32x4 pre;
      gate_tile<A, B>(p, H0, f, tg, r, g, pre);
      float gv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float dg;
        act_of(pre[i], p.double_sigmoid, gv[i], dg);
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int col = 32 * tg + 16 * half + r;
        ffn_f32x4 acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < S::CF; ++kc)
          acc = mfma(xh[c0 + kc], frag(p.w1t[f] + col * (2 * A) + 32 * kc + 8 * g), acc);
        const int src = 8 * half + (r >> 1) + 16 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          O[(4 * g + i) * S::OS + col] = f32_to_bf16(acc[i] * __shfl(gv[i], src, kWave));
      }
    }
    wave_sync();
#pragma unroll 1
    for (int t = 0; t < 2 * A / 16; ++t) {
      ffn_f32x4 acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 2 * B / 32; ++kc)
        acc = mfma(*reinterpret_cast<const ffn_u32x4*>(O + r * S::OS + 32 * kc + 8 * g),
                   frag(p.w2t[f] + (16 * t + r) * (2 * B) + 32 * kc + 8 * g), acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) Y[(4 * g + i) * S::YS + S::doff(f) + 16 * t + r] = acc[i];
    }
    wave_sync();  // G and O are rewritten for the next frequency
  }
  // out = x + y, node r's chunks
  if (valid) {
#pragma unroll
    for (int c = 0; c < S::CH; ++c) {
      float v[8];
      unpack8(xr[c], v);
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] += Y[r * S::YS + 32 * c + 8 * g + u];
      *reinterpret_cast<ffn_u32x4*>(p.out + node * S::D + 32 * c + 8 * g) = pack8(v);
    }
  }
}

template <int A, int B>
__global__ __launch_bounds__(64) void ffn_backward_kernel(FfnArgs p) {
  using S = Shape<A, B>;
  __shared__ __align__(16) uint16_t H0[16 * S::HS];
  __shared__ __align__(16) uint16_t DP[16 * S::HS];  // dpre of the current frequency, rounded
  __shared__ __align__(16) uint16_t DH[16 * S::OS];  // dhidden of the current frequency, rounded
  __shared__ __align__(16) float DX[16 * S::YS];   // d xhat, then the parameter-gradient products
  const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16, node = n0 + r;
  const bool valid = node < p.N;
  ffn_u32x4 xr[S::CH], dzr[S::CH];
#pragma unroll
  for (int c = 0; c < S::CH; ++c) {
    xr[c] = valid ? frag(p.x + node * S::D + 32 * c + 8 * g) : ffn_u32x4{0u, 0u, 0u, 0u};
    dzr[c] = valid ? frag(p.dz + node * S::D + 32 * c + 8 * g) : ffn_u32x4{0u, 0u, 0u, 0u};
  }
  float mu, inv_d;
  ffn_u32x4 xh[S::CH];
  normalise<A, B>(p, xr, g, true, valid ? node : 0, mu, inv_d, xh);
  if (valid) {
#pragma unroll
    for (int c = 0; c < S::CH; ++c) *reinterpret_cast<ffn_u32x4*>(p.xhat + node * S::D + 32 * c + 8 * g) = xh[c];
  }
  // row index of output-layout row i (node n0 + 4 g + i) and whether it exists
  bool rv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) rv[i] = n0 + 4 * g + i < p.N;
  hidden0_tiles<A, B>(p, xh, r, g, [&](int t, const ffn_f32x4& h0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t hb = f32_to_bf16(h0[i]);
      H0[(4 * g + i) * S::HS + 16 * t + r] = hb;
      if (rv[i]) p.hidden0[(n0 + 4 * g + i) * B + 16 * t + r] = bf16_to_f32(hb);
    }
  });
  wave_sync();
  // dhidden_0 accumulates the SiLU branch and both gates' branches
  ffn_f32x4 dh0[B / 16];
#pragma unroll
  for (int t = 0; t < B / 16; ++t) {
    ffn_f32x4 dout{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < S::C0; ++kc) dout = mfma(dzr[kc], frag(p.w2n[0] + (16 * t + r) * A + 32 * kc + 8 * g), dout);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float h = bf16_to_f32(H0[(4 * g + i) * S::HS + 16 * t + r]);
      float sv, ds;
      act_of(h, 0, sv, ds);
      dh0[t][i] = dout[i] * ds;
      if (rv[i]) p.outs[0][(n0 + 4 * g + i) * B + 16 * t + r] = f32_to_bf16(sv);
    }
  }
#pragma unroll 1
  for (int f = 1; f <= 2; ++f) {
    // gate tile tg serves hidden tiles 2 tg, 2 tg + 1 (as in the forward)
    const int c0 = S::C0 + (f - 1) * S::CF;
#pragma unroll 1
    for (int tg = 0; tg < B / 16; ++tg) {
      ffn_f32x4 pre;
      gate_tile<A, B>(p, H0, f, tg, r, g, pre);
      float gv[4], dgv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) act_of(pre[i], p.double_sigmoid, gv[i], dgv[i]);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int col = 32 * tg + 16 * half + r;
        ffn_f32x4 hid{0.f, 0.f, 0.f, 0.f}, dout{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < S::CF; ++kc) {
          hid = mfma(xh[c0 + kc], frag(p.w1t[f] + col * (2 * A) + 32 * kc + 8 * g), hid);
          dout = mfma(dzr[c0 + kc], frag(p.w2n[f] + col * (2 * A) + 32 * kc + 8 * g), dout);
        }
        const int src = 8 * half + (r >> 1) + 16 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 4 * g + i;
          const float gme = __shfl(gv[i], src, kWave), dgme = __shfl(dgv[i], src, kWave);
          const float dhv = dout[i] * gme;
          // d gate of copy col / 2: both coordinates (lanes r and r ^ 1)
          float dgate = dout[i] * hid[i];
          dgate += __shfl_xor(dgate, 1, kWave);
          const uint16_t dpb = f32_to_bf16(dgate * dgme), dhb = f32_to_bf16(dhv);
          DH[row * S::OS + col] = dhb;
          if ((r & 1) == 0) DP[row * S::HS + col / 2] = dpb;
          if (rv[i]) {
            const int64_t nr = n0 + row;
            p.outs[f][nr * (2 * B) + col] = f32_to_bf16(hid[i] * gme);
            p.dhidden[f][nr * (2 * B) + col] = dhb;
            if ((r & 1) == 0) p.dpre[nr * (2 * B) + (f - 1) * B + col / 2] = dpb;
          }
        }
      }
    }
    wave_sync();
    // dhidden_0 += dpre_f Wg_f; d xhat_f = dhidden_f M1_f^T
#pragma unroll
    for (int t = 0; t < B / 16; ++t) {
#pragma unroll 1
      for (int kc = 0; kc < B / 32; ++kc)
        dh0[t] = mfma(*reinterpret_cast<const ffn_u32x4*>(DP + r * S::HS + 32 * kc + 8 * g),
                      frag(p.wgt + (16 * t + r) * (2 * B) + (f - 1) * B + 32 * kc + 8 * g), dh0[t]);
    }
#pragma unroll 1
    for (int t = 0; t < 2 * A / 16; ++t) {
      ffn_f32x4 acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 2 * B / 32; ++kc)
        acc = mfma(*reinterpret_cast<const ffn_u32x4*>(DH + r * S::OS + 32 * kc + 8 * g),
                   frag(p.w1n[f] + (16 * t + r) * (2 * B) + 32 * kc + 8 * g), acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) DX[(4 * g + i) * S::YS + S::doff(f) + 16 * t + r] = acc[i];
    }
    wave_sync();
  }
  // frequency 0: dhidden_0 out and through M1_0^T
#pragma unroll
  for (int t = 0; t < B / 16; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t dhb = f32_to_bf16(dh0[t][i]);
      DH[(4 * g + i) * S::OS + 16 * t + r] = dhb;
      if (rv[i]) p.dhidden[0][(n0 + 4 * g + i) * B + 16 * t + r] = dhb;
    }
  wave_sync();
#pragma unroll 1
  for (int t = 0; t < A / 16; ++t) {
    ffn_f32x4 acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < B / 32; ++kc)
      acc = mfma(*reinterpret_cast<const ffn_u32x4*>(DH + r * S::OS + 32 * kc + 8 * g),
                 frag(p.w1n[0] + (16 * t + r) * B + 32 * kc + 8 * g), acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) DX[(4 * g + i) * S::YS + 16 * t + r] = acc[i];
  }
  wave_sync();
  // the layer norm's backward for node r, from d xhat in LDS
  // xn: node r's normalised values before the gains, from its bfloat16 chunks
  auto xn_of = [&](int c, int u) {
    float v[8];
    unpack8(xr[c], v);
    return (c < S::C0 ? v[u] - mu : v[u]) * inv_d;
  };
  float gy[S::CH][8];
  float pdot = 0.f, g0 = 0.f;
#pragma unroll
  for (int c = 0; c < S::CH; ++c)
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = 32 * c + 8 * g + u;
      gy[c][u] = DX[r * S::YS + k];
      const float gh = gy[c][u] * p.gamma[k];
      pdot += gh * xn_of(c, u);
      if (c < S::C0) g0 += gh;
    }
  pdot = node_sum(pdot);
  g0 = node_sum(g0) / float(A);
  // d(mean square)/dx_k: 2 / A at frequency 0, 1 / A above, over 2 x 3 present frequencies
  const float w0 = 2.f / float(A) / 6.f, w1 = 1.f / float(A) / 6.f;
  wave_sync();  // every lane has read its d xhat
#pragma unroll
  for (int c = 0; c < S::CH; ++c) {
    float dz[8], dxv[8];
    unpack8(dzr[c], dz);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = 32 * c + 8 * g + u;
      const bool scalar = c < S::C0;
      const float gh = gy[c][u] * p.gamma[k];
      const float xn = xn_of(c, u);
      dxv[u] = dz[u] + inv_d * (gh - (scalar ? g0 : 0.f) - pdot * xn * (scalar ? w0 : w1));
      // the parameter-gradient products of this node, zero for rows past N
      DX[r * S::YS + k] = valid ? gy[c][u] * xn : 0.f;
    }
    if (valid) *reinterpret_cast<ffn_u32x4*>(p.dx + node * S::D + 32 * c + 8 * g) = pack8(dxv);
  }
  wave_sync();
  // dgamma: the tile's 16 nodes summed per coordinate in a fixed order; dbeta from gy of the scalars
  float* part = p.partial + (int64_t)blockIdx.x * (S::D + A);
  for (int k = lane; k < S::D; k += kWave) {
    float s = 0.f;
#pragma unroll
    for (int n = 0; n < 16; ++n) s += DX[n * S::YS + k];
    part[k] = s;
  }
  wave_sync();
  // dbeta: the scalars' gy over the tile's nodes
#pragma unroll
  for (int c = 0; c < S::C0; ++c)
#pragma unroll
    for (int u = 0; u < 8; ++u) DX[r * S::YS + 32 * c + 8 * g + u] = valid ? gy[c][u] : 0.f;
  wave_sync();
  for (int k = lane; k < A; k += kWave) {
    float s = 0.f;
#pragma unroll
    for (int n = 0; n < 16; ++n) s += DX[n * S::YS + k];
    part[S::D + k] = s;
  }
}

int fill(FfnArgs& a, int64_t N, int64_t A, int64_t B, double eps, int double_sigmoid, const uint16_t* x,
         const float* gamma, const float* beta, const uint16_t* const* w1t, const uint16_t* const* w1n, const float* b1,
         const uint16_t* wg, const uint16_t* wgt, const float* bg, const uint16_t* const* w2t,
         const uint16_t* const* w2n, const float* b2) {
  GM_REQUIRE(N >= 0, "N must be non-negative");
  GM_REQUIRE(A == 32 && (B == 64 || B == 128), "the fused feed-forward serves A = 32 copies and B = 64 or 128");
  GM_REQUIRE(eps > 0, "eps must be positive");
  a = FfnArgs{};
  a.N = N;
  a.eps = (float)eps;
  a.double_sigmoid = double_sigmoid != 0;
  a.x = x;
  a.gamma = gamma;
  a.beta = beta;
  a.b1 = b1;
  a.wg = wg;
  a.wgt = wgt;
  a.bg = bg;
  a.b2 = b2;
  if (N == 0) return GM_OK;
  GM_REQUIRE(x && aligned(x, 16) && gamma, "x (16-byte aligned) and gamma must be device pointers");
  GM_REQUIRE(wg && wgt && aligned(wg, 16) && aligned(wgt, 16), "the gate weights must be 16-byte aligned");
  for (int f = 0; f < 3; ++f) {
    GM_REQUIRE(w1t[f] && w2t[f] && aligned(w1t[f], 16) && aligned(w2t[f], 16),
               "every weight block must be a 16-byte aligned device pointer");
    a.w1t[f] = w1t[f];
    a.w2t[f] = w2t[f];
    if (w1n) {  // the backward's other orientation of the blocks
      GM_REQUIRE(w1n[f] && w2n[f] && aligned(w1n[f], 16) && aligned(w2n[f], 16),
                 "every weight block must be a 16-byte aligned device pointer");
      a.w1n[f] = w1n[f];
      a.w2n[f] = w2n[f];
    }
  }
  return GM_OK;
}

template <int A, int B>
void launch(bool forward, const FfnArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.N + 15) / 16)), block(64);
  if (forward)
    hipLaunchKernelGGL((ffn_forward_kernel<A, B>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((ffn_backward_kernel<A, B>), grid, block, 0, s, a);
}

void launch_any(bool forward, int64_t B, const FfnArgs& a, hipStream_t s) {
  if (B == 64)
    launch<32, 64>(forward, a, s);
  else
    launch<32, 128>(forward, a, s);
}

}  // namespace
}  // namespace gm

extern "C" int64_t gm_ffn_partial_rows(int64_t N) { return (N + 15) / 16; }

extern "C" int gm_ffn_forward_bf16(const uint16_t* x, int64_t N, int64_t A, int64_t B, double eps, int double_sigmoid,
                                   const float* gamma, const float* beta, const uint16_t* const* w1t,
                                   const float* b1, const uint16_t* wg, const float* bg, const uint16_t* const* w2t,
                                   const float* b2, uint16_t* out, float* mean, float* inv_d, void* stream) {
  gm::FfnArgs a;
  GM_REQUIRE(w1t && w2t, "w1t and w2t must be host arrays of three device pointers");
  int rc = gm::fill(a, N, A, B, eps, double_sigmoid, x, gamma, beta, w1t, nullptr, b1, wg, wg, bg, w2t, nullptr, b2);
  if (rc != GM_OK) return rc;
  if (N == 0) return GM_OK;
  GM_REQUIRE(out && gm::aligned(out, 16) && mean && inv_d, "out (16-byte aligned), mean and inv_d must be device pointers");
  a.out = out;
  a.mean = mean;
  a.inv_d = inv_d;
  gm::launch_any(true, B, a, (hipStream_t)stream);
  return gm::check_launch("ffn_forward");
}

extern "C" int gm_ffn_backward_bf16(const uint16_t* dz, const uint16_t* x, int64_t N, int64_t A, int64_t B,
                                    double eps, int double_sigmoid, const float* gamma, const float* beta,
                                    const uint16_t* const* w1t, const uint16_t* const* w1n, const float* b1,
                                    const uint16_t* wg, const uint16_t* wgt, const float* bg,
                                    const uint16_t* const* w2t, const uint16_t* const* w2n, const float* mean,
                                    const float* inv_d, uint16_t* dx, uint16_t* xhat, float* hidden0,
                                    uint16_t* const* outs, uint16_t* const* dhidden, uint16_t* dpre, float* partial,
                                    void* stream) {
  gm::FfnArgs a;
  GM_REQUIRE(w1t && w1n && w2t && w2n && outs && dhidden, "the weight and output arrays must be host arrays of three");
  int rc = gm::fill(a, N, A, B, eps, double_sigmoid, x, gamma, beta, w1t, w1n, b1, wg, wgt, bg, w2t, w2n, nullptr);
  if (rc != GM_OK) return rc;
  if (N == 0) return GM_OK;
  GM_REQUIRE(dz && gm::aligned(dz, 16) && mean && inv_d, "dz (16-byte aligned), mean and inv_d must be device pointers");
  GM_REQUIRE(dx && gm::aligned(dx, 16) && xhat && gm::aligned(xhat, 16) && hidden0 && dpre && partial,
             "dx and xhat (16-byte aligned), hidden0, dpre and partial must be device pointers");
  for (int f = 0; f < 3; ++f) {
    GM_REQUIRE(outs[f] && dhidden[f], "outs and dhidden must hold three device pointers");
    a.outs[f] = outs[f];
    a.dhidden[f] = dhidden[f];
  }
  a.dz = dz;
  a.mean = const_cast<float*>(mean);
  a.inv_d = const_cast<float*>(inv_d);
  a.dx = dx;
  a.xhat = xhat;
  a.hidden0 = hidden0;
  a.dpre = dpre;
  a.partial = partial;
  gm::launch_any(false, B, a, (hipStream_t)stream);
  return gm::check_launch("ffn_backward");
}
