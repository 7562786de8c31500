// fp32 matrix products on the bf16 matrix cores of gfx950.
//
// On this part the fp32 MFMA (v_mfma_f32_16x16x4_f32) issues at the same
// rate as fp32 vector arithmetic, while v_mfma_f32_16x16x32_bf16 performs
// eight times the multiply-adds in half the cycles.  An fp32 value x is the
// exact sum of three bf16 values
//
//   x = hi + mid + lo,   hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid)
//
// (round to nearest at each step; x has 24 significant bits, each piece
// takes the next 8, so the last one is exact and |mid| <= 2^-8 |x|,
// |lo| <= 2^-16 |x|).  Every product of two pieces is exact in fp32, and
//
//   a b = ah bh + (ah bm + am bh) + (am bm + ah bl + al bh) + O(2^-24 |a b|)
//
// so six bf16 products accumulated in fp32 give an fp32 product to within
// the rounding of fp32 itself (the three dropped products are below 2^-24
// |a b| together).  Six products on the bf16 MFMA cost 3 K / 32 instructions
// of half the fp32 instruction's issue time for a K-deep contraction, against
// K / 4 fp32 instructions: 2.67x less matrix-core time, paid for with the
// splitting arithmetic (11 VALU instructions per pair of values).
//
// Operand slots: lane l of a 16x16x32 product supplies eight bf16 values of
// row l % 16 of A and eight of column l % 16 of B, and the product pairs slot
// u of A's lane (i, g) with slot u of B's lane (j, g), g = l / 16.  Which
// contraction index a slot stands for is the caller's choice, as long as A
// and B agree; the kernels here put two piece products of four contraction
// indices in a lane's eight slots (four indices per 32-bit pair of slots,
// first value in the low half).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>

namespace gm {

// Whether the kernels that have both forms take the split bf16 products
// (GM_SPLIT_PRODUCTS=0: the fp32 MFMA throughout).
inline bool split_products() {
  static const bool on = [] {
    const char* v = std::getenv("GM_SPLIT_PRODUCTS");
    return v == nullptr || v[0] != '0';
  }();
  return on;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// The three pieces of two values, each a packed bf16 pair (x0 in the low half).
struct SplitPair {
  uint32_t hi, mid, lo;
};

__device__ __forceinline__ uint32_t pack_bf16(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{x0, x1}), bf16x2));
}

// A packed pair back to fp32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

__device__ __forceinline__ SplitPair split_pair(float x0, float x1) {
  SplitPair s;
  s.hi = pack_bf16(x0, x1);
  const float r0 = x0 - bf16_lo(s.hi), r1 = x1 - bf16_hi(s.hi);
  s.mid = pack_bf16(r0, r1);
  s.lo = pack_bf16(r0 - bf16_lo(s.mid), r1 - bf16_hi(s.mid));
  return s;
}

// Four consecutive contraction values' pieces: (hi, mid, lo) as two packed pairs each.
struct Split4 {
  uint32_t hi[2], mid[2], lo[2];
};

__device__ __forceinline__ Split4 split4(float x0, float x1, float x2, float x3) {
  const SplitPair a = split_pair(x0, x1), b = split_pair(x2, x3);
  return Split4{{a.hi, b.hi}, {a.mid, b.mid}, {a.lo, b.lo}};
}

// Eight slots from two four-value pieces: slots 0..3 = p, 4..7 = r.
__device__ __forceinline__ u32x4 slots(const uint32_t (&p)[2], const uint32_t (&r)[2]) {
  return u32x4{p[0], p[1], r[0], r[1]};
}

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// The A operands of one side of a split product over four contraction
// indices: [hi, mid] and [hi, lo].  With the other side's B operands
// [hi, hi], [mid, mid] and [lo, hi] the three instructions form the six
// piece products hh, mh, hm, mm, hl, lh.
struct SplitA {
  u32x4 hm, hl;
};
struct SplitB {
  u32x4 hh, mm, lh;
};

__device__ __forceinline__ SplitA split_a(float x0, float x1, float x2, float x3) {
  const Split4 s = split4(x0, x1, x2, x3);
  return SplitA{slots(s.hi, s.mid), slots(s.hi, s.lo)};
}

__device__ __forceinline__ SplitB split_b(float x0, float x1, float x2, float x3) {
  const Split4 s = split4(x0, x1, x2, x3);
  return SplitB{slots(s.hi, s.hi), slots(s.mid, s.mid), slots(s.lo, s.hi)};
}

// c + A B over four contraction indices in fp32 accuracy: the smallest
// products first.
__device__ __forceinline__ f32x4 mfma_split(const SplitA& a, const SplitB& b, f32x4 c) {
  c = mfma_bf16(a.hl, b.lh, c);  // hi lo + lo hi
  c = mfma_bf16(a.hm, b.mm, c);  // hi mid + mid mid
  c = mfma_bf16(a.hm, b.hh, c);  // hi hi + mid hi
  return c;
}

}  // namespace gm
