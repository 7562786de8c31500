// The attention/depthwise descriptor as the kernels read it.
#pragma once
#include <cstdint>

#include "gm_hip.h"

namespace gm {

// One row per frequency f: n, copies per head a, flat offset, coefficient
// offset, dim (1 or 2).  Column c of head h inside row f lies in
// [off + h * a * dim, off + (h + 1) * a * dim).
struct AttnLayout {
  int F, H, D, orders;
  int head_width;  // sum_f a_f dim_f: one head's reals
  int n[GM_ATTN_MAX_F], a[GM_ATTN_MAX_F], off[GM_ATTN_MAX_F], coff[GM_ATTN_MAX_F], dim[GM_ATTN_MAX_F];
};

int parse_attention_layout(const int64_t* desc, int64_t F, int64_t H, int64_t D, int64_t orders, AttnLayout& L);

// Per-head chunks of four consecutive reals (four scalars, or two complex
// pairs of one frequency): chunk c of head h starts at base[c] + h * stride[c]
// and its frequency is order[c].  Valid when every head segment is a multiple
// of four reals at a four-aligned offset.
constexpr int kMaxChunks = 16;
struct Chunks {
  int count;
  int base[kMaxChunks], stride[kMaxChunks], order[kMaxChunks];
};

// Also requires the rows to tile [0, D) exactly, since the fast kernels write
// only the chunks' columns of dq and dk.
inline bool make_chunks(const AttnLayout& L, Chunks& C) {
  C.count = 0;
  if (L.D % 4 != 0) return false;
  bool seen[GM_ATTN_MAX_D] = {};
  for (int f = 0; f < L.F; ++f)
    for (int c = L.off[f]; c < L.off[f] + L.H * L.a[f] * L.dim[f]; ++c) {
      if (seen[c]) return false;
      seen[c] = true;
    }
  for (int c = 0; c < L.D; ++c)
    if (!seen[c]) return false;
  for (int f = 0; f < L.F; ++f) {
    const int width = L.a[f] * L.dim[f];
    if (width % 4 != 0 || L.off[f] % 4 != 0) return false;
    for (int u = 0; u < width; u += 4) {
      if (C.count == kMaxChunks) return false;
      C.base[C.count] = L.off[f] + u;
      C.stride[C.count] = width;
      C.order[C.count] = L.n[f];
      ++C.count;
    }
  }
  return C.count > 0;
}

}  // namespace gm
