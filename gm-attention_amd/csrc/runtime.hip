// Error state and version of libgmhip.so.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "common.hpp"
#include "layout.hpp"

namespace gm {

namespace {
thread_local std::string last_error;
}

void set_error(const std::string& message) { last_error = message; }

int fail(int code, const std::string& message) {
  last_error = message;
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(GM_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(err));
  return GM_OK;
}

int64_t resident_blocks(const void* kernel, int threads, size_t lds) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int64_t> cache;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();  // not left for the next launch check
    return 0;
  }
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(dev, kernel);
  const auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int cus = 0, per = 0;
  int64_t slots = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, lds) == hipSuccess)
    slots = (int64_t)cus * per;
  else
    (void)hipGetLastError();
  cache[key] = slots;
  return slots;
}

int parse_attention_layout(const int64_t* desc, int64_t F, int64_t H, int64_t D, int64_t orders, AttnLayout& L) {
  GM_REQUIRE(desc != nullptr, "desc must be a host pointer to (F, 5) int64");
  GM_REQUIRE(F >= 0 && F <= GM_ATTN_MAX_F, "desc must have at most 8 frequency rows");
  GM_REQUIRE(H >= 1 && H <= GM_ATTN_MAX_H, "at most 16 heads");
  GM_REQUIRE(D >= 1 && D <= GM_ATTN_MAX_D, "D must be in [1, 1024]");
  GM_REQUIRE(orders >= 1, "the phase tables need at least one order");
  L.F = (int)F;
  L.H = (int)H;
  L.D = (int)D;
  L.orders = (int)orders;
  L.head_width = 0;
  for (int f = 0; f < F; ++f) {
    const int64_t* row = desc + f * GM_ATTN_DESC;
    const int64_t n = row[0], a = row[1], off = row[2], coff = row[3], dim = row[4];
    GM_REQUIRE(n >= 0 && n < orders, "a descriptor frequency exceeds the phase tables");
    GM_REQUIRE(dim == (n == 0 ? 1 : 2), "descriptor dim must be 1 at frequency 0 and 2 above");
    GM_REQUIRE(a >= 0 && off >= 0 && coff >= 0, "descriptor entries must be non-negative");
    GM_REQUIRE(off + H * a * dim <= D, "a descriptor row runs past the flat width D");
    L.n[f] = (int)n;
    L.a[f] = (int)a;
    L.off[f] = (int)off;
    L.coff[f] = (int)coff;
    L.dim[f] = (int)dim;
    L.head_width += (int)(a * dim);
  }
  return GM_OK;
}

}  // namespace gm

extern "C" const char* gm_last_error(void) { return gm::last_error.c_str(); }

extern "C" int gm_abi_version(void) { return 3; }

extern "C" int gm_xcd_block_map(int64_t nb, int kind, const int64_t* ptr, int64_t n_items, int per, int64_t* out) {
  GM_REQUIRE(nb >= 1 && out != nullptr, "nb must be positive and out a host array of nb entries");
  GM_REQUIRE(kind >= 0 && kind <= 2, "kind must be 0 (contiguous), 1 (spread) or 2 (balanced)");
  GM_REQUIRE(kind != 2 || (ptr != nullptr && n_items >= 1 && per >= 1), "the balanced map needs the CSR offsets");
  for (int64_t b = 0; b < nb; ++b)
    out[b] = kind == 0 ? gm::xcd_block(b, nb)
                       : (kind == 1 ? gm::xcd_spread_block(b, nb) : gm::xcd_balanced_block(b, nb, ptr, n_items, per));
  return GM_OK;
}
