// Deterministic, counter-based parameter initialisation on the host.
//
// The reference leaves several parameters as torch.empty (model/modules.py:63-69,
// model/hawk.py:16, model/retnet.py:35-36) and fills everything from a
// checkpoint. "Random-init weights, seed 0" therefore needs an explicit spec:
// every element is a pure function of (seed, parameter name, element index),
//   key  = mix64(fnv1a64(name) ^ mix64(seed))
//   bits = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)       (splitmix64 finaliser)
//   u    = (bits >> 40) * 2^-24                              (exact in fp32)
//   v    = lo + (hi - lo) * u                                (fp32, two roundings)
// so any machine regenerates bit-identical weights without shipping them.
// The per-parameter ranges restate check_cell_rewrite.py:187-210.
#include <algorithm>
#include <cstdint>
#include <thread>
#include <vector>

#include "common.h"

namespace {

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

#pragma clang fp contract(off)
void fill_range(float* dst, int64_t begin, int64_t end, uint64_t key, float lo, float hi) {
  const float span = hi - lo;
  for (int64_t i = begin; i < end; ++i) {
    const uint64_t bits = mix64(key + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ULL);
    const float u = (float)(bits >> 40) * 0x1p-24f;
    const float p = span * u;
    dst[i] = lo + p;
  }
}

}  // namespace

extern "C" {

uint64_t hk_param_key(uint64_t seed, const char* name) {
  uint64_t h = 0xcbf29ce484222325ULL;
  for (const unsigned char* p = (const unsigned char*)name; *p; ++p) {
    h ^= *p;
    h *= 0x100000001b3ULL;
  }
  return mix64(h ^ mix64(seed));
}

int hk_fill_uniform_host(float* dst, int64_t n, uint64_t key, float lo, float hi, int threads) {
  HK_REQUIRE(dst != nullptr || n == 0, "hk_fill_uniform_host: null destination");
  HK_REQUIRE(n >= 0, "hk_fill_uniform_host: negative size");
  threads = std::max(1, std::min(threads, 64));
  const int64_t min_chunk = 1 << 20;
  const int64_t nt = std::max<int64_t>(1, std::min<int64_t>(threads, (n + min_chunk - 1) / min_chunk));
  if (nt == 1) {
    fill_range(dst, 0, n, key, lo, hi);
    return HK_OK;
  }
  std::vector<std::thread> pool;
  const int64_t per = (n + nt - 1) / nt;
  for (int64_t t = 0; t < nt; ++t) {
    const int64_t b = t * per, e = std::min(n, b + per);
    if (b >= e) break;
    pool.emplace_back(fill_range, dst, b, e, key, lo, hi);
  }
  for (auto& th : pool) th.join();
  return HK_OK;
}

// Host conversion to the CastLinear 16-bit formats, with the same routine
// the kernels use (common.h).
int hk_to_lp_host(const float* src, uint16_t* dst, int64_t n, int fmt) {
  HK_REQUIRE((src && dst) || n == 0, "hk_to_lp_host: null argument");
  HK_REQUIRE(n >= 0 && (fmt == hk::kLpBF16 || fmt == hk::kLpF16),
             "hk_to_lp_host: bad size or format %d", fmt);
  for (int64_t i = 0; i < n; ++i) dst[i] = hk::f32_to_lp_bits(src[i], fmt);
  return HK_OK;
}

}  // extern "C"
