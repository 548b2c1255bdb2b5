// Shared helpers for the HIP/CDNA4 (gfx950) recurrent-step library.
//
// Status codes returned by every extern "C" entry point (never exceptions
// across the ABI): 0 ok, negative = error class; hk_last_error() holds text.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#define HK_OK 0
#define HK_ERR_ARG (-1)       // bad shape / pointer / size (the reference asserts)
#define HK_ERR_HIP (-2)       // a HIP runtime call failed
#define HK_ERR_CAPACITY (-3)  // more rows / runs than the engine was sized for
#define HK_ERR_STATE (-4)     // engine used before weights were bound, etc.

namespace hk {

void set_error(const char* fmt, ...);

constexpr int kWave = 64;

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// softplus with torch's default beta=1, threshold=20: x above the threshold
// is returned unchanged, otherwise log1p(exp(x)).
__device__ __forceinline__ float softplus(float x) {
  return x > 20.0f ? x : log1pf(expf(x));
}

// log(sigmoid(x)) in the overflow-free form min(x, 0) - log1p(exp(-|x|)).
__device__ __forceinline__ float logsigmoid(float x) {
  return fminf(x, 0.0f) - log1pf(expf(-fabsf(x)));
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// Short-latency forms for the step-serial recurrences, on the hardware
// base-2 exponential / logarithm and reciprocal (v_exp_f32, v_log_f32,
// v_rcp_f32, each about 1 ulp): e^x = 2^(x log2 e), log1p(y) = log2(1 + y)
// ln 2. The rounding of x log2 e adds |x| * 2^-24 relative error to e^x
// (under 1e-6 for |x| < 16); log1p loses relative accuracy for y < 2^-24
// but keeps an absolute error under 2^-24, which is what logsigmoid needs.
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_logsigmoid(float x) {
  return fminf(x, 0.0f) - __builtin_amdgcn_logf(1.0f + fast_exp(-fabsf(x))) * 0.693147180559945309f;
}
__device__ __forceinline__ float fast_sigmoid(float x) { return fast_rcp(1.0f + fast_exp(-x)); }
// tanh z = sign(z) (1 - e) / (1 + e), e = e^{-2|z|} in (0, 1]: no overflow.
__device__ __forceinline__ float fast_tanh(float z) {
  const float e = fast_exp(-2.0f * fabsf(z));
  return copysignf((1.0f - e) * fast_rcp(1.0f + e), z);
}

__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

// Round-to-nearest-even fp32 -> bf16 bits (no NaN inputs on this path, but a
// NaN stays a NaN: the quiet bit is forced). The device converts with the
// hardware instruction (v_cvt_pk_bf16_f32 on gfx950): the kernels' float mode
// is round-to-nearest-even with subnormals kept, so it rounds every non-NaN
// input as the integer form below, which the host uses. That form is written
// as selects, not early returns.
__host__ __device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? ((u >> 16) | 0x40u) : r);
#endif
}

__host__ __device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

__host__ __device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

// Round-to-nearest-even fp32 -> IEEE binary16 bits, overflow to infinity
// (torch's fp32 -> fp16 cast). Normal results: drop 13 mantissa bits with a
// round-half-even bias, the carry stepping into the exponent. Subnormal
// results: adding 0.5 (whose ulp is 2^-24, the fp16 subnormal step) makes
// the fp32 adder round |f| to a multiple of 2^-24; the low bits of the sum
// are that multiple. Every case is computed and the result selected (no
// branches): NaN -> quiet NaN, |f| >= 65520 (rounds past 65504) or infinity
// -> infinity, |f| >= 2^-14 -> normal, else subnormal or zero. The device
// uses the hardware conversion (v_cvt_f16_f32), which rounds every non-NaN
// input the same way under the kernels' float mode (round-to-nearest-even,
// fp16 subnormals kept).
__host__ __device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (_Float16)f);
#else
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7fffffffu;
  const uint32_t r = a - 0x38000000u;  // rebias the exponent (127 -> 15)
  const uint32_t normal = (r + 0xfffu + ((r >> 13) & 1u)) >> 13;
  const uint32_t sub =
      __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, a) + 0.5f) - 0x3f000000u;
  uint32_t v = a >= 0x38800000u ? normal : sub;
  v = a >= 0x477ff000u ? 0x7c00u : v;
  v = a > 0x7f800000u ? 0x7e00u : v;
  return (uint16_t)(sign | v);
#endif
}

// fp16 bits -> fp32 (exact: every fp16 value is an fp32 value).
__host__ __device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
#if defined(__HIP_DEVICE_COMPILE__)
  return (float)__builtin_bit_cast(_Float16, h);
#else
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  // zero / subnormal: m * 2^-24, exact in fp32; infinity / NaN; normal
  const uint32_t sub = __builtin_bit_cast(uint32_t, (float)m * 5.9604644775390625e-08f);
  uint32_t v = e == 31u ? 0x7f800000u | (m << 13) : ((e + 112u) << 23) | (m << 13);
  v = e == 0u ? sub : v;
  return __builtin_bit_cast(float, sign | v);
#endif
}

// The 16-bit compute formats of CastLinear (example_model.py:150-155).
enum LpFmt : int { kLpBF16 = 0, kLpF16 = 1 };

__host__ __device__ __forceinline__ uint16_t f32_to_lp_bits(float f, int fmt) {
  return fmt == kLpF16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f);
}
__host__ __device__ __forceinline__ float round_lp(float f, int fmt) {
  return fmt == kLpF16 ? f16_bits_to_f32(f32_to_f16_bits(f)) : round_bf16(f);
}
// The same with the format fixed at compile time.
template <int FMT>
__host__ __device__ __forceinline__ uint16_t f32_to_lp_bits_t(float f) {
  return FMT == kLpF16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f);
}
template <int FMT>
__host__ __device__ __forceinline__ float round_lp_t(float f) {
  return FMT == kLpF16 ? f16_bits_to_f32(f32_to_f16_bits(f)) : round_bf16(f);
}

// Global-memory loads through explicit address-space-1 pointers. Pointers
// that reach a kernel inside an argument struct are generic to the compiler,
// which then emits flat loads (slower, and their waits also cover LDS);
// these helpers give global_load_* with scalar base addressing.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 gload16(const void* p) {
  return *(const __attribute__((address_space(1))) u32x4*)(p);
}
__device__ __forceinline__ float4 gload_f4(const float* p) {
  const u32x4 v = gload16(p);
  return make_float4(__builtin_bit_cast(float, v.x), __builtin_bit_cast(float, v.y),
                     __builtin_bit_cast(float, v.z), __builtin_bit_cast(float, v.w));
}
__device__ __forceinline__ float gload(const float* p) {
  return *(const __attribute__((address_space(1))) float*)(p);
}
__device__ __forceinline__ void gstore(float* p, float v) {
  *(__attribute__((address_space(1))) float*)(p) = v;
}

// Work-group barrier for communication through LDS only. __syncthreads()
// also orders global memory, which on gfx950 means waiting for every
// outstanding vector-memory load of the wave (s_waitcnt vmcnt(0)) and so
// drains any prefetch in flight; this one waits only for LDS operations.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wave-wide sum with DPP-free shuffles (xor butterfly over 64 lanes).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Wave sums of NV values at once (NV a power of two, <= 64): each level of
// the xor butterfly halves the values a lane keeps (lane bit d picks which
// half), so NV sums take NV - 1 + 6 - log2(NV) shuffles instead of 6 * NV.
// The result is the sum of value i = lane >> (6 - log2(NV)) over the wave:
// lane i * 64 / NV (and every lane of its group) holds sum i.
template <int NV>
__device__ __forceinline__ float transposed_wave_sum(float (&v)[NV]) {
  static_assert(NV >= 1 && NV <= 64 && (NV & (NV - 1)) == 0, "power of two up to 64");
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int n = NV, d = 32; n > 1; n >>= 1, d >>= 1) {
    const bool hi = (lane & d) != 0;
#pragma unroll
    for (int i = 0; i < n / 2; ++i) {
      // selects on values (not on element addresses, which the compiler may
      // turn into indexed private-memory accesses)
      const float lo_v = v[i], hi_v = v[n / 2 + i];
      const float keep = hi ? hi_v : lo_v;
      const float send = hi ? lo_v : hi_v;
      v[i] = keep + __shfl_xor(send, d, 64);
    }
  }
  float r = v[0];
#pragma unroll
  for (int d = 32 / NV; d >= 1; d >>= 1) r += __shfl_xor(r, d, 64);
  return r;
}

// Element i of the sum of n planes `stride` floats apart, added in plane
// order (split-row scan outputs).
__device__ __forceinline__ float plane_sum(const float* p, int64_t i, int n, int64_t stride) {
  float v = p[i];
  for (int q = 1; q < n; ++q) v += p[i + q * stride];
  return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `red` must hold
// blockDim.x / 64 floats of LDS. Every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  v = wave_sum(v);
  lds_barrier();
  if (lane == 0) red[wave] = v;
  lds_barrier();
  float t = 0.0f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

}  // namespace hk

#define HK_CHECK_HIP(expr)                                                        \
  do {                                                                            \
    hipError_t e_ = (expr);                                                       \
    if (e_ != hipSuccess) {                                                       \
      hk::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                    __LINE__);                                                    \
      return HK_ERR_HIP;                                                          \
    }                                                                             \
  } while (0)

#define HK_REQUIRE(cond, ...)     \
  do {                            \
    if (!(cond)) {                \
      hk::set_error(__VA_ARGS__); \
      return HK_ERR_ARG;          \
    }                             \
  } while (0)

#define HK_LAUNCH_CHECK()                                                              \
  do {                                                                                 \
    hipError_t e_ = hipGetLastError();                                                 \
    if (e_ != hipSuccess) {                                                            \
      hk::set_error("kernel launch failed: %s (%s:%d)", hipGetErrorString(e_), __FILE__, \
                    __LINE__);                                                         \
      return HK_ERR_HIP;                                                               \
    }                                                                                  \
  } while (0)
