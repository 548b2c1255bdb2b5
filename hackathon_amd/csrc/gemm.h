// Projection GEMMs on gfx950 matrix cores: Y[M,N] = A[M,K] . W[N,K]^T with a
// fused epilogue. Three operand types share one kernel template:
//   bf16 (v_mfma_f32_16x16x32_bf16) and fp16 (v_mfma_f32_16x16x32_f16) - the
//        reduced-precision linears, output rounded to the operand format
//        after the bias add exactly as CastLinear does
//        (example_model.py:92-95);
//   fp32 (v_mfma_f32_16x16x4_f32)   - the fp32 path and the linears kept fp32
//        (example_model.py:106), plus the fp32 BlockLinear products
//        (model/modules.py:71-79), batched over the diagonal blocks; with
//        GemmArgs::split_wscale set, the same fp32 operands multiply on f16
//        matrix cores as value plus remainder (v_mfma_f32_16x16x32_f16).
// fp32 products of at most 16 rows (any batch description, every epilogue;
// split_wscale is not used there: exact fp32), and packed 16-bit
// projections of at most 16 rows, run on kernels of their own that stream W
// through registers without splitting K.
#pragma once

#include "common.h"

namespace hk {

enum class GemmType { kBF16 = 0, kF32 = 1, kF16 = 2 };

// Work-group counts of the packed kernel's tile rule (measured on the
// ensemble's projection shapes): alone on the device, 160 (most of the 256
// CUs; CastLinear replay 14.8 us per launch against 16.6 at 112); inside a
// four-stream tick, 112 for GEMMs of more than 64 rows (larger tiles re-read
// less and crowd the other streams less: C4 tick 9.21-9.24 ms against
// 9.34-9.37 at 160).
constexpr int kMinTilesAlone = 160;
constexpr int kMinTilesShared = 112;

struct GemmEpilogue {
  const float* bias = nullptr;      // [N] (per batch: + b*c_bstride)
  const float* residual = nullptr;  // [M, ldr] added last
  int64_t ldr = 0;
  float* out = nullptr;             // fp32 result [M, ldo]
  int64_t ldo = 0;
  uint16_t* out_lp = nullptr;       // optional 16-bit copy [M, ldl] in format lp_fmt
  int64_t ldl = 0;
  int lp_fmt = kLpBF16;             // LpFmt of round_lp and out_lp
  bool round_lp = false;            // round (acc + bias) to lp_fmt first
  int act = 0;                      // 0 none, 1 relu (after rounding)
  // Mamba2's dt (model/mamba2.py:92-97), fp32 products only: with dt_a set
  // the result is dt = softplus(acc + bias) (in out), and
  // dt_decay[m, n] = exp(dt_a[n] * dt).
  const float* dt_a = nullptr;
  float* dt_decay = nullptr;
  int64_t ldd = 0;
};

struct GemmArgs {
  GemmType type = GemmType::kBF16;
  const void* A = nullptr;  // [M, lda] of bf16, fp16 or fp32
  int64_t lda = 0;
  const void* W = nullptr;  // [N, ldw] of bf16, fp16 or fp32
  int64_t ldw = 0;
  int M = 0, N = 0, K = 0;
  // Block-diagonal batches: batch b reads A + b*a_bstride (elements), W +
  // b*w_bstride, and writes columns offset by b*c_bstride.
  int batch = 1;
  int64_t a_bstride = 0, w_bstride = 0, c_bstride = 0;
  // Optional, for batches of blocks over two inputs: batch b >= a2_from
  // reads A2 instead of A, and with a_period > 0 the A offset is
  // (b % a_period) * a_bstride (W and the output still step by b).
  const void* A2 = nullptr;
  int a2_from = 0;
  int a_period = 0;
  // 16-bit W held in the fragment-packed layout of pack_lp_weight (ldw is
  // then unused; N and K must be multiples of 32 and 64).
  bool w_packed = false;
  // Packed kernel's tile rule: the largest tile that still gives at least
  // this many work-groups without splitting K (0: kMinTilesAlone, for a GEMM
  // that has the device to itself; the engine's ticks, where three other
  // streams share the device, pass kMinTilesShared).
  int min_tiles = 0;
  // fp32 operands only: > 0 runs the product on f16 matrix cores, each
  // operand as an f16 value plus its f16 remainder (hi.hi + hi.lo + lo.hi,
  // fp32 accumulation), W multiplied by this power of two first and the
  // result by its inverse (the caller picks it so that |w| * scale < 2^14);
  // A must stay below 65504 in magnitude.
  float split_wscale = 0.0f;
  GemmEpilogue ep;
};

// Split-K state of one stream's GEMMs (the GEMMs of one workspace must not
// overlap in time). `arrivals` holds one counter per output tile, zero
// between launches: the kernel's last split of a tile resets it.
struct GemmWorkspace {
  float* partial = nullptr;  // split-K partial sums
  int64_t partial_elems = 0;
  int* arrivals = nullptr;   // zero-initialised by the owner
  int64_t arrival_elems = 0;
};

// K must be a multiple of 64 (bf16, fp16) or 16 (fp32); lda/ldw multiples of 8 / 4.
int gemm(const GemmArgs& g, const GemmWorkspace& ws, hipStream_t stream, int splits_hint = 0);

// Packed layout of a 16-bit weight W[N][K] (row-major, ldw = K) for the
// matrix cores: 16-bit element (n, k) goes to
//   ((((n / 32) * (K / 32) + k / 32) * 2 + (n % 32) / 16) * 64 + lane) * 8 + k % 8,
//   lane = n % 16 + 16 * ((k % 32) / 8),
// i.e. for each 32-column block, each 32-deep k block is two 1 KB MFMA B
// fragments (16 columns each) in lane order, and the 64-deep slab a wave
// multiplies is 4 KB contiguous. N must be a multiple of 32, K of 64.
bool packable(int N, int K);
int pack_lp_weight(const uint16_t* src, uint16_t* dst, int N, int K, hipStream_t stream);
// fp32 rows [rows][K] (rows a multiple of 32) -> rounded to format fmt and
// packed (the packed rows r .. r + rows of a larger W start at r*K).
int pack_f32_to_lp(const float* src, uint16_t* dst, int rows, int K, int fmt, hipStream_t stream);

}  // namespace hk
