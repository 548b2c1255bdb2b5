// Projection GEMM kernel (see gemm.h).
//
// 64x64 output tile per 256-thread work-group, 4 wave64s in a 2x2 layout,
// each wave owning a 32x32 sub-tile = 2x2 MFMA 16x16 fragments. K advances in
// 64-byte slabs (32 bf16 or 16 fp32) staged through LDS; the next slab is
// fetched into registers while the current one is multiplied. Rows are padded
// by 16 bytes in LDS so the 16-byte fragment reads of one wave spread over
// the banks.
//
// The flat work-group id is remapped so that consecutive tiles (the M tiles
// that share one slab of W) land on the same XCD and therefore the same L2:
// hardware dispatch sends work-group i to XCD i % 8.
//
// Split-K: with splits > 1 each split writes raw partial sums and a second
// kernel adds them in split order (deterministic) and applies the epilogue.
#include <algorithm>

#include "gemm.h"

namespace hk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BM = 64;
constexpr int BN = 64;

template <GemmType T>
struct Tr;
template <>
struct Tr<GemmType::kBF16> {
  using E = uint16_t;
  static constexpr int BK = 32;
};
template <>
struct Tr<GemmType::kF32> {
  using E = float;
  static constexpr int BK = 16;
};

__device__ __forceinline__ void apply_store(const GemmEpilogue& ep, float v, int m, int nc) {
  if (ep.bias) v += ep.bias[nc];
  if (ep.round_lp) v = round_bf16(v);
  if (ep.act == 1) v = fmaxf(v, 0.0f);
  if (ep.residual) v += ep.residual[(int64_t)m * ep.ldr + nc];
  if (ep.out) ep.out[(int64_t)m * ep.ldo + nc] = v;
  if (ep.out_lp) ep.out_lp[(int64_t)m * ep.ldl + nc] = f32_to_bf16_bits(v);
}

template <GemmType T>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g, float* partial, int splits,
                                                    int tiles_m, int tiles_n) {
  using E = typename Tr<T>::E;
  constexpr int BK = Tr<T>::BK;
  constexpr int EPC = 16 / sizeof(E);     // elements per 16-byte chunk
  constexpr int LROW = BK + EPC;          // padded LDS row, elements
  __shared__ __align__(16) E As[BM * LROW];
  __shared__ __align__(16) E Bs[BN * LROW];

  const int nwg = gridDim.x;
  int bid = blockIdx.x;
  const int full = (nwg / 8) * 8;
  if (bid < full) bid = (bid % 8) * (full / 8) + bid / 8;
  const int tm = bid % tiles_m;
  int rest = bid / tiles_m;
  const int tn = rest % tiles_n;
  rest /= tiles_n;
  const int split = rest % splits;
  const int b = rest / splits;

  const int tid = threadIdx.x;
  const int lrow = tid >> 2;
  const int lchk = tid & 3;
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const E* Ab = static_cast<const E*>(g.A) + (int64_t)b * g.a_bstride;
  const E* Wb = static_cast<const E*>(g.W) + (int64_t)b * g.w_bstride;
  const int a_row = (m0 + lrow) < g.M ? m0 + lrow : 0;
  const int w_row = (n0 + lrow) < g.N ? n0 + lrow : 0;
  const E* a_src = Ab + (int64_t)a_row * g.lda + lchk * EPC;
  const E* w_src = Wb + (int64_t)w_row * g.ldw + lchk * EPC;

  const int ktiles = g.K / BK;
  const int per = (ktiles + splits - 1) / splits;
  const int kt0 = split * per;
  const int kt1 = min(ktiles, kt0 + per);

  // Register ring of kRing K-slabs: the load of slab kt+kRing is issued when
  // slab kt is consumed, so each load has kRing-1 slabs of MFMA work to land.
  // The loop is unrolled by kRing so every ring index is a compile-time
  // constant (the ring stays in VGPRs), and the barriers wait on LDS only.
  constexpr int kRing = 4;
  // Loads are unconditional so the wait counts stay static: rows past M or N
  // read row 0 (their products land only in output rows/columns that are
  // never stored), and slabs past the split's end re-read its last slab.
  const int kt_last = max(kt1 - 1, 0);
  u32x4 ra[kRing], rw[kRing];
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    const int kt = min(kt0 + j, kt_last);
    ra[j] = gload16(a_src + (int64_t)kt * BK);
    rw[j] = gload16(w_src + (int64_t)kt * BK);
  }

  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int fr = lane & 15;   // fragment row (A) / column (B)
  const int fk = lane >> 4;   // k group within the MFMA
  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int kb = kt0; kb < kt1; kb += kRing) {
#pragma unroll
    for (int j = 0; j < kRing; ++j) {
      const int kt = kb + j;
      if (kt < kt1) {
        *reinterpret_cast<u32x4*>(&As[lrow * LROW + lchk * EPC]) = ra[j];
        *reinterpret_cast<u32x4*>(&Bs[lrow * LROW + lchk * EPC]) = rw[j];
        lds_barrier();
        {
          const int nk = min(kt + kRing, kt_last);
          ra[j] = gload16(a_src + (int64_t)nk * BK);
          rw[j] = gload16(w_src + (int64_t)nk * BK);
        }
        if constexpr (T == GemmType::kBF16) {
          bf16x8 af[2], bfr[2];
#pragma unroll
          for (int i = 0; i < 2; ++i)
            af[i] = *reinterpret_cast<const bf16x8*>(&As[(wm * 32 + i * 16 + fr) * LROW + fk * 8]);
#pragma unroll
          for (int q = 0; q < 2; ++q)
            bfr[q] = *reinterpret_cast<const bf16x8*>(&Bs[(wn * 32 + q * 16 + fr) * LROW + fk * 8]);
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q)
              acc[i][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[q], acc[i][q], 0, 0, 0);
        } else {
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4) {
            float af[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) af[i] = As[(wm * 32 + i * 16 + fr) * LROW + s4 * 4 + fk];
#pragma unroll
            for (int q = 0; q < 2; ++q) bfr[q] = Bs[(wn * 32 + q * 16 + fr) * LROW + s4 * 4 + fk];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
              for (int q = 0; q < 2; ++q)
                acc[i][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bfr[q], acc[i][q], 0, 0, 0);
          }
        }
        lds_barrier();
      }
    }
  }

  // Fragment (i, j): lane holds rows 4*fk + e, column fr.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 32 + j * 16 + fr;
      if (n >= g.N) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * 32 + i * 16 + fk * 4 + e;
        if (m >= g.M) continue;
        const float v = acc[i][j][e];
        if (splits == 1) {
          apply_store(g.ep, v, m, n + (int)((int64_t)b * g.c_bstride));
        } else {
          partial[(((int64_t)b * splits + split) * g.M + m) * g.N + n] = v;
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs g, const float* partial,
                                                            int splits) {
  const int64_t total = (int64_t)g.batch * g.M * g.N;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int n = (int)(idx % g.N);
    const int64_t bm = idx / g.N;
    const int m = (int)(bm % g.M);
    const int b = (int)(bm / g.M);
    const float* p = partial + ((int64_t)b * splits * g.M + m) * g.N + n;
    float v = 0.0f;
    for (int s = 0; s < splits; ++s) v += p[(int64_t)s * g.M * g.N];
    apply_store(g.ep, v, m, n + (int)((int64_t)b * g.c_bstride));
  }
}

}  // namespace

int gemm(const GemmArgs& g, const GemmWorkspace& ws, hipStream_t stream, int splits_hint) {
  HK_REQUIRE(g.A && g.W && (g.ep.out || g.ep.out_lp), "gemm: null operand");
  HK_REQUIRE(g.M >= 0 && g.N > 0 && g.K > 0 && g.batch > 0, "gemm: bad shape M=%d N=%d K=%d",
             g.M, g.N, g.K);
  const int BK = g.type == GemmType::kBF16 ? Tr<GemmType::kBF16>::BK : Tr<GemmType::kF32>::BK;
  const int align = g.type == GemmType::kBF16 ? 8 : 4;
  HK_REQUIRE(g.K % BK == 0, "gemm: K=%d is not a multiple of %d", g.K, BK);
  HK_REQUIRE(g.lda % align == 0 && g.ldw % align == 0 && g.a_bstride % align == 0 &&
                 g.w_bstride % align == 0,
             "gemm: leading dimensions must keep 16-byte alignment");
  if (g.M == 0) return HK_OK;
  const int tiles_m = (g.M + BM - 1) / BM;
  const int tiles_n = (g.N + BN - 1) / BN;
  const int64_t tiles = (int64_t)tiles_m * tiles_n * g.batch;
  const int ktiles = g.K / BK;
  int splits = splits_hint;
  if (splits <= 0) {
    splits = (int)((1024 + tiles - 1) / tiles);
    splits = std::min(splits, std::max(1, ktiles / 4));
    splits = std::min(splits, 32);
  }
  splits = std::max(1, std::min(splits, ktiles));
  while (splits > 1 && (int64_t)splits * g.batch * g.M * g.N > ws.partial_elems) --splits;
  const int64_t nwg = tiles * splits;
  HK_REQUIRE(nwg < (1LL << 31), "gemm: grid too large");
  if (g.type == GemmType::kBF16) {
    hipLaunchKernelGGL(gemm_kernel<GemmType::kBF16>, dim3((unsigned)nwg), dim3(256), 0, stream,
                       g, ws.partial, splits, tiles_m, tiles_n);
  } else {
    hipLaunchKernelGGL(gemm_kernel<GemmType::kF32>, dim3((unsigned)nwg), dim3(256), 0, stream, g,
                       ws.partial, splits, tiles_m, tiles_n);
  }
  HK_LAUNCH_CHECK();
  if (splits > 1) {
    const int64_t total = (int64_t)g.batch * g.M * g.N;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, g, ws.partial,
                       splits);
    HK_LAUNCH_CHECK();
  }
  return HK_OK;
}

}  // namespace hk
