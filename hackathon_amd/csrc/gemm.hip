// Projection GEMM kernels (see gemm.h). Four kernels:
// - gemm_wp_kernel, for the engine's 16-bit CastLinear projections, whose
//   weights are stored packed in MFMA fragment order (described at the
//   kernel);
// - gemm_kernel, below, for fp32 products (the fp32 mode's linears and the
//   BlockLinear batches) and 16-bit weights in row-major layout;
// - gemm_skinny_kernel and gemm_skinny_wp_kernel, for fp32 products and
//   packed 16-bit projections of at most 16 rows (described at the kernels).
//
// gemm_kernel: 64x64 output tile per 256-thread work-group, 4 wave64s in a 2x2 layout,
// each wave owning a 32x32 sub-tile = 2x2 MFMA 16x16 fragments. K advances in
// 128-byte slabs (64 bf16/fp16 or 32 fp32 per row) that travel global -> LDS
// directly (global_load_lds_dwordx4) through a ring of kStages LDS stages,
// with one barrier per slab and counted vmcnt waits, so kStages - 2 slabs stay
// in flight behind the one being multiplied. Three stages (48 KB) measure as
// fast as four to six (the L2 -> LDS rate per CU, not latency, bounds a
// slab) and let three work-groups share a CU, so launches of just over 256
// or 512 work-groups leave no tail round. Chunks are XOR-swizzled within a
// row so the 16-byte fragment reads of one wave spread over the LDS banks.
//
// The flat work-group id is remapped so that consecutive tiles (the M tiles
// that share one slab of W) land on the same XCD and therefore the same L2:
// hardware dispatch sends work-group i to XCD i % 8.
//
// Split-K: with splits > 1 each split writes its raw partial sums with
// agent-coherent stores, waits until they have landed and counts itself in at
// the tile's arrival counter. The split that arrives last reads the other
// partials back (agent-coherent loads), adds all of them in split order
// (deterministic, independent of arrival order), applies the epilogue and
// resets the counter for the next launch.
#include <algorithm>
#include <cmath>

#include "gemm.h"

namespace hk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BM = 64;
constexpr int BN = 64;
#ifndef HK_GEMM_STAGES
#define HK_GEMM_STAGES 3
#endif
constexpr int kStages = HK_GEMM_STAGES;  // LDS ring depth (16 KB per stage)

template <GemmType T>
struct Tr;
template <>
struct Tr<GemmType::kBF16> {
  using E = uint16_t;
  static constexpr int BK = 64;       // 128-byte slab rows
};
template <>
struct Tr<GemmType::kF16> {
  using E = uint16_t;
  static constexpr int BK = 64;       // 128-byte slab rows
};
template <>
struct Tr<GemmType::kF32> {
  using E = float;
  static constexpr int BK = 32;       // 128-byte slab rows
  static constexpr int BK_NARROW = 16;  // for K a multiple of 16 only
};

typedef const __attribute__((address_space(1))) void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

// Raw buffer resource word 3 (gfx9: 32-bit data format, no stride, no
// swizzle), and the cache-policy operand of a buffer access that is coherent
// across the device's XCDs (sc1, as agent-scope atomics compile to).
constexpr int kBufWord3 = 0x00020000;
constexpr int kCoherentSc1 = 16;

// LDS address (byte offset) of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// 16-byte LDS read issued as inline asm: LDS written by global_load_lds
// transfers is outside what the compiler can order exactly across the
// pipelined loop (it would wait for every transfer in flight before each
// read), so the reads are hidden from it and ordered by hand: the transfers
// by the counted vmcnt wait before the stage's barrier, the reads by
// ds_wait4 below, which also ties the read registers to their uses.
__device__ __forceinline__ u32x4 ds_read16(uint32_t addr) {
  u32x4 v;
  __asm__ volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ void ds_wait4(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : : "memory");
}

// s_waitcnt with only the vector-memory count constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// vmcnt(k * D) for a runtime k in [0, S-2].
template <int D, int S>
__device__ __forceinline__ void wait_slabs(int k) {
  static_assert(S <= 6, "stages");
  if (k >= S - 2) {
    wait_vmcnt<(S - 2) * D>();
  } else if (k == 3) {
    wait_vmcnt<3 * D>();
  } else if (k == 2) {
    wait_vmcnt<2 * D>();
  } else if (k == 1) {
    wait_vmcnt<D>();
  } else {
    wait_vmcnt<0>();
  }
}

// Eight fp32 values (two groups of four) * scale as f16 values (hi) and the
// f16 of their remainders (lo): hi + lo holds 22 significant bits of each.
__device__ __forceinline__ void split_f16x8(u32x4 a, u32x4 b, float scale, halfx8& hi,
                                            halfx8& lo) {
  const floatx4 fa = __builtin_bit_cast(floatx4, a), fb = __builtin_bit_cast(floatx4, b);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x0 = fa[e] * scale, x1 = fb[e] * scale;
    const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
    hi[e] = h0;
    hi[4 + e] = h1;
    lo[e] = (_Float16)(x0 - (float)h0);
    lo[4 + e] = (_Float16)(x1 - (float)h1);
  }
}

template <GemmType T, int BK, int S, bool SPLIT = false>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g, float* partial, int* arrivals,
                                                    int splits, int tiles_m, int tiles_n) {
  using E = typename Tr<T>::E;
  constexpr int EPC = 16 / sizeof(E);   // elements per 16-byte chunk
  constexpr int CPR = BK / EPC;         // chunks per slab row (8, or 4 when narrow)
  constexpr int ROWB = CPR * 16;        // bytes per slab row
  constexpr int OPB = BM * ROWB;        // bytes of one operand's slab
  constexpr int STB = 2 * OPB;          // one stage: the A and the W slab
  constexpr int RPC = 64 / CPR;         // slab rows per 1 KB wave transfer
  constexpr int CPW = BM / RPC / 4;     // transfers per wave per operand
  constexpr int SWM = CPR - 1;          // swizzle mask
  constexpr int D = 2 * CPW;            // transfers per wave per slab
  static_assert(S >= 3 && S <= 6, "stages");
  // One LDS array per stage: with the stage index a compile-time constant
  // the compiler can tell a read of one stage from a transfer into another
  // and adds no wait of its own.
  __shared__ __align__(16) unsigned char st0[STB], st1[STB], st2[STB], st3[STB], st4[STB],
      st5[STB];
  unsigned char* const stage[6] = {st0, st1, st2, st3, st4, st5};

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
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const void* Asrc = (g.A2 != nullptr && b >= g.a2_from) ? g.A2 : g.A;
  const E* Ab = static_cast<const E*>(Asrc) +
                (int64_t)(g.a_period > 0 ? b % g.a_period : b) * g.a_bstride;
  const E* Wb = static_cast<const E*>(g.W) + (int64_t)b * g.w_bstride;

  // Slabs travel global -> LDS directly (global_load_lds_dwordx4): lane l of
  // a wave's 1 KB transfer lands at byte 16*l, i.e. slab row q*RPC + l/CPR,
  // physical chunk l % CPR, which holds logical chunk
  // (l % CPR) ^ ((row >> 1) & SWM). The XOR spreads the 16 rows one MFMA
  // fragment read touches over distinct banks. Rows past M or N read row 0
  // (their products reach only outputs that are never stored).
  const E* a_src[CPW];
  const E* w_src[CPW];
  int xoff[CPW];  // LDS byte offset of the wave's transfer within an operand slab
#pragma unroll
  for (int h = 0; h < CPW; ++h) {
    const int q = wave * CPW + h;
    const int row = q * RPC + lane / CPR;
    const int lc = (lane % CPR) ^ ((row >> 1) & SWM);
    const int ar = m0 + row, wr = n0 + row;
    a_src[h] = Ab + (int64_t)(ar < g.M ? ar : 0) * g.lda + lc * EPC;
    w_src[h] = Wb + (int64_t)(wr < g.N ? wr : 0) * g.ldw + lc * EPC;
    xoff[h] = q * 1024;
  }

  const int ktiles = g.K / BK;
  const int per = (ktiles + splits - 1) / splits;
  const int kt0 = split * per;
  const int kt1 = min(ktiles, kt0 + per);
  const int nslab = max(kt1 - kt0, 0);
  // Every slab is D transfers per wave; the wait before slab i allows the
  // transfers of the slabs issued after it (at most S-2) to stay in flight.
  auto issue = [&](unsigned char* st, int kt) {
#pragma unroll
    for (int h = 0; h < CPW; ++h) {
      __builtin_amdgcn_global_load_lds((gptr_t)(a_src[h] + (int64_t)kt * BK),
                                       (lptr_t)(st + xoff[h]), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((gptr_t)(w_src[h] + (int64_t)kt * BK),
                                       (lptr_t)(st + OPB + xoff[h]), 16, 0, 0);
    }
  };

  const int fr = lane & 15;   // fragment row (A) / column (B)
  const int fk = lane >> 4;   // k group within the MFMA
  const int wm = wave >> 1;
  const int wn = wave & 1;
  // Byte offsets of this lane's fragment rows within a stage, and their
  // swizzle keys.
  uint32_t arow[2], brow[2];
  int akey[2], bkey[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ra = wm * 32 + i * 16 + fr, rb = wn * 32 + i * 16 + fr;
    arow[i] = ra * ROWB;
    brow[i] = OPB + rb * ROWB;
    akey[i] = (ra >> 1) & SWM;
    bkey[i] = (rb >> 1) & SWM;
  }
  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // The bias of this lane's two output columns, fetched before the slabs
  // (older than every transfer, so the counted waits cover it too).
  float bias_v[2] = {0.0f, 0.0f};
  if (g.ep.bias) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 32 + j * 16 + fr;
      if (n < g.N) bias_v[j] = g.ep.bias[n + (int)((int64_t)b * g.c_bstride)];
    }
  }

#pragma unroll
  for (int s2 = 0; s2 < S - 1; ++s2)
    if (s2 < nslab) issue(stage[s2], kt0 + s2);

  for (int kb = 0; kb < nslab; kb += S) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int i = kb + j;
      if (i < nslab) {
        // Slab i is complete once at most the S-2 later slabs' transfers are
        // outstanding; the barrier then also shows every wave's transfers and
        // retires all reads of stage (j - 1) mod S, the next transfer's target.
        // (A raw s_barrier: a workgroup fence would also wait for every LDS
        // transfer in flight. The empty asm blocks keep LDS accesses from
        // moving across it; earlier reads have retired before their MFMAs.)
        wait_slabs<D, S>(min(S - 2, nslab - 1 - i));
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        if (i + S - 1 < nslab) issue(stage[(j + S - 1) % S], kt0 + i + S - 1);
        const uint32_t st = lds_addr(stage[j]);
        if constexpr (SPLIT) {
          // fp32 operands on f16 matrix cores: a lane's 8 values of a row
          // (k = 4*fk + c and 16 + 4*fk + c; A and B share the map, which
          // is all the product needs) become an f16 value plus its f16
          // remainder each (W scaled by a power of two first), and
          // hi.hi + hi.lo + lo.hi accumulate in fp32 (v_mfma_f32_16x16x32_f16).
          u32x4 fa[2][2], fb[2][2];  // [ks][fragment]
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            fa[ks][0] = ds_read16(st + arow[0] + (((ks * 4 + fk) ^ akey[0]) << 4));
            fa[ks][1] = ds_read16(st + arow[1] + (((ks * 4 + fk) ^ akey[1]) << 4));
            fb[ks][0] = ds_read16(st + brow[0] + (((ks * 4 + fk) ^ bkey[0]) << 4));
            fb[ks][1] = ds_read16(st + brow[1] + (((ks * 4 + fk) ^ bkey[1]) << 4));
          }
          ds_wait4(fa[0][0], fa[0][1], fb[0][0], fb[0][1]);
          ds_wait4(fa[1][0], fa[1][1], fb[1][0], fb[1][1]);
          halfx8 ahi[2], alo[2], bhi[2], blo[2];
#pragma unroll
          for (int i2 = 0; i2 < 2; ++i2) {
            split_f16x8(fa[0][i2], fa[1][i2], 1.0f, ahi[i2], alo[i2]);
            split_f16x8(fb[0][i2], fb[1][i2], g.split_wscale, bhi[i2], blo[i2]);
          }
#pragma unroll
          for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              acc[ii][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[ii], bhi[q], acc[ii][q], 0, 0, 0);
              acc[ii][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[ii], blo[q], acc[ii][q], 0, 0, 0);
              acc[ii][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[ii], bhi[q], acc[ii][q], 0, 0, 0);
            }
        } else {
#pragma unroll
        for (int ks = 0; ks < BK * (int)sizeof(E) / 64; ++ks) {
          // Four 16-byte fragment reads (A rows i, B columns i) of one
          // 64-byte k step, issued together; see ds_read16.
          u32x4 fa0 = ds_read16(st + arow[0] + (((ks * 4 + fk) ^ akey[0]) << 4));
          u32x4 fa1 = ds_read16(st + arow[1] + (((ks * 4 + fk) ^ akey[1]) << 4));
          u32x4 fb0 = ds_read16(st + brow[0] + (((ks * 4 + fk) ^ bkey[0]) << 4));
          u32x4 fb1 = ds_read16(st + brow[1] + (((ks * 4 + fk) ^ bkey[1]) << 4));
          ds_wait4(fa0, fa1, fb0, fb1);
          const u32x4 fa[2] = {fa0, fa1}, fb[2] = {fb0, fb1};
          if constexpr (T == GemmType::kBF16) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
              for (int q = 0; q < 2; ++q)
                acc[ii][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, fa[ii]), __builtin_bit_cast(bf16x8, fb[q]),
                    acc[ii][q], 0, 0, 0);
          } else if constexpr (T == GemmType::kF16) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
              for (int q = 0; q < 2; ++q)
                acc[ii][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(halfx8, fa[ii]), __builtin_bit_cast(halfx8, fb[q]),
                    acc[ii][q], 0, 0, 0);
          } else {
            // k-step (ks, c) of a lane in k group fk covers k = 16*ks + 4*fk
            // + c for A and B alike, so one 16-byte read feeds four MFMAs.
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
              const floatx4 av = __builtin_bit_cast(floatx4, fa[ii]);
#pragma unroll
              for (int q = 0; q < 2; ++q) {
                const floatx4 bv = __builtin_bit_cast(floatx4, fb[q]);
                acc[ii][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc[ii][q], 0, 0, 0);
                acc[ii][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc[ii][q], 0, 0, 0);
                acc[ii][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc[ii][q], 0, 0, 0);
                acc[ii][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc[ii][q], 0, 0, 0);
              }
            }
          }
        }
        }
      }
    }
  }
  // (Every transfer was waited for before its slab; nothing is in flight.)
  if constexpr (SPLIT) {
    const float inv = 1.0f / g.split_wscale;  // a power of two: exact
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] *= inv;
  }

  // Fragment (i, j): lane holds rows 4*fk + e, column fr.
  if (splits > 1) {
    // (The host keeps splits * batch * M * N within the int range.)
    const int MN = g.M * g.N;
    float* const pb = partial + (int64_t)b * splits * MN;
    int off[2][2][4];  // this lane's elements within one split's [M, N]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int n = n0 + wn * 32 + j * 16 + fr;
          const int m = m0 + wm * 32 + i * 16 + fk * 4 + e;
          off[i][j][e] = (n < g.N && m < g.M) ? m * g.N + n : -1;
        }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (off[i][j][e] >= 0)
            __hip_atomic_store(pb + split * MN + off[i][j][e], acc[i][j][e], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    // Release side: the partials are stored with agent scope (sc1, written
    // through this XCD's L2), so once every lane's stores are acknowledged
    // (vmcnt 0) and every wave has passed the barrier, they are visible to
    // any XCD before the tile counter sees this split. An agent-scope
    // release fence would also write back the whole L2 (buffer_wbl2): the
    // CastLinear replay measured 16.6 against 13.8 us per launch with one.
    wait_vmcnt<0>();
    __shared__ int last_split;
    __syncthreads();
    int* const arrival = arrivals + ((int64_t)b * tiles_n + tn) * tiles_m + tm;
    if (tid == 0)
      last_split = __hip_atomic_fetch_add(arrival, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
    __syncthreads();
    if (!last_split) return;
    // Acquire side: the last split's loads of the other partials are
    // issued only after the counter's returned value (through LDS and the
    // barrier) selected this work-group, and they are agent-scope loads
    // (sc1) that no line of this CU's L1 or of a non-coherent L2 state
    // serves. An agent-scope acquire fence here would also invalidate the
    // XCD's L2 (buffer_inv sc1): the CastLinear replay measured 0.199
    // against 0.210 of HBM peak, and the C4 tick 8.78 against 8.70 ms.
    if (tid == 0) __hip_atomic_store(arrival, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Sum in split order, four splits' loads in flight at a time; this
    // split's own part comes from its registers.
    floatx4 sum[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) sum[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < splits; s0 += 4) {
      float t[4][2][2][4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int sp = s0 + q;
        const bool other = sp < splits && sp != split;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              t[q][i][j][e] = (other && off[i][j][e] >= 0)
                                  ? __hip_atomic_load(pb + sp * MN + off[i][j][e],
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                  : acc[i][j][e];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (s0 + q < splits)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
              for (int e = 0; e < 4; ++e) sum[i][j][e] += t[q][i][j][e];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = sum[i][j];
  }

  // All residual reads before any store: the residual may be the output
  // itself (x += f(x)); element by element in place is exact, and issuing
  // the reads first avoids a store-to-load ordering wait per element.
  const GemmEpilogue& ep = g.ep;
  float res[2][2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = n0 + wn * 32 + j * 16 + fr;
        const int m = m0 + wm * 32 + i * 16 + fk * 4 + e;
        res[i][j][e] = (ep.residual && n < g.N && m < g.M)
                           ? ep.residual[(int64_t)m * ep.ldr + n + (int64_t)b * g.c_bstride]
                           : 0.0f;
      }
  // Every value first, then every store (no register of a pending store
  // is rewritten while stores are in flight).
  float outv[2][2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[i][j][e] + bias_v[j];
        if (ep.round_lp) v = round_lp(v, ep.lp_fmt);
        if (ep.act == 1) v = fmaxf(v, 0.0f);
        outv[i][j][e] = v + res[i][j][e];
        if (ep.dt_a) outv[i][j][e] = softplus(outv[i][j][e]);
      }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 32 + j * 16 + fr;
      if (n >= g.N) continue;
      const int nc = n + (int)((int64_t)b * g.c_bstride);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * 32 + i * 16 + fk * 4 + e;
        if (m >= g.M) continue;
        if (ep.out) ep.out[(int64_t)m * ep.ldo + nc] = outv[i][j][e];
        if (ep.out_lp) ep.out_lp[(int64_t)m * ep.ldl + nc] = f32_to_lp_bits(outv[i][j][e], ep.lp_fmt);
        if (ep.dt_decay) ep.dt_decay[(int64_t)m * ep.ldd + nc] = expf(ep.dt_a[n] * outv[i][j][e]);
      }
    }
  }
}

// Skinny fp32 products: at most 16 rows of A (kSkinnyRows), e.g. the fp32
// mode's four symbols, one request each. The 64x64 tile above would stage
// and multiply 64 rows of A per slab for these, and its split-K partial sums
// add a chain of dependent round trips (store, counter, reload) to every
// launch; the product is a stream of W. Here a work-group of 16 waves owns
// 16 output columns and all of K: the waves take interleaved 16-deep k steps
// (together 1 KB of each W row per round), each step one A fragment and one
// W fragment loaded straight into registers (16 rows x 64 bytes each) and
// four v_mfma_f32_16x16x4f32 (A rows past M read row 0; their outputs are
// never stored). Two steps per round; a round past a wave's last step loads
// its first step again and skips the products, so every load is unconditional.
// The waves' sums meet in LDS and are added in wave order (deterministic).
// (Measured alone, M = 4, W streamed from HBM, microseconds per launch, this
// kernel / gemm_kernel: 8192x2048 17.3 / 28.9, 2048x4096 14.9 / 20.5,
// 4096x2048 9.7 / 18.6, 8448x2048 22.6 / 42.2, 2048x2048 8.9 / 15.5, 64x2048
// 8.2 / 13.5. A form with 64-column work-groups and gemm_kernel's split K
// ran 22.8, 20.7, 17.4, 27.1, 18.8 and 14.7: the split's round trips cost
// more than its parallelism gains.)
constexpr int kSkinnyRows = 16;
constexpr int kSkinnyWaves = 16;
constexpr int kSkinnyU = 2;  // k steps per wave per round of loads

__global__ __launch_bounds__(64 * kSkinnyWaves) void gemm_skinny_kernel(GemmArgs g, int tiles_n) {
  constexpr int NWV = kSkinnyWaves;
  constexpr int U = kSkinnyU;
  const int nwg = gridDim.x;
  int bid = blockIdx.x;
  const int full = (nwg / 8) * 8;
  if (bid < full) bid = (bid % 8) * (full / 8) + bid / 8;
  const int tn = bid % tiles_n;
  const int b = bid / tiles_n;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int fr = lane & 15;  // A row / W column of the fragments
  const int fk = lane >> 4;  // k group: k = 16*step + 4*fk + c
  const int n0 = tn * 16;
  const int M = g.M;
  const void* Asrc = (g.A2 != nullptr && b >= g.a2_from) ? g.A2 : g.A;
  const float* Ab = static_cast<const float*>(Asrc) +
                    (int64_t)(g.a_period > 0 ? b % g.a_period : b) * g.a_bstride;
  const float* Wb = static_cast<const float*>(g.W) + (int64_t)b * g.w_bstride;
  const float* a_src = Ab + (int64_t)(fr < M ? fr : 0) * g.lda + 4 * fk;
  const int wr = n0 + fr;
  const float* w_src = Wb + (int64_t)(wr < g.N ? wr : 0) * g.ldw + 4 * fk;

  // this wave's 16-deep k steps: wave, wave + NWV, ...
  const int ksteps = g.K / 16;
  const int nsteps = ksteps > wave ? (ksteps - wave + NWV - 1) / NWV : 0;

  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < nsteps; s0 += U) {
    floatx4 av[U], wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = s0 + u < nsteps ? s0 + u : 0;
      const int64_t k = (int64_t)(wave + NWV * st) * 16;
      av[u] = *reinterpret_cast<const floatx4*>(a_src + k);
      wv[u] = *reinterpret_cast<const floatx4*>(w_src + k);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s0 + u < nsteps) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u].x, wv[u].x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u].y, wv[u].y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u].z, wv[u].z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u].w, wv[u].w, acc, 0, 0, 0);
      }
    }
  }

  // Waves 1.. hand their sums to wave 0, which adds them in wave order.
  __shared__ floatx4 red[NWV - 1][64];
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int w = 0; w < NWV - 1; ++w) acc += red[w][lane];

  // The fragment: lane holds rows 4*fk + e of column n0 + fr.
  const int n = n0 + fr;
  // The epilogue of gemm_kernel: residual reads first (the residual may be
  // the output itself), then every value, then every store.
  if (n >= g.N) return;
  const GemmEpilogue& ep = g.ep;
  const int64_t cb = (int64_t)b * g.c_bstride;
  const float bias_v = ep.bias ? ep.bias[n + cb] : 0.0f;
  float res[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = 4 * fk + e;
    res[e] = (ep.residual && m < M) ? ep.residual[(int64_t)m * ep.ldr + n + cb] : 0.0f;
  }
  float outv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = acc[e] + bias_v;
    if (ep.round_lp) v = round_lp(v, ep.lp_fmt);
    if (ep.act == 1) v = fmaxf(v, 0.0f);
    outv[e] = v + res[e];
    if (ep.dt_a) outv[e] = softplus(outv[e]);
  }
  const int64_t nc = n + cb;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = 4 * fk + e;
    if (m >= M) continue;
    if (ep.out) ep.out[(int64_t)m * ep.ldo + nc] = outv[e];
    if (ep.out_lp) ep.out_lp[(int64_t)m * ep.ldl + nc] = f32_to_lp_bits(outv[e], ep.lp_fmt);
    if (ep.dt_decay) ep.dt_decay[(int64_t)m * ep.ldd + nc] = expf(ep.dt_a[n] * outv[e]);
  }
}

// The 16-bit CastLinear projection of at most 16 rows on packed weights:
// gemm_skinny_kernel's scheme on v_mfma_f32_16x16x32_bf16 / _f16. A
// work-group of 16 waves owns one 16-column MFMA fragment of a packed
// 32-column block and all of K; each 32-deep k step is one 1 KB contiguous W
// fragment and one A fragment (16 rows x 64 bytes; rows past M read row 0),
// taken in interleaved steps by the waves, two per round, loads
// unconditional (a round past a wave's last step reloads its first). The
// waves' sums meet in LDS in wave order; wave 0 applies gemm_wp_kernel's
// epilogue (bias, rounding to the operand format, relu, residual, fp32 and
// 16-bit stores).
template <GemmType T>
__global__ __launch_bounds__(64 * kSkinnyWaves) void gemm_skinny_wp_kernel(GemmArgs g,
                                                                           int tiles_n) {
  constexpr int NWV = kSkinnyWaves;
  constexpr int U = kSkinnyU;
  constexpr int FMT = T == GemmType::kF16 ? kLpF16 : kLpBF16;
  typedef uint16_t E;
  const int nwg = gridDim.x;
  int bid = blockIdx.x;
  const int full = (nwg / 8) * 8;
  if (bid < full) bid = (bid % 8) * (full / 8) + bid / 8;
  const int tn = bid % tiles_n;  // 16-column fragment: block tn / 2, half tn % 2
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int fr = lane & 15;
  const int fq = lane >> 4;
  const int M = g.M;
  const int kb32 = g.K / 32;
  const E* a_src = static_cast<const E*>(g.A) + (int64_t)(fr < M ? fr : 0) * g.lda + 8 * fq;
  // fragment (block, kb, half) starts at ((block * kb32 + kb) * 2 + half) * 512
  const E* w_src = static_cast<const E*>(g.W) +
                   (((int64_t)(tn >> 1) * kb32) * 2 + (tn & 1)) * 512 + 8 * lane;
  const int nsteps = kb32 > wave ? (kb32 - wave + NWV - 1) / NWV : 0;

  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < nsteps; s0 += U) {
    u32x4 av[U], wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = s0 + u < nsteps ? s0 + u : 0;
      const int kb = wave + NWV * st;
      av[u] = *reinterpret_cast<const u32x4*>(a_src + (int64_t)kb * 32);
      wv[u] = *reinterpret_cast<const u32x4*>(w_src + (int64_t)kb * 1024);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s0 + u < nsteps) {
        if constexpr (T == GemmType::kBF16)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[u]),
                                                        __builtin_bit_cast(bf16x8, wv[u]), acc, 0,
                                                        0, 0);
        else
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(halfx8, av[u]),
                                                       __builtin_bit_cast(halfx8, wv[u]), acc, 0,
                                                       0, 0);
      }
    }
  }

  __shared__ floatx4 red[NWV - 1][64];
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int w = 0; w < NWV - 1; ++w) acc += red[w][lane];

  // lane holds rows 4*fq + e of column n (N is a multiple of 32: every
  // column exists)
  const int n = tn * 16 + fr;
  const GemmEpilogue& ep = g.ep;
  const float bias_v = ep.bias ? ep.bias[n] : 0.0f;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = acc[e] + bias_v;
    if (ep.round_lp) v[e] = round_lp_t<FMT>(v[e]);
    if (ep.act == 1) v[e] = fmaxf(v[e], 0.0f);
  }
  if (ep.residual) {
    float res[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 4 * fq + e;
      res[e] = m < M ? ep.residual[(int64_t)m * ep.ldr + n] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += res[e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = 4 * fq + e;
    if (m >= M) continue;
    if (ep.out) ep.out[(int64_t)m * ep.ldo + n] = v[e];
    if (ep.out_lp) ep.out_lp[(int64_t)m * ep.ldl + n] = f32_to_lp_bits_t<FMT>(v[e]);
  }
}

// lgkmcnt(0) tying every register of r (in groups of 8 or 4) to the wait.
template <int N>
__device__ __forceinline__ void ds_wait_all(u32x4 (&r)[N]) {
  static_assert(N % 4 == 0, "groups of four");
#pragma unroll
  for (int i = 0; i + 8 <= N; i += 8)
    __asm__ volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(r[i]), "+v"(r[i + 1]), "+v"(r[i + 2]), "+v"(r[i + 3]), "+v"(r[i + 4]),
                       "+v"(r[i + 5]), "+v"(r[i + 6]), "+v"(r[i + 7])
                     :
                     : "memory");
  if constexpr (N % 8 == 4)
    __asm__ volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(r[N - 4]), "+v"(r[N - 3]), "+v"(r[N - 2]), "+v"(r[N - 1])
                     :
                     : "memory");
}

// ---------------------------------------------------------------------------
// Packed-weight tile for the 16-bit projections (W in the pack_lp_weight
// layout). NW waves per work-group, each owning 32 output columns (two MFMA
// B fragments) and every one of the tile's 16*MF rows.
//
// W is the operand each element of which feeds exactly one wave, and packed
// it is 4 KB contiguous per wave and slab: it travels global -> VGPR with
// fully coalesced 1 KB loads and never touches LDS. A (row-major) is shared
// by all waves and travels global -> LDS (global_load_lds_dwordx4, 8 rows x
// 128 bytes per 1 KB transfer) through a ring of R slabs, XOR-swizzled as in
// the 64x64 kernel; each wave reads its A fragments from there. (An A
// fragment is 16 rows x 64 bytes, so loading it straight from row-major
// memory touches 16 rows per instruction and runs several times slower.)
// R - 1 slabs of A and W loads stay in flight behind the slab being
// multiplied; every slab, including padding slabs past the range, issues
// the same loads, so each ring slot is written the same way in every
// iteration.
template <GemmType T, int MF, int NW, int R>
__global__ __launch_bounds__(64 * NW) void gemm_wp_kernel(GemmArgs g, float* partial,
                                                          int* arrivals, int splits, int tiles_m,
                                                          int tiles_n) {
  static_assert(T != GemmType::kF32, "16-bit operands only");
  constexpr int BMT = 16 * MF;          // tile rows
  constexpr int BNT = 32 * NW;          // tile columns
  constexpr int ASLAB = BMT * 128;      // one A slab in LDS
  constexpr int TPW = 2 * MF / NW;      // A transfers (1 KB) per wave per slab
  constexpr int G = TPW + 4;            // vector-memory instructions per wave per slab
  static_assert(TPW >= 1 && TPW * NW == 2 * MF, "A transfers must split evenly over waves");
  static_assert(R >= 2 && (R - 2) * G < 64, "ring depth");
  static_assert(R * ASLAB <= 96 * 1024, "LDS ring");
  typedef uint16_t E;
  __shared__ __align__(16) unsigned char ring[R * ASLAB];

  const int nwg = gridDim.x;
  int bid = blockIdx.x;
  const int full = (nwg / 8) * 8;
  if (bid < full) bid = (bid % 8) * (full / 8) + bid / 8;
  const int tm = bid % tiles_m;
  const int rest = bid / tiles_m;
  const int tn = rest % tiles_n;
  const int split = rest / tiles_n;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int fr = lane & 15;
  const int fq = lane >> 4;
  const int m0 = tm * BMT;
  const int nw0 = tn * BNT + 32 * wave;  // this wave's first column
  const bool cols_live = nw0 < g.N;
  const E* const A = static_cast<const E*>(g.A);
  const E* const W = static_cast<const E*>(g.W);
  const int kb32 = g.K / 32;

  // A transfers: wave w issues t = w*TPW .. w*TPW + TPW - 1, transfer t
  // covering slab rows 8t .. 8t + 7; lane l lands at byte 16 l: row
  // 8t + l / 8, physical chunk l % 8 holding logical chunk
  // (l % 8) ^ ((row >> 1) & 7). Rows past M read row 0.
  const E* a_src[TPW];
  int a_off[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int t = wave * TPW + u;
    const int row = 8 * t + lane / 8;
    const int lc = (lane % 8) ^ ((row >> 1) & 7);
    const int ar = m0 + row;
    a_src[u] = A + (int64_t)(ar < g.M ? ar : 0) * g.lda + lc * 8;
    a_off[u] = t * 1024;
  }
  // W: this wave's 32-column block (block 0 for a wave past N: its loads
  // stay in range, its products are never stored).
  const E* const w_src = W + (int64_t)(cols_live ? nw0 / 32 : 0) * kb32 * 1024 + lane * 8;

  const int ktiles = g.K / 64;
  const int per = (ktiles + splits - 1) / splits;
  const int kt0 = split * per;
  const int nslab = max(min(ktiles, kt0 + per) - kt0, 0);

  // A fragment rows of this lane within a slab, and their swizzle keys.
  uint32_t arow[MF];
  int akey[MF];
#pragma unroll
  for (int i = 0; i < MF; ++i) {
    const int ra = 16 * i + fr;
    arow[i] = ra * 128;
    akey[i] = (ra >> 1) & 7;
  }

  float bias_v[2] = {0.0f, 0.0f};
  if (g.ep.bias && cols_live) {
#pragma unroll
    for (int c = 0; c < 2; ++c) bias_v[c] = g.ep.bias[nw0 + 16 * c + fr];
  }

  floatx4 acc[MF][2];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[i][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  u32x4 wreg[R][4];  // [ring slot][k step * 2 + column fragment]
  auto issue = [&](int i, int r, u32x4 (&dst)[4]) {
    const int ks = kt0 + (i < nslab ? i : 0);
    unsigned char* const st = ring + r * ASLAB;
#pragma unroll
    for (int u = 0; u < TPW; ++u)
      __builtin_amdgcn_global_load_lds((gptr_t)(a_src[u] + (int64_t)ks * 64), (lptr_t)(st + a_off[u]),
                                       16, 0, 0);
    const E* const wp = w_src + (int64_t)ks * 2048;
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = gload16(wp + q * 512);
  };

  const int npad = (nslab + R - 1) / R * R;
#pragma unroll
  for (int r = 0; r < R - 1; ++r) issue(r, r, wreg[r]);

  for (int ib = 0; ib < npad; ib += R) {
#pragma unroll
    for (int jj = 0; jj < R; ++jj) {
      const int i = ib + jj;
      // Slab i's loads are complete once only the R - 2 later slabs' are
      // outstanding; the barrier then shows every wave's A transfers and
      // retires all reads of ring slot (jj - 1) mod R, the next target.
      wait_vmcnt<(R - 2) * G>();
      __asm__ volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      __asm__ volatile("" ::: "memory");
      issue(i + R - 1, (jj + R - 1) % R, wreg[(jj + R - 1) % R]);
      if (cols_live && i < nslab) {
        const uint32_t st = lds_addr(ring) + (uint32_t)jj * ASLAB;
        u32x4 af[2 * MF];  // [k step * MF + row fragment]
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int m = 0; m < MF; ++m)
            af[h * MF + m] = ds_read16(st + arow[m] + (((h * 4 + fq) ^ akey[m]) << 4));
        ds_wait_all(af);
        const u32x4(&b)[4] = wreg[jj];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int m = 0; m < MF; ++m)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              if constexpr (T == GemmType::kBF16) {
                acc[m][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, af[h * MF + m]), __builtin_bit_cast(bf16x8, b[2 * h + c]),
                    acc[m][c], 0, 0, 0);
              } else {
                acc[m][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(halfx8, af[h * MF + m]), __builtin_bit_cast(halfx8, b[2 * h + c]),
                    acc[m][c], 0, 0, 0);
              }
            }
      }
    }
  }
  // The padding slabs' loads are still in flight: all of them land before
  // the work-group goes on.
  wait_vmcnt<0>();

  // Fragment (m, c): lane holds rows 16 m + 4 fq + e, column 16 c + fr.
  if (splits > 1) {
    // Partials in fragment order, [tile][split][wave][fragment][lane] of
    // float4 (tile = tn * tiles_m + tm): a lane's four values of a fragment
    // are one 16-byte agent-coherent (sc1) store and load, and a wave's
    // access is 1 KB contiguous. Waves past N store and read nothing.
    constexpr int TILE = BMT * BNT;  // floats per tile and split
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        partial + ((int64_t)tn * tiles_m + tm) * splits * TILE, 0, splits * TILE * 4,
        kBufWord3);
    const int lane_b = (wave * MF * 2 * 64 + lane) * 16;
    if (cols_live) {
#pragma unroll
      for (int m = 0; m < MF; ++m)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[m][c]), prs,
                                                 lane_b + (m * 2 + c) * 1024, split * TILE * 4,
                                                 kCoherentSc1);
    }
    // Release side: the partials are stored with agent scope (sc1, written
    // through this XCD's L2), so once every lane's stores are acknowledged
    // (vmcnt 0) and every wave has passed the barrier, they are visible to
    // any XCD before the tile counter sees this split. An agent-scope
    // release fence would also write back the whole L2 (buffer_wbl2): the
    // CastLinear replay measured 16.6 against 13.8 us per launch with one.
    wait_vmcnt<0>();
    __shared__ int last_split;
    __syncthreads();
    int* const arrival = arrivals + (int64_t)tn * tiles_m + tm;
    if (tid == 0)
      last_split = __hip_atomic_fetch_add(arrival, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
    __syncthreads();
    if (!last_split) return;
    // Acquire side: the last split's loads of the other partials are
    // issued only after the counter's returned value (through LDS and the
    // barrier) selected this work-group, and they are agent-scope loads
    // (sc1) that no line of this CU's L1 or of a non-coherent L2 state
    // serves. An agent-scope acquire fence here would also invalidate the
    // XCD's L2 (buffer_inv sc1): the CastLinear replay measured 0.199
    // against 0.210 of HBM peak, and the C4 tick 8.78 against 8.70 ms.
    if (tid == 0) __hip_atomic_store(arrival, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!cols_live) return;
    // Sum in split order; this split's own part comes from its registers.
    floatx4 sum[MF][2];
#pragma unroll
    for (int m = 0; m < MF; ++m)
#pragma unroll
      for (int c = 0; c < 2; ++c) sum[m][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int sp = 0; sp < splits; ++sp) {
      floatx4 t[MF][2];
      if (sp != split) {
#pragma unroll
        for (int m = 0; m < MF; ++m)
#pragma unroll
          for (int c = 0; c < 2; ++c)
            t[m][c] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(prs, lane_b + (m * 2 + c) * 1024,
                                                               sp * TILE * 4, kCoherentSc1));
      } else {
#pragma unroll
        for (int m = 0; m < MF; ++m)
#pragma unroll
          for (int c = 0; c < 2; ++c) t[m][c] = acc[m][c];
      }
#pragma unroll
      for (int m = 0; m < MF; ++m)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) sum[m][c][e] += t[m][c][e];
    }
#pragma unroll
    for (int m = 0; m < MF; ++m)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[m][c] = sum[m][c];
  }
  if (!cols_live) return;

  // Epilogue: bias, rounding to the operand format, relu, residual, stores.
  // Each option is one uniform branch around a loop over all of the lane's
  // values, so the per-value code is straight-line; a tile whose rows all
  // lie inside the output stores without bounds checks. The residual may be
  // the output itself (x += f(x)): every residual read comes before any
  // store.
  constexpr int FMT = T == GemmType::kF16 ? kLpF16 : kLpBF16;
  typedef __attribute__((address_space(1))) float gf32;
  typedef __attribute__((address_space(1))) uint16_t gu16;
  const GemmEpilogue& ep = g.ep;
  float v[MF][2][4];
#pragma unroll
  for (int m = 0; m < MF; ++m)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[m][c][e] = acc[m][c][e] + bias_v[c];
  if (ep.round_lp) {
#pragma unroll
    for (int m = 0; m < MF; ++m)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[m][c][e] = round_lp_t<FMT>(v[m][c][e]);
  }
  if (ep.act == 1) {
#pragma unroll
    for (int m = 0; m < MF; ++m)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[m][c][e] = fmaxf(v[m][c][e], 0.0f);
  }
  const int r0 = m0 + 4 * fq;  // element (m, c, e): row r0 + 16 m + e, column c0 + 16 c
  const int c0 = nw0 + fr;
  if (m0 + BMT <= g.M) {
    if (ep.residual) {
      float res[MF][2][4];
#pragma unroll
      for (int m = 0; m < MF; ++m)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            res[m][c][e] = *(const gf32*)(ep.residual + (int64_t)(r0 + 16 * m + e) * ep.ldr + c0 + 16 * c);
#pragma unroll
      for (int m = 0; m < MF; ++m)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[m][c][e] += res[m][c][e];
    }
    if (ep.out) {
#pragma unroll
      for (int m = 0; m < MF; ++m)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            *(gf32*)(ep.out + (int64_t)(r0 + 16 * m + e) * ep.ldo + c0 + 16 * c) = v[m][c][e];
    }
    if (ep.out_lp) {
#pragma unroll
      for (int m = 0; m < MF; ++m)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            *(gu16*)(ep.out_lp + (int64_t)(r0 + 16 * m + e) * ep.ldl + c0 + 16 * c) =
                f32_to_lp_bits_t<FMT>(v[m][c][e]);
    }
    return;
  }
  // The tile's last rows run past M: every access checks its row.
  if (ep.residual) {
#pragma unroll
    for (int m = 0; m < MF; ++m)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = r0 + 16 * m + e;
          if (r < g.M) v[m][c][e] += ep.residual[(int64_t)r * ep.ldr + c0 + 16 * c];
        }
  }
#pragma unroll
  for (int m = 0; m < MF; ++m)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = r0 + 16 * m + e;
        if (r < g.M) {
          if (ep.out) ep.out[(int64_t)r * ep.ldo + c0 + 16 * c] = v[m][c][e];
          if (ep.out_lp) ep.out_lp[(int64_t)r * ep.ldl + c0 + 16 * c] = f32_to_lp_bits_t<FMT>(v[m][c][e]);
        }
      }
}

// Row-major 16-bit W[N][K] -> the packed layout (one thread per 16-byte
// chunk of the destination: lane l of fragment f reads 8 consecutive k of
// one row).
__global__ void pack_lp_weight_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                      int N, int K) {
  const int64_t chunks = (int64_t)N * K / 8;
  const int kb32 = K / 32;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < chunks;
       q += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(q % 64);
    const int64_t f = q / 64;             // fragment: ((nb * kb32 + kb) * 2 + hf)
    const int hf = (int)(f % 2);
    const int64_t blk = f / 2;
    const int kb = (int)(blk % kb32);
    const int nb = (int)(blk / kb32);
    const int n = nb * 32 + hf * 16 + lane % 16;
    const int k = kb * 32 + 8 * (lane / 16);
    const u32x4 v = gload16(src + (int64_t)n * K + k);
    *reinterpret_cast<u32x4*>(dst + q * 8) = v;
  }
}

// The same from fp32 rows, rounding each value to the 16-bit format on the
// way (the engine's weight binding).
__global__ void pack_f32_to_lp_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                      int rows, int K, int fmt) {
  const int64_t chunks = (int64_t)rows * K / 8;
  const int kb32 = K / 32;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < chunks;
       q += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(q % 64);
    const int64_t f = q / 64;
    const int hf = (int)(f % 2);
    const int64_t blk = f / 2;
    const int kb = (int)(blk % kb32);
    const int nb = (int)(blk / kb32);
    const int n = nb * 32 + hf * 16 + lane % 16;
    const int k = kb * 32 + 8 * (lane / 16);
    const float* p = src + (int64_t)n * K + k;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (uint32_t)f32_to_lp_bits(p[2 * j], fmt) | ((uint32_t)f32_to_lp_bits(p[2 * j + 1], fmt) << 16);
    *reinterpret_cast<u32x4*>(dst + q * 8) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

template <GemmType T, int MF, int NW, int R>
void launch_wp(const GemmArgs& g, const GemmWorkspace& ws, hipStream_t stream, int splits,
               int tiles_m, int tiles_n) {
  hipLaunchKernelGGL((gemm_wp_kernel<T, MF, NW, R>), dim3((unsigned)(tiles_m * tiles_n * splits)),
                     dim3(64 * NW), 0, stream, g, ws.partial, ws.arrivals, splits, tiles_m,
                     tiles_n);
}

// The packed-weight kernel for one GEMM (batch 1, W packed).
int gemm_wp(const GemmArgs& g, const GemmWorkspace& ws, hipStream_t stream, int splits_hint) {
  HK_REQUIRE(g.type != GemmType::kF32 && g.batch == 1 && g.A2 == nullptr && g.a_period == 0,
             "gemm: a packed weight needs a 16-bit single GEMM");
  HK_REQUIRE(g.ep.dt_a == nullptr, "gemm: the dt epilogue is for fp32 products");
  HK_REQUIRE(packable(g.N, g.K), "gemm: packed weight shape N=%d K=%d", g.N, g.K);
  const int fmt = g.type == GemmType::kF16 ? kLpF16 : kLpBF16;
  HK_REQUIRE(!(g.ep.round_lp || g.ep.out_lp) || g.ep.lp_fmt == fmt,
             "gemm: the packed kernel rounds to its operand format");
  if (g.M <= kSkinnyRows) {
    const int tiles_n = g.N / 16;
    if (g.type == GemmType::kF16)
      hipLaunchKernelGGL((gemm_skinny_wp_kernel<GemmType::kF16>), dim3((unsigned)tiles_n),
                         dim3(64 * kSkinnyWaves), 0, stream, g, tiles_n);
    else
      hipLaunchKernelGGL((gemm_skinny_wp_kernel<GemmType::kBF16>), dim3((unsigned)tiles_n),
                         dim3(64 * kSkinnyWaves), 0, stream, g, tiles_n);
    HK_LAUNCH_CHECK();
    return HK_OK;
  }
  // Tile: the largest of 64x128, 64x64, 32x64, 32x32 (rows x columns) that
  // still gives at least min_tiles work-groups without splitting K; failing
  // that the smallest, with K split to fill the device. Measured on the
  // ensemble's shapes (M 77-256, N 2048-8448, K 128-4096): taller tiles or
  // split K lose to more, smaller work-groups, because each CU's concurrent
  // L2 misses, not its MFMA or LDS rate, bound these GEMMs. The one
  // exception is a long K (4096): one tile size up with K split in two
  // gains (alone on the device 256x2048x4096 15.5 against 16.9 us,
  // 179x2048x4096 15.6 / 16.5, 77x2048x4096 11.5 / 15.6; in the C4 tick
  // 8.95-8.97 against 9.04-9.06 ms). Every K = 2048 shape loses with any
  // split, and 128x128 tiles lose everywhere.
  const int min_tiles = g.min_tiles > 0 ? g.min_tiles : kMinTilesAlone;
  static const int kTiles[4][2] = {{4, 4}, {4, 2}, {2, 2}, {2, 1}};  // (MF, NW)
  auto tiles_of = [&](int c) {
    return (int64_t)((g.M + 16 * kTiles[c][0] - 1) / (16 * kTiles[c][0])) *
           ((g.N + 32 * kTiles[c][1] - 1) / (32 * kTiles[c][1]));
  };
  int pick = 3;
  bool fits = false;
  for (int c = 0; c < 4 && !fits; ++c) {
    if (tiles_of(c) >= min_tiles) {
      pick = c;
      fits = true;
    }
  }
  int long_k_splits = 0;
  if (fits && pick > 0 && g.K >= 4096 && 2 * tiles_of(pick - 1) >= min_tiles) {
    --pick;
    long_k_splits = 2;
  } else if (!fits && g.K >= 4096) {
    // too few rows for even the smallest tile: 32x64 tiles with K split up
    // to 4 ways (64x2048x4096 9.4 against 11.0 us for 32x32 split 2)
    pick = 2;
    long_k_splits = (int)std::min<int64_t>(4, std::max<int64_t>(2, (256 + tiles_of(2) - 1) / tiles_of(2)));
  }
  const int mf = kTiles[pick][0];
  const int nw = kTiles[pick][1];
  constexpr int R = 4;
  const int tiles_m = (g.M + 16 * mf - 1) / (16 * mf);
  const int tiles_n = (g.N + 32 * nw - 1) / (32 * nw);
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  const int ktiles = g.K / 64;
  int splits = splits_hint;
  if (splits <= 0 && long_k_splits > 0) {
    splits = long_k_splits;
  } else if (splits <= 0) {
    splits = tiles >= min_tiles ? 1 : (int)((256 + tiles - 1) / tiles);
    splits = std::min(splits, std::max(1, ktiles / 4));
    splits = std::min(splits, 16);
  }
  splits = std::max(1, std::min(splits, ktiles));
  // (partials are whole tiles: 16*mf x 32*nw floats per tile and split)
  while (splits > 1 && (int64_t)splits * tiles * (16 * mf) * (32 * nw) > ws.partial_elems) --splits;
  if (tiles > ws.arrival_elems || ws.arrivals == nullptr) splits = 1;
  const int per = (ktiles + splits - 1) / splits;
  splits = (ktiles + per - 1) / per;
  HK_REQUIRE(tiles * splits < (1LL << 31), "gemm: grid too large");
  HK_REQUIRE(splits == 1 || (int64_t)splits * (16 * mf) * (32 * nw) * 4 < (1LL << 31),
             "gemm: split tile too large");
  const bool f16 = g.type == GemmType::kF16;
#define HK_WP_CASE(MF_, NW_, R_)                                                             \
  if (mf == MF_ && nw == NW_ && R == R_) {                                                  \
    if (f16)                                                                                \
      launch_wp<GemmType::kF16, MF_, NW_, R_>(g, ws, stream, splits, tiles_m, tiles_n);     \
    else                                                                                    \
      launch_wp<GemmType::kBF16, MF_, NW_, R_>(g, ws, stream, splits, tiles_m, tiles_n);    \
    HK_LAUNCH_CHECK();                                                                      \
    return HK_OK;                                                                           \
  }
  HK_WP_CASE(4, 4, 4)
  HK_WP_CASE(4, 2, 4)
  HK_WP_CASE(2, 2, 4)
  HK_WP_CASE(2, 1, 4)
#undef HK_WP_CASE
  HK_REQUIRE(false, "gemm: no packed kernel for MF=%d NW=%d R=%d", mf, nw, R);
  return HK_ERR_ARG;
}

// fp32 products of at most kSkinnyRows rows (any batch description).
int gemm_skinny(const GemmArgs& g, hipStream_t stream) {
  const int tiles_n = (g.N + 15) / 16;
  const int64_t tiles = (int64_t)tiles_n * g.batch;
  HK_REQUIRE(tiles < (1LL << 31), "gemm: grid too large");
  hipLaunchKernelGGL(gemm_skinny_kernel, dim3((unsigned)tiles), dim3(64 * kSkinnyWaves), 0, stream,
                     g, tiles_n);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

}  // namespace

bool packable(int N, int K) { return N > 0 && K > 0 && N % 32 == 0 && K % 64 == 0; }

int pack_lp_weight(const uint16_t* src, uint16_t* dst, int N, int K, hipStream_t stream) {
  HK_REQUIRE(src && dst, "pack_lp_weight: null operand");
  HK_REQUIRE(packable(N, K), "pack_lp_weight: N=%d K=%d (N a multiple of 32, K of 64)", N, K);
  HK_REQUIRE(((uintptr_t)src & 15u) == 0 && ((uintptr_t)dst & 15u) == 0,
             "pack_lp_weight: operands must be 16-byte aligned");
  const int64_t chunks = (int64_t)N * K / 8;
  const unsigned blocks = (unsigned)std::min<int64_t>((chunks + 255) / 256, 4096);
  hipLaunchKernelGGL(pack_lp_weight_kernel, dim3(blocks), dim3(256), 0, stream, src, dst, N, K);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int pack_f32_to_lp(const float* src, uint16_t* dst, int rows, int K, int fmt, hipStream_t stream) {
  HK_REQUIRE(src && dst, "pack_f32_to_lp: null operand");
  HK_REQUIRE(rows > 0 && rows % 32 == 0 && K > 0 && K % 64 == 0,
             "pack_f32_to_lp: rows=%d K=%d (rows a multiple of 32, K of 64)", rows, K);
  HK_REQUIRE(((uintptr_t)dst & 15u) == 0, "pack_f32_to_lp: destination must be 16-byte aligned");
  const int64_t chunks = (int64_t)rows * K / 8;
  const unsigned blocks = (unsigned)std::min<int64_t>((chunks + 255) / 256, 4096);
  hipLaunchKernelGGL(pack_f32_to_lp_kernel, dim3(blocks), dim3(256), 0, stream, src, dst, rows, K,
                     fmt);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int gemm(const GemmArgs& g, const GemmWorkspace& ws, hipStream_t stream, int splits_hint) {
  HK_REQUIRE(g.A && g.W && (g.ep.out || g.ep.out_lp), "gemm: null operand");
  HK_REQUIRE(g.a_period >= 0 && g.a2_from >= 0, "gemm: bad batch-source description");
  HK_REQUIRE(g.M >= 0 && g.N > 0 && g.K > 0 && g.batch > 0, "gemm: bad shape M=%d N=%d K=%d",
             g.M, g.N, g.K);
  int wexp = 0;
  HK_REQUIRE(g.split_wscale == 0.0f ||
                 (std::isfinite(g.split_wscale) && std::frexp(g.split_wscale, &wexp) == 0.5f),
             "gemm: split_wscale %g is not a positive power of two", (double)g.split_wscale);
  const bool narrow = g.type == GemmType::kF32 && g.K % Tr<GemmType::kF32>::BK != 0;
  const bool half = g.type != GemmType::kF32;  // bf16 or fp16 operands
  const int BK = half     ? Tr<GemmType::kBF16>::BK
                 : narrow ? Tr<GemmType::kF32>::BK_NARROW
                          : Tr<GemmType::kF32>::BK;
  const int align = half ? 8 : 4;
  HK_REQUIRE(g.K % BK == 0, "gemm: K=%d is not a multiple of %d", g.K, BK);
  HK_REQUIRE(g.lda % align == 0 && g.ldw % align == 0 && g.a_bstride % align == 0 &&
                 g.w_bstride % align == 0,
             "gemm: leading dimensions must keep 16-byte alignment");
  if (g.M == 0) return HK_OK;
  if (g.w_packed) return gemm_wp(g, ws, stream, splits_hint);
  if (g.type == GemmType::kF32 && g.M <= kSkinnyRows) return gemm_skinny(g, stream);
  const int tiles_m = (g.M + BM - 1) / BM;
  const int tiles_n = (g.N + BN - 1) / BN;
  const int64_t tiles = (int64_t)tiles_m * tiles_n * g.batch;
  const int ktiles = g.K / BK;
  int splits = splits_hint;
  if (splits <= 0) {
    // About one work-group per CU (the slab ring covers the latency), each
    // split at least 8 slabs long.
    splits = (int)((256 + tiles - 1) / tiles);
    splits = std::min(splits, std::max(1, ktiles / 8));
    splits = std::min(splits, 32);
  }
  splits = std::max(1, std::min(splits, ktiles));
  while (splits > 1 && (int64_t)splits * g.batch * g.M * g.N > ws.partial_elems) --splits;
  if (tiles > ws.arrival_elems || ws.arrivals == nullptr) splits = 1;
  const int64_t nwg = tiles * splits;
  HK_REQUIRE(nwg < (1LL << 31), "gemm: grid too large");
  if (g.type == GemmType::kBF16) {
    hipLaunchKernelGGL((gemm_kernel<GemmType::kBF16, Tr<GemmType::kBF16>::BK, kStages>),
                       dim3((unsigned)nwg), dim3(256), 0, stream, g, ws.partial, ws.arrivals, splits,
                       tiles_m, tiles_n);
  } else if (g.type == GemmType::kF16) {
    hipLaunchKernelGGL((gemm_kernel<GemmType::kF16, Tr<GemmType::kF16>::BK, kStages>),
                       dim3((unsigned)nwg), dim3(256), 0, stream, g, ws.partial, ws.arrivals, splits,
                       tiles_m, tiles_n);
  } else if (!narrow && g.split_wscale > 0.0f) {
    hipLaunchKernelGGL((gemm_kernel<GemmType::kF32, Tr<GemmType::kF32>::BK, kStages, true>),
                       dim3((unsigned)nwg), dim3(256), 0, stream, g, ws.partial, ws.arrivals, splits,
                       tiles_m, tiles_n);
  } else if (!narrow) {
    hipLaunchKernelGGL((gemm_kernel<GemmType::kF32, Tr<GemmType::kF32>::BK, kStages>),
                       dim3((unsigned)nwg), dim3(256), 0, stream, g, ws.partial, ws.arrivals, splits,
                       tiles_m, tiles_n);
  } else {
    hipLaunchKernelGGL((gemm_kernel<GemmType::kF32, Tr<GemmType::kF32>::BK_NARROW, kStages>),
                       dim3((unsigned)nwg), dim3(256), 0, stream, g, ws.partial, ws.arrivals, splits,
                       tiles_m, tiles_n);
  }
  HK_LAUNCH_CHECK();
  return HK_OK;
}

}  // namespace hk
