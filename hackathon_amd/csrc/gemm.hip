// Projection GEMM kernel (see gemm.h).
//
// 64x64 output tile per 256-thread work-group, 4 wave64s in a 2x2 layout,
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

template <GemmType T, int BK, int S>
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
  // (Every transfer was waited for before its slab; nothing is in flight.)

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
    // Every partial store of this lane acknowledged at the agent-coherent
    // level, then every wave's, before the tile counter sees this split.
    wait_vmcnt<0>();
    __shared__ int last_split;
    __syncthreads();
    int* const arrival = arrivals + ((int64_t)b * tiles_n + tn) * tiles_m + tm;
    if (tid == 0)
      last_split = __hip_atomic_fetch_add(arrival, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
    __syncthreads();
    if (!last_split) return;
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
      }
    }
  }
}

}  // namespace

int gemm(const GemmArgs& g, const GemmWorkspace& ws, hipStream_t stream, int splits_hint) {
  HK_REQUIRE(g.A && g.W && (g.ep.out || g.ep.out_lp), "gemm: null operand");
  HK_REQUIRE(g.a_period >= 0 && g.a2_from >= 0, "gemm: bad batch-source description");
  HK_REQUIRE(g.M >= 0 && g.N > 0 && g.K > 0 && g.batch > 0, "gemm: bad shape M=%d N=%d K=%d",
             g.M, g.N, g.K);
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
