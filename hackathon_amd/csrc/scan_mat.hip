// Matrix-state scan kernel for gfx950 (see scan_mat.h for the recurrence).
//
// One 256-thread work-group (4 wave64s) owns one (run, head, 64-column tile).
// Lane = column, so every state row is one coalesced 256-byte access per wave;
// wave w holds rows [w*RPW, (w+1)*RPW) of the tile in VGPRs for the whole run,
// so the state crosses HBM exactly twice per tick however long the run is.
// The contraction over rows is in-lane (RPW FMAs into 4 accumulators), then a
// 4-way cross-wave sum through LDS. Per-step row vectors (scale*beta, w),
// gamma and alpha are staged into LDS eight steps at a time with all loads in
// flight together, so a long run pays one load latency per eight steps.
#include <cstdint>

#include "scan_mat.h"

namespace hk {
namespace {

constexpr int kSteps = 8;  // steps whose row vectors are staged per LDS block
static_assert(kSteps >= kLogCapMax, "a log fits one staging block");

typedef const __attribute__((address_space(1))) void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

// s_waitcnt with only the vector-memory count constrained to zero (gfx9
// encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
__device__ __forceinline__ void wait_vmem_all() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
  __asm__ volatile("" ::: "memory");
}

// Copies n_chunks 16-byte chunks global -> LDS with global_load_lds, one
// 1 KB transfer (64 lanes) per instruction, transfers dealt to the NW waves:
// chunk c lands at LDS byte 16 c of dst, read from src(c). Lanes past the
// last chunk read chunk 0 again and write the LDS after the used area, which
// must have room for whole transfers.
template <int NW, typename Src>
__device__ __forceinline__ void dma_chunks(float* dst, int n_chunks, int wave, int lane, Src src) {
  const int n_tr = (n_chunks + 63) / 64;
  for (int q = wave; q < n_tr; q += NW) {
    const int c = q * 64 + lane;
    __builtin_amdgcn_global_load_lds((gptr_t)src(c < n_chunks ? c : 0), (lptr_t)(dst + q * 256),
                                     16, 0, 0);
  }
}

// Raw buffer resource over `bytes` bytes from `base` (gfx9 word 3: 32-bit
// data format, no stride, no swizzle). A buffer access takes the row offset
// as a scalar operand and the lane's column offset as its one vector operand,
// and one past `bytes` reads zero and drops stores instead of faulting.
constexpr int kBufWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, kBufWord3);
}

// NW waves split the tile's rows (RPW each); every lane owns VW adjacent
// columns, so a work-group covers 64*VW columns and each wave instruction
// moves 256*VW contiguous bytes of a state row.
// The 512-row tile (8 waves x 64 rows) is held to 128 VGPRs (4 waves per
// SIMD) so that two work-groups share a CU: one streams its state tile in or
// out while the other computes.
// SPLIT: the launch splits tile rows (row_parts > 1); without it the
// row-part arithmetic folds away. FULL: every wave's slice of every tile
// exists (part rows = NW * RPW, whole column tiles), so the tile moves
// without predication.
template <int RPW, int NW, int VW, bool VEC, bool SPLIT, bool FULL>
__global__ __launch_bounds__(64 * NW, (NW == 8 && RPW == 64) ? 4 : 1) void mat_scan_kernel(
    MatScanDesc d) {
  constexpr int kRows = NW * RPW;
  constexpr int NT = 64 * NW;
  constexpr int CW = 64 * VW;  // columns per work-group
  __shared__ __align__(16) float sb[kSteps][kRows];  // scale * beta
  __shared__ __align__(16) float sw[kSteps][kRows];  // w
  __shared__ __align__(16) float sg[kSteps][CW];     // gamma of this column tile
  __shared__ float sa[kSteps];                       // alpha
  __shared__ __align__(16) float red[2][NW][CW];
  // The pending log's entries (full tiles: copied global -> LDS while the
  // tile and the first block's step vectors load, in whole 1 KB transfers).
  constexpr int kLogB = (kSteps * kRows + 255) / 256 * 256;
  constexpr int kLogG = (kSteps * CW + 255) / 256 * 256;
  __shared__ __align__(16) float slb[kLogB];  // [entry][kRows]
  __shared__ __align__(16) float slg[kLogG];  // [entry][CW]
  __shared__ float shdr[64];                   // log header: n, F, a_0 ..
  constexpr bool kLateLog = RPW <= 32;         // log applied in the staging

  // Column tile varies fastest in dispatch order: the work-groups of one
  // (run, head) tile stream adjacent segments of the same rows together.
  const int run = blockIdx.z;
  const int parts = SPLIT ? d.row_parts : 1;
  const int part = SPLIT ? (int)blockIdx.y % parts : 0;
  const int head = SPLIT ? (int)blockIdx.y / parts : (int)blockIdx.y;
  const int prows = d.rows / parts;  // this part's tile rows
  const int row_off = part * prows;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col0 = blockIdx.x * CW;
  const int colv = col0 + lane * VW;  // first of this lane's VW columns
  bool cok[VW];
#pragma unroll
  for (int v = 0; v < VW; ++v) cok[v] = colv + v < d.cols;

  int slot, r0, len;
  if (d.per_row) {
    slot = run;
    r0 = run;
    len = (d.mask == nullptr || d.mask[run]) ? 1 : 0;
  } else {
    slot = d.slot_ids[run];
    r0 = d.run_off[run];
    len = d.run_off[run + 1] - r0;
  }
  float* out_base = d.out + (int64_t)head * d.out_head_stride + (int64_t)part * d.out_part_stride;
  if (len == 0) {
    // Idle row (reference API): state untouched, output defined as zero.
    if (wave == 0) {
#pragma unroll
      for (int v = 0; v < VW; ++v)
        if (cok[v]) out_base[(int64_t)r0 * d.out_row_stride + colv + v] = 0.0f;
    }
    return;
  }

  // Rows past the part's rows hold zero in LDS and in the tile, so they
  // contribute nothing and need no branch in the inner loop.
  for (int i = tid; i < kSteps * kRows; i += NT) {
    const int r = i % kRows;
    if (r >= prows) {
      sb[i / kRows][r] = 0.0f;
      sw[i / kRows][r] = 0.0f;
    }
  }

  // The pending log's count (a scalar load). Up to 32 rows per wave its
  // factor and coefficients go global -> LDS (one dword per lane from wave 0,
  // lanes past the header repeat its last word) and are read from there after
  // the first staging barrier; with 64 they are scalar loads.
  int log_n = 0;
  bool defer = false;
  const float* lh = d.log_hdr + ((int64_t)slot * d.heads + head) * kLogHdr;
  if (d.log_cap > 0) {
    log_n = (int)lh[0];
    defer = log_n + len <= d.log_cap;
    if (kLateLog && wave == 0 && log_n > 0)
      __builtin_amdgcn_global_load_lds((gptr_t)(lh + (lane < kLogHdr ? lane : kLogHdr - 1)),
                                       (lptr_t)shdr, 4, 0, 0);
  }
  const int64_t le0 = ((int64_t)slot * d.heads + head) * d.log_cap;  // first log entry

  // Uniform tile base (scalar registers) + 32-bit per-lane offsets: a tile
  // spans well under 2^32 elements, and this keeps 64-bit address math out
  // of the unrolled row loops.
  float* tbase = d.state + (int64_t)slot * d.slot_stride + (int64_t)head * d.head_stride +
                 (int64_t)row_off * d.row_stride;
  const int rbase = wave * RPW;
  const uint32_t rstride = (uint32_t)d.row_stride;
  const uint32_t off0 = (uint32_t)colv * (uint32_t)d.col_stride + (uint32_t)rbase * rstride;
  const int rlim = prows - rbase;  // rows of this wave's slice that exist
  // FULL: the tile moves without predication through a buffer resource on
  // the wave's first row, row i at scalar offset i * row bytes, the lane's
  // columns at one vector offset, so the RPW loads issue back to back and
  // hold no per-row address registers. The resource spans exactly the slice.
  constexpr bool full = FULL;
  const int rsb = 4 * (int)d.row_stride;  // row bytes
  const int lane_b = 4 * colv * (int)d.col_stride;
  const __amdgpu_buffer_rsrc_t rs =
      tile_rsrc(tbase + (int64_t)rbase * d.row_stride,
                4u * (uint32_t)((RPW - 1) * d.row_stride + (int64_t)(col0 + CW - 1) * d.col_stride + 1));
  float s[RPW][VW];
  if constexpr (full) {
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      if constexpr (VW == 2) {  // unit column stride
        // two adjacent 32-bit loads, which the compiler merges into one
        // buffer_load_dwordx2 (its 64-bit load builtin emits a single dword)
        s[i][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, lane_b, i * rsb, 0));
        s[i][1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, lane_b + 4, i * rsb, 0));
      } else {
        s[i][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, lane_b, i * rsb, 0));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const uint32_t o = off0 + (uint32_t)i * rstride;
      if constexpr (VW == 2) {
        float2 v2 = make_float2(0.0f, 0.0f);
        if (cok[0] && cok[1] && i < rlim) v2 = *reinterpret_cast<const float2*>(tbase + o);
        s[i][0] = v2.x;
        s[i][1] = v2.y;
      } else {
#pragma unroll
        for (int v = 0; v < VW; ++v)
          s[i][v] = (cok[v] && i < rlim) ? tbase[o + (uint32_t)v * (uint32_t)d.col_stride] : 0.0f;
      }
    }
  }

  // ---- deferred write-back: the tile is materialised from B and the log
  // (s = F s, then s = fma(b_j, a_j g_j, s) in entry order, as mat_log_flush
  // does). The entries reach LDS behind the tile's loads: full tiles by
  // global -> LDS transfers, other tiles by loads (rows past the part's rows
  // zero). Up to 32 rows per wave the log is applied after the first staging
  // barrier, so the step vectors' loads overlap it; with 64 the registers
  // held across the staging do not fit beside the tile, and it is applied
  // here with plain loads.
  if (log_n > 0) {
    const float* lb = d.log_b + le0 * d.rows + row_off;
    const float* lg = d.log_g + le0 * d.cols + col0;
    if constexpr (kLateLog) {
      if constexpr (FULL) {
        constexpr int bq = kRows / 4;  // chunks per entry (prows == kRows)
        constexpr int gq = CW / 4;
        dma_chunks<NW>(slb, log_n * bq, wave, lane, [&](int c) {
          const int j = c / bq;
          return lb + (int64_t)j * d.rows + 4 * (c - j * bq);
        });
        dma_chunks<NW>(slg, log_n * gq, wave, lane, [&](int c) {
          const int j = c / gq;
          return lg + (int64_t)j * d.cols + 4 * (c - j * gq);
        });
      } else {
        for (int i = tid; i < log_n * kRows; i += NT) {
          const int j = i / kRows;
          const int r = i - j * kRows;
          slb[i] = r < prows ? lb[(int64_t)j * d.rows + r] : 0.0f;
        }
        for (int i = tid; i < log_n * CW; i += NT) {
          const int j = i / CW;
          const int c = i - j * CW;
          slg[i] = col0 + c < d.cols ? lg[(int64_t)j * d.cols + c] : 0.0f;
        }
      }
    } else {
      for (int i = tid; i < log_n * prows; i += NT) {
        const int j = i / prows;
        sb[j][i - j * prows] = lb[(int64_t)j * d.rows + (i - j * prows)];
      }
      for (int i = tid; i < log_n * CW; i += NT) {
        const int j = i / CW;
        const int c = i - j * CW;
        sg[j][c] = col0 + c < d.cols ? lg[(int64_t)j * d.cols + c] : 0.0f;
      }
      lds_barrier();
      const float F = lh[1];
      for (int j = 0; j < log_n; ++j) {
        const float a = lh[2 + j];
        const float f = j == 0 ? F : 1.0f;
        float gj[VW];
#pragma unroll
        for (int v = 0; v < VW; ++v) gj[v] = a * sg[j][lane * VW + v];
#pragma unroll
        for (int i = 0; i < RPW; i += 4) {
          const float4 bv = *reinterpret_cast<const float4*>(&sb[j][rbase + i]);
          const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
          for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int v = 0; v < VW; ++v) s[i + k][v] = fmaf(bb[k], gj[v], f * s[i + k][v]);
        }
      }
      lds_barrier();  // the step staging below rewrites sb / sg
    }
  }

  const float* beta_h = d.beta.ptr + (int64_t)head * d.beta.head_stride + row_off;
  const float* w_h = d.w.ptr + (int64_t)head * d.w.head_stride + row_off;
  for (int t0 = 0; t0 < len; t0 += kSteps) {
    const int ns = min(kSteps, len - t0);
    const int64_t row0 = r0 + t0;
    // ---- stage ns steps of row vectors, all loads in flight at once
    if constexpr (VEC) {
      constexpr int V = (kSteps * kRows / 4 + NT - 1) / NT;
      const int vpr = prows >> 2;  // float4 per step
      const int nv = ns * vpr;
      float4 vb[V], vw[V];
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const int i = min(u * NT + tid, nv - 1);
        const int st = i / vpr;
        const int k4 = i - st * vpr;
        const int64_t row = row0 + st;
        vb[u] = reinterpret_cast<const float4*>(beta_h + row * d.beta.row_stride)[k4];
        vw[u] = reinterpret_cast<const float4*>(w_h + row * d.w.row_stride)[k4];
      }
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const int i = u * NT + tid;
        if (i < nv) {
          const int st = i / vpr;
          const int k4 = i - st * vpr;
          const int64_t row = row0 + st;
          const float sc = d.scale.ptr ? d.scale.ptr[row * d.scale.row_stride +
                                                     head * d.scale.head_stride]
                                       : 1.0f;
          // (i*k), (dt*b): the association the reference uses
          float4 b4 = vb[u];
          b4.x = sc * b4.x;
          b4.y = sc * b4.y;
          b4.z = sc * b4.z;
          b4.w = sc * b4.w;
          *reinterpret_cast<float4*>(&sb[st][4 * k4]) = b4;
          *reinterpret_cast<float4*>(&sw[st][4 * k4]) = vw[u];
        }
      }
    } else {
      for (int i = tid; i < ns * prows; i += NT) {
        const int st = i / prows;
        const int k = i - st * prows;
        const int64_t row = row0 + st;
        const float sc = d.scale.ptr ? d.scale.ptr[row * d.scale.row_stride +
                                                   head * d.scale.head_stride]
                                     : 1.0f;
        sb[st][k] = sc * beta_h[row * d.beta.row_stride + k];
        sw[st][k] = w_h[row * d.w.row_stride + k];
      }
    }
    for (int i = tid; i < ns * CW; i += NT) {
      const int st = i / CW;
      const int c = col0 + (i - st * CW);
      const int64_t row = row0 + st;
      sg[st][i - st * CW] = c < d.cols ? d.gamma.ptr[row * d.gamma.row_stride +
                                                     head * d.gamma.head_stride + c]
                                       : 0.0f;
    }
    if (tid < ns) {
      const int64_t row = row0 + tid;
      sa[tid] = d.alpha.ptr[row * d.alpha.row_stride + head * d.alpha.head_stride];
    }
    // the log's transfers (this wave's) are in LDS before the barrier
    if (kLateLog && log_n > 0 && t0 == 0) wait_vmem_all();
    lds_barrier();
    if (kLateLog && log_n > 0 && t0 == 0) {
      for (int j = 0; j < log_n; ++j) {
        const float a = shdr[2 + j];
        const float f = j == 0 ? shdr[1] : 1.0f;
        float gj[VW];
#pragma unroll
        for (int v = 0; v < VW; ++v) gj[v] = a * slg[j * CW + lane * VW + v];
#pragma unroll
        for (int i = 0; i < RPW; i += 4) {
          const float4 bv = *reinterpret_cast<const float4*>(&slb[j * kRows + rbase + i]);
          const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
          for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int v = 0; v < VW; ++v) s[i + k][v] = fmaf(bb[k], gj[v], f * s[i + k][v]);
        }
      }
    }

    // ---- advance the tile through the staged steps
    for (int st = 0; st < ns; ++st) {
      const float a = sa[st];
      float g[VW];
#pragma unroll
      for (int v = 0; v < VW; ++v) g[v] = sg[st][lane * VW + v];
      float acc[VW][2];
#pragma unroll
      for (int v = 0; v < VW; ++v) acc[v][0] = acc[v][1] = 0.0f;
#pragma unroll
      for (int i = 0; i < RPW; i += 4) {
        const float4 bv = *reinterpret_cast<const float4*>(&sb[st][rbase + i]);
        const float4 wv = *reinterpret_cast<const float4*>(&sw[st][rbase + i]);
        const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
        const float ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
          for (int v = 0; v < VW; ++v) {
            s[i + k][v] = a * s[i + k][v] + bb[k] * g[v];
            acc[v][k & 1] += ww[k] * s[i + k][v];
          }
        }
      }
      const int par = st & 1;
#pragma unroll
      for (int v = 0; v < VW; ++v) red[par][wave][lane * VW + v] = acc[v][0] + acc[v][1];
      lds_barrier();
      if (tid < CW && col0 + tid < d.cols) {
        float o = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) o += red[par][w2][tid];
        out_base[(row0 + st) * d.out_row_stride + col0 + tid] = o;
      }
    }
    lds_barrier();  // the next block's staging overwrites sb/sw/sg/sa
  }

  if (defer) {
    // B stays; the run's steps (len <= log_cap <= kSteps: all in the one
    // staging block, still in LDS) become log entries log_n .. log_n+len-1.
    // Column tile 0 writes each part's rows of b; part 0 each tile's g.
    const int64_t le = le0 + log_n;
    if (blockIdx.x == 0) {
      float* lb = d.log_b + le * d.rows + row_off;
      for (int i = tid; i < len * prows; i += NT) {
        const int t = i / prows;
        lb[(int64_t)t * d.rows + (i - t * prows)] = sb[t][i - t * prows];
      }
    }
    if (part == 0) {
      float* lg = d.log_g + le * d.cols + col0;
      for (int i = tid; i < len * CW; i += NT) {
        const int t = i / CW;
        const int c = i - t * CW;
        if (col0 + c < d.cols) lg[(int64_t)t * d.cols + c] = sg[t][c];
      }
    }
    return;
  }

  if constexpr (full) {
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      if constexpr (VW == 2) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, s[i][0]), rs, lane_b,
                                              i * rsb, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, s[i][1]), rs,
                                              lane_b + 4, i * rsb, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, s[i][0]), rs, lane_b,
                                              i * rsb, 0);
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const uint32_t o = off0 + (uint32_t)i * rstride;
    if constexpr (VW == 2) {
      if (cok[0] && cok[1] && i < rlim)
        *reinterpret_cast<float2*>(tbase + o) = make_float2(s[i][0], s[i][1]);
    } else {
#pragma unroll
      for (int v = 0; v < VW; ++v)
        if (cok[v] && i < rlim) tbase[o + (uint32_t)v * (uint32_t)d.col_stride] = s[i][v];
    }
  }
}

// Log header update after a scan launch, one thread per (run, head): a run
// that was deferred (n + len <= cap) appends len entries, entry t weighted
// by the product of the run's later alphas, and scales the older entries
// and F by the product of all of them; any other run left B materialised,
// so its log empties (n = 0, F = 1).
__global__ void mat_log_commit_kernel(LogCommit c) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < c.jobs()) log_commit_one(c, i);
}

// B <- F B + sum_j b_j (a_j g_j) for slots slot0 + blockIdx.z, one row per
// work-group (the same operation order as the scan's materialisation).
__global__ void mat_log_flush_kernel(MatScanDesc d, int slot0) {
  const int row = blockIdx.x;
  const int head = blockIdx.y;
  const int slot = slot0 + blockIdx.z;
  const float* lh = d.log_hdr + ((int64_t)slot * d.heads + head) * kLogHdr;
  const int n = (int)lh[0];
  if (n == 0) return;
  const float F = lh[1];
  const int64_t le = ((int64_t)slot * d.heads + head) * d.log_cap;
  float* b = d.state + (int64_t)slot * d.slot_stride + (int64_t)head * d.head_stride +
             (int64_t)row * d.row_stride;
  for (int c = threadIdx.x; c < d.cols; c += blockDim.x) {
    float v = b[(int64_t)c * d.col_stride] * F;
    for (int j = 0; j < n; ++j) {
      const float gj = lh[2 + j] * d.log_g[(le + j) * d.cols + c];
      v = fmaf(d.log_b[(le + j) * d.rows + row], gj, v);
    }
    b[(int64_t)c * d.col_stride] = v;
  }
}

// Empties the logs of slots slots[i] (or slot0 + i when slots is null).
__global__ void mat_log_clear_kernel(float* hdr, int heads, const int* slots, int slot0, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * heads) return;
  const int k = i / heads;
  const int slot = slots ? slots[k] : slot0 + k;
  float* h = hdr + ((int64_t)slot * heads + (i - k * heads)) * kLogHdr;
  h[0] = 0.0f;
  h[1] = 1.0f;
}

// Appends counts[k] zero-valued entries (row and column vectors zero,
// coefficient 1) to the logs of slot slots[k], up to the capacity: the
// leaf's value F*B + sum_j a_j b_j g_j^T is unchanged. One thread per
// (slot, head).
__global__ void mat_log_fill_kernel(float* hdr, float* lb, float* lg, int heads, int cap,
                                    int rows, int cols, const int* slots, const int* counts,
                                    int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * heads) return;
  const int k = i / heads;
  const int64_t sh = (int64_t)slots[k] * heads + (i - k * heads);
  float* h = hdr + sh * kLogHdr;
  const int have = (int)h[0];
  const int add = min(counts[k], cap - have);
  if (add <= 0) return;
  for (int j = have; j < have + add; ++j) {
    h[2 + j] = 1.0f;
    float* b = lb + (sh * cap + j) * rows;
    for (int r = 0; r < rows; ++r) b[r] = 0.0f;
    float* g = lg + (sh * cap + j) * cols;
    for (int c = 0; c < cols; ++c) g[c] = 0.0f;
  }
  h[0] = (float)(have + add);
}

}  // namespace

int mat_log_fill(const MatScanDesc& d, const int* slots_dev, const int* counts_dev, int n,
                 hipStream_t stream) {
  if (d.log_cap == 0 || n == 0) return HK_OK;
  HK_REQUIRE(n > 0 && d.log_hdr && d.log_b && d.log_g && slots_dev && counts_dev,
             "mat_log_fill: bad arguments");
  const int total = n * d.heads;
  hipLaunchKernelGGL(mat_log_fill_kernel, dim3((total + 255) / 256), dim3(256), 0, stream,
                     d.log_hdr, d.log_b, d.log_g, d.heads, d.log_cap, d.rows, d.cols, slots_dev,
                     counts_dev, n);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

LogCommit log_commit_of(const MatScanDesc& d) {
  LogCommit c;
  if (d.log_cap == 0 || d.n_runs == 0 || d.per_row) return c;
  c.slot_ids = d.slot_ids;
  c.run_off = d.run_off;
  c.n_runs = d.n_runs;
  c.heads = d.heads;
  c.alpha = d.alpha;
  c.log_hdr = d.log_hdr;
  c.log_cap = d.log_cap;
  return c;
}

int launch_mat_log_commit(const MatScanDesc& d, hipStream_t stream) {
  if (d.log_cap == 0 || d.n_runs == 0) return HK_OK;
  HK_REQUIRE(!d.per_row && d.slot_ids && d.run_off && d.log_hdr, "mat_log_commit: need runs");
  const LogCommit c = log_commit_of(d);
  hipLaunchKernelGGL(mat_log_commit_kernel, dim3((c.jobs() + 255) / 256), dim3(256), 0, stream, c);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int mat_log_flush(const MatScanDesc& d, int slot0, int n, hipStream_t stream) {
  if (d.log_cap == 0 || n == 0) return HK_OK;
  HK_REQUIRE(d.state && d.log_hdr && d.log_b && d.log_g && n > 0 && n <= 65535 &&
                 d.heads <= 65535,
             "mat_log_flush: bad arguments");
  hipLaunchKernelGGL(mat_log_flush_kernel, dim3(d.rows, d.heads, n), dim3(256), 0, stream, d,
                     slot0);
  HK_LAUNCH_CHECK();
  const int total = n * d.heads;
  hipLaunchKernelGGL(mat_log_clear_kernel, dim3((total + 255) / 256), dim3(256), 0, stream,
                     d.log_hdr, d.heads, nullptr, slot0, n);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int mat_log_clear(const MatScanDesc& d, const int* slots_dev, int slot0, int n,
                  hipStream_t stream) {
  if (d.log_cap == 0 || n == 0) return HK_OK;
  HK_REQUIRE(n > 0 && d.log_hdr, "mat_log_clear: bad arguments");
  const int total = n * d.heads;
  hipLaunchKernelGGL(mat_log_clear_kernel, dim3((total + 255) / 256), dim3(256), 0, stream,
                     d.log_hdr, d.heads, slots_dev, slot0, n);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int launch_mat_scan(const MatScanDesc& d, hipStream_t stream) {
  HK_REQUIRE(d.state && d.out && d.alpha.ptr && d.beta.ptr && d.gamma.ptr && d.w.ptr,
             "mat_scan: null operand");
  HK_REQUIRE(d.rows > 0 && d.cols > 0 && d.heads > 0, "mat_scan: empty tile %dx%d heads %d",
             d.rows, d.cols, d.heads);
  HK_REQUIRE(d.per_row || (d.slot_ids && d.run_off), "mat_scan: need run descriptors");
  HK_REQUIRE(d.row_parts >= 1 && (d.row_parts == 1 || d.rows % (4 * d.row_parts) == 0),
             "mat_scan: %d rows do not split into %d parts of a multiple of 4", d.rows,
             d.row_parts);
  HK_REQUIRE((int64_t)d.heads * d.row_parts <= 65535, "mat_scan: too many heads");
  HK_REQUIRE(d.log_cap == 0 || (d.log_cap <= kLogCapMax && d.log_cap <= kLogHdr - 2 &&
                                !d.per_row && d.log_hdr && d.log_b && d.log_g),
             "mat_scan: bad write-back log");
  const int prows = d.rows / d.row_parts;
  HK_REQUIRE((int64_t)d.rows * d.row_stride + (int64_t)d.cols * d.col_stride < (1LL << 30),
             "mat_scan: tile too large for 32-bit byte offsets");
  if (d.n_runs == 0) return HK_OK;
  HK_REQUIRE(d.n_runs <= 65535, "mat_scan: at most 65535 runs per launch");
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool vec = prows % 4 == 0 && al16(d.beta.ptr) && al16(d.w.ptr) &&
                   d.beta.row_stride % 4 == 0 && d.beta.head_stride % 4 == 0 &&
                   d.w.row_stride % 4 == 0 && d.w.head_stride % 4 == 0;
  // 256-row tiles with whole 128-column tiles, unit column stride and 8-byte
  // aligned rows: 8 waves x float2 columns. 512-row tiles: 8 waves x 64 rows
  // (wider tiles there exceed the register file of an 8-wave work-group).
  const bool wide = prows > 128 && d.cols % 128 == 0 && d.col_stride == 1 &&
                    d.row_stride % 2 == 0 && d.head_stride % 2 == 0 && d.slot_stride % 2 == 0 &&
                    (reinterpret_cast<uintptr_t>(d.state) & 7) == 0;
#define HK_SCAN_LAUNCH_F(R, NW, VW, SP, FU)                                                \
  {                                                                                          \
    dim3 grid((d.cols + 64 * VW - 1) / (64 * VW), d.heads * d.row_parts, d.n_runs);          \
    if (vec)                                                                                 \
      hipLaunchKernelGGL((mat_scan_kernel<R, NW, VW, true, SP, FU>), grid, dim3(64 * NW), 0,   \
                         stream, d);                                                         \
    else                                                                                     \
      hipLaunchKernelGGL((mat_scan_kernel<R, NW, VW, false, SP, FU>), grid, dim3(64 * NW), 0,  \
                         stream, d);                                                         \
  }
#define HK_SCAN_LAUNCH_S(R, NW, VW, SP)                                   \
  {                                                                        \
    if (prows == R * NW && d.cols % (64 * VW) == 0)                        \
      HK_SCAN_LAUNCH_F(R, NW, VW, SP, true)                                \
    else                                                                   \
      HK_SCAN_LAUNCH_F(R, NW, VW, SP, false)                               \
  }
#define HK_SCAN_LAUNCH(R, NW, VW)                              \
  {                                                            \
    if (d.row_parts > 1) HK_SCAN_LAUNCH_S(R, NW, VW, true)     \
    else HK_SCAN_LAUNCH_S(R, NW, VW, false)                    \
  }
  if (prows <= 32) {
    HK_SCAN_LAUNCH(8, 4, 1)
  } else if (prows <= 64) {
    HK_SCAN_LAUNCH(16, 4, 1)
  } else if (prows <= 128) {
    HK_SCAN_LAUNCH(32, 4, 1)
  } else if (prows <= 256) {
    if (wide) HK_SCAN_LAUNCH(32, 8, 2) else HK_SCAN_LAUNCH(64, 4, 1)
  } else if (prows <= 512) {
    HK_SCAN_LAUNCH(64, 8, 1)
  } else {
    HK_REQUIRE(false, "mat_scan: %d rows per part exceed the 512-row tile", prows);
  }
#undef HK_SCAN_LAUNCH
#undef HK_SCAN_LAUNCH_S
#undef HK_SCAN_LAUNCH_F
  HK_LAUNCH_CHECK();
  return HK_OK;
}

}  // namespace hk
