// Row-wise kernels: norms and the fused elementwise tails of each layer.
//
// One work-group per request row. Normalisations keep the reference's
// formulas (mean of squares / biased variance over the normalised extent,
// eps inside the square root); reductions run in a fixed order, so a row's
// result does not depend on the batch it rides in.
#include <algorithm>

#include "ops.h"

namespace hk {
namespace {

// Row held in registers: thread t owns columns t + 256*i (i < V), loaded
// together (clamped, masked) before any reduction, so a row costs one load
// latency instead of one per 256 columns and pass. Per-thread partial sums
// run in increasing column order, then the block sum.
template <int V>
struct RowRegs {
  float v[V];
  __device__ __forceinline__ void load(const float* __restrict__ xr, int width) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int c = threadIdx.x + 256 * i;
      const float x = xr[min(c, width - 1)];
      v[i] = c < width ? x : 0.0f;
    }
  }
  __device__ __forceinline__ float sum(int width) const {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (threadIdx.x + 256 * i < width) s += v[i];
    return s;
  }
  __device__ __forceinline__ float sumsq(int width, float mean) const {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (threadIdx.x + 256 * i < width) {
        const float d = v[i] - mean;
        s += d * d;
      }
    return s;
  }
};

// out = x * rsqrt(mean(x^2) + eps) * w
template <int V>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, int64_t ldx,
                                                      const float* __restrict__ w, float eps,
                                                      int width, float* __restrict__ out,
                                                      int64_t ldo, uint16_t* __restrict__ out_lp, int lp_fmt,
                                                      int64_t ldl) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  RowRegs<V> r;
  r.load(x + row * ldx, width);
  const float ss = block_sum(r.sumsq(width, 0.0f), red);
  const float inv = 1.0f / sqrtf(ss / (float)width + eps);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c < width) {
      const float o = (r.v[i] * inv) * w[c];
      if (out) out[row * ldo + c] = o;
      if (out_lp) out_lp[row * ldl + c] = f32_to_lp_bits(o, lp_fmt);
    }
  }
}

// out = LayerNorm(x) * w (+ residual), eps 1e-5, no bias
template <int V>
__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ w,
                                                        const float* __restrict__ residual,
                                                        int width, float* __restrict__ out,
                                                        uint16_t* __restrict__ out_lp, int lp_fmt) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  RowRegs<V> r;
  r.load(x + row * width, width);
  const float mean = block_sum(r.sum(width), red) / (float)width;
  const float rstd = 1.0f / sqrtf(block_sum(r.sumsq(width, mean), red) / (float)width + 1e-5f);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c < width) {
      float o = ((r.v[i] - mean) * rstd) * w[c];
      if (residual) o += residual[row * width + c];
      if (out) out[row * width + c] = o;
      if (out_lp) out_lp[row * width + c] = f32_to_lp_bits(o, lp_fmt);
    }
  }
}

// a = RMSNorm(x) * w_rms (fp32 and optional bf16 copy); xn = LayerNorm(a) * w_ln.
template <int V>
__global__ __launch_bounds__(256) void rms_ln_kernel(const float* __restrict__ x,
                                                     const float* __restrict__ w_rms, float eps,
                                                     const float* __restrict__ w_ln, int width,
                                                     float* __restrict__ a,
                                                     uint16_t* __restrict__ a_lp, int lp_fmt,
                                                     float* __restrict__ xn) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  RowRegs<V> r;
  r.load(x + row * width, width);
  const float ss = block_sum(r.sumsq(width, 0.0f), red);
  const float inv = 1.0f / sqrtf(ss / (float)width + eps);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + 256 * i;
    r.v[i] = c < width ? (r.v[i] * inv) * w_rms[min(c, width - 1)] : 0.0f;
    if (c < width) {
      a[row * width + c] = r.v[i];
      if (a_lp) a_lp[row * width + c] = f32_to_lp_bits(r.v[i], lp_fmt);
    }
  }
  const float mean = block_sum(r.sum(width), red) / (float)width;
  const float rstd = 1.0f / sqrtf(block_sum(r.sumsq(width, mean), red) / (float)width + 1e-5f);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c < width) xn[row * width + c] = ((r.v[i] - mean) * rstd) * w_ln[c];
  }
}

// x = LayerNorm(y) * w_ln + x (in place); a = RMSNorm(x) * w_rms (fp32, bf16).
template <int V>
__global__ __launch_bounds__(256) void ln_res_rms_kernel(const float* __restrict__ y,
                                                         const float* __restrict__ w_ln,
                                                         float* __restrict__ x,
                                                         const float* __restrict__ w_rms,
                                                         float eps, int width,
                                                         float* __restrict__ a,
                                                         uint16_t* __restrict__ a_lp, int lp_fmt) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  RowRegs<V> r, xr;
  r.load(y + row * width, width);
  xr.load(x + row * width, width);
  const float mean = block_sum(r.sum(width), red) / (float)width;
  const float rstd = 1.0f / sqrtf(block_sum(r.sumsq(width, mean), red) / (float)width + 1e-5f);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + 256 * i;
    r.v[i] = c < width ? ((r.v[i] - mean) * rstd) * w_ln[min(c, width - 1)] + xr.v[i] : 0.0f;
    if (c < width) x[row * width + c] = r.v[i];
  }
  const float ss = block_sum(r.sumsq(width, 0.0f), red);
  const float inv = 1.0f / sqrtf(ss / (float)width + eps);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c < width) {
      const float o = (r.v[i] * inv) * w_rms[c];
      a[row * width + c] = o;
      if (a_lp) a_lp[row * width + c] = f32_to_lp_bits(o, lp_fmt);
    }
  }
}

__global__ void stage_features_kernel(const float* __restrict__ feat, int n_rows, int f, int kpad,
                                      float* __restrict__ out, uint16_t* __restrict__ out_lp, int lp_fmt) {
  const int64_t total = (int64_t)n_rows * kpad;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / kpad;
    const int c = (int)(i % kpad);
    const float v = c < f ? feat[r * f + c] : 0.0f;
    if (out) out[i] = v;
    if (out_lp) out_lp[i] = f32_to_lp_bits(v, lp_fmt);
  }
}

// Row values held in registers (inner <= 256 * kMambaPostMax).
constexpr int kMambaPostMax = 32;
__global__ __launch_bounds__(256) void mamba2_post_kernel(
    const float* __restrict__ ssm_out, int n_parts, int64_t part_stride,
    const float* __restrict__ x, int64_t ldx, const float* __restrict__ z, int64_t ldz,
    const float* __restrict__ d, const float* __restrict__ w, int inner, int head_size,
    float* __restrict__ out, uint16_t* __restrict__ out_lp, int lp_fmt, int n_rows, LogCommit lc) {
  if ((int)blockIdx.x >= n_rows) {  // the scan's log-header update (LogCommit)
    const int i = ((int)blockIdx.x - n_rows) * (int)blockDim.x + (int)threadIdx.x;
    if (i < lc.jobs()) log_commit_one(lc, i);
    return;
  }
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  const float* zr = z + row * ldz;
  float yv[kMambaPostMax];
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < kMambaPostMax; ++u) {
    const int c = threadIdx.x + 256 * u;
    yv[u] = 0.0f;
    if (c < inner) {
      const float so = plane_sum(ssm_out, row * inner + c, n_parts, part_stride);
      yv[u] = (so + d[c / head_size] * xr[c]) * silu(zr[c]);
      ss += yv[u] * yv[u];
    }
  }
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)inner + 1e-5f);
#pragma unroll
  for (int u = 0; u < kMambaPostMax; ++u) {
    const int c = threadIdx.x + 256 * u;
    if (c < inner) {
      const float o = (yv[u] * inv) * w[c];
      if (out) out[row * inner + c] = o;
      if (out_lp) out_lp[row * inner + c] = f32_to_lp_bits(o, lp_fmt);
    }
  }
}

// One wave per head.
// A head's values held in registers (head_size <= 64 * kHeadPostMax).
constexpr int kHeadPostMax = 16;
__global__ void retnet_post_kernel(const float* __restrict__ o, int n_parts, int64_t part_stride,
                                   const float* __restrict__ g, int64_t ldg, int hidden,
                                   int head_size, float* __restrict__ out,
                                   uint16_t* __restrict__ out_lp, int lp_fmt, int n_rows, LogCommit lc,
                                   RetnetAdvance adv) {
  if ((int)blockIdx.x >= n_rows) {  // the scan's log-header update, then the position bookkeeping
    const int i = ((int)blockIdx.x - n_rows) * (int)blockDim.x + (int)threadIdx.x;
    if (i < lc.jobs())
      log_commit_one(lc, i);
    else if (i - lc.jobs() < adv.jobs())
      retnet_advance_one(adv, i - lc.jobs());
    return;
  }
  const int64_t row = blockIdx.x;
  const int head = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t ob = row * hidden + (int64_t)head * head_size;
  const float* grow = g + row * ldg + (int64_t)head * head_size;
  float ov[kHeadPostMax];
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < kHeadPostMax; ++u) {
    const int j = lane + 64 * u;
    ov[u] = j < head_size ? plane_sum(o, ob + j, n_parts, part_stride) : 0.0f;
    ss += ov[u] * ov[u];
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)head_size + 1e-6f);
#pragma unroll
  for (int u = 0; u < kHeadPostMax; ++u) {
    const int j = lane + 64 * u;
    if (j < head_size) {
      const float v = silu(grow[j]) * (ov[u] * inv);
      if (out) out[ob + j] = v;
      if (out_lp) out_lp[ob + j] = f32_to_lp_bits(v, lp_fmt);
    }
  }
}

// One wave per group, then a block-wide LayerNorm over the whole row.
__global__ void slstm_post_kernel(const float* __restrict__ y, const float* __restrict__ skip,
                                  const float* __restrict__ gn_w, const float* __restrict__ gn_b,
                                  const float* __restrict__ ln_w, int hidden, int gsize,
                                  float* __restrict__ x1, float* __restrict__ xn,
                                  uint16_t* __restrict__ xn_lp, int lp_fmt) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const int grp = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t base = row * hidden + (int64_t)grp * gsize;
  float s = 0.0f;
#pragma unroll 8
  for (int j = lane; j < gsize; j += 64) s += y[base + j];
  const float mean = wave_sum(s) / (float)gsize;
  float v = 0.0f;
#pragma unroll 8
  for (int j = lane; j < gsize; j += 64) {
    const float dlt = y[base + j] - mean;
    v += dlt * dlt;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(v) / (float)gsize + 1e-5f);
  float rs = 0.0f;
#pragma unroll 8
  for (int j = lane; j < gsize; j += 64) {
    const int c = grp * gsize + j;
    const float o = ((y[base + j] - mean) * rstd) * gn_w[c] + gn_b[c] + skip[base + j];
    x1[base + j] = o;
    rs += o;
  }
  __threadfence_block();
  const float rmean = block_sum(rs, red) / (float)hidden;
  float rv = 0.0f;
#pragma unroll 8
  for (int j = lane; j < gsize; j += 64) {
    const float dlt = x1[base + j] - rmean;
    rv += dlt * dlt;
  }
  const float rrstd = 1.0f / sqrtf(block_sum(rv, red) / (float)hidden + 1e-5f);
#pragma unroll 8
  for (int j = lane; j < gsize; j += 64) {
    const int c = grp * gsize + j;
    const float o = ((x1[base + j] - rmean) * rrstd) * ln_w[c];
    if (xn) xn[base + j] = o;
    if (xn_lp) xn_lp[base + j] = f32_to_lp_bits(o, lp_fmt);
  }
}

// One wave per head (= GroupNorm group); U values per lane (head size <=
// 64 U). Every operand of the head is loaded before the two reductions, so
// the kernel waits for memory once. FULL: the head size is exactly 64 U and
// nothing is predicated.
template <int U, bool FULL>
__global__ void mlstm_post_kernel(const float* __restrict__ num, int n_parts, int64_t part_stride,
                                  const float* __restrict__ den, int den_ld,
                                  const float* __restrict__ gn_w, const float* __restrict__ gn_b,
                                  const float* __restrict__ skip_w,
                                  const float* __restrict__ x_conv,
                                  const float* __restrict__ x_gate, int64_t ld_gate, int inner,
                                  int hs, float* __restrict__ out, uint16_t* __restrict__ out_lp, int lp_fmt, int n_rows, LogCommit lc,
                                  ConvCommit cc) {
  if ((int)blockIdx.x >= n_rows) {  // the scan's log-header update (LogCommit)
    const int i = ((int)blockIdx.x - n_rows) * (int)blockDim.x + (int)threadIdx.x;
    if (i < lc.jobs()) log_commit_one(lc, i);
    return;
  }
  const int64_t row = blockIdx.x;
  const int head = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // The last row of each run leaves the conv state: the inputs of positions
  // p-2 .. p (p its position), those before the run from the old state
  // (read here, before any write; every reader of it ran before this kernel).
  if (cc.state != nullptr && (row + 1 == n_rows || cc.row_pos[row + 1] == 0)) {
    const int p = cc.row_pos[row];
    float* st = cc.state + (int64_t)cc.row_slot[row] * cc.slot_stride;
    float nv[3][U];
#pragma unroll
    for (int k = 0; k < 3; ++k)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = head * hs + lane + 64 * u;
        nv[k][u] = 0.0f;
        if (FULL || lane + 64 * u < hs)
          nv[k][u] = p - 2 + k >= 0 ? cc.x[(row - (2 - k)) * cc.ldx + c]
                                    : st[(int64_t)(1 + p + k) * inner + c];
      }
#pragma unroll
    for (int k = 0; k < 3; ++k)
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (FULL || lane + 64 * u < hs) st[(int64_t)k * inner + head * hs + lane + 64 * u] = nv[k][u];
  }
  const int64_t base = row * inner + (int64_t)head * hs;
  const float* gate = x_gate + row * ld_gate + (int64_t)head * hs;
  float hv[U], gw[U], gb[U], sk[U], xc[U], xg[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = lane + 64 * u;
    const bool ok = FULL || j < hs;
    const int c = head * hs + j;
    hv[u] = ok ? plane_sum(num, base + j, n_parts, part_stride) : 0.0f;
    gw[u] = ok ? gn_w[c] : 0.0f;
    gb[u] = ok ? gn_b[c] : 0.0f;
    sk[u] = ok ? skip_w[c] : 0.0f;
    xc[u] = ok ? x_conv[base + j] : 0.0f;
    xg[u] = ok ? gate[j] : 0.0f;
  }
  const float dn = den[row * den_ld + head];
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    // num / den of this lane's elements; absent ones stay zero
    hv[u] = (FULL || lane + 64 * u < hs) ? hv[u] / dn : 0.0f;
    s += hv[u];
  }
  const float mean = wave_sum(s) / (float)hs;
  float v = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float dlt = (FULL || lane + 64 * u < hs) ? hv[u] - mean : 0.0f;
    v += dlt * dlt;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(v) / (float)hs + 1e-5f);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = lane + 64 * u;
    if (FULL || j < hs) {
      const float gnv = ((hv[u] - mean) * rstd) * gw[u] + gb[u];
      const float h = (gnv + sk[u] * xc[u]) * silu(xg[u]);
      if (out) out[base + j] = h;
      if (out_lp) out_lp[base + j] = f32_to_lp_bits(h, lp_fmt);
    }
  }
}

// One wave per row.
__global__ void output_proj_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                   const float* __restrict__ b, int n_rows, int hidden,
                                   float* __restrict__ preds, int pred_ld, int col) {
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int lane = threadIdx.x & 63;
  const float* xr = x + row * hidden;
  float s = 0.0f;
#pragma unroll 8
  for (int c = lane; c < hidden; c += 64) s += xr[c] * w[c];
  s = wave_sum(s);
  if (lane == 0) preds[row * pred_ld + col] = s + b[0];
}

__global__ void mlstm_qkv_kernel(const float* __restrict__ x_conv, const float* __restrict__ x_m,
                                 int64_t ld_xm, const float* __restrict__ wq,
                                 const float* __restrict__ wk, const float* __restrict__ wv,
                                 int n_rows, int inner, int blk, float k_div,
                                 float* __restrict__ qkv, float* __restrict__ ks) {
  const int64_t total = (int64_t)n_rows * inner;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / inner;
    const int c = (int)(i % inner);
    const int nb = c / blk;  // block index
    const int kk = c % blk;  // output index within the block
    const float* xc = x_conv + r * inner + (int64_t)nb * blk;
    const float* xm = x_m + r * ld_xm + (int64_t)nb * blk;
    const int64_t woff = ((int64_t)nb * blk + kk) * blk;  // W[nb][kk][:]
    float q = 0.0f, k = 0.0f, v = 0.0f;
    for (int h = 0; h < blk; ++h) {
      q += xc[h] * wq[woff + h];
      k += xc[h] * wk[woff + h];
      v += xm[h] * wv[woff + h];
    }
    float* out = qkv + r * 3 * (int64_t)inner;
    out[c] = q;
    out[inner + c] = k;
    out[2 * inner + c] = v;
    ks[r * inner + c] = k / k_div;
  }
}

// mLSTM q/k/v BlockLinear with 4x4 blocks (model/xlstm.py:191-193,
// :220-222) fused with the block's causal conv (model/xlstm.py:217-218) and
// the input / forget gate projections of the cell, [igate; fgate](cat(q, k,
// v)) (model/xlstm.py:29-30, :52-54), for R rows x one column segment per
// work-group: each thread computes whole 4-column blocks of the conv output
// (from x_m's rows and, before a run, the slot's conv state; stored for the
// block's tail), of q, k and v with 16-byte loads, stores them, and
// accumulates their NOUT gate-row products; the work-group's NOUT sums (in
// a fixed order) are segment seg's partial pre-activations, plane seg of
// if_part [segs][n_rows][NOUT]; plane 0 also carries the bias.
template <int NOUT, int R>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void mlstm_qkv_if_kernel(
    ConvIn conv, const float* __restrict__ x_m, int64_t ld_xm,
    const float* __restrict__ wq, const float* __restrict__ wk, const float* __restrict__ wv,
    int n_rows, int inner, float k_div, const float* __restrict__ w_if,
    const float* __restrict__ b_if, float* __restrict__ qkv, float* __restrict__ ks,
    float* __restrict__ if_part) {
  static_assert(R * NOUT <= 64, "one butterfly for all sums");
  __shared__ float red[4][R * NOUT];
  const int seg = blockIdx.x;
  const int rbase = blockIdx.y * R;  // rows rbase .. rbase + R - 1 (past n_rows: the last row)
  const int tid = threadIdx.x;
  const int per = (inner >> 2) / gridDim.x;  // 4-column blocks per segment
  const int64_t wl = (int64_t)3 * inner;
  int rows[R], pos[R];
  const float* cst[R];  // the conv state of the row's slot
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rows[r] = min(rbase + r, n_rows - 1);
    pos[r] = conv.row_pos[rows[r]];
    cst[r] = conv.state + (int64_t)conv.row_slot[rows[r]] * conv.slot_stride;
  }
  auto dot4 = [](float4 a, float4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; };
  // One channel of the conv, in conv_scan's order of operations.
  auto conv1 = [](float b, float w0, float w1, float w2, float w3, float s0, float s1, float s2,
                  float x) {
    float v = b + w0 * s0;
    v += w1 * s1;
    v += w2 * s2;
    v += w3 * x;
    return silu(v);
  };
  float acc[R * NOUT];
#pragma unroll
  for (int i = 0; i < R * NOUT; ++i) acc[i] = 0.0f;
  for (int nb = seg * per + tid; nb < (seg + 1) * per; nb += 256) {
    // The block's weights are loaded once for all R rows; every operand is
    // loaded before any is used (one L2 round trip per block).
    // xs[r][k]: the input k positions before row r's (k = 1..3; index
    // k - 1), from x_m inside the run, else from the conv state.
    float4 xc[R], xm[R], xs[R][3];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      xm[r] = reinterpret_cast<const float4*>(x_m + (int64_t)rows[r] * ld_xm)[nb];
#pragma unroll
      for (int k = 1; k <= 3; ++k) {
        const float* src = pos[r] >= k ? x_m + (int64_t)(rows[r] - k) * ld_xm
                                       : cst[r] + (int64_t)(3 + pos[r] - k) * inner;
        xs[r][k - 1] = reinterpret_cast<const float4*>(src)[nb];
      }
    }
    const float4 cw0 = reinterpret_cast<const float4*>(conv.w)[nb];
    const float4 cw1 = reinterpret_cast<const float4*>(conv.w + inner)[nb];
    const float4 cw2 = reinterpret_cast<const float4*>(conv.w + 2 * (int64_t)inner)[nb];
    const float4 cw3 = reinterpret_cast<const float4*>(conv.w + 3 * (int64_t)inner)[nb];
    const float4 cb = reinterpret_cast<const float4*>(conv.b)[nb];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float4 s0 = xs[r][2], s1 = xs[r][1], s2 = xs[r][0], x0 = xm[r];
      xc[r] = make_float4(conv1(cb.x, cw0.x, cw1.x, cw2.x, cw3.x, s0.x, s1.x, s2.x, x0.x),
                          conv1(cb.y, cw0.y, cw1.y, cw2.y, cw3.y, s0.y, s1.y, s2.y, x0.y),
                          conv1(cb.z, cw0.z, cw1.z, cw2.z, cw3.z, s0.z, s1.z, s2.z, x0.z),
                          conv1(cb.w, cw0.w, cw1.w, cw2.w, cw3.w, s0.w, s1.w, s2.w, x0.w));
      if (rbase + r < n_rows)
        reinterpret_cast<float4*>(conv.out + (int64_t)rows[r] * inner)[nb] = xc[r];
    }
    // W[nb][o][h]: block nb's 4x4 weights, row o = output column 4nb + o
    float4 bq[4], bk[4], bv[4];
#pragma unroll
    for (int o = 0; o < 4; ++o) {
      bq[o] = reinterpret_cast<const float4*>(wq)[(int64_t)nb * 4 + o];
      bk[o] = reinterpret_cast<const float4*>(wk)[(int64_t)nb * 4 + o];
      bv[o] = reinterpret_cast<const float4*>(wv)[(int64_t)nb * 4 + o];
    }
    float4 q[R], k[R], v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      q[r] = make_float4(dot4(xc[r], bq[0]), dot4(xc[r], bq[1]), dot4(xc[r], bq[2]), dot4(xc[r], bq[3]));
      k[r] = make_float4(dot4(xc[r], bk[0]), dot4(xc[r], bk[1]), dot4(xc[r], bk[2]), dot4(xc[r], bk[3]));
      v[r] = make_float4(dot4(xm[r], bv[0]), dot4(xm[r], bv[1]), dot4(xm[r], bv[2]), dot4(xm[r], bv[3]));
      if (rbase + r < n_rows) {
        float4* q4o = reinterpret_cast<float4*>(qkv + (int64_t)rows[r] * 3 * inner);
        q4o[nb] = q[r];
        q4o[(inner >> 2) + nb] = k[r];
        q4o[(inner >> 1) + nb] = v[r];
        reinterpret_cast<float4*>(ks + (int64_t)rows[r] * inner)[nb] =
            make_float4(k[r].x / k_div, k[r].y / k_div, k[r].z / k_div, k[r].w / k_div);
      }
    }
    // the gate rows' 16-byte pieces of this block's q, k and v columns
#pragma unroll
    for (int n = 0; n < NOUT; ++n) {
      const float4* wn = reinterpret_cast<const float4*>(w_if + n * wl);
      const float4 w0 = wn[nb], w1 = wn[(inner >> 2) + nb], w2 = wn[(inner >> 1) + nb];
#pragma unroll
      for (int r = 0; r < R; ++r)
        acc[r * NOUT + n] += dot4(q[r], w0) + dot4(k[r], w1) + dot4(v[r], w2);
    }
  }
  // lane (64 / (R*NOUT)) * i of each wave holds the wave's sum i = r*NOUT + n
  constexpr int NV = R * NOUT;
  const float ws = transposed_wave_sum<NV>(acc);
  const int lane = tid & 63, wave = tid >> 6;
  if (lane % (64 / NV) == 0) red[wave][lane / (64 / NV)] = ws;
  lds_barrier();
  if (tid < NV) {
    const int r = tid / NOUT, n = tid % NOUT;
    if (rbase + r < n_rows) {
      float t = seg == 0 ? b_if[n] : 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) t += red[w2][tid];
      if_part[((int64_t)seg * n_rows + rbase + r) * NOUT + n] = t;
    }
  }
}

__global__ void to_lp_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                             int64_t n, int lp_fmt) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = f32_to_lp_bits(src[i], lp_fmt);
}

__global__ void round_lp_inplace_kernel(float* __restrict__ v, int64_t n, int lp_fmt) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    v[i] = round_lp(v[i], lp_fmt);
}

__global__ void fill_f32_kernel(float* __restrict__ dst, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = v;
}

inline unsigned grid_for(int64_t total, int block = 256) {
  int64_t g = (total + block - 1) / block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (unsigned)g;
}

}  // namespace

// Dispatch on the row width: V elements per thread, width <= 256 * V.
#define HK_ROW_DISPATCH(width, LAUNCH)                                     \
  do {                                                                     \
    HK_REQUIRE((width) >= 1 && (width) <= 8192, "row width %d unsupported (at most 8192)", \
               (int)(width));                                              \
    if ((width) <= 256) { LAUNCH(1); }                                     \
    else if ((width) <= 1024) { LAUNCH(4); }                               \
    else if ((width) <= 2048) { LAUNCH(8); }                               \
    else if ((width) <= 4096) { LAUNCH(16); }                              \
    else { LAUNCH(32); }                                                   \
  } while (0)

int rmsnorm_rows(const float* x, int64_t ldx, const float* w, float eps, int n_rows, int width,
                 float* out, int64_t ldo, uint16_t* out_lp, int lp_fmt, int64_t ldl, hipStream_t s) {
  if (n_rows == 0) return HK_OK;
#define L(V)                                                                              \
  hipLaunchKernelGGL(rmsnorm_kernel<V>, dim3(n_rows), dim3(256), 0, s, x, ldx, w, eps, width, \
                     out, ldo, out_lp, lp_fmt, ldl)
  HK_ROW_DISPATCH(width, L);
#undef L
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int rms_ln_rows(const float* x, const float* w_rms, float eps, const float* w_ln, int n_rows,
                int width, float* a, uint16_t* a_lp, int lp_fmt, float* xn, hipStream_t s) {
  if (n_rows == 0) return HK_OK;
#define L(V)                                                                                \
  hipLaunchKernelGGL(rms_ln_kernel<V>, dim3(n_rows), dim3(256), 0, s, x, w_rms, eps, w_ln, width, \
                     a, a_lp, lp_fmt, xn)
  HK_ROW_DISPATCH(width, L);
#undef L
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int ln_res_rms_rows(const float* y, const float* w_ln, float* x, const float* w_rms, float eps,
                    int n_rows, int width, float* a, uint16_t* a_lp, int lp_fmt, hipStream_t s) {
  if (n_rows == 0) return HK_OK;
#define L(V)                                                                                  \
  hipLaunchKernelGGL(ln_res_rms_kernel<V>, dim3(n_rows), dim3(256), 0, s, y, w_ln, x, w_rms, eps, \
                     width, a, a_lp, lp_fmt)
  HK_ROW_DISPATCH(width, L);
#undef L
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int stage_features(const float* feat, int n_rows, int f, int kpad, float* out, uint16_t* out_lp, int lp_fmt,
                   hipStream_t s) {
  if (n_rows == 0) return HK_OK;
  hipLaunchKernelGGL(stage_features_kernel, dim3(grid_for((int64_t)n_rows * kpad)), dim3(256), 0,
                     s, feat, n_rows, f, kpad, out, out_lp, lp_fmt);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

// Rows plus the work-groups of a LogCommit job of `threads`-thread groups.
unsigned rows_and_commit(int n_rows, const LogCommit& lc, int threads) {
  return (unsigned)(n_rows + (lc.jobs() + threads - 1) / threads);
}

int mamba2_post(const float* ssm_out, int n_parts, int64_t part_stride, const float* x,
                int64_t ldx, const float* z, int64_t ldz, const float* d, const float* w,
                int n_rows, int inner, int head_size, float* out, uint16_t* out_lp, int lp_fmt,
                const LogCommit& lc, hipStream_t s) {
  if (n_rows == 0 && lc.jobs() == 0) return HK_OK;
  HK_REQUIRE(inner <= 256 * kMambaPostMax && n_parts >= 1,
             "mamba2_post: inner %d above %d or no planes", inner, 256 * kMambaPostMax);
  hipLaunchKernelGGL(mamba2_post_kernel, dim3(rows_and_commit(n_rows, lc, 256)), dim3(256), 0, s,
                     ssm_out, n_parts, part_stride, x, ldx, z, ldz, d, w, inner, head_size, out,
                     out_lp, lp_fmt, n_rows, lc);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int retnet_post(const float* o, int n_parts, int64_t part_stride, const float* g, int64_t ldg,
                int n_rows, int hidden, int head_size, float* out, uint16_t* out_lp, int lp_fmt,
                const LogCommit& lc, const RetnetAdvance& adv, hipStream_t s) {
  if (n_rows == 0 && lc.jobs() == 0 && adv.jobs() == 0) return HK_OK;
  const int heads = hidden / head_size;
  HK_REQUIRE(heads * head_size == hidden && heads <= 16 && head_size <= 64 * kHeadPostMax &&
                 n_parts >= 1,
             "retnet_post: %d heads of %d unsupported", heads, head_size);
  HK_REQUIRE(adv.jobs() == 0 || (adv.slot_ids && adv.run_off && adv.decay && adv.scales),
             "retnet_post: incomplete position bookkeeping");
  const int threads = 64 * heads;
  const unsigned grid =
      (unsigned)(n_rows + (lc.jobs() + adv.jobs() + threads - 1) / threads);
  hipLaunchKernelGGL(retnet_post_kernel, dim3(grid), dim3(threads), 0, s, o, n_parts, part_stride,
                     g, ldg, hidden, head_size, out, out_lp, lp_fmt, n_rows, lc, adv);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int slstm_post(const float* y, const float* skip, const float* gn_w, const float* gn_b,
               int groups, const float* ln_w, int n_rows, int hidden, float* x1, float* xn,
               uint16_t* xn_lp, int lp_fmt, hipStream_t s) {
  if (n_rows == 0) return HK_OK;
  HK_REQUIRE(groups >= 1 && groups <= 16 && hidden % groups == 0,
             "slstm_post: %d groups unsupported", groups);
  hipLaunchKernelGGL(slstm_post_kernel, dim3(n_rows), dim3(64 * groups), 0, s, y, skip, gn_w,
                     gn_b, ln_w, hidden, hidden / groups, x1, xn, xn_lp, lp_fmt);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int layernorm_rows(const float* x, const float* w, const float* residual, int n_rows, int width,
                   float* out, uint16_t* out_lp, int lp_fmt, hipStream_t s) {
  if (n_rows == 0) return HK_OK;
#define L(V)                                                                                \
  hipLaunchKernelGGL(layernorm_kernel<V>, dim3(n_rows), dim3(256), 0, s, x, w, residual, width, \
                     out, out_lp, lp_fmt)
  HK_ROW_DISPATCH(width, L);
#undef L
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int mlstm_post(const float* num, int n_parts, int64_t part_stride, const float* den, int den_ld,
               const float* gn_w, const float* gn_b, const float* skip_w, const float* x_conv,
               const float* x_gate, int64_t ld_gate, int n_rows, int inner, int heads,
               float* out, uint16_t* out_lp, int lp_fmt, const LogCommit& lc,
               const ConvCommit& cc, hipStream_t s) {
  if (n_rows == 0 && lc.jobs() == 0) return HK_OK;
  HK_REQUIRE(heads >= 1 && heads <= 16 && inner % heads == 0 &&
                 inner / heads <= 64 * kHeadPostMax && n_parts >= 1,
             "mlstm_post: %d heads of %d unsupported", heads, inner / std::max(heads, 1));
  HK_REQUIRE(!cc.state || (cc.row_pos && cc.row_slot && cc.x),
             "mlstm_post: conv state update without row descriptors or inputs");
  const int hs = inner / heads;
#define HK_POST(U, F)                                                                     \
  hipLaunchKernelGGL((mlstm_post_kernel<U, F>), dim3(rows_and_commit(n_rows, lc, 64 * heads)), \
                     dim3(64 * heads), 0, s, num, n_parts, part_stride, den, den_ld, gn_w, gn_b, \
                     skip_w, x_conv, x_gate, ld_gate, inner, hs, out, out_lp, lp_fmt, n_rows, lc, \
                     cc)
  if (hs == 512) {
    HK_POST(8, true);
  } else if (hs == 256) {
    HK_POST(4, true);
  } else if (hs == 128) {
    HK_POST(2, true);
  } else if (hs == 64) {
    HK_POST(1, true);
  } else {
    HK_POST(kHeadPostMax, false);
  }
#undef HK_POST
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int output_proj(const float* x, const float* w, const float* b, int n_rows, int hidden,
                float* preds, int pred_ld, int col, hipStream_t s) {
  if (n_rows == 0) return HK_OK;
  hipLaunchKernelGGL(output_proj_kernel, dim3((n_rows + 3) / 4), dim3(256), 0, s, x, w, b, n_rows,
                     hidden, preds, pred_ld, col);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int mlstm_qkv(const float* x_conv, const float* x_m, int64_t ld_xm, const float* wq,
              const float* wk, const float* wv, int n_rows, int inner, int blk, float k_div,
              float* qkv, float* ks, hipStream_t s) {
  if (n_rows == 0) return HK_OK;
  hipLaunchKernelGGL(mlstm_qkv_kernel, dim3(grid_for((int64_t)n_rows * inner)), dim3(256), 0, s,
                     x_conv, x_m, ld_xm, wq, wk, wv, n_rows, inner, blk, k_div, qkv, ks);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int mlstm_qkv_if(const ConvIn& conv, const float* x_m, int64_t ld_xm, const float* wq,
                 const float* wk, const float* wv, int n_rows, int inner, float k_div,
                 const float* w_if, const float* b_if, int n_out, float* qkv, float* ks,
                 float* if_part, int segs, hipStream_t s) {
  if (n_rows == 0) return HK_OK;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  HK_REQUIRE(conv.state && conv.w && conv.b && conv.row_pos && conv.row_slot && conv.out,
             "mlstm_qkv_if: null conv operand");
  HK_REQUIRE(mlstm_qkv_if_supported(inner, n_out, segs) && ld_xm % 4 == 0 &&
                 conv.slot_stride % 4 == 0 && al16(conv.state) && al16(conv.w) && al16(conv.b) &&
                 al16(conv.out) && al16(x_m) && al16(wq) && al16(wk) && al16(wv) && al16(w_if) &&
                 al16(qkv) && al16(ks),
             "mlstm_qkv_if: inner %d, %d gate rows, %d segments or alignment unsupported", inner,
             n_out, segs);
  // R rows per work-group share each block's weight loads (R * n_out <= 64).
  const dim3 block(256);
#define HK_QKV_IF(NOUT, R)                                                                      \
  hipLaunchKernelGGL((mlstm_qkv_if_kernel<NOUT, R>), dim3(segs, (n_rows + (R)-1) / (R)), block, \
                     0, s, conv, x_m, ld_xm, wq, wk, wv, n_rows, inner, k_div, w_if, b_if, qkv, \
                     ks, if_part)
  switch (n_out) {
    case 4: HK_QKV_IF(4, 4); break;
    case 8: HK_QKV_IF(8, 4); break;
    case 16: HK_QKV_IF(16, 4); break;
    default: HK_QKV_IF(32, 2); break;
  }
#undef HK_QKV_IF
  HK_LAUNCH_CHECK();
  return HK_OK;
}

bool mlstm_qkv_if_supported(int inner, int n_out, int segs) {
  return (n_out == 4 || n_out == 8 || n_out == 16 || n_out == 32) && inner % 4 == 0 && segs >= 1 &&
         (inner / 4) % segs == 0;
}

int to_lp(const float* src, uint16_t* dst, int64_t n, int lp_fmt, hipStream_t s) {
  if (n == 0) return HK_OK;
  hipLaunchKernelGGL(to_lp_kernel, dim3(grid_for(n)), dim3(256), 0, s, src, dst, n, lp_fmt);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int round_lp_inplace(float* v, int64_t n, int lp_fmt, hipStream_t s) {
  if (n == 0) return HK_OK;
  hipLaunchKernelGGL(round_lp_inplace_kernel, dim3(grid_for(n)), dim3(256), 0, s, v, n, lp_fmt);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int fill_f32(float* dst, int64_t n, float v, hipStream_t s) {
  if (n == 0) return HK_OK;
  hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, dst, n, v);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

}  // namespace hk
