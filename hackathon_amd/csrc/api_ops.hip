// extern "C" entry points for the reference's fused state-step API
// (model/kernels.py:346-401): state updated in place on active rows, idle rows
// untouched, idle outputs zero. Shapes follow the reference's (B, n, h, k)
// layout; every operand is a contiguous fp32 device array.
#include <cstring>
#include <string>

#include "common.h"
#include "gemm.h"
#include "scan_mat.h"

namespace hk {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

namespace {

// Element at a 32-bit byte offset from a wave-uniform base (global memory
// access with a scalar base and a vector offset).
__device__ __forceinline__ float* at_bytes(float* base, uint32_t bytes) {
  return reinterpret_cast<float*>(reinterpret_cast<char*>(base) + bytes);
}

// One chunk of RC state rows h0 .. h0+RC-1 of mamba2_row_step_kernel (sb,
// xr, yo already offset to row h0). GUARD = false: every row and column of
// the chunk exists (no predication, so the loads issue back to back).
template <int CPL, int RC, bool GUARD>
__device__ __forceinline__ void mamba2_chunk(float* sb, const float* xr, float* yo, int rows_left,
                                             float a, const float (&coef)[CPL],
                                             const float (&cw)[CPL], const bool (&cok)[CPL],
                                             int lane, int size_c) {
  float sv[RC][CPL], xv[RC], p[RC];
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    const bool hok = !GUARD || i < rows_left;
    xv[i] = hok ? xr[i] : 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t off = 4u * (uint32_t)(i * size_c + lane + 64 * j);
      sv[i][j] = (!GUARD || (hok && cok[j])) ? *at_bytes(sb, off) : 0.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      sv[i][j] = a * sv[i][j] + coef[j] * xv[i];
      acc += cw[j] * sv[i][j];
    }
    p[i] = acc;
  }
#pragma unroll
  for (int i = 0; i < RC; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t off = 4u * (uint32_t)(i * size_c + lane + 64 * j);
      if (!GUARD || (i < rows_left && cok[j])) *at_bytes(sb, off) = sv[i][j];
    }
  const float sum = transposed_wave_sum<RC>(p);  // lane i * 64 / RC holds row i
  constexpr int kShift = RC == 16 ? 2 : RC == 8 ? 3 : RC == 4 ? 4 : RC == 2 ? 5 : 6;
  const int r = lane >> kShift;
  if ((lane & ((1 << kShift) - 1)) == 0 && (!GUARD || r < rows_left)) yo[r] = sum;
}

// Mamba2 step in the reference's state layout [B][heads][h][c], where c (the
// axis y contracts over) is contiguous: one work-group per (row, head), lane
// = column c (CPL columns per lane, so a state row is one coalesced wave
// access), each wave 16 rows h at a time (full chunks unpredicated, a
// ragged one 4 rows at a time); the row sums over c come out of one
// transposed butterfly. Idle rows: state untouched, output zero.
template <int CPL>
__global__ __launch_bounds__(256) void mamba2_row_step_kernel(
    float* __restrict__ ssm, const float* __restrict__ x, const float* __restrict__ b,
    const float* __restrict__ c, const float* __restrict__ dt, const float* __restrict__ decay,
    const uint8_t* __restrict__ mask, float* __restrict__ y, int heads, int size_h, int size_c) {
  const int head = blockIdx.x;
  const int row = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t rh = (int64_t)row * heads + head;
  float* yo = y + rh * size_h;
  if (mask != nullptr && mask[row] == 0) {
    for (int h = threadIdx.x; h < size_h; h += blockDim.x) yo[h] = 0.0f;
    return;
  }
  const float a = decay[rh];
  const float sdt = dt[rh];
  float coef[CPL], cw[CPL];
  bool cok[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int ci = lane + 64 * j;
    cok[j] = ci < size_c;
    coef[j] = cok[j] ? sdt * b[(int64_t)row * size_c + ci] : 0.0f;  // (dt * b), then * x
    cw[j] = cok[j] ? c[(int64_t)row * size_c + ci] : 0.0f;
  }
  float* st = ssm + rh * size_h * size_c;
  const float* xr = x + rh * size_h;
  const bool full_c = size_c == 64 * CPL;
  for (int h0 = wave * 16; h0 < size_h; h0 += 64) {
    float* sb = st + (int64_t)h0 * size_c;  // uniform per wave
    if (full_c && h0 + 16 <= size_h) {
      mamba2_chunk<CPL, 16, false>(sb, xr + h0, yo + h0, 16, a, coef, cw, cok, lane, size_c);
    } else {
      for (int r = 0; r < 16 && h0 + r < size_h; r += 4)
        mamba2_chunk<CPL, 4, true>(sb + (int64_t)r * size_c, xr + h0 + r, yo + h0 + r,
                                   size_h - h0 - r, a, coef, cw, cok, lane, size_c);
    }
  }
}

// One chunk of RC state rows h0 .. h0+RC-1 of hcontract_row_step_kernel.
// GUARD = false: every row and column of the chunk exists (no predication,
// so the row scalars and the state loads issue back to back).
template <int CPL, int RC, bool GUARD>
__device__ __forceinline__ void hcontract_chunk(float* sb, const float* bh, const float* wh,
                                                int rows_left, float a, float sc,
                                                const float (&g)[CPL], const bool (&cok)[CPL],
                                                float (&acc)[CPL], int lane, int size_k) {
  float sv[RC][CPL], bb[RC], ww[RC];
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    const bool hok = !GUARD || i < rows_left;
    bb[i] = hok ? sc * bh[i] : 0.0f;  // (scale * beta): the reference's association
    ww[i] = hok ? wh[i] : 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t off = 4u * (uint32_t)(i * size_k + lane + 64 * j);
      sv[i][j] = (!GUARD || (hok && cok[j])) ? *at_bytes(sb, off) : 0.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < RC; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      sv[i][j] = a * sv[i][j] + bb[i] * g[j];
      acc[j] += ww[i] * sv[i][j];
    }
#pragma unroll
  for (int i = 0; i < RC; ++i)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t off = 4u * (uint32_t)(i * size_k + lane + 64 * j);
      if (!GUARD || (i < rows_left && cok[j])) *at_bytes(sb, off) = sv[i][j];
    }
}

// One step of S <- alpha S + (scale beta) (x) gamma, out_k = sum_h w_h
// S_new[h, k] on the reference's [B][heads][h][k] layout (k contiguous:
// mlstm_step, retnet_step). One work-group per (row, head); lane = column k
// (CPL columns per lane); wave v takes chunks of RC = 16 / CPL rows, 4 RC
// apart, starting at row v RC, the chunk's 16 state values per lane loaded
// together. The four waves' column sums meet once in LDS, added in wave
// order. Idle rows: state untouched, output zero.
template <int CPL, int RC = 16 / CPL>
__global__ __launch_bounds__(256) void hcontract_row_step_kernel(
    float* __restrict__ S, const float* __restrict__ alpha, int64_t alpha_head_stride,
    int64_t alpha_row_stride, const float* __restrict__ scale, const float* __restrict__ beta,
    const float* __restrict__ gamma, const float* __restrict__ w, const uint8_t* __restrict__ mask,
    float* __restrict__ out, int heads, int size_h, int size_k) {
  __shared__ float red[4][64 * CPL];
  const int head = blockIdx.x;
  const int row = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t rh = (int64_t)row * heads + head;
  float* o = out + rh * size_k;
  if (mask != nullptr && mask[row] == 0) {
    for (int k = threadIdx.x; k < size_k; k += blockDim.x) o[k] = 0.0f;
    return;
  }
  const float a = alpha[(int64_t)row * alpha_row_stride + (int64_t)head * alpha_head_stride];
  const float sc = scale ? scale[rh] : 1.0f;
  float g[CPL], acc[CPL];
  bool cok[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    cok[j] = c < size_k;
    g[j] = cok[j] ? gamma[rh * size_k + c] : 0.0f;
    acc[j] = 0.0f;
  }
  float* st = S + rh * size_h * size_k;
  const float* bh = beta + rh * size_h;
  const float* wh = w + rh * size_h;
  const bool full_k = size_k == 64 * CPL;
  for (int h0 = wave * RC; h0 < size_h; h0 += 4 * RC) {
    float* sb = st + (int64_t)h0 * size_k;  // uniform per wave
    if (full_k && h0 + RC <= size_h) {
      hcontract_chunk<CPL, RC, false>(sb, bh + h0, wh + h0, RC, a, sc, g, cok, acc, lane, size_k);
    } else {  // ragged chunk: 4 rows at a time (keeps the register count of the full path)
      for (int r = 0; r < RC && h0 + r < size_h; r += 4)
        hcontract_chunk<CPL, 4, true>(sb + (int64_t)r * size_k, bh + h0 + r, wh + h0 + r,
                                      size_h - h0 - r, a, sc, g, cok, acc, lane, size_k);
    }
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j) red[wave][lane + 64 * j] = acc[j];
  lds_barrier();
  for (int k = threadIdx.x; k < size_k; k += blockDim.x)
    o[k] = ((red[0][k] + red[1][k]) + red[2][k]) + red[3][k];
}

// Depthwise causal conv step in the reference's layout: state [B][C][K-1]
// (oldest tap first), weight [C][K]. One thread per (row, channel); the
// window is [state, x] and the taps are added in window order after the
// bias, as the engine's run kernel does.
constexpr int kConvMaxTaps = 8;

__global__ __launch_bounds__(256) void conv1d_step_kernel(
    float* __restrict__ state, const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ bias, const uint8_t* __restrict__ mask, float* __restrict__ out,
    int64_t n, int channels, int taps) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t row = i / channels;
  const int ch = (int)(i - row * channels);
  if (mask != nullptr && mask[row] == 0) {
    out[i] = 0.0f;
    return;
  }
  float win[kConvMaxTaps];
  float* st = state + i * (taps - 1);
  for (int j = 0; j < taps - 1; ++j) win[j] = st[j];
  win[taps - 1] = x[i];
  const float* wr = w + (int64_t)ch * taps;
  float v = (bias ? bias[ch] : 0.0f) + wr[0] * win[0];
  for (int j = 1; j < taps; ++j) v += wr[j] * win[j];
  out[i] = v;
  for (int j = 0; j < taps - 1; ++j) st[j] = win[j + 1];
}

// RG-LRU elementwise step on the gate pre-activations: h' = h a^(c r) +
// sqrt(1 - a^(2 c r)) (i x), i = sigmoid(gi), r = sigmoid(gr), the same
// operations in the same order as the engine's run kernel.
__global__ __launch_bounds__(256) void rglru_step_kernel(
    float* __restrict__ h, const float* __restrict__ x, const float* __restrict__ gi,
    const float* __restrict__ gr, const float* __restrict__ a, float c_exp,
    const uint8_t* __restrict__ mask, float* __restrict__ out, int64_t n, int width) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t row = i / width;
  const int ch = (int)(i - row * width);
  if (mask != nullptr && mask[row] == 0) {
    if (out) out[i] = 0.0f;
    return;
  }
  const float it = sigmoid(gi[i]);
  const float rt = sigmoid(gr[i]);
  const float at = powf(a[ch], c_exp * rt);
  const float mult = sqrtf(1.0f - at * at);
  const float hn = (h[i] * at) + (mult * (it * x[i]));
  h[i] = hn;
  if (out) out[i] = hn;
}

// sLSTM cell step on the four gate pre-activations (stabilised exponential
// gates; the same operations as the engine's round kernel).
__global__ __launch_bounds__(256) void slstm_step_kernel(
    float* __restrict__ c_state, float* __restrict__ n_state, float* __restrict__ m_state,
    const float* __restrict__ ip, const float* __restrict__ fp, const float* __restrict__ zp,
    const float* __restrict__ op, const uint8_t* __restrict__ mask, float* __restrict__ y,
    int64_t n, int width) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  if (mask != nullptr && mask[i / width] == 0) {
    y[i] = 0.0f;
    return;
  }
  const float lfm = m_state[i] + logsigmoid(fp[i]);
  const float mn = fmaxf(ip[i], lfm);
  const float og = sigmoid(op[i]);
  const float ig = expf(ip[i] - mn);
  const float fg = expf(lfm - mn);
  const float cn = fg * c_state[i] + ig * tanhf(zp[i]);
  const float nn = fg * n_state[i] + ig;
  c_state[i] = cn;
  n_state[i] = nn;
  m_state[i] = mn;
  y[i] = og * cn / (nn + 1e-6f);
}

// BlockLinear with blocks too small or unaligned for the matrix-core GEMM:
// one thread per output, the dot product over the block in input order.
__global__ __launch_bounds__(256) void block_linear_kernel(
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ out, int64_t n, int blocks, int bs) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int width = blocks * bs;
  const int64_t row = i / width;
  const int col = (int)(i - row * width);
  const int blk = col / bs;
  const float* xr = x + row * width + (int64_t)blk * bs;
  const float* wr = w + (int64_t)col * bs;  // W[blk][o][:], col = blk*bs + o
  float acc = 0.0f;
  for (int h = 0; h < bs; ++h) acc = fmaf(xr[h], wr[h], acc);
  out[i] = bias ? acc + bias[col] : acc;
}

int elementwise_grid(int64_t n, unsigned* blocks) {
  const int64_t b = (n + 255) / 256;
  HK_REQUIRE(b < (1LL << 31), "too many elements (%lld)", (long long)n);
  *blocks = (unsigned)b;
  return HK_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

int hcontract_row_step(float* S, const float* alpha, int64_t alpha_head_stride,
                       int64_t alpha_row_stride, const float* scale, const float* beta,
                       const float* gamma, const float* w, const uint8_t* mask, float* out,
                       int batch, int heads, int size_h, int size_k, hipStream_t s) {
  const dim3 grid(heads, batch), block(256);
#define HK_HC(C)                                                                           \
  hipLaunchKernelGGL(hcontract_row_step_kernel<C>, grid, block, 0, s, S, alpha,            \
                     alpha_head_stride, alpha_row_stride, scale, beta, gamma, w, mask, out, \
                     heads, size_h, size_k)
  if (size_k <= 64) {
    HK_HC(1);
  } else if (size_k <= 128) {
    HK_HC(2);
  } else {
    HK_HC(4);
  }
#undef HK_HC
  HK_LAUNCH_CHECK();
  return HK_OK;
}

namespace {

}  // namespace

}  // namespace hk

extern "C" {

const char* hk_last_error(void) { return hk::g_last_error.c_str(); }

int hk_version(void) { return 2; }

int hk_mlstm_step(float* cell, const float* q, const float* k, const float* v,
                  const float* i_gate, const float* f_gate, const uint8_t* mask, float* out,
                  int batch, int heads, int size_h, int size_k, void* stream) {
  HK_REQUIRE(batch >= 0 && heads > 0 && size_h > 0 && size_k > 0,
             "hk_mlstm_step: bad shape B=%d n=%d h=%d k=%d", batch, heads, size_h, size_k);
  if (batch == 0) return HK_OK;
  if (size_k <= 256 && batch <= 65535 && heads <= 65535) {
    return hk::hcontract_row_step(cell, f_gate, 1, heads, i_gate, k, v, q, mask, out, batch,
                                  heads, size_h, size_k, (hipStream_t)stream);
  }
  hk::MatScanDesc d;
  d.state = cell;
  d.rows = size_h;
  d.cols = size_k;
  d.heads = heads;
  d.row_stride = size_k;
  d.col_stride = 1;
  d.head_stride = (int64_t)size_h * size_k;
  d.slot_stride = (int64_t)heads * size_h * size_k;
  d.per_row = true;
  d.mask = mask;
  d.n_runs = batch;
  d.alpha = {f_gate, heads, 1};
  d.scale = {i_gate, heads, 1};
  d.beta = {k, (int64_t)heads * size_h, size_h};
  d.gamma = {v, (int64_t)heads * size_k, size_k};
  d.w = {q, (int64_t)heads * size_h, size_h};
  d.out = out;
  d.out_row_stride = (int64_t)heads * size_k;
  d.out_head_stride = size_k;
  return hk::launch_mat_scan(d, (hipStream_t)stream);
}

int hk_retnet_step(float* state, const float* k_rope, const float* v, const float* q_scaled,
                   const float* decay, const uint8_t* mask, float* out, int batch, int heads,
                   int size_h, int size_k, void* stream) {
  HK_REQUIRE(batch >= 0 && heads > 0 && size_h > 0 && size_k > 0,
             "hk_retnet_step: bad shape B=%d n=%d h=%d k=%d", batch, heads, size_h, size_k);
  if (batch == 0) return HK_OK;
  if (size_k <= 256 && batch <= 65535 && heads <= 65535) {
    // one decay per head, shared by every row
    return hk::hcontract_row_step(state, decay, 1, 0, nullptr, k_rope, v, q_scaled, mask, out,
                                  batch, heads, size_h, size_k, (hipStream_t)stream);
  }
  hk::MatScanDesc d;
  d.state = state;
  d.rows = size_h;
  d.cols = size_k;
  d.heads = heads;
  d.row_stride = size_k;
  d.col_stride = 1;
  d.head_stride = (int64_t)size_h * size_k;
  d.slot_stride = (int64_t)heads * size_h * size_k;
  d.per_row = true;
  d.mask = mask;
  d.n_runs = batch;
  d.alpha = {decay, 0, 1};  // one decay per head, shared by every row
  d.scale = {nullptr, 0, 0};
  d.beta = {k_rope, (int64_t)heads * size_h, size_h};
  d.gamma = {v, (int64_t)heads * size_k, size_k};
  d.w = {q_scaled, (int64_t)heads * size_h, size_h};
  d.out = out;
  d.out_row_stride = (int64_t)heads * size_k;
  d.out_head_stride = size_k;
  return hk::launch_mat_scan(d, (hipStream_t)stream);
}

int hk_mamba2_step(float* ssm, const float* x, const float* b, const float* c, const float* dt,
                   const float* decay, const uint8_t* mask, float* y, int batch, int heads,
                   int size_h, int size_c, void* stream) {
  HK_REQUIRE(batch >= 0 && heads > 0 && size_h > 0 && size_c > 0,
             "hk_mamba2_step: bad shape B=%d n=%d h=%d c=%d", batch, heads, size_h, size_c);
  if (batch == 0) return HK_OK;
  if (size_c <= 256 && batch <= 65535 && heads <= 65535) {
    const dim3 grid(heads, batch), block(256);
    hipStream_t s = (hipStream_t)stream;
#define HK_M2(C)                                                                              \
  hipLaunchKernelGGL(hk::mamba2_row_step_kernel<C>, grid, block, 0, s, ssm, x, b, c, dt, decay, \
                     mask, y, heads, size_h, size_c)
    if (size_c <= 64) {
      HK_M2(1);
    } else if (size_c <= 128) {
      HK_M2(2);
    } else {
      HK_M2(4);
    }
#undef HK_M2
    HK_LAUNCH_CHECK();
    return HK_OK;
  }
  // Wider states: the matrix scan with tile rows = c (stride 1) and tile
  // columns = h (stride size_c).
  hk::MatScanDesc d;
  d.state = ssm;
  d.rows = size_c;
  d.cols = size_h;
  d.heads = heads;
  d.row_stride = 1;
  d.col_stride = size_c;
  d.head_stride = (int64_t)size_h * size_c;
  d.slot_stride = (int64_t)heads * size_h * size_c;
  d.per_row = true;
  d.mask = mask;
  d.n_runs = batch;
  d.alpha = {decay, heads, 1};
  d.scale = {dt, heads, 1};
  d.beta = {b, size_c, 0};  // b and c are per row, shared by every head
  d.gamma = {x, (int64_t)heads * size_h, size_h};
  d.w = {c, size_c, 0};
  d.out = y;
  d.out_row_stride = (int64_t)heads * size_h;
  d.out_head_stride = size_h;
  return hk::launch_mat_scan(d, (hipStream_t)stream);
}

int hk_conv1d_step(float* state, const float* x, const float* weight, const float* bias,
                   const uint8_t* mask, float* out, int batch, int channels, int kernel_size,
                   void* stream) {
  HK_REQUIRE(batch >= 0 && channels > 0 && kernel_size >= 1 &&
                 kernel_size <= hk::kConvMaxTaps,
             "hk_conv1d_step: bad shape B=%d C=%d K=%d (K in 1..%d)", batch, channels,
             kernel_size, hk::kConvMaxTaps);
  HK_REQUIRE(state || kernel_size == 1, "hk_conv1d_step: null state");
  HK_REQUIRE(x && weight && out, "hk_conv1d_step: null operand");
  const int64_t n = (int64_t)batch * channels;
  if (n == 0) return HK_OK;
  unsigned blocks;
  const int st = hk::elementwise_grid(n, &blocks);
  if (st != HK_OK) return st;
  hipLaunchKernelGGL(hk::conv1d_step_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     state, x, weight, bias, mask, out, n, channels, kernel_size);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int hk_block_linear(const float* x, const float* weight, const float* bias, float* out, int batch,
                    int blocks, int block_size, void* stream) {
  HK_REQUIRE(batch >= 0 && blocks > 0 && block_size > 0,
             "hk_block_linear: bad shape B=%d blocks=%d size=%d", batch, blocks, block_size);
  HK_REQUIRE(x && weight && out, "hk_block_linear: null operand");
  if (batch == 0) return HK_OK;
  hipStream_t s = (hipStream_t)stream;
  if (block_size % 16 == 0 && hk::aligned16(x) && hk::aligned16(weight) && hk::aligned16(out)) {
    // Matrix cores: the blocks are the batches of one fp32 GEMM launch.
    hk::GemmArgs g;
    g.type = hk::GemmType::kF32;
    g.A = x;
    g.lda = (int64_t)blocks * block_size;
    g.W = weight;
    g.ldw = block_size;
    g.M = batch;
    g.N = block_size;
    g.K = block_size;
    g.batch = blocks;
    g.a_bstride = block_size;
    g.w_bstride = (int64_t)block_size * block_size;
    g.c_bstride = block_size;
    g.ep.bias = bias;
    g.ep.out = out;
    g.ep.ldo = (int64_t)blocks * block_size;
    return hk::gemm(g, hk::GemmWorkspace{}, s);
  }
  const int64_t n = (int64_t)batch * blocks * block_size;
  unsigned nb;
  const int st = hk::elementwise_grid(n, &nb);
  if (st != HK_OK) return st;
  hipLaunchKernelGGL(hk::block_linear_kernel, dim3(nb), dim3(256), 0, s, x, weight, bias, out, n,
                     blocks, block_size);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

// CastLinear.forward on 16-bit operands: the engine's projection GEMM with
// its CastLinear epilogue. Workspace layout: kCastArrivals arrival counters,
// then split-K partial sums.
int hk_cast_linear(const uint16_t* x, const uint16_t* w, const float* bias, float* out, int M,
                   int N, int K, int fmt, void* workspace, int64_t workspace_bytes,
                   void* stream) {
  constexpr int64_t kCastArrivals = 1 << 16;
  HK_REQUIRE(x && w && out, "hk_cast_linear: null operand");
  HK_REQUIRE(M >= 0 && N > 0 && K > 0 && K % 64 == 0,
             "hk_cast_linear: bad shape M=%d N=%d K=%d (K a multiple of 64)", M, N, K);
  HK_REQUIRE(fmt == hk::kLpBF16 || fmt == hk::kLpF16, "hk_cast_linear: format %d", fmt);
  HK_REQUIRE(hk::aligned16(x) && hk::aligned16(w), "hk_cast_linear: operands must be 16-byte aligned");
  HK_REQUIRE(workspace == nullptr || workspace_bytes >= kCastArrivals * 4,
             "hk_cast_linear: a workspace needs at least %lld bytes", (long long)kCastArrivals * 4);
  if (M == 0) return HK_OK;
  hk::GemmArgs g;
  g.type = fmt == hk::kLpF16 ? hk::GemmType::kF16 : hk::GemmType::kBF16;
  g.A = x;
  g.lda = K;
  g.W = w;
  g.ldw = K;
  g.M = M;
  g.N = N;
  g.K = K;
  g.ep.bias = bias;
  g.ep.round_lp = true;
  g.ep.lp_fmt = fmt;
  g.ep.out = out;
  g.ep.ldo = N;
  hk::GemmWorkspace ws;
  if (workspace != nullptr) {
    ws.arrivals = static_cast<int*>(workspace);
    ws.arrival_elems = kCastArrivals;
    ws.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCastArrivals * 4);
    ws.partial_elems = (workspace_bytes - kCastArrivals * 4) / 4;
  }
  return hk::gemm(g, ws, (hipStream_t)stream);
}

int hk_pack_cast_weight(const uint16_t* w, uint16_t* packed, int N, int K, void* stream) {
  return hk::pack_lp_weight(w, packed, N, K, (hipStream_t)stream);
}

int hk_cast_linear_packed(const uint16_t* x, const uint16_t* w_packed, const float* bias,
                          float* out, int M, int N, int K, int fmt, int min_work_groups,
                          void* workspace, int64_t workspace_bytes, void* stream) {
  constexpr int64_t kCastArrivals = 1 << 16;
  HK_REQUIRE(x && w_packed && out, "hk_cast_linear_packed: null operand");
  HK_REQUIRE(M >= 0 && hk::packable(N, K),
             "hk_cast_linear_packed: bad shape M=%d N=%d K=%d (N a multiple of 32, K of 64)", M,
             N, K);
  HK_REQUIRE(fmt == hk::kLpBF16 || fmt == hk::kLpF16, "hk_cast_linear_packed: format %d", fmt);
  HK_REQUIRE(hk::aligned16(x) && hk::aligned16(w_packed),
             "hk_cast_linear_packed: operands must be 16-byte aligned");
  HK_REQUIRE(min_work_groups >= 0, "hk_cast_linear_packed: min_work_groups=%d", min_work_groups);
  HK_REQUIRE(workspace == nullptr || workspace_bytes >= kCastArrivals * 4,
             "hk_cast_linear_packed: a workspace needs at least %lld bytes",
             (long long)kCastArrivals * 4);
  if (M == 0) return HK_OK;
  hk::GemmArgs g;
  g.type = fmt == hk::kLpF16 ? hk::GemmType::kF16 : hk::GemmType::kBF16;
  g.A = x;
  g.lda = K;
  g.W = w_packed;
  g.w_packed = true;
  g.min_tiles = min_work_groups;
  g.M = M;
  g.N = N;
  g.K = K;
  g.ep.bias = bias;
  g.ep.round_lp = true;
  g.ep.lp_fmt = fmt;
  g.ep.out = out;
  g.ep.ldo = N;
  hk::GemmWorkspace ws;
  if (workspace != nullptr) {
    ws.arrivals = static_cast<int*>(workspace);
    ws.arrival_elems = kCastArrivals;
    ws.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCastArrivals * 4);
    ws.partial_elems = (workspace_bytes - kCastArrivals * 4) / 4;
  }
  return hk::gemm(g, ws, (hipStream_t)stream);
}

int hk_rglru_step(float* h, const float* x, const float* gate_i, const float* gate_r,
                  const float* a, float c, const uint8_t* mask, float* out, int batch, int width,
                  void* stream) {
  HK_REQUIRE(batch >= 0 && width > 0, "hk_rglru_step: bad shape B=%d H=%d", batch, width);
  HK_REQUIRE(h && x && gate_i && gate_r && a, "hk_rglru_step: null operand");
  const int64_t n = (int64_t)batch * width;
  if (n == 0) return HK_OK;
  unsigned blocks;
  const int st = hk::elementwise_grid(n, &blocks);
  if (st != HK_OK) return st;
  hipLaunchKernelGGL(hk::rglru_step_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, h, x,
                     gate_i, gate_r, a, c, mask, out, n, width);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int hk_slstm_step(float* c_state, float* n_state, float* m_state, const float* i_pre,
                  const float* f_pre, const float* z_pre, const float* o_pre,
                  const uint8_t* mask, float* y, int batch, int width, void* stream) {
  HK_REQUIRE(batch >= 0 && width > 0, "hk_slstm_step: bad shape B=%d H=%d", batch, width);
  HK_REQUIRE(c_state && n_state && m_state && i_pre && f_pre && z_pre && o_pre && y,
             "hk_slstm_step: null operand");
  const int64_t n = (int64_t)batch * width;
  if (n == 0) return HK_OK;
  unsigned blocks;
  const int st = hk::elementwise_grid(n, &blocks);
  if (st != HK_OK) return st;
  hipLaunchKernelGGL(hk::slstm_step_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     c_state, n_state, m_state, i_pre, f_pre, z_pre, o_pre, mask, y, n, width);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

}  // extern "C"
