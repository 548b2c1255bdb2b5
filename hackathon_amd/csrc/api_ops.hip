// extern "C" entry points for the reference's fused state-step API
// (model/kernels.py:346-401): state updated in place on active rows, idle rows
// untouched, idle outputs zero. Shapes follow the reference's (B, n, h, k)
// layout; every operand is a contiguous fp32 device array.
#include <cstring>
#include <string>

#include "common.h"
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

// Mamba2 step in the reference's state layout [B][heads][h][c], where c (the
// axis y contracts over) is contiguous: one work-group per (row, head), lane
// = column c (CPL columns per lane, so a state row is one coalesced wave
// access), each wave 16 rows h at a time; the 16 row sums over c come out
// of one transposed butterfly (lane 4i holds row i). Idle rows: state
// untouched, output zero.
template <int CPL>
__global__ __launch_bounds__(256) void mamba2_row_step_kernel(
    float* __restrict__ ssm, const float* __restrict__ x, const float* __restrict__ b,
    const float* __restrict__ c, const float* __restrict__ dt, const float* __restrict__ decay,
    const uint8_t* __restrict__ mask, float* __restrict__ y, int heads, int size_h, int size_c) {
  const int head = blockIdx.x;
  const int row = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
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
  for (int h0 = wave * 16; h0 < size_h; h0 += 64) {
    float sv[16][CPL], xv[16], p[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const bool hok = h0 + i < size_h;
      xv[i] = hok ? xr[h0 + i] : 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        sv[i][j] = (hok && cok[j]) ? st[(int64_t)(h0 + i) * size_c + lane + 64 * j] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        sv[i][j] = a * sv[i][j] + coef[j] * xv[i];
        acc += cw[j] * sv[i][j];
      }
      p[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        if (h0 + i < size_h && cok[j]) st[(int64_t)(h0 + i) * size_c + lane + 64 * j] = sv[i][j];
    const float sum = transposed_wave_sum<16>(p);
    if ((lane & 3) == 0 && h0 + (lane >> 2) < size_h) yo[h0 + (lane >> 2)] = sum;
  }
}

}  // namespace

}  // namespace hk

extern "C" {

const char* hk_last_error(void) { return hk::g_last_error.c_str(); }

int hk_version(void) { return 1; }

int hk_mlstm_step(float* cell, const float* q, const float* k, const float* v,
                  const float* i_gate, const float* f_gate, const uint8_t* mask, float* out,
                  int batch, int heads, int size_h, int size_k, void* stream) {
  HK_REQUIRE(batch >= 0 && heads > 0 && size_h > 0 && size_k > 0,
             "hk_mlstm_step: bad shape B=%d n=%d h=%d k=%d", batch, heads, size_h, size_k);
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

}  // extern "C"
