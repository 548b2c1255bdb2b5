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
  // The reference layout keeps c (the contracted axis) contiguous: tile rows
  // are c with stride 1, tile columns are h with stride size_c.
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
