// Matrix-state scan: the one recurrence shared by the three large per-symbol
// states (xLSTM mLSTM cell, RetNet retention state, Mamba2 SSM state).
//
// For every step t of a symbol's run, with S a rows x cols fp32 tile per head:
//   S[r][c]  <- alpha_t * S[r][c] + (scale_t * beta_t[r]) * gamma_t[c]
//   out_t[c]  = sum_r w_t[r] * S_new[r][c]
// mLSTM  (model/kernels.py:143-151): alpha=f, scale=i, beta=k, gamma=v, w=q
// RetNet (model/kernels.py:154-160): alpha=decay[head], scale=1, beta=k_rope,
//                                    gamma=v, w=q_scaled
// Mamba2 (model/kernels.py:163-171): alpha=decay, scale=dt, beta=b, gamma=x,
//                                    w=c (rows = the contracted bc axis)
#pragma once

#include "common.h"

namespace hk {

constexpr int kLogHdr = 16;  // floats per (slot, head) log header
constexpr int kLogCapMax = 8;

struct Operand {
  const float* ptr = nullptr;  // nullptr => the value 1.0 (scale only)
  int64_t row_stride = 0;      // elements between request rows
  int64_t head_stride = 0;     // elements between heads
};

struct MatScanDesc {
  float* state = nullptr;
  int64_t slot_stride = 0, head_stride = 0, row_stride = 0, col_stride = 1;
  int rows = 0, cols = 0, heads = 0;
  // Run descriptors: run i advances slot slot_ids[i] over request rows
  // run_off[i] .. run_off[i+1]-1, in order. With `per_row` set instead, run i
  // is request row i of slot i and advances iff mask is null or mask[i] != 0
  // (the reference kernel API, model/kernels.py:28-34).
  const int* slot_ids = nullptr;
  const int* run_off = nullptr;
  bool per_row = false;
  const uint8_t* mask = nullptr;
  int n_runs = 0;
  Operand alpha, scale, beta, gamma, w;
  float* out = nullptr;
  int64_t out_row_stride = 0, out_head_stride = 0;
  // Row split: with row_parts > 1 (rows a multiple of 4 * row_parts) each
  // (run, head, column tile) is advanced by row_parts work-groups, part p
  // owning rows [p * rows / row_parts, (p + 1) * rows / row_parts); part p
  // writes its share of out_t (the sum over its rows) to out + p *
  // out_part_stride, and the caller adds the planes in part order. The
  // update of a state row never reads another row, so only the output sum
  // is split; a long run then has row_parts times the parallelism per step.
  int row_parts = 1;
  int64_t out_part_stride = 0;
  // Deferred write-back (log_cap > 0). A slot's tile is
  //   S = F * B + sum_{j < n} a_j b_j g_j^T
  // with B the tile at `state` and n <= log_cap pending rank-1 updates
  // (b_j: scale * beta of a past step, g_j: its gamma, a_j: the product of
  // the alphas applied since). A run of len steps with n + len <= log_cap
  // leaves B untouched and appends its steps to the log; any other run
  // writes the materialised tile back and empties the log. The scan only
  // reads the log header; launch_mat_log_commit (after the scan, on the same
  // stream) updates it. State reads stay one tile per run, state writes
  // drop to one tile per log_cap steps of short runs.
  float* log_hdr = nullptr;  // [slot][head][kLogHdr]: n, F, a_0 .. a_{cap-1}
  float* log_b = nullptr;    // [slot][head][cap][rows]
  float* log_g = nullptr;    // [slot][head][cap][cols]
  int log_cap = 0;
};

// The log-header update of one scan launch (deferred write-back), as a job
// that runs after the scan: job i advances the header of (run i / heads,
// head i % heads). A run that fit the log appends its steps (entry n + t
// gets the product of the run's alphas after step t; F and the older
// coefficients are scaled by the product of all of them); any other run's
// tile was written back, so its log is emptied. The scan kernel reads the
// header only, so the update waits for the whole launch; the tower's post
// kernel (which also follows the scan and does not read the header) runs
// it in extra work-groups, which saves a launch per layer.
struct LogCommit {
  const int* slot_ids = nullptr;
  const int* run_off = nullptr;
  int n_runs = 0, heads = 0;
  Operand alpha;
  float* log_hdr = nullptr;
  int log_cap = 0;  // 0: no log, no jobs
  __host__ __device__ int jobs() const { return log_cap > 0 ? n_runs * heads : 0; }
};

__device__ __forceinline__ void log_commit_one(const LogCommit& c, int i) {
  const int run = i / c.heads;
  const int head = i - run * c.heads;
  const int slot = c.slot_ids[run];
  const int r0 = c.run_off[run];
  const int len = c.run_off[run + 1] - r0;
  // The header and the run's first kLogCapMax alphas are loaded together,
  // before any store (a store ahead of a load of another array would keep
  // the loads in order, one memory round trip per step).
  float* h = c.log_hdr + ((int64_t)slot * c.heads + head) * kLogHdr;
  float hv[2 + kLogCapMax];
#pragma unroll
  for (int j = 0; j < 2 + kLogCapMax; ++j) hv[j] = h[j];
  const float* ap =
      c.alpha.ptr + (int64_t)r0 * c.alpha.row_stride + (int64_t)head * c.alpha.head_stride;
  float a[kLogCapMax];
#pragma unroll
  for (int t = 0; t < kLogCapMax; ++t) a[t] = t < len ? ap[(int64_t)t * c.alpha.row_stride] : 1.0f;
  const int n = (int)hv[0];
  if (n + len <= c.log_cap) {
    float p = 1.0f;  // product of the alphas after step t
#pragma unroll
    for (int t = kLogCapMax - 1; t >= 0; --t) {
      if (t < len) {
        h[2 + n + t] = p;
        p *= a[t];
      }
    }
#pragma unroll
    for (int j = 0; j < kLogCapMax; ++j)
      if (j < n) h[2 + j] = hv[2 + j] * p;
    h[1] = hv[1] * p;
    h[0] = (float)(n + len);
  } else {
    h[0] = 0.0f;
    h[1] = 1.0f;
  }
}

// The job of a scan described by d (no jobs without a log or runs).
LogCommit log_commit_of(const MatScanDesc& d);

int launch_mat_scan(const MatScanDesc& d, hipStream_t stream);
// The LogCommit job of a scan launch as a launch of its own; run after it.
int launch_mat_log_commit(const MatScanDesc& d, hipStream_t stream);
// Materialises slots [slot0, slot0 + n) into B and empties their logs.
int mat_log_flush(const MatScanDesc& d, int slot0, int n, hipStream_t stream);
// Empties the logs of n slots after their B was set directly: slots_dev[i]
// (a device list) or, with slots_dev null, slot0 + i.
int mat_log_clear(const MatScanDesc& d, const int* slots_dev, int slot0, int n,
                  hipStream_t stream);
// Appends counts_dev[i] zero-valued entries to the logs of slot slots_dev[i]
// (each head; at most up to the capacity): the leaf's value is unchanged.
int mat_log_fill(const MatScanDesc& d, const int* slots_dev, const int* counts_dev, int n,
                 hipStream_t stream);

}  // namespace hk
