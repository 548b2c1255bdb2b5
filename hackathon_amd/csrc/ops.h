// Row-wise and per-run kernels of the ensemble step (launchers).
//
// Row kernels take request rows r in [0, n). Run kernels take run
// descriptors: run i advances slot slot_ids[i] over rows run_off[i] ..
// run_off[i+1]-1 in order; runs are sorted by non-increasing length.
#pragma once

#include "common.h"
#include "scan_mat.h"

namespace hk {

struct Runs {
  const int* slot_ids = nullptr;  // device [n_runs]
  const int* run_off = nullptr;   // device [n_runs + 1]
  int n_runs = 0;
  int n_rows = 0;
  int max_len = 0;                // steps of the longest run (host)
  const int* row_pos = nullptr;   // device [n_rows]: position of each row in its run
  const int* row_slot = nullptr;  // device [n_rows]: slot of each row's run
};

// A width-4 causal conv (model/modules.py:23-49) computed by the kernel
// that consumes it: row r at position p of its run reads the inputs of
// positions p-3 .. p, those before the run from the slot's conv state
// (3 rows of `channels`, oldest first); out = silu(conv).
struct ConvIn {
  const float* state = nullptr;  // [slot][3][channels]
  int64_t slot_stride = 0;
  const float* w = nullptr;       // [4][channels] (tap 0 multiplies the oldest input)
  const float* b = nullptr;       // [channels]
  const int* row_pos = nullptr;
  const int* row_slot = nullptr;
  float* out = nullptr;           // [n_rows][channels], for later readers
};

// The conv state a run leaves (its last 3 inputs, behind the old state's
// newest ones when the run is shorter than 3), written by a kernel that runs
// after every reader of the old state: the last row of each run writes it.
struct ConvCommit {
  float* state = nullptr;  // null: nothing to write
  int64_t slot_stride = 0;
  const int* row_pos = nullptr;
  const int* row_slot = nullptr;
  const float* x = nullptr;  // the conv's inputs [n_rows][ldx]
  int64_t ldx = 0;
};

// ---- row kernels (rowops.hip) ---------------------------------------------

// out = x * rsqrt(mean(x^2) + eps) * w (model/inference_model.py:58,60;
// model/mamba2.py:45). out_lp (16-bit copy in format lp_fmt, LpFmt) optional.
int rmsnorm_rows(const float* x, int64_t ldx, const float* w, float eps, int n_rows, int width,
                 float* out, int64_t ldo, uint16_t* out_lp, int lp_fmt, int64_t ldl, hipStream_t s);

// Features [n, f] -> zero-padded GEMM operand [n, kpad] (fp32 and/or 16-bit).
int stage_features(const float* feat, int n_rows, int f, int kpad, float* out, uint16_t* out_lp, int lp_fmt,
                   hipStream_t s);

// Mamba2 tail before out_proj (model/mamba2.py:158-164):
// y = (ssm_out + d[head] * x) * silu(z); RMSNorm(eps 1e-5) * w. ssm_out is
// the sum of n_parts planes part_stride floats apart (split-row scan).
int mamba2_post(const float* ssm_out, int n_parts, int64_t part_stride, const float* x,
                int64_t ldx, const float* z, int64_t ldz, const float* d, const float* w,
                int n_rows, int inner, int head_size, float* out, uint16_t* out_lp, int lp_fmt,
                const LogCommit& lc, hipStream_t s);

// The RetNet position bookkeeping a tick leaves per (slot, head)
// (model/retnet.py:264-269): offsets += run length, and the scale advanced
// s' = s*gamma + 1 once per step; one job per (run, head), run after every
// reader of the old values.
struct RetnetAdvance {
  const int* slot_ids = nullptr;
  const int* run_off = nullptr;
  int n_runs = 0, heads = 0;
  const float* decay = nullptr;  // [heads]
  int* offsets = nullptr;        // [slot]; null: no jobs
  float* scales = nullptr;       // [slot][heads]
  __host__ __device__ int jobs() const { return offsets ? n_runs * heads : 0; }
};

// Job i of a RetnetAdvance: (run i / heads, head i % heads). The scale steps
// through the run with the expression retnet_prep steps it with per row.
__device__ __forceinline__ void retnet_advance_one(const RetnetAdvance& a, int i) {
  const int run = i / a.heads;
  const int head = i - run * a.heads;
  const int slot = a.slot_ids[run];
  const int len = a.run_off[run + 1] - a.run_off[run];
  float sc = a.scales[(int64_t)slot * a.heads + head];
  const float gam = a.decay[head];
  for (int t = 0; t < len; ++t) sc = sc * gam + 1.0f;
  a.scales[(int64_t)slot * a.heads + head] = sc;
  if (head == 0) a.offsets[slot] += len;
}

// RetNet tail before out_proj (model/retnet.py:168-169): per-head RMSNorm
// (eps 1e-6, no affine), times silu(g). o is the sum of n_parts planes.
// Extra work: the scan's log-header update (lc) and the tick's position
// bookkeeping (adv).
int retnet_post(const float* o, int n_parts, int64_t part_stride, const float* g, int64_t ldg,
                int n_rows, int hidden, int head_size, float* out, uint16_t* out_lp, int lp_fmt,
                const LogCommit& lc, const RetnetAdvance& adv, hipStream_t s);

// sLSTM block tail + mLSTM block norm (model/xlstm.py:422-424, :308):
// x1 = GroupNorm(groups)(y) + skip; xn = LayerNorm(x1) * w_ln.
int slstm_post(const float* y, const float* skip, const float* gn_w, const float* gn_b,
               int groups, const float* ln_w, int n_rows, int hidden, float* x1, float* xn,
               uint16_t* xn_lp, int lp_fmt, hipStream_t s);

// Fused row pairs of the xLSTM block (model/inference_model.py:63-68 around
// model/xlstm.py:355-367): a = RMSNorm(x) * w_rms, xn = LayerNorm(a) * w_ln;
// and x = LayerNorm(y) * w_ln + x, a = RMSNorm(x) * w_rms.
int rms_ln_rows(const float* x, const float* w_rms, float eps, const float* w_ln, int n_rows,
                int width, float* a, uint16_t* a_lp, int lp_fmt, float* xn, hipStream_t s);
int ln_res_rms_rows(const float* y, const float* w_ln, float* x, const float* w_rms, float eps,
                    int n_rows, int width, float* a, uint16_t* a_lp, int lp_fmt, hipStream_t s);

// out = LayerNorm(x) * w (+ residual) (no bias; eps 1e-5).
int layernorm_rows(const float* x, const float* w, const float* residual, int n_rows, int width,
                   float* out, uint16_t* out_lp, int lp_fmt, hipStream_t s);

// mLSTM cell/block tail (model/xlstm.py:236-241, :321-322):
// out = GroupNorm(num / den) ; h = (out + skip * x_conv) * silu(x_gate).
// num is the sum of n_parts planes part_stride floats apart.
// Extra work: the scan's log-header update (lc) and the conv state of the
// block's conv (cc, over `inner` channels).
int mlstm_post(const float* num, int n_parts, int64_t part_stride, const float* den, int den_ld,
               const float* gn_w, const float* gn_b, const float* skip_w, const float* x_conv,
               const float* x_gate, int64_t ld_gate, int n_rows, int inner, int heads,
               float* out, uint16_t* out_lp, int lp_fmt, const LogCommit& lc,
               const ConvCommit& cc, hipStream_t s);

// preds[r, col] = x[r] . w + b (shared output_proj, model/inference_model.py:142).
int output_proj(const float* x, const float* w, const float* b, int n_rows, int hidden,
                float* preds, int pred_ld, int col, hipStream_t s);

// mLSTM q/k/v BlockLinear (model/xlstm.py:191-193, :220-222), blk x blk blocks:
// qkv[:, 0:I] = q, [:, I:2I] = k, [:, 2I:3I] = v; ks = k / k_div.
int mlstm_qkv(const float* x_conv, const float* x_m, int64_t ld_xm, const float* wq,
              const float* wk, const float* wv, int n_rows, int inner, int blk, float k_div,
              float* qkv, float* ks, hipStream_t s);

// mlstm_qkv with blk 4 fused with the block's conv (x_conv = conv over the
// first `inner` columns of x_m, written to conv.out) and the cell's input /
// forget gate projections (model/xlstm.py:29-30, :52-54): w_if
// [n_out][3*inner] (igate rows, then fgate rows), b_if [n_out]. The
// pre-activations land as `segs` partial planes if_part [segs][n_rows][n_out],
// to be added in plane order (plane 0 holds the bias).
bool mlstm_qkv_if_supported(int inner, int n_out, int segs);
int mlstm_qkv_if(const ConvIn& conv, const float* x_m, int64_t ld_xm, const float* wq,
                 const float* wk, const float* wv, int n_rows, int inner, float k_div,
                 const float* w_if, const float* b_if, int n_out, float* qkv, float* ks,
                 float* if_part, int segs, hipStream_t s);

// 16-bit copy (LpFmt lp_fmt) of an fp32 matrix (weights at bind time).
int to_lp(const float* src, uint16_t* dst, int64_t n, int lp_fmt, hipStream_t s);
// v[i] = v[i] rounded through the 16-bit format lp_fmt, in place.
int round_lp_inplace(float* v, int64_t n, int lp_fmt, hipStream_t s);
// fill with a constant
int fill_f32(float* dst, int64_t n, float v, hipStream_t s);

// ---- run kernels (scans.hip) ----------------------------------------------

// Depthwise causal conv over each run (model/modules.py:45-49), kernel 4:
// window = [state(3 oldest..newest), x]; out = bias + sum_j w[j] * window[j];
// state <- last three inputs. state is [slot][3][C], w is [4][C] (tap-major).
int conv_scan(const Runs& r, const float* in, int64_t ld_in, int channels, float* state,
              int64_t slot_stride, const float* w, const float* bias, int act_silu, float* out,
              int64_t ldo, hipStream_t s);

// RetNet rotary + scale recurrence (model/retnet.py:239-269, :340) for
// each row, from the offsets and scales the slot held before the tick (the
// bookkeeping that advances them is RetnetAdvance). Needs r.row_pos and
// r.row_slot.
int retnet_prep(const Runs& r, const float* qkvg, int64_t ld, int hidden, int heads,
                float k_scaling, const float* angle, const float* decay, int* offsets,
                float* scales, float* k_rope, float* q_scaled, hipStream_t s);

// Hawk RG-LRU over each run, times gelu(gate) (model/hawk.py:31-37, :77, :83).
int rglru_scan(const Runs& r, const float* x, const float* gi, const float* gr, int64_t ldg,
               const float* gate, int64_t ld_gate, const float* a, float c_exp, int hidden,
               float* h_state, float* out, uint16_t* out_lp, int lp_fmt, hipStream_t s);

// One sLSTM step for the first n_active runs (model/xlstm.py:414-421, :355-369).
int slstm_round(const Runs& r, int step, int n_active, const float* gin, int hidden, int heads,
                const float* w_state, const float* b_state, const float* h_state, float* c_state,
                float* n_state, float* m_state, float* y, hipStream_t s);
// The whole tick's sLSTM recurrence in one persistent launch (all steps);
// also writes h_state. act_dev[t] = runs active at step t. xch: [n_rows]
// [hidden] 64-bit exchange words; tag: nonzero and different from every
// earlier launch's on the same buffer; err: set to 1 if a poll timed out.
// split: the recurrent product on split-f16 matrix cores (head sizes
// 64-512; the reduced-precision modes), else on fp32 matrix cores.
bool slstm_persist_supported(int hidden, int heads);
int slstm_persist(const Runs& r, const int* act_dev, int n_rounds, const float* gin, int hidden,
                  int heads, const float* w_state, const float* b_state, float* h_state,
                  float* c_state, float* n_state, float* m_state, float* y,
                  unsigned long long* xch, unsigned int tag, int* err, uint64_t* trace,
                  bool split, hipStream_t s);
// Whether two persistent launches (each at most max_runs runs over
// max_rounds steps) can be co-resident at once, so that two run groups'
// recurrences may overlap.
int slstm_persist_pair_fits(int hidden, int heads, int max_runs, int max_rounds, bool split,
                            bool* ok);
// After the last round: h_state[slot] = y[last row of the run].
int slstm_final(const Runs& r, const float* y, int hidden, float* h_state, hipStream_t s);

// mLSTM gate / normaliser recurrence (model/xlstm.py:61-74, :140-142). The
// gate pre-activations if_pre [rows][2*heads] (i then f) are the sum of
// n_parts planes part_stride floats apart, added in plane order.
int mlstm_gates(const Runs& r, const float* if_pre, int n_parts, int64_t part_stride, int heads,
                const float* qkv, int inner, const float* ks, float* n_state, float* m_state,
                float* ig, float* fg, float* den, hipStream_t s);

}  // namespace hk
