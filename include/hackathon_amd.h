/*
 * hackathon_amd.h - C-ABI of libhackathon_amd.so, the MI355X (gfx950) engine
 * for one-step recurrent inference of the 4-tower ensemble (xLSTM, Mamba2,
 * RetNet, Hawk).
 *
 * Conventions
 * - Every entry point returns int status: 0 ok, -1 bad argument, -2 HIP
 *   failure, -3 capacity exceeded, -4 wrong engine state. Nothing throws or
 *   aborts across the ABI; hk_last_error() describes the last failure on the
 *   calling thread.
 * - Pointers are device pointers unless named *_host. Work is enqueued on the
 *   `stream` argument (a hipStream_t; NULL = the default stream) and is
 *   asynchronous unless the comment says otherwise.
 * - All tensors are dense, row-major, fp32 unless stated.
 *
 * The reference is pure Python; each entry point names the reference
 * interface (file:line in huixu11/hackathon) it replaces. The Python layer in
 * hackathon_amd/ mirrors those interfaces on top of this ABI.
 */
#ifndef HACKATHON_AMD_H
#define HACKATHON_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library version (increments on ABI changes). */
int hk_version(void);

/* Text of the last error on this thread ("" if none). */
const char* hk_last_error(void);

/* ---------------------------------------------------------------------------
 * Fused state steps, the reference's kernel API.
 * Replaces model/kernels.py:346-360 (mlstm_step), :363-376 (retnet_step),
 * :379-401 (mamba2_step), contract at model/kernels.py:28-34: the state is
 * updated in place on rows with mask[b] != 0 (mask NULL = all rows), idle
 * rows are left bit-identical, and `out` is written for every row (zeros on
 * idle rows). mask is a bool array of `batch` bytes.
 * ------------------------------------------------------------------------- */

/* cell[B,n,h,k] <- f[B,n]*cell + (i[B,n]*k[B,n,h]) (x) v[B,n,k];
 * out[B,n,k] = sum_h q[B,n,h] * cell_new[B,n,h,k]. */
int hk_mlstm_step(float* cell, const float* q, const float* k, const float* v,
                  const float* i_gate, const float* f_gate, const uint8_t* mask, float* out,
                  int batch, int heads, int size_h, int size_k, void* stream);

/* state[B,n,h,k] <- decay[n]*state + k_rope[B,n,h] (x) v[B,n,k];
 * out[B,n,k] = sum_h q_scaled[B,n,h] * state_new[B,n,h,k]. */
int hk_retnet_step(float* state, const float* k_rope, const float* v, const float* q_scaled,
                   const float* decay, const uint8_t* mask, float* out, int batch, int heads,
                   int size_h, int size_k, void* stream);

/* ssm[B,n,h,c] <- decay[B,n]*ssm + (dt[B,n]*b[B,c]) (x) x[B,n,h];
 * y[B,n,h] = sum_c c[B,c] * ssm_new[B,n,h,c]. */
int hk_mamba2_step(float* ssm, const float* x, const float* b, const float* c, const float* dt,
                   const float* decay, const uint8_t* mask, float* y, int batch, int heads,
                   int size_h, int size_c, void* stream);

/* ---------------------------------------------------------------------------
 * The other per-step operators of the towers, same contract as above (state
 * in place on active rows, idle rows bit-identical, zero outputs on idle
 * rows, mask NULL = all rows). The reference computes these with torch
 * modules and blends small state leaves with where(mask, new, old)
 * (example_model.py:907-949); on active rows the results are those modules'.
 * ------------------------------------------------------------------------- */

/* CausalConv1d.forward (model/modules.py:23-49): window = [state[b,c,0..K-2],
 * x[b,c]]; out[b,c] = bias[c] + sum_j weight[c,j] * window[j] (bias NULL =
 * none); state[b,c,:] <- window[1..K-1]. state [B,C,K-1], weight [C,K] (the
 * conv's [C,1,K]), 1 <= K <= 8. Mamba2's x/b/c convs (model/mamba2.py:84-86),
 * the xLSTM blocks' and Hawk's conv all go through this one operator. */
int hk_conv1d_step(float* state, const float* x, const float* weight, const float* bias,
                   const uint8_t* mask, float* out, int batch, int channels, int kernel_size,
                   void* stream);

/* BlockLinear.forward (model/modules.py:71-79): out[b, n*bs + k] =
 * sum_h x[b, n*bs + h] * weight[n,k,h] (+ bias[n*bs + k]); x, out
 * [B, blocks*bs], weight [blocks, bs, bs] (blocks, out, in). No state, no
 * mask. Block sizes that are multiples of 16 with 16-byte aligned operands
 * run on the fp32 matrix cores. */
int hk_block_linear(const float* x, const float* weight, const float* bias, float* out, int batch,
                    int blocks, int block_size, void* stream);

/* CastLinear.forward (example_model.py:92-95) on operands already in the
 * 16-bit format fmt (0 bf16, 1 fp16): out[m,n] = fp32 of round_fmt(sum_k
 * x[m,k] w[n,k] + bias[n]) (fp32 accumulation, the bias added in fp32, one
 * rounding to fmt, as torch's 16-bit linear rounds its result before the
 * cast back to fp32). x [M,K], w [N,K] (nn.Linear layout), K a multiple of
 * 64, both 16-byte aligned; bias [N] fp32 holding values representable in
 * fmt (CastLinear's 16-bit bias), NULL = none; out [M,N] fp32. The engine's
 * projection GEMM. workspace (NULL = none) lets it split K over several
 * work-groups: workspace_bytes >= 256 KiB, zero-filled before its first use
 * (calls leave it zeroed); calls sharing one workspace must not overlap. */
int hk_cast_linear(const uint16_t* x, const uint16_t* w, const float* bias, float* out, int M,
                   int N, int K, int fmt, void* workspace, int64_t workspace_bytes, void* stream);

/* A CastLinear weight (example_model.py:82-95, the 16-bit W of
 * convert_linears :109-148) rearranged once, at load time, into the layout
 * the engine's projection GEMM streams: w [N,K] 16-bit row-major -> packed
 * [N*K] (N a multiple of 32, K of 64, both 16-byte aligned). For each block
 * of 32 output columns and 32-deep block of K, two 1 KB matrix-core operand
 * fragments of 16 columns in lane order (element (n, k) at
 * ((((n/32)*(K/32) + k/32)*2 + (n%32)/16)*64 + n%16 + 16*((k%32)/8))*8 + k%8).
 * Stream-ordered on `stream`. */
int hk_pack_cast_weight(const uint16_t* w, uint16_t* packed, int N, int K, void* stream);

/* hk_cast_linear with the weight in the hk_pack_cast_weight layout: the
 * kernel the engine runs for every CastLinear projection (the weight slots
 * are packed at binding). Same operands, result and workspace rules as
 * hk_cast_linear; N a multiple of 32. min_work_groups selects the tile: the
 * largest that still gives that many work-groups without splitting K (0:
 * 160, for a GEMM that has the device to itself; the engine's four-stream
 * ticks use 112 above 64 rows). The result does not depend on it beyond fp32 summation
 * order. */
int hk_cast_linear_packed(const uint16_t* x, const uint16_t* w_packed, const float* bias,
                          float* out, int M, int N, int K, int fmt, int min_work_groups,
                          void* workspace, int64_t workspace_bytes, void* stream);

/* RGLRU.forward after its two BlockLinears (model/hawk.py:31-37):
 * i = sigmoid(gate_i), r = sigmoid(gate_r), a_t = a ** (c * r),
 * h <- h * a_t + sqrt(1 - a_t^2) * (i * x); out (NULL = none) = new h on
 * active rows. h, x, gate_i, gate_r, out [B,H]; a [H]; the reference's c is 8. */
int hk_rglru_step(float* h, const float* x, const float* gate_i, const float* gate_r,
                  const float* a, float c, const uint8_t* mask, float* out, int batch, int width,
                  void* stream);

/* SLSTMCell.forward (model/xlstm.py:247-274) on the gate pre-activations
 * (input BlockLinear + state BlockLinear + bias, model/xlstm.py:319-322):
 * m' = max(i, m + logsigmoid(f)), i' = exp(i - m'), f' = exp(m + logsigmoid(f)
 * - m'), c' = f' c + i' tanh(z), n' = f' n + i', y = sigmoid(o) c' / (n' +
 * 1e-6). c, n, m [B,H] updated in place (m starts at -inf, model/xlstm.py:280);
 * y [B,H]. */
int hk_slstm_step(float* c_state, float* n_state, float* m_state, const float* i_pre,
                  const float* f_pre, const float* z_pre, const float* o_pre,
                  const uint8_t* mask, float* y, int batch, int width, void* stream);

/* ---------------------------------------------------------------------------
 * Host-side tick packing (host memory, no GPU).
 * Replaces the per-round loops of process_batch (example_model.py:819-905).
 * ------------------------------------------------------------------------- */

/* Items = the batch's symbols in dict order; item i has item_len[i] requests
 * (numbered item by item) and slot item_slot[i] (-1 = no slot: answered with
 * zeros, example_model.py:826-839). Writes the runs for hk_engine_tick
 * (slot_ids[n_runs], run_off[n_runs+1]: one per slotted item with requests,
 * by non-increasing length, ties in item order), req_row[n_req] (each
 * request's row, -1 if unslotted) and resp_req[n_req] (the request answered
 * at each response position: unslotted items' requests first, then round by
 * round, items in dict order within a round, example_model.py:881-899).
 * Slots must be distinct. Arrays are host memory; slot_ids and run_off hold
 * at least n_items (+1) entries. */
int hk_pack_tick(const int* item_slot, const int* item_len, int n_items, int* slot_ids,
                 int* run_off, int* req_row, int* resp_req, int* n_runs_out, int* n_rows_out);

/* ---------------------------------------------------------------------------
 * Deterministic parameter initialisation (host, no GPU).
 * The reference fills its torch.empty parameters from a checkpoint
 * (example_model.py:296-302); the build's "random-init weights" restate the
 * ranges of check_cell_rewrite.py:187-210 with a counter-based generator, so
 * every value is a pure function of (seed, parameter name, index).
 * ------------------------------------------------------------------------- */

/* key = mix64(fnv1a64(name) ^ mix64(seed)) */
uint64_t hk_param_key(uint64_t seed, const char* name);

/* dst[i] = lo + (hi - lo) * u_i, u_i = (mix64(key + (i+1)*golden) >> 40) * 2^-24,
 * fp32 with two roundings; `threads` host threads. */
int hk_fill_uniform_host(float* dst, int64_t n, uint64_t key, float lo, float hi, int threads);

/* dst[i] = the 16-bit pattern of src[i] in CastLinear format fmt (0 bf16,
 * 1 fp16), round to nearest even, fp16 overflowing to infinity: torch's
 * .to(torch.bfloat16) / .to(torch.float16), which CastLinear applies to its
 * weights, biases, inputs and outputs (example_model.py:82-95). The engine's
 * kernels round the same way (the device's conversion instructions, every
 * non-NaN input alike). Host memory, no GPU. */
int hk_to_lp_host(const float* src, uint16_t* dst, int64_t n, int fmt);

/* ---------------------------------------------------------------------------
 * Ensemble engine: packed weights + slot-indexed HBM state store + tick.
 * Replaces MultiTowerModel(config) + init_state + forward
 * (model/inference_model.py:103-146) and the per-round step of
 * NnInferenceClient (example_model.py:400-429, :848-883).
 * ------------------------------------------------------------------------- */

/* cfg[11] = {hidden, proj, depth, heads, features, mamba_head, mamba_bc,
 *            capacity (slots), max_rows, max_runs, lp}: lp 0 = every linear
 *            fp32, 1 = bf16 CastLinear, 2 = fp16 CastLinear (the reference's
 *            LINEAR_DTYPE values fp32 / bf16 / fp16, example_model.py:150-157).
 * Allocates weights, the state store (capacity slots) and workspaces on the
 * current device. Replaces ModelConfig/MultiTowerModel construction
 * (model/inference_model.py:21-27, :103-117) and convert_linears
 * (example_model.py:109-148). */
int hk_engine_create(const int* cfg, int n_cfg, void** out_handle);

/* Frees everything the engine owns (synchronises the device first). */
int hk_engine_destroy(void* handle);

/* Number of fp32 values weight slot (tower, layer, slot) expects; tower -1 /
 * layer -1 addresses the shared output_proj, layer -1 the tower's input
 * projections. */
int hk_engine_param_numel(void* handle, int tower, int layer, int slot, int64_t* numel);

/* Synchronous bind of one packed weight slot from host fp32 values; converted
 * to the engine's 16-bit format (bf16 or fp16, round to nearest even) on the
 * device for CastLinear weights, biases rounded through it
 * (example_model.py:82-90). Replaces load_state_dict + convert_linears
 * (example_model.py:301-331). */
int hk_engine_load_param(void* handle, int tower, int layer, int slot, const float* host,
                         int64_t numel);

/* hk_engine_load_param without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under graph capture, serving loops that swap weights in place, harnesses
 * that forbid hipMalloc). CastLinear weights are staged through a 16 MiB
 * array that the library holds in every GPU's memory for the life of the
 * process, 4 Mi values at a time, so a slot of any size binds; results are
 * bit-identical to hk_engine_load_param's. Synchronous. The engine's device
 * must be current. Calls on one GPU share its array; a lock per GPU makes
 * calls from several threads of the process take turns with it. */
int hk_engine_load_param_noalloc(void* handle, int tower, int layer, int slot, const float* host,
                                 int64_t numel);

/* Elements per slot of state leaf `leaf` of tower `tower`. */
int hk_engine_state_numel(void* handle, int tower, int leaf, int64_t* per_slot);

/* Stream-ordered copy of leaf `leaf` of block `layer` for slots
 * [slot0, slot0+nslots) to (to_engine=0) or from (to_engine=1) the device
 * buffer `buf`. Used to export/import state in the reference's
 * init_state layout (model/inference_model.py:145-146). */
int hk_engine_state_copy(void* handle, int tower, int layer, int leaf, int slot0, int nslots,
                         void* buf, int to_engine, void* stream);

/* Resets slots to init_state values (zeros; sLSTM running max -inf,
 * model/xlstm.py:375); n < 0 resets every slot. */
int hk_engine_reset_slots(void* handle, const int* slots_host, int n, void* stream);

/* Appends counts_host[i] zero-valued entries to every pending-update log
 * (matrix-state write-back log, each layer and head) of slot slots_host[i],
 * up to the log capacity (8): the state the slots stand for is unchanged,
 * while later ticks read and write the logs as they do in a long-running
 * store. Measurement support with no reference counterpart (the reference
 * writes every state back each round): it starts a benchmark window at the
 * log occupancy a long run reaches. Synchronous. */
int hk_engine_log_fill(void* handle, const int* slots_host, const int* counts_host, int n,
                       void* stream);

/* One tick: n_runs runs, run i = slot slot_ids_host[i] advanced over request
 * rows run_off_host[i] .. run_off_host[i+1]-1 in order; runs sorted by
 * non-increasing length, slots distinct. features_dev [n_rows, features]
 * fp32, preds_dev [n_rows, 4] (one column per tower). Equivalent to the
 * reference's rounds (example_model.py:885-899), each a masked forward +
 * _blend_state (example_model.py:400-429, :907-949). Returns -3 when the
 * tick exceeds max_rows / max_runs. The side streams' launches are enqueued
 * by three engine-owned host threads (started on the first tick) while the
 * calling thread enqueues its stream's; the call returns once all are
 * enqueued. Not reentrant: one calling thread per engine at a time. */
int hk_engine_tick(void* handle, const int* slot_ids_host, const int* run_off_host, int n_runs,
                   const float* features_dev, float* preds_dev, void* stream);

/* hipGraph replay of small ticks. Replaces the reference's captured step
 * (_capture_step / _replay_graph, example_model.py:444-492), which records
 * one full-capacity round once and replays it for every round. Here ticks of
 * at most max_rows rows are captured once per tick shape (the run lengths;
 * descriptors, features and predictions go through fixed device buffers) and
 * replayed from a cache of at most max_graphs shapes, least recently used
 * evicted; hk_engine_tick then enqueues one copy in, one graph launch and
 * one copy out. Results are bit-identical to the eager tick's. max_rows 0
 * (the default) enqueues every tick's kernels eagerly and frees the cache.
 * Not used while hk_engine_profile records. The graph launch replays its
 * nodes from the calling thread, so one tick at a time a replayed tick ends
 * later than an eager one (whose side streams are enqueued by the engine's
 * threads); back to back they run alike. */
int hk_engine_graphs(void* handle, int max_rows, int max_graphs);

/* Shapes cached, graphs captured and ticks replayed so far. No reference
 * counterpart (test and measurement support). */
int hk_engine_graph_info(void* handle, int64_t* cached, int64_t* captures, int64_t* replays);

/* Waits for the work enqueued on `stream` (a tick's stream: every tick joins
 * its side streams back into it, so this covers whole ticks; other work on
 * the device is not waited for); returns -2 if a persistent kernel's step
 * barrier timed out in an earlier tick (its results are then invalid), else 0.
 * No reference counterpart: the reference has no in-kernel barriers; its
 * per-round host read-back (example_model.py:880) is the wait this replaces. */
int hk_engine_check(void* handle, void* stream);

/* Measurement hook (no reference counterpart; the reference times with CUDA
 * events and torch.profiler, profile_step.py:337-397): with bit k of `kinds`
 * set, every launch of kind k (0 mLSTM scan, 1 Mamba2 scan, 2 RetNet scan,
 * 3 sLSTM recurrence, 4 projection GEMM) is bracketed by HIP events on its
 * stream; 0 stops. Clears earlier records. */
int hk_engine_profile(void* handle, int kinds);

/* Waits for the recorded launches of `kind`, returns their count and summed
 * duration in ms, and clears the records. */
int hk_engine_profile_read(void* handle, int kind, int* count, double* total_ms);

#ifdef __cplusplus
}
#endif

#endif /* HACKATHON_AMD_H */
