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

#ifdef __cplusplus
}
#endif

#endif /* HACKATHON_AMD_H */
