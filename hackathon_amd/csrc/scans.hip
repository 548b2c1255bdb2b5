// Per-run scan kernels: each work-group walks one symbol's run of requests
// in order, carrying that symbol's small recurrent state in registers, so the
// state is read once and written once per tick.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "ops.h"

namespace hk {
namespace {

constexpr int kConvChunk = 16;
// grid (runs, ceil(C/256)); thread per channel.
__global__ __launch_bounds__(256) void conv_scan_kernel(
    const int* __restrict__ slot_ids, const int* __restrict__ run_off, const float* __restrict__ in,
    int64_t ld_in, int channels, float* __restrict__ state, int64_t slot_stride,
    const float* __restrict__ w, const float* __restrict__ bias, int act_silu,
    float* __restrict__ out, int64_t ldo) {
  const int run = blockIdx.x;
  const int c = blockIdx.y * 256 + threadIdx.x;
  if (c >= channels) return;
  const int slot = slot_ids[run];
  const int r0 = run_off[run];
  const int r1 = run_off[run + 1];
  if (r1 <= r0) return;
  float* st = state + (int64_t)slot * slot_stride;
  float s0 = st[c], s1 = st[channels + c], s2 = st[2 * channels + c];
  const float w0 = w[c], w1 = w[channels + c], w2 = w[2 * channels + c], w3 = w[3 * channels + c];
  const float b = bias[c];
  // The run's inputs stream through two register buffers of kConvChunk
  // rows: the next chunk's loads are in flight while this one is computed
  // (rows past the run read its last row, unused).
  float xa[kConvChunk], xb[kConvChunk];
  auto load = [&](float (&x)[kConvChunk], int rb) {
#pragma unroll
    for (int k = 0; k < kConvChunk; ++k) x[k] = in[(int64_t)min(rb + k, r1 - 1) * ld_in + c];
  };
  auto step = [&](const float (&x)[kConvChunk], int rb) {
#pragma unroll
    for (int k = 0; k < kConvChunk; ++k) {
      if (rb + k < r1) {
        float v = b + w0 * s0;
        v += w1 * s1;
        v += w2 * s2;
        v += w3 * x[k];
        out[(int64_t)(rb + k) * ldo + c] = act_silu ? silu(v) : v;
        s0 = s1;
        s1 = s2;
        s2 = x[k];
      }
    }
  };
  load(xa, r0);
  for (int rb = r0; rb < r1; rb += 2 * kConvChunk) {
    // (most runs fit one chunk: no prefetch of chunks past the run)
    if (rb + kConvChunk < r1) load(xb, rb + kConvChunk);
    step(xa, rb);
    if (rb + kConvChunk >= r1) break;
    if (rb + 2 * kConvChunk < r1) load(xa, rb + 2 * kConvChunk);
    step(xb, rb + kConvChunk);
  }
  st[c] = s0;
  st[channels + c] = s1;
  st[2 * channels + c] = s2;
}

// grid (rows, ceil(hidden/256)); thread per (row, channel): every row is
// independent once its run is known (binary search over the run offsets,
// uniform per work-group). The scale recurrence s' = s*gamma + 1 is stepped
// from the slot's stored scale through the row's position in its run, the
// same operations in the same order as a sequential pass.
__global__ __launch_bounds__(256) void retnet_prep_kernel(
    const int* __restrict__ row_pos, const int* __restrict__ row_slot,
    const float* __restrict__ qkvg, int64_t ld, int hidden, int head_size, float k_scaling,
    const float* __restrict__ angle, const float* __restrict__ decay,
    const int* __restrict__ offsets, const float* __restrict__ scales, float* __restrict__ k_rope,
    float* __restrict__ q_scaled) {
  const int r = blockIdx.x;
  const int c = blockIdx.y * 256 + threadIdx.x;
  if (c >= hidden) return;
  const int heads = hidden / head_size;
  const int head = c / head_size;
  const int j = c % head_size;
  const int partner = (j & 1) ? c - 1 : c + 1;
  const float sign = (j & 1) ? 1.0f : -1.0f;  // rotate_every_two: (-x1, x0)
  const int slot = row_slot[r];
  const int t = row_pos[r];
  const float gam = decay[head];
  float sc = scales[(int64_t)slot * heads + head];
  for (int i = 0; i <= t; ++i) sc = sc * gam + 1.0f;
  const float* row = qkvg + (int64_t)r * ld;
  const float theta = (float)(offsets[slot] + t) * angle[j];
  const float sn = sinf(theta);
  const float cs = cosf(theta);
  const float q = row[c];
  const float qp = sign * row[partner];
  const float k = row[hidden + c] * k_scaling;
  const float kp = sign * (row[hidden + partner] * k_scaling);
  const float qr = q * cs + qp * sn;
  const float kr = k * cs + kp * sn;
  const float sf = 1.0f / sqrtf(sc);
  k_rope[(int64_t)r * hidden + c] = kr;
  q_scaled[(int64_t)r * hidden + c] = qr * sf;
}


// RG-LRU over each run's rows (model/hawk.py:31-37, with the output gate
// of model/hawk.py:83). grid (runs, ceil(hidden/64)); 256 threads = 64
// channels x 4 row lanes. Only h' = h*a_t + u_t is sequential over a run's
// rows; the gates (a_t = a^(c r_t), u_t = sqrt(1 - a_t^2) i_t x_t and the
// output gate gelu(g_t)), the bulk of the arithmetic, are independent per
// row. A run's rows go through in chunks of kRgChunk: each row lane forms
// the gates of every fourth row of the chunk into LDS (the next chunk's
// inputs already loading into registers), then row lane 0 runs the
// recurrence over the chunk and writes the outputs, so a long run's serial
// chain holds two multiplies and an add per row.
constexpr int kRgChunk = 16;
constexpr int kRgLanes = 4;                  // row lanes per channel
constexpr int kRgPer = kRgChunk / kRgLanes;  // rows per lane per chunk
__global__ __launch_bounds__(256) void rglru_scan_kernel(
    const int* __restrict__ slot_ids, const int* __restrict__ run_off, const float* __restrict__ x,
    const float* __restrict__ gi, const float* __restrict__ gr, int64_t ldg,
    const float* __restrict__ gate, int64_t ld_gate, const float* __restrict__ a, float c_exp,
    int hidden, float* __restrict__ h_state, float* __restrict__ out,
    uint16_t* __restrict__ out_lp, int lp_fmt) {
  __shared__ float s_at[2][kRgChunk][64], s_ut[2][kRgChunk][64], s_og[2][kRgChunk][64];
  const int run = blockIdx.x;
  const int cl = threadIdx.x & 63;
  const int lr = threadIdx.x >> 6;  // row lane (= wave)
  const int c = blockIdx.y * 64 + cl;
  const bool live = c < hidden;
  const int cc = live ? c : 0;      // loads of a channel past hidden read channel 0
  const int slot = slot_ids[run];
  const int r0 = run_off[run];
  const int r1 = run_off[run + 1];
  if (r1 <= r0) return;
  const float base = a[cc];
  struct Rows {
    float i[kRgPer], r[kRgPer], x[kRgPer], g[kRgPer];
  };
  // this lane's rows of the chunk at rb: rb + lr + kRgLanes*k (rows past the
  // run read its last row; their gates are never used)
  auto load = [&](Rows& v, int rb) {
#pragma unroll
    for (int k = 0; k < kRgPer; ++k) {
      if (k > 0 && rb + lr + kRgLanes * k >= r1) break;
      const int64_t ri = (int64_t)min(rb + lr + kRgLanes * k, r1 - 1);
      v.i[k] = gi[ri * ldg + cc];
      v.r[k] = gr[ri * ldg + cc];
      v.x[k] = x[ri * hidden + cc];
      v.g[k] = gate[ri * ld_gate + cc];
    }
  };
  auto gates = [&](const Rows& v, int rb, int buf) {
    // Each product and sum rounded on its own, as the reference's tensor
    // ops do (model/hawk.py:35-37): no multiply-add is fused. Rows past the
    // run are skipped (most runs are a few rows long).
#pragma clang fp contract(off)
#pragma unroll
    for (int k = 0; k < kRgPer; ++k) {
      if (rb + lr + kRgLanes * k >= r1) break;
      const float it = sigmoid(v.i[k]);
      const float rt = sigmoid(v.r[k]);
      const float at = powf(base, c_exp * rt);
      const float mult = sqrtf(1.0f - at * at);
      const int j = lr + kRgLanes * k;
      s_at[buf][j][cl] = at;
      s_ut[buf][j][cl] = mult * (it * v.x[k]);
      s_og[buf][j][cl] = gelu_erf(v.g[k]);
    }
  };
  float h = lr == 0 ? h_state[(int64_t)slot * hidden + cc] : 0.0f;
  Rows v;
  load(v, r0);
  int buf = 0;
  for (int rb = r0; rb < r1; rb += kRgChunk, buf ^= 1) {
    gates(v, rb, buf);
    if (rb + kRgChunk < r1) load(v, rb + kRgChunk);
    // the chunk's gates are in LDS; buffer buf was last read two chunks ago,
    // before the previous barrier
    lds_barrier();
    if (lr == 0 && live) {
#pragma clang fp contract(off)
      const int n = min(kRgChunk, r1 - rb);
      for (int j = 0; j < n; ++j) {
        h = (h * s_at[buf][j][cl]) + s_ut[buf][j][cl];
        const float o = s_og[buf][j][cl] * h;
        const int64_t ri = (int64_t)(rb + j);
        if (out) out[ri * hidden + c] = o;
        if (out_lp) out_lp[ri * hidden + c] = f32_to_lp_bits(o, lp_fmt);
      }
    }
  }
  if (lr == 0 && live) h_state[(int64_t)slot * hidden + c] = h;
}

// One sLSTM step. grid (heads, units/16, ceil(n_active/16)); 256 threads =
// 4 waves, wave g computes gate g (i, f, z, o) for 16 units x 16 runs:
// lane = (unit u = lane%16, k-quarter = lane/16), then a 4-lane butterfly.
constexpr int kSlRuns = 16;
constexpr int kSlUnits = 16;

__global__ __launch_bounds__(256) void slstm_round_kernel(
    const int* __restrict__ slot_ids, const int* __restrict__ run_off, int step, int n_active,
    const float* __restrict__ gin, int hidden, int hs, const float* __restrict__ w_state,
    const float* __restrict__ b_state, const float* __restrict__ h_state,
    float* __restrict__ c_state, float* __restrict__ n_state, float* __restrict__ m_state,
    float* __restrict__ y) {
  extern __shared__ __align__(16) float smem[];
  float* hp = smem;                            // [kSlRuns][hs]
  float* gsum = smem + kSlRuns * hs;           // [4][kSlRuns][kSlUnits]
  const int head = blockIdx.x;
  const int u0 = blockIdx.y * kSlUnits;
  const int rb = blockIdx.z * kSlRuns;
  const int nr = min(kSlRuns, n_active - rb);
  const int heads = hidden / hs;

  // Stage h_{t-1} of each run's head block.
  for (int i = threadIdx.x; i < kSlRuns * hs; i += 256) {
    const int rr = i / hs;
    const int k = i % hs;
    float v = 0.0f;
    if (rr < nr) {
      const int run = rb + rr;
      const int row = run_off[run] + step;
      v = step == 0 ? h_state[(int64_t)slot_ids[run] * hidden + head * hs + k]
                    : y[(int64_t)(row - 1) * hidden + head * hs + k];
    }
    hp[i] = v;
  }
  lds_barrier();

  const int g = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int u = lane & 15;
  const int kq = lane >> 4;
  const int kchunk = hs / 4;
  // W[g][head][unit][k] (BlockLinear weight (blocks, out, in)).
  const float* wrow =
      w_state + (((int64_t)g * heads + head) * hs + (u0 + u)) * hs + (int64_t)kq * kchunk;
  float acc[kSlRuns];
#pragma unroll
  for (int i = 0; i < kSlRuns; ++i) acc[i] = 0.0f;
  for (int k = 0; k < kchunk; ++k) {
    const float wv = wrow[k];
    const float* hk = hp + kq * kchunk + k;
#pragma unroll
    for (int i = 0; i < kSlRuns; ++i) acc[i] += wv * hk[i * hs];
  }
#pragma unroll
  for (int i = 0; i < kSlRuns; ++i) {
    float v = acc[i];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    acc[i] = v;
  }
  if (kq == 0) {
#pragma unroll
    for (int i = 0; i < kSlRuns; ++i) gsum[(g * kSlRuns + i) * kSlUnits + u] = acc[i];
  }
  lds_barrier();

  const int rr = threadIdx.x / kSlUnits;
  const int uu = threadIdx.x % kSlUnits;
  if (rr >= nr) return;
  const int run = rb + rr;
  const int slot = slot_ids[run];
  const int row = run_off[run] + step;
  const int col = head * hs + u0 + uu;
  const float* gr = gin + (int64_t)row * 4 * hidden;
  const float ip = gr[col] + (gsum[(0 * kSlRuns + rr) * kSlUnits + uu] + b_state[col]);
  const float fp = gr[hidden + col] + (gsum[(1 * kSlRuns + rr) * kSlUnits + uu] + b_state[hidden + col]);
  const float zp =
      gr[2 * hidden + col] + (gsum[(2 * kSlRuns + rr) * kSlUnits + uu] + b_state[2 * hidden + col]);
  const float op =
      gr[3 * hidden + col] + (gsum[(3 * kSlRuns + rr) * kSlUnits + uu] + b_state[3 * hidden + col]);
  const int64_t si = (int64_t)slot * hidden + col;
  const float m = m_state[si];
  const float lfm = m + logsigmoid(fp);
  const float mn = fmaxf(ip, lfm);
  const float og = sigmoid(op);
  const float ig = expf(ip - mn);
  const float fg = expf(lfm - mn);
  const float cn = fg * c_state[si] + ig * tanhf(zp);
  const float nn = fg * n_state[si] + ig;
  c_state[si] = cn;
  n_state[si] = nn;
  m_state[si] = mn;
  y[(int64_t)row * hidden + col] = og * cn / (nn + 1e-6f);
}

// Persistent sLSTM recurrence for a whole tick: one launch per layer instead
// of one launch per step. Work-group g (512 threads, 8 waves) owns 16 units
// of one head: 64 gate rows (unit*4 + gate) x hs inputs of the recurrent
// weights, held in VGPRs for every step as MFMA A fragments (wave =
// (16-row tile, k half)). Step t, per chunk of up to 16 active runs: stage
// h_{t-1} of the chunk's runs in LDS; G[64 rows x runs] = W . H; add the two
// k halves through LDS; then the cell update, one (run, unit) per thread.
// The product, for head sizes 64-512: split f16 on v_mfma_f32_16x16x32_f16,
// W*S and h*kHScale each as an f16 value plus its f16 remainder (22
// significant bits), G = hi.hi + (hi.lo + lo.hi) with fp32 accumulation and
// an exact power-of-two unscale: the dropped lo.lo term is below 2^-22 of
// each product, under the rounding of an fp32 dot product of this length,
// and the step costs 24 matrix instructions per wave (fp32 matrix cores
// took 64 of twice the cycles each; at 16 runs the fp32 product bound the
// step). For head size 32: v_mfma_f32_16x16x4_f32 when the chunk has more
// than kValuRuns runs, else VALU dot products over the same weights.
//
// h_t crosses work-groups (and XCDs) through an exchange buffer of 64-bit
// words (value bits | tag << 32) stored and loaded with agent-scope atomics.
// The tag is this launch's number, so a reader that sees its tag in a word
// also sees that word's value: no barrier between the head's work-groups is
// needed, and each row of the buffer is written once per launch. A reader
// polls with a bounded spin; on timeout it sets the error flag and every
// wave of every work-group leaves.
constexpr int kPersistRuns = 16;   // runs per chunk = one MFMA n-tile
constexpr int kValuRuns = 4;       // chunks up to this size use the VALU product
constexpr int kPersistThreads = 512;
// LDS a persistent work-group asks for at least, so that it has its CU to
// itself: other streams' kernels sharing those CUs slow the recurrence's
// step chain about as much as they gain (C4 tick 9.40-9.45 ms against
// 9.42-9.50 with the CUs shared, interleaved runs on two boxes).
constexpr size_t kPersistLdsFloor = 140 * 1024;
// Bounded wait: each poll re-reads a wave's words (a memory round trip of a
// microsecond or more), so this bounds a wait to well under a few seconds,
// far above a legitimate step even when other streams' kernels delay some
// work-groups' start.
constexpr int kSpinLimit = 1 << 19;

struct SlstmPersistArgs {
  const int* slot_ids;
  const int* run_off;
  const int* act;      // act[t] = runs with length > t (runs sorted by length)
  int n_rounds;
  int n_runs;
  const float* gin;    // [rows][4*hidden] input-side gate pre-activations
  int hidden;
  int heads;
  const float* w_state;  // [4][heads][hs][hs]
  const float* b_state;  // [4][hidden]
  float* h_state;
  float* c_state;
  float* n_state;
  float* m_state;
  float* y;                 // [rows][hidden]
  unsigned long long* xch;  // [rows][hidden] exchange words
  unsigned int tag;         // nonzero; differs from the tags of earlier launches
  int* err;                 // set to 1 on a poll timeout
  uint64_t* trace;          // optional [n_rounds][8] wall-clock stamps of work-group 0
};

typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef _Float16 halfx8_t __attribute__((ext_vector_type(8)));

// The split-f16 product stages h as h * kHScale (hi = f16 of it, lo = f16 of
// the remainder): every h the recurrence produces has |h| < 1 (|c| <= n),
// the scale keeps small values clear of f16 subnormals, and |h| below
// 65504 / kHScale stays finite.
constexpr float kHScale = 256.0f;

// Power of two that puts a row's largest |w| (m) in [2^13, 2^14), so that
// w*S splits into an f16 hi part and an f16 remainder with 22 significant
// bits together and no overflow (S = 2^100 for an all-zero row).
__device__ __forceinline__ float row_split_scale(float m) {
  const int ex = (int)((__float_as_uint(m) >> 23) & 0xffu);
  return ldexpf(1.0f, min(max(140 - ex, -100), 100));
}

__device__ __forceinline__ void stage_split4(_Float16* hi, _Float16* lo, float4 v) {
  const float x[4] = {v.x * kHScale, v.y * kHScale, v.z * kHScale, v.w * kHScale};
  _Float16 h[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[e] = (_Float16)x[e];
    l[e] = (_Float16)(x[e] - (float)h[e]);
  }
  typedef _Float16 halfx4_t __attribute__((ext_vector_type(4)));
  *reinterpret_cast<halfx4_t*>(hi) = halfx4_t{h[0], h[1], h[2], h[3]};
  *reinterpret_cast<halfx4_t*>(lo) = halfx4_t{l[0], l[1], l[2], l[3]};
}

// LDS ints of the run descriptors (run_off, slot_ids, act), kept even so
// that what follows stays 8-byte aligned.
__host__ __device__ __forceinline__ int persist_meta_ints(int n_runs, int n_rounds) {
  return (2 * n_runs + 1 + n_rounds + 1) & ~1;
}

__device__ __forceinline__ unsigned long long xch_word(float v, unsigned int tag) {
  return (unsigned long long)__float_as_uint(v) | ((unsigned long long)tag << 32);
}

// Waits until every word of this wave at offs[u] (u < N) carries `tag`; the
// words' values land in val[]. Returns false on timeout or a raised error
// flag (then the flag is set). All N loads of a poll are issued before the
// first wait.
template <int N>
__device__ __forceinline__ bool poll_words(const unsigned long long* base, const uint32_t* offs,
                                           unsigned int tag, int* err, float* val) {
  int spins = 0;
  for (;;) {
    unsigned long long w[N];
#pragma unroll
    for (int u = 0; u < N; ++u)
      w[u] = __hip_atomic_load(base + offs[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool ok = true;
#pragma unroll
    for (int u = 0; u < N; ++u) {
      ok = ok && (unsigned int)(w[u] >> 32) == tag;
      val[u] = __uint_as_float((unsigned int)w[u]);
    }
    if (__all(ok)) return true;
    __builtin_amdgcn_s_sleep(1);
    ++spins;
    if (spins > kSpinLimit ||
        ((spins & 255) == 0 &&
         __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)) {
      __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}

// poll_words over the first n (uniform, 1 <= n <= N) of N offsets, with the
// load count rounded up to a power of two (the extra offsets are valid).
template <int N>
__device__ __forceinline__ bool poll_first(const unsigned long long* base, const uint32_t* offs,
                                           unsigned int tag, int* err, float* val, int n) {
  if constexpr (N >= 2) {
    if (n <= N / 2) return poll_first<N / 2>(base, offs, tag, err, val, n);
  }
  return poll_words<N>(base, offs, tag, err, val);
}

template <int HS, bool SPLIT>
__global__ __launch_bounds__(kPersistThreads) void slstm_persist_kernel(SlstmPersistArgs a) {
  extern __shared__ __align__(16) float smem[];
  constexpr int hs = HS;
  constexpr int wpg = hs / 16;      // work-groups per head
  constexpr int NT = kPersistThreads;
  constexpr int PAD = hs + 8;       // LDS row stride of h (spreads runs over banks)
  constexpr int KH = hs / 2;        // k per wave
  constexpr int KG = KH / 16;       // groups of 4 MFMA k-steps per wave
  // With SPLIT, head sizes 64-512 multiply on split f16 (hi/lo) matrix
  // cores; head size 32, and every head size without SPLIT (the fp32 mode),
  // on fp32 matrix cores.
  constexpr bool kF16 = SPLIT && HS >= 64;
  constexpr int PADH = PAD;         // f16 row stride of the split h planes
  float* hbuf = smem;                               // [16][PAD] (fp32 path)
  // split-f16 path: the same bytes as two [16][PADH] planes of f16, h*kHScale
  // rounded (hi) and its remainder (lo)
  _Float16* hhi = reinterpret_cast<_Float16*>(smem);
  _Float16* hlo = hhi + kPersistRuns * PADH;
  float* gsum = hbuf + kPersistRuns * PAD;          // [16 runs][64 rows], k half 0
  float* xbuf = gsum + kPersistRuns * 64;           // [16 runs][64 rows], k half 1
  // The run descriptors, copied to LDS once: every step reads them, and a
  // global load there would put a memory latency ahead of each step's poll.
  int* l_off = reinterpret_cast<int*>(xbuf + kPersistRuns * 64);  // [n_runs + 1]
  int* l_slot = l_off + a.n_runs + 1;                             // [n_runs]
  int* l_act = l_slot + a.n_runs;                                 // [n_rounds]
  __shared__ int s_abort;
  // The recurrence is latency-bound and shares its CUs with other streams'
  // kernels: its waves take instruction-issue priority over theirs.
  __builtin_amdgcn_s_setprio(3);
  const int H = a.hidden;
  const int head = blockIdx.x / wpg;
  const int u0 = (blockIdx.x % wpg) * 16;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int mt = wave & 3;          // rows 16*mt .. +15
  const int kh = wave >> 2;         // k half
  const int fr = lane & 15;         // A row / B column (run) / C column
  const int fk = lane >> 4;         // k sub-group / C row group

  // Weights, fp32 path (head size 32): A fragments of v_mfma_f32_16x16x4f32;
  // for k-step group g and step c this lane covers k = kh*KH + 16*g + 4*fk
  // + c of row 16*mt + fr (A and B use the same map).
  // Split-f16 path (head sizes 64-512): A fragments of
  // v_mfma_f32_16x16x32_f16 for k-step s: k = kh*KH + 32*s + 8*fk .. +7 of
  // row 16*mt + fr, each weight w*S (S a power of two per row, |w*S| <
  // 2^14) held as hi = f16(w*S) and lo = f16(w*S - hi).
  constexpr int KS = kF16 ? KH / 32 : 1;
  float w[kF16 ? 1 : 4 * KG];
  halfx8_t whi[KS], wlo[KS];
  float inv_row[4] = {1.0f, 1.0f, 1.0f, 1.0f};  // 1/(S_row * kHScale), output rows 4*fk + e
  {
    const int row = 16 * mt + fr;
    const int unit = row >> 2, gate = row & 3;
    const float* rsrc = a.w_state + (((int64_t)gate * a.heads + head) * hs + (u0 + unit)) * hs;
    if constexpr (!kF16) {
      const float* src = rsrc + kh * KH + 4 * fk;
#pragma unroll
      for (int g = 0; g < KG; ++g) {
        const float4 v = *reinterpret_cast<const float4*>(src + 16 * g);
        w[4 * g + 0] = v.x;
        w[4 * g + 1] = v.y;
        w[4 * g + 2] = v.z;
        w[4 * g + 3] = v.w;
      }
    } else {
      const float* src = rsrc + kh * KH + 8 * fk;
      float wf[KS][8];
      float m = 0.0f;
#pragma unroll
      for (int q = 0; q < KS; ++q) {
        const float4 v0 = *reinterpret_cast<const float4*>(src + 32 * q);
        const float4 v1 = *reinterpret_cast<const float4*>(src + 32 * q + 4);
        wf[q][0] = v0.x; wf[q][1] = v0.y; wf[q][2] = v0.z; wf[q][3] = v0.w;
        wf[q][4] = v1.x; wf[q][5] = v1.y; wf[q][6] = v1.z; wf[q][7] = v1.w;
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(wf[q][e]));
      }
      // the row's largest |w|: over the four k groups, then the two k halves
      m = fmaxf(m, __shfl_xor(m, 16, 64));
      m = fmaxf(m, __shfl_xor(m, 32, 64));
      float* rmax = gsum;  // [2][64], before the step loop uses gsum
      if (fk == 0) rmax[kh * 64 + row] = m;
      lds_barrier();
      const float rs = row_split_scale(fmaxf(rmax[row], rmax[64 + row]));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int orow = 16 * mt + 4 * fk + e;
        inv_row[e] = 1.0f / (row_split_scale(fmaxf(rmax[orow], rmax[64 + orow])) * kHScale);
      }
      lds_barrier();
#pragma unroll
      for (int q = 0; q < KS; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = wf[q][e] * rs;
          const _Float16 h = (_Float16)v;
          whi[q][e] = h;
          wlo[q][e] = (_Float16)(v - (float)h);
        }
    }
  }
  // Cell-update role (threads 0..255): unit uu, run jr of each chunk.
  const int uu = tid & 15;
  const int jr = tid >> 4;
  const int ccol = head * hs + u0 + uu;
  float bi = 0.f, bf = 0.f, bz = 0.f, bo = 0.f;
  if (tid < 256) {
    bi = a.b_state[ccol];
    bf = a.b_state[H + ccol];
    bz = a.b_state[2 * H + ccol];
    bo = a.b_state[3 * H + ccol];
  }
  if (tid == 0) s_abort = 0;
  for (int i = tid; i <= a.n_runs; i += NT) l_off[i] = a.run_off[i];
  for (int i = tid; i < a.n_runs; i += NT) l_slot[i] = a.slot_ids[i];
  for (int i = tid; i < a.n_rounds; i += NT) l_act[i] = a.act[i];
  lds_barrier();

  // Optional phase stamps of work-group 0 (thread 0), kept in LDS during the
  // recurrence so that taking them adds no memory waits, stored at the end.
  const bool tr = a.trace != nullptr && blockIdx.x == 0 && tid == 0;
  uint64_t* ltr = reinterpret_cast<uint64_t*>(l_off + persist_meta_ints(a.n_runs, a.n_rounds));
  for (int t = 0; t < a.n_rounds; ++t) {
    const int na = l_act[t];
    if (tr) ltr[t * 8 + 0] = __builtin_amdgcn_s_memrealtime();
    for (int c0 = 0; c0 < na; c0 += kPersistRuns) {
      const int nj = min(kPersistRuns, na - c0);
      // Operands of this thread's cell update, fetched before the h staging
      // so their latency overlaps it.
      const bool cell = tid < 256 && jr < nj;
      float pi = 0.f, pf = 0.f, pz = 0.f, po = 0.f, pc = 0.f, pn = 0.f, pm = 0.f;
      int64_t psi = 0, prow = 0;
      if (cell) {
        const int run = c0 + jr;
        const int row = l_off[run] + t;
        const float* gr = a.gin + (int64_t)row * 4 * H;
        psi = (int64_t)l_slot[run] * H + ccol;
        prow = row;
        pi = gr[ccol];
        pf = gr[H + ccol];
        pz = gr[2 * H + ccol];
        po = gr[3 * H + ccol];
        pc = a.c_state[psi];
        pn = a.n_state[psi];
        pm = a.m_state[psi];
      }
      // Stage h_{t-1} of the chunk's runs into hbuf[j][k]. Loads are
      // unconditional (index clamped to a valid element) so the staging
      // registers never go to scratch; only the LDS stores are predicated.
      if (t == 0) {
        // from the state store (written before this launch)
        constexpr int vph = hs / 4;
        constexpr int kV = (kPersistRuns * vph + NT - 1) / NT;
        const int nvec = nj * vph;
        float4 v[kV];
#pragma unroll
        for (int u = 0; u < kV; ++u) {
          const int i = min(u * NT + tid, nvec - 1);
          const int j = i / vph;
          v[u] = reinterpret_cast<const float4*>(a.h_state + (int64_t)l_slot[c0 + j] * H +
                                                 head * hs)[i - j * vph];
        }
        if (tr && c0 == 0) ltr[t * 8 + 1] = __builtin_amdgcn_s_memrealtime();
#pragma unroll
        for (int u = 0; u < kV; ++u) {
          const int i = u * NT + tid;
          if (i < nvec) {
            const int j = i / vph;
            if constexpr (kF16) {
              stage_split4(hhi + j * PADH + 4 * (i - j * vph), hlo + j * PADH + 4 * (i - j * vph),
                           v[u]);
            } else {
              *reinterpret_cast<float4*>(hbuf + j * PAD + 4 * (i - j * vph)) = v[u];
            }
          }
        }
      } else {
        // written by the head's work-groups at step t-1 of this launch
        constexpr int kS = (kPersistRuns * hs + NT - 1) / NT;
        const int nel = nj * hs;
        uint32_t offs[kS];
        float v[kS];
#pragma unroll
        for (int u = 0; u < kS; ++u) {
          const int i = min(u * NT + tid, nel - 1);
          const int j = i / hs;
          offs[u] = (uint32_t)(l_off[c0 + j] + t - 1) * (uint32_t)H + head * hs + (i - j * hs);
        }
        // Waves whose words all lie past the chunk poll the clamped last word.
        if (!poll_first<kS>(a.xch, offs, a.tag, a.err, v, (nel + NT - 1) / NT)) s_abort = 1;
        if (tr && c0 == 0) ltr[t * 8 + 1] = __builtin_amdgcn_s_memrealtime();
#pragma unroll
        for (int u = 0; u < kS; ++u) {
          const int i = u * NT + tid;
          if (i < nel) {
            const int j = i / hs;
            if constexpr (kF16) {
              const float x = v[u] * kHScale;
              const _Float16 h = (_Float16)x;
              hhi[j * PADH + (i - j * hs)] = h;
              hlo[j * PADH + (i - j * hs)] = (_Float16)(x - (float)h);
            } else {
              hbuf[j * PAD + (i - j * hs)] = v[u];
            }
          }
        }
      }
      lds_barrier();
      if (s_abort) return;
      if (tr && c0 == 0) ltr[t * 8 + 2] = __builtin_amdgcn_s_memrealtime();
      // Each k half writes its partial gate sums to its own LDS plane
      // (gsum: k half 0, xbuf: k half 1); the cell update adds the two.
      float* half = kh == 0 ? gsum : xbuf;
      if constexpr (kF16) {
        // G = W . H as hi*hi + (hi*lo + lo*hi) over this k half, every
        // chunk size, then unscaled (powers of two: exact). Columns fr >= nj
        // read run 0's row again (their results are dropped): lanes reading
        // one address share an LDS access, so a chunk of few runs reads
        // little more than its own rows.
        // four accumulator chains (hi.hi of even and of odd k-steps, hi.lo,
        // lo.hi), so consecutive matrix instructions seldom wait on each other
        floatx4_t a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0, c0 = a0, c1 = a0;
        const int fb = fr < nj ? fr : 0;
        const _Float16* bh = hhi + fb * PADH + kh * KH + 8 * fk;
        const _Float16* bl = hlo + fb * PADH + kh * KH + 8 * fk;
#pragma unroll
        for (int q = 0; q < KS; ++q) {
          const halfx8_t b_hi = *reinterpret_cast<const halfx8_t*>(bh + 32 * q);
          const halfx8_t b_lo = *reinterpret_cast<const halfx8_t*>(bl + 32 * q);
          if (q % 2 == 0) {
            a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi[q], b_hi, a0, 0, 0, 0);
          } else {
            a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi[q], b_hi, a1, 0, 0, 0);
          }
          c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi[q], b_lo, c0, 0, 0, 0);
          c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(wlo[q], b_hi, c1, 0, 0, 0);
        }
        const floatx4_t acc = (a0 + a1) + (c0 + c1);
        *reinterpret_cast<float4*>(half + fr * 64 + 16 * mt + 4 * fk) =
            make_float4(acc[0] * inv_row[0], acc[1] * inv_row[1], acc[2] * inv_row[2],
                        acc[3] * inv_row[3]);
      } else if (nj > kValuRuns) {
        // Columns fr >= nj read run 0's row again (one shared LDS access);
        // their results are dropped. Four independent accumulator chains
        // (one per step c of a group), summed at the end, so consecutive
        // MFMAs do not wait on each other.
        floatx4_t a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0, a2 = a0, a3 = a0;
        const float* hb = hbuf + (fr < nj ? fr : 0) * PAD + kh * KH + 4 * fk;
#pragma unroll
        for (int g = 0; g < KG; ++g) {
          const float4 hv = *reinterpret_cast<const float4*>(hb + 16 * g);
          a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 * g + 0], hv.x, a0, 0, 0, 0);
          a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 * g + 1], hv.y, a1, 0, 0, 0);
          a2 = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 * g + 2], hv.z, a2, 0, 0, 0);
          a3 = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 * g + 3], hv.w, a3, 0, 0, 0);
        }
        const floatx4_t acc = (a0 + a1) + (a2 + a3);
        // acc[e] = G[row 16*mt + 4*fk + e][run fr], partial over this k half.
        *reinterpret_cast<float4*>(half + fr * 64 + 16 * mt + 4 * fk) =
            make_float4(acc[0], acc[1], acc[2], acc[3]);
      } else {
        // VALU product, one run at a time (a rolled loop keeps the code
        // small: this runs once per step and must stay in the instruction
        // cache): lane (fr, fk) dots its register row slice with run j's h
        // (one LDS word per k, shared by the 16 lanes of a k group), then
        // the four k groups are summed across lanes.
        const float* hb = hbuf + kh * KH + 4 * fk;
#pragma unroll 1
        for (int j = 0; j < nj; ++j) {
          float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
          for (int g = 0; g < KG; ++g) {
            const float4 hv = *reinterpret_cast<const float4*>(hb + j * PAD + 16 * g);
            s0 = fmaf(w[4 * g + 0], hv.x, s0);
            s1 = fmaf(w[4 * g + 1], hv.y, s1);
            s2 = fmaf(w[4 * g + 2], hv.z, s2);
            s3 = fmaf(w[4 * g + 3], hv.w, s3);
          }
          float p = (s0 + s1) + (s2 + s3);
          p += __shfl_xor(p, 16);
          p += __shfl_xor(p, 32);
          if (fk == 0) half[j * 64 + 16 * mt + fr] = p;
        }
      }
      lds_barrier();
      if (tr && c0 == 0) ltr[t * 8 + 3] = __builtin_amdgcn_s_memrealtime();
      if (cell) {
        const float4 g0 = *reinterpret_cast<const float4*>(gsum + jr * 64 + uu * 4);
        const float4 g1 = *reinterpret_cast<const float4*>(xbuf + jr * 64 + uu * 4);
        const float ip = pi + ((g0.x + g1.x) + bi);
        const float fp = pf + ((g0.y + g1.y) + bf);
        const float zp = pz + ((g0.z + g1.z) + bz);
        const float op = po + ((g0.w + g1.w) + bo);
        const float lfm = pm + fast_logsigmoid(fp);
        const float mn = fmaxf(ip, lfm);
        const float og = fast_sigmoid(op);
        const float ig = fast_exp(ip - mn);
        const float fg = fast_exp(lfm - mn);
        const float cn = fg * pc + ig * fast_tanh(zp);
        const float nn = fg * pn + ig;
        const float h = og * cn * fast_rcp(nn + 1e-6f);
        a.c_state[psi] = cn;
        a.n_state[psi] = nn;
        a.m_state[psi] = mn;
        a.y[prow * H + ccol] = h;
        __hip_atomic_store(a.xch + prow * H + ccol, xch_word(h, a.tag), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      if (tr && c0 == 0) ltr[t * 8 + 4] = __builtin_amdgcn_s_memrealtime();
      // The next chunk's staging writes hbuf only (read before the barrier
      // above); gsum and xbuf are rewritten only after its staging barrier.
    }
    if (tr) ltr[t * 8 + 5] = __builtin_amdgcn_s_memrealtime();
  }
  if (a.trace != nullptr && blockIdx.x == 0) {
    lds_barrier();
    for (int i = tid; i < a.n_rounds * 8; i += NT) a.trace[i] = ltr[i];
  }
  // h_state <- h of each run's last step, for this work-group's units. Step
  // 0 of every work-group of the head reads h_state (chunk by chunk), so it
  // is written only once all of them are past that staging: each writes the
  // step-0 words of the last run in its last step-0 chunk, after all of its
  // step-0 staging, so wait for those words.
  {
    constexpr int kS = (hs + NT - 1) / NT;
    uint32_t offs[kS];
    float v[kS];
    const uint32_t row = (uint32_t)l_off[a.n_runs - 1];
#pragma unroll
    for (int u = 0; u < kS; ++u)
      offs[u] = row * (uint32_t)H + head * hs + min(u * NT + tid, hs - 1);
    if (!poll_words<kS>(a.xch, offs, a.tag, a.err, v)) s_abort = 1;
    lds_barrier();
    if (s_abort) return;
  }
  // The words were written by other threads of this work-group: read them
  // through the tag as well (the loop count is uniform so every lane polls).
  const int total = a.n_runs * 16;
  for (int base = 0; base < total; base += NT) {
    const int i = min(base + tid, total - 1);
    const int run = i >> 4;
    const int col = head * hs + u0 + (i & 15);
    const uint32_t off = (uint32_t)(l_off[run + 1] - 1) * (uint32_t)H + col;
    float hv;
    if (!poll_words<1>(a.xch, &off, a.tag, a.err, &hv)) return;
    if (base + tid < total) a.h_state[(int64_t)l_slot[run] * H + col] = hv;
  }
}

__global__ void slstm_final_kernel(const int* __restrict__ slot_ids,
                                   const int* __restrict__ run_off, const float* __restrict__ y,
                                   int hidden, float* __restrict__ h_state) {
  const int run = blockIdx.x;
  const int last = run_off[run + 1] - 1;
  const int slot = slot_ids[run];
  for (int c = threadIdx.x; c < hidden; c += blockDim.x)
    h_state[(int64_t)slot * hidden + c] = y[(int64_t)last * hidden + c];
}

// mLSTM gate / normaliser recurrence (model/xlstm.py:61-74, :140-142), one
// work-group of NWV waves per (run, head): thread i holds elements
// [i*PER, i*PER + PER) of the head's normaliser n (threads past hs hold
// zeros). Steps run in order in blocks of kGateBlock:
//  - the stabiliser chain m_t = max(i_t, m_{t-1} + logsigmoid(f_t)) and the
//    gates i', f' of the block's steps first (wave-uniform values; the gate
//    pre-activations may arrive as n_parts partial sums, added in order);
//  - then n_t = f'_t n_{t-1} + i'_t k_t and each thread's part of q_t . n_t
//    for every step of the block;
//  - then the block's dot products are summed together: a transposed
//    butterfly leaves step j's wave sum in lane 8j after 10 shuffles (one
//    wave sum per step would take 6 dependent shuffles each), and the waves'
//    sums meet in LDS.
// The rows of the next two blocks are prefetched into a register double
// buffer; loads are unconditional (rows clamped to the run) so that the
// compiler's wait counts stay exact.
constexpr int kGateBlock = 8;
template <int NWV, int PER>
__global__ __launch_bounds__(64 * NWV) void mlstm_gates_kernel(
    const int* __restrict__ slot_ids, const int* __restrict__ run_off, const float* __restrict__ if_pre,
    int n_parts, int64_t part_stride, int heads, const float* __restrict__ qkv, int inner, const float* __restrict__ ks,
    float* __restrict__ n_state, float* __restrict__ m_state, float* __restrict__ ig_out,
    float* __restrict__ fg_out, float* __restrict__ den_out) {
  constexpr int B = kGateBlock;
  using VecT = typename std::conditional<PER == 1, float,
               typename std::conditional<PER == 2, float2, float4>::type>::type;
  __shared__ float red[2][NWV][B];
  const int run = blockIdx.x / heads;
  const int head = blockIdx.x - run * heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hs = inner / heads;
  const int slot = slot_ids[run];
  const int r0 = run_off[run];
  const int len = run_off[run + 1] - r0;
  const int rl = r0 + len - 1;
  const int e0 = tid * PER;
  const float okf = e0 < hs ? 1.0f : 0.0f;
  const int ec = e0 < hs ? e0 : 0;  // clamped chunk (chunk 0 always exists)
  float* nst = n_state + ((int64_t)slot * heads + head) * hs + ec;
  auto get = [](const float* p, float* v) {
    const VecT x = *reinterpret_cast<const VecT*>(p);
    if constexpr (PER == 1) {
      v[0] = x;
    } else if constexpr (PER == 2) {
      v[0] = x.x;
      v[1] = x.y;
    } else {
      v[0] = x.x;
      v[1] = x.y;
      v[2] = x.z;
      v[3] = x.w;
    }
  };
  float nv[PER];
  get(nst, nv);
#pragma unroll
  for (int p = 0; p < PER; ++p) nv[p] *= okf;
  float m = m_state[(int64_t)slot * heads + head];

  const float* qh = qkv + (int64_t)head * hs + ec;
  const float* kh = ks + (int64_t)head * hs + ec;
  // gate pre-activations: lane j < 8 holds i of step j, lane 8 + j holds f
  const int gj = lane & 7;
  const float* gh = if_pre + head + ((lane & 8) ? heads : 0);
  float rq[2][B][PER], rk[2][B][PER], rg[2];
  auto fill = [&](float (&q)[B][PER], float (&k)[B][PER], float& g, int tb) {
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int64_t row = min(r0 + tb + j, rl);
      get(qh + row * 3 * inner, q[j]);
      get(kh + row * inner, k[j]);
    }
    const float* gp = gh + (int64_t)min(r0 + tb + gj, rl) * 2 * heads;
    g = gp[0];
    for (int p = 1; p < n_parts; ++p) g += gp[p * part_stride];
  };
  fill(rq[0], rk[0], rg[0], 0);
  fill(rq[1], rk[1], rg[1], B);

  auto block = [&](const float (&q)[B][PER], const float (&k)[B][PER], float g, int tb, int par) {
    float ig[B], fg[B], em[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const float ri = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), j));
      const float rf = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), 8 + j));
      const float lf = fast_logsigmoid(rf);
      const float mn = fmaxf(ri, m + lf);
      ig[j] = fast_exp(ri - mn);
      fg[j] = fast_exp(lf + m - mn);
      em[j] = fast_exp(-mn);
      if (tb + j < len) m = mn;
    }
    float pd[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      if (tb + j < len) {
#pragma unroll
        for (int p = 0; p < PER; ++p) nv[p] = fg[j] * nv[p] + ig[j] * (okf * k[j][p]);
      }
      float d = 0.0f;
#pragma unroll
      for (int p = 0; p < PER; ++p) d += q[j][p] * nv[p];
      pd[j] = d;
    }
    // lane 8j holds step j's wave sum
    float a1 = transposed_wave_sum<B>(pd);
    const int myj = lane >> 3;
    if constexpr (NWV > 1) {
      if ((lane & 7) == 0) red[par][wave][myj] = a1;
      lds_barrier();
      a1 = 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < NWV; ++w2) a1 += red[par][w2][myj];
    }
    if (wave == 0 && (lane & 7) == 0 && tb + myj < len) {
      float sig = ig[0], sfg = fg[0], sem = em[0];
#pragma unroll
      for (int j = 1; j < B; ++j) {
        sig = myj == j ? ig[j] : sig;
        sfg = myj == j ? fg[j] : sfg;
        sem = myj == j ? em[j] : sem;
      }
      const int64_t row = r0 + tb + myj;
      ig_out[row * heads + head] = sig;
      fg_out[row * heads + head] = sfg;
      den_out[row * heads + head] = fmaxf(fabsf(a1), sem) + 1e-6f;
    }
  };

  for (int tb = 0; tb < len; tb += 2 * B) {
    block(rq[0], rk[0], rg[0], tb, 0);
    if (tb + B >= len) break;  // the second block would hold no step of the run
    fill(rq[0], rk[0], rg[0], tb + 2 * B);
    block(rq[1], rk[1], rg[1], tb + B, 1);
    fill(rq[1], rk[1], rg[1], tb + 3 * B);
  }
  if (e0 < hs) {
    VecT x;
    if constexpr (PER == 1) {
      x = nv[0];
    } else if constexpr (PER == 2) {
      x = make_float2(nv[0], nv[1]);
    } else {
      x = make_float4(nv[0], nv[1], nv[2], nv[3]);
    }
    *reinterpret_cast<VecT*>(nst) = x;
  }
  if (tid == 0) m_state[(int64_t)slot * heads + head] = m;
}

}  // namespace

int conv_scan(const Runs& r, const float* in, int64_t ld_in, int channels, float* state,
              int64_t slot_stride, const float* w, const float* bias, int act_silu, float* out,
              int64_t ldo, hipStream_t s) {
  if (r.n_runs == 0) return HK_OK;
  dim3 grid(r.n_runs, (channels + 255) / 256);
  hipLaunchKernelGGL(conv_scan_kernel, grid, dim3(256), 0, s, r.slot_ids, r.run_off, in, ld_in,
                     channels, state, slot_stride, w, bias, act_silu, out, ldo);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int retnet_prep(const Runs& r, const float* qkvg, int64_t ld, int hidden, int heads,
                float k_scaling, const float* angle, const float* decay, int* offsets,
                float* scales, float* k_rope, float* q_scaled, hipStream_t s) {
  if (r.n_runs == 0) return HK_OK;
  HK_REQUIRE(hidden % heads == 0 && (hidden / heads) % 2 == 0, "retnet_prep: bad head size");
  HK_REQUIRE(r.n_rows > 0, "retnet_prep: bad row count %d", r.n_rows);
  HK_REQUIRE(r.row_pos && r.row_slot, "retnet_prep: needs the rows' run positions and slots");
  dim3 grid(r.n_rows, (hidden + 255) / 256);
  hipLaunchKernelGGL(retnet_prep_kernel, grid, dim3(256), 0, s, r.row_pos, r.row_slot, qkvg, ld,
                     hidden, hidden / heads, k_scaling, angle, decay, offsets, scales, k_rope,
                     q_scaled);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int rglru_scan(const Runs& r, const float* x, const float* gi, const float* gr, int64_t ldg,
               const float* gate, int64_t ld_gate, const float* a, float c_exp, int hidden,
               float* h_state, float* out, uint16_t* out_lp, int lp_fmt, hipStream_t s) {
  if (r.n_runs == 0) return HK_OK;
  dim3 grid(r.n_runs, (hidden + 63) / 64);
  hipLaunchKernelGGL(rglru_scan_kernel, grid, dim3(256), 0, s, r.slot_ids, r.run_off, x, gi, gr,
                     ldg, gate, ld_gate, a, c_exp, hidden, h_state, out, out_lp, lp_fmt);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int slstm_round(const Runs& r, int step, int n_active, const float* gin, int hidden, int heads,
                const float* w_state, const float* b_state, const float* h_state, float* c_state,
                float* n_state, float* m_state, float* y, hipStream_t s) {
  if (n_active == 0) return HK_OK;
  const int hs = hidden / heads;
  HK_REQUIRE(hs * heads == hidden && hs % kSlUnits == 0 && hs % 4 == 0,
             "slstm_round: head size %d unsupported", hs);
  const size_t smem = (size_t)(kSlRuns * hs + 4 * kSlRuns * kSlUnits) * sizeof(float);
  HK_REQUIRE(smem <= 64 * 1024, "slstm_round: head size %d too large for LDS staging", hs);
  dim3 grid(heads, hs / kSlUnits, (n_active + kSlRuns - 1) / kSlRuns);
  hipLaunchKernelGGL(slstm_round_kernel, grid, dim3(256), smem, s, r.slot_ids, r.run_off, step,
                     n_active, gin, hidden, hs, w_state, b_state, h_state, c_state, n_state,
                     m_state, y);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

bool slstm_persist_supported(int hidden, int heads) {
  const int hs = hidden / heads;
  return hs * heads == hidden && (hs == 32 || hs == 64 || hs == 128 || hs == 256 || hs == 512);
}

// The step barriers need every work-group of the launch resident at once.
// The grid (heads * hs/16 <= 128 work-groups of one CU each) is checked
// against the device's CU count times the kernel's occupancy per CU; given
// that, an ordinary launch is enough: work-groups that cannot start yet wait
// only for other kernels' work-groups, which never wait on this kernel. (A
// cooperative launch would also exclude concurrent kernels of the other
// streams for the whole recurrence.)
template <int HS, bool SPLIT>
int launch_persist(const SlstmPersistArgs& a, size_t smem, hipStream_t s) {
  const dim3 grid(a.heads * (HS / 16)), block(kPersistThreads);
  // per process (one device type), for the last LDS size asked for; two
  // threads may launch at once (the engine's two xLSTM run groups)
  static std::mutex mu;
  static int cus = -1;
  static size_t fits_smem = 0;
  static int64_t fits = -1;
  {
    std::lock_guard<std::mutex> lk(mu);
    if (cus < 0) {
      int dev = 0;
      HK_CHECK_HIP(hipGetDevice(&dev));
      HK_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    }
    if (fits < 0 || smem != fits_smem) {
      int per_cu = 0;
      HK_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, slstm_persist_kernel<HS, SPLIT>, kPersistThreads, smem));
      fits = (int64_t)cus * per_cu;
      fits_smem = smem;
    }
  }
  HK_REQUIRE((int64_t)grid.x <= fits, "slstm_persist: %u work-groups cannot be co-resident (%d)",
             grid.x, fits);
  hipLaunchKernelGGL((slstm_persist_kernel<HS, SPLIT>), grid, block, smem, s, a);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

// LDS bytes a persistent launch over n_runs runs and n_rounds steps uses.
size_t persist_smem(int hs, int n_runs, int n_rounds) {
  return (size_t)(kPersistRuns * (hs + 8) + 2 * kPersistRuns * 64) * sizeof(float) +
         (size_t)persist_meta_ints(n_runs, n_rounds) * sizeof(int);
}

// LDS bytes it asks for (see kPersistLdsFloor).
size_t persist_smem_launch(size_t used) { return std::max(used, kPersistLdsFloor); }

template <int HS, bool SPLIT>
int persist_pair_fits(size_t smem, int heads, bool* ok) {
  int dev = 0, cus = 0, per_cu = 0;
  HK_CHECK_HIP(hipGetDevice(&dev));
  HK_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  HK_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
      &per_cu, slstm_persist_kernel<HS, SPLIT>, kPersistThreads, smem));
  *ok = 2LL * heads * (HS / 16) <= (int64_t)cus * per_cu;
  return HK_OK;
}

int slstm_persist_pair_fits(int hidden, int heads, int max_runs, int max_rounds, bool split,
                            bool* ok) {
  *ok = false;
  if (!slstm_persist_supported(hidden, heads)) return HK_OK;
  const int hs = hidden / heads;
  const size_t smem = persist_smem_launch(persist_smem(hs, max_runs, max_rounds));
#define HK_FITS(HS)                                                                  \
  return split ? persist_pair_fits<HS, true>(smem, heads, ok)                       \
               : persist_pair_fits<HS, false>(smem, heads, ok)
  switch (hs) {
    case 32: HK_FITS(32);
    case 64: HK_FITS(64);
    case 128: HK_FITS(128);
    case 256: HK_FITS(256);
    default: HK_FITS(512);
  }
#undef HK_FITS
}

int slstm_persist(const Runs& r, const int* act_dev, int n_rounds, const float* gin, int hidden,
                  int heads, const float* w_state, const float* b_state, float* h_state,
                  float* c_state, float* n_state, float* m_state, float* y,
                  unsigned long long* xch, unsigned int tag, int* err, uint64_t* trace,
                  bool split, hipStream_t s) {
  if (r.n_runs == 0 || n_rounds == 0) return HK_OK;
  HK_REQUIRE(slstm_persist_supported(hidden, heads), "slstm_persist: head size unsupported");
  HK_REQUIRE(tag != 0 && xch != nullptr, "slstm_persist: exchange buffer and nonzero tag needed");
  HK_REQUIRE((int64_t)r.n_rows * hidden < (1LL << 32), "slstm_persist: exchange buffer too large");
  const int hs = hidden / heads;
  SlstmPersistArgs a{r.slot_ids, r.run_off, act_dev, n_rounds, r.n_runs, gin, hidden, heads,
                     w_state, b_state, h_state, c_state, n_state, m_state, y, xch, tag, err,
                     trace};
  size_t smem = persist_smem(hs, r.n_runs, n_rounds);
  HK_REQUIRE(smem <= 96 * 1024, "slstm_persist: %d runs over %d steps exceed the LDS descriptor copy",
             r.n_runs, n_rounds);
  if (trace != nullptr) {
    HK_REQUIRE(n_rounds <= 512, "slstm_persist: tracing supports at most 512 steps");
    smem += (size_t)n_rounds * 8 * sizeof(uint64_t);
  }
  smem = persist_smem_launch(smem);
#define HK_LAUNCH(HS) \
  return split ? launch_persist<HS, true>(a, smem, s) : launch_persist<HS, false>(a, smem, s)
  switch (hs) {
    case 32: HK_LAUNCH(32);
    case 64: HK_LAUNCH(64);
    case 128: HK_LAUNCH(128);
    case 256: HK_LAUNCH(256);
    default: HK_LAUNCH(512);
  }
#undef HK_LAUNCH
}

int slstm_final(const Runs& r, const float* y, int hidden, float* h_state, hipStream_t s) {
  if (r.n_runs == 0) return HK_OK;
  hipLaunchKernelGGL(slstm_final_kernel, dim3(r.n_runs), dim3(256), 0, s, r.slot_ids, r.run_off,
                     y, hidden, h_state);
  HK_LAUNCH_CHECK();
  return HK_OK;
}

int mlstm_gates(const Runs& r, const float* if_pre, int n_parts, int64_t part_stride, int heads,
                const float* qkv, int inner, const float* ks, float* n_state, float* m_state,
                float* ig, float* fg, float* den, hipStream_t s) {
  if (r.n_runs == 0) return HK_OK;
  HK_REQUIRE(n_parts >= 1 && n_parts <= 8, "mlstm_gates: 1 to 8 partial gate sums");
  const int hs = inner / heads;
  HK_REQUIRE(inner % heads == 0 && hs >= 1 && hs <= 1024,
             "mlstm_gates: head size %d unsupported (at most 1024)", hs);
  // NWV waves of 64 threads, PER consecutive elements per thread
  const int nwv = std::min(4, (hs + 63) / 64);
  const int per = hs <= 64 * nwv ? 1 : (hs <= 128 * nwv ? 2 : 4);
  HK_REQUIRE(hs % per == 0 && inner % per == 0 &&
                 (reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(ks) |
                  reinterpret_cast<uintptr_t>(n_state)) % (4 * per) == 0,
             "mlstm_gates: head size %d needs %d-float aligned rows", hs, per);
  const dim3 grid(r.n_runs * heads), block(64 * nwv);
#define HK_GATES(W, P)                                                                    \
  hipLaunchKernelGGL((mlstm_gates_kernel<W, P>), grid, block, 0, s, r.slot_ids, r.run_off, \
                     if_pre, n_parts, part_stride, heads, qkv, inner, ks, n_state, m_state, ig, \
                     fg, den)
  if (nwv == 1) {
    HK_GATES(1, 1);
  } else if (nwv == 2) {
    HK_GATES(2, 1);
  } else if (nwv == 3) {
    HK_GATES(3, 1);
  } else if (per == 1) {
    HK_GATES(4, 1);
  } else if (per == 2) {
    HK_GATES(4, 2);
  } else {
    HK_GATES(4, 4);
  }
#undef HK_GATES
  HK_LAUNCH_CHECK();
  return HK_OK;
}

}  // namespace hk
