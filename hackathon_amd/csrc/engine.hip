// The ensemble engine: packed weights, a slot-indexed recurrent state store
// resident in HBM, and the layer-major tick.
//
// A tick receives a batch of requests grouped into runs, one run per symbol
// (its slot) holding that symbol's requests in arrival order, runs sorted by
// non-increasing length. Every layer processes all requests of the tick at
// once: projections are GEMMs over every request row, and each recurrent
// layer scans each run in order while holding the symbol's state tile on
// chip, so a symbol's state crosses HBM twice per tick however many requests
// it has. The maths is exactly the reference's round-by-round evaluation
// (example_model.py:885-899): rows never mix (example_model.py:422-427) and
// each symbol's requests are applied in list order.
//
// Per request, per tower (model/inference_model.py:85-95, :55-68):
//   x = input_down(relu(input_up(features)))
//   12 x { x += layer(RMSNorm(x)); x += fc2(relu(fc1(RMSNorm(x)))) }
//   pred[tower] = output_proj(x)                          (shared weights)
#include <algorithm>
#include <cmath>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "common.h"
#include "gemm.h"
#include "ops.h"
#include "scan_mat.h"

extern "C" const char* hk_last_error(void);  // api_ops.hip: this thread's last error text

namespace hk {
namespace {

// Staging area of hk_engine_load_param_noalloc: 4 Mi fp32 values (16 MiB) in
// every GPU's memory for the life of the process. Host code never passes the
// symbol itself to the device: each device's copy has its own address,
// resolved once per device by scratch_on_current_device().
constexpr int64_t kScratchFloats = 4LL << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_dev[kMaxDevices] = {};
// Held by a binding for as long as it stages through a device's array, so
// that two bindings on one device (from two engines or threads) never
// overwrite each other's chunks.
std::mutex g_scratch_use_mu[kMaxDevices];

// The device address of `scratch` on the current device.
int scratch_on_current_device(float** out) {
  int dev = 0;
  HK_CHECK_HIP(hipGetDevice(&dev));
  HK_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    HK_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_dev[dev];
  return HK_OK;
}

enum TowerType { kXLSTM = 0, kMamba2 = 1, kRetNet = 2, kHawk = 3 };
constexpr int kTowers = 4;
constexpr int kMaxIfSegments = 4;  // partial planes of the mLSTM gate pre-activations
// Matrix-scan launches whose longest run has at least kRowSplitMinLen steps
// are latency-bound on that run: their tile rows are split over up to
// kMaxRowParts work-groups, and the scan's consumer adds the output planes.
constexpr int kMaxRowParts = 4;
// Pending rank-1 updates a matrix-state tile may carry before its write-back
// (one staging block of the scan).
constexpr int kLogCap = 8;
constexpr int kRowSplitMinLen = 16;

// ---- weight slots ----------------------------------------------------------
// Block-level slots common to every tower type.
enum { B_NORM1, B_NORM2, B_FC1_W, B_FC1_B, B_FC2_W, B_FC2_B, B_LAYER0 };
enum {  // xLSTM layer
  X_S_NORM = B_LAYER0, X_S_CONV_W, X_S_CONV_B, X_S_IN_W, X_S_ST_W, X_S_ST_B, X_S_GN_W, X_S_GN_B,
  X_L_NORM, X_L_XG_W, X_L_QKV_W, X_L_CONV_W, X_L_CONV_B, X_L_IF_W, X_L_IF_B, X_L_GN_W, X_L_GN_B,
  X_L_DOWN_W, X_L_SKIP, X_F_NORM, X_NSLOTS
};
enum {  // Mamba2 layer
  M_PROJ_W = B_LAYER0, M_DT_W, M_DT_B, M_CONV_W, M_CONV_B, M_A, M_D, M_NORM, M_OUT_W, M_NSLOTS
};
enum { R_QKVG_W = B_LAYER0, R_OUT_W, R_DECAY, R_ANGLE, R_NSLOTS };  // RetNet layer
enum { K_PROJ_W = B_LAYER0, K_CONV_W, K_CONV_B, K_GATES_W, K_A, K_OUT_W, K_NSLOTS };  // Hawk
enum { T_UP_W, T_UP_B, T_DOWN_W, T_DOWN_B, T_NSLOTS };  // tower level (layer = -1)
enum { G_OUT_W, G_OUT_B, G_NSLOTS };                     // global (tower = -1)

// State leaves, in the reference's init_state order per block.
enum { XS_S_CONV, XS_S_H, XS_S_C, XS_S_N, XS_S_M, XS_L_CONV, XS_L_C, XS_L_N, XS_L_M, XS_N };
enum { MS_CONV, MS_SSM, MS_N };
enum { RS_OFF, RS_SCALE, RS_S, RS_N };
enum { KS_CONV, KS_H, KS_N };

struct SlotDef {
  const char* name;
  int64_t numel;
  bool lp;          // a CastLinear weight: 16-bit storage in reduced-precision mode
  bool lp_bias;     // a CastLinear bias: rounded to 16 bits in reduced-precision mode
  int k = 0;        // a CastLinear weight's input width (its N is numel / k)
};

struct Slot {
  SlotDef def{};
  void* ptr = nullptr;   // device storage (16-bit when def.lp && lowp, else fp32)
  bool packed = false;   // 16-bit weight held in the pack_lp_weight layout
  bool bound = false;
  // fp32 slots: the power of two that puts the largest |w| in [2^13, 2^14),
  // for products run as split f16 (GemmArgs::split_wscale); set at binding
  float split_scale = 1.0f;
};

// Power of two that puts max |w| of an fp32 weight in [2^13, 2^14) (1 for
// an all-zero or non-finite maximum).
float split_scale_of(const float* w, int64_t n) {
  float m = 0.0f;
  for (int64_t i = 0; i < n; ++i) m = std::fmax(m, std::fabs(w[i]));
  if (!(m > 0.0f) || !std::isfinite(m)) return 1.0f;
  const int e = std::ilogb(m);  // m in [2^e, 2^(e+1))
  return std::ldexp(1.0f, std::min(std::max(13 - e, -100), 100));
}

struct Dims {
  int H, P, D, nh, F, Fpad;
  int nh_s, bs_s;        // sLSTM heads / head size
  int I, hs_m;           // mLSTM inner / head size
  int Im, hm, bc, nhm;   // Mamba2 inner / head / bc / heads
  int hs_r;              // RetNet head size
  int nb_h, bs_h;        // Hawk RG-LRU blocks
};

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

std::vector<SlotDef> block_slots(const Dims& d, int tower) {
  std::vector<SlotDef> v = {
      {"norm1.weight", d.H, false, false},
      {"norm2.weight", d.H, false, false},
      {"mlp.fc1.weight", (int64_t)d.P * d.H, true, false, d.H},
      {"mlp.fc1.bias", d.P, false, true},
      {"mlp.fc2.weight", (int64_t)d.H * d.P, true, false, d.P},
      {"mlp.fc2.bias", d.H, false, true},
  };
  switch (tower) {
    case kXLSTM: {
      const int64_t I = d.I;
      v.push_back({"slstm.norm.weight", d.H, false, false});
      v.push_back({"slstm.conv (4 taps x H)", 4LL * d.H, false, false});
      v.push_back({"slstm.conv1d.conv.bias", d.H, false, false});
      v.push_back({"slstm.{i,f,z,o}gate_input.weight", 4LL * d.H * d.bs_s, false, false});
      v.push_back({"slstm.{i,f,z,o}gate_state.weight", 4LL * d.H * d.bs_s, false, false});
      v.push_back({"slstm.{i,f,z,o}gate_state.bias", 4LL * d.H, false, false});
      v.push_back({"slstm.group_norm.weight", d.H, false, false});
      v.push_back({"slstm.group_norm.bias", d.H, false, false});
      v.push_back({"mlstm.norm.weight", d.H, false, false});
      v.push_back({"mlstm.{x_proj,gate_proj}.weight", 2 * I * d.H, true, false, d.H});
      v.push_back({"mlstm.{q,k,v}_proj.weight", 3 * I * 4, false, false});
      v.push_back({"mlstm.conv (4 taps x I)", 4 * I, false, false});
      v.push_back({"mlstm.conv1d.conv.bias", I, false, false});
      v.push_back({"mlstm.mlstm_cell.{igate,fgate}_proj.weight", 2LL * d.nh * 3 * I, false, false});
      v.push_back({"mlstm.mlstm_cell.{igate,fgate}_proj.bias", 2LL * d.nh, false, false});
      v.push_back({"mlstm.mlstm_cell.outnorm.weight", I, false, false});
      v.push_back({"mlstm.mlstm_cell.outnorm.bias", I, false, false});
      v.push_back({"mlstm.proj_down.weight", (int64_t)d.H * I, true, false, (int)I});
      v.push_back({"mlstm.learnable_skip", I, false, false});
      v.push_back({"final_norm.weight", d.H, false, false});
      break;
    }
    case kMamba2: {
      const int64_t C = d.Im + 2LL * d.bc;
      v.push_back({"{input,b,c,z}_proj.weight", (C + d.Im) * d.H, true, false, d.H});
      v.push_back({"dt_proj.weight", (int64_t)d.nhm * d.H, false, false});
      v.push_back({"dt_proj.bias", d.nhm, false, false});
      v.push_back({"{input,b,c}_conv (4 taps x C)", 4 * C, false, false});
      v.push_back({"{input,b,c}_conv.conv.bias", C, false, false});
      v.push_back({"a", d.nhm, false, false});
      v.push_back({"d", d.nhm, false, false});
      v.push_back({"norm.weight", d.Im, false, false});
      v.push_back({"out_proj.weight", (int64_t)d.H * d.Im, true, false, d.Im});
      break;
    }
    case kRetNet: {
      v.push_back({"{q,k,v,g}_proj.weight", 4LL * d.H * d.H, true, false, d.H});
      v.push_back({"out_proj.weight", (int64_t)d.H * d.H, true, false, d.H});
      v.push_back({"decay", d.nh, false, false});
      v.push_back({"angle", d.hs_r, false, false});
      break;
    }
    case kHawk: {
      v.push_back({"{gate,recurrent}_proj.weight", 2LL * d.H * d.H, true, false, d.H});
      v.push_back({"conv (4 taps x H)", 4LL * d.H, false, false});
      v.push_back({"conv.conv.bias", d.H, false, false});
      v.push_back({"rglru.{input,recurrence}_gate.weight", 2LL * d.H * d.bs_h, false, false});
      v.push_back({"rglru.a", d.H, false, false});
      v.push_back({"out_proj.weight", (int64_t)d.H * d.H, true, false, d.H});
      break;
    }
  }
  return v;
}

std::vector<SlotDef> tower_slots(const Dims& d) {
  return {{"input_up.weight (K padded)", (int64_t)d.P * d.Fpad, true, false, d.Fpad},
          {"input_up.bias", d.P, false, true},
          {"input_down.weight", (int64_t)d.H * d.P, true, false, d.P},
          {"input_down.bias", d.H, false, true}};
}

std::vector<SlotDef> global_slots(const Dims& d) {
  return {{"output_proj.weight", d.H, false, false}, {"output_proj.bias", 1, false, false}};
}

std::vector<int64_t> state_leaves(const Dims& d, int tower) {
  switch (tower) {
    case kXLSTM:
      return {3LL * d.H, d.H, d.H, d.H, d.H, 3LL * d.I, (int64_t)d.nh * d.hs_m * d.hs_m,
              (int64_t)d.nh * d.hs_m, d.nh};
    case kMamba2:
      return {3LL * (d.Im + 2 * d.bc), (int64_t)d.nhm * d.bc * d.hm};
    case kRetNet:
      return {1, d.nh, (int64_t)d.nh * d.hs_r * d.hs_r};
    default:
      return {3LL * d.H, d.H};
  }
}

// ---- device buffers ----------------------------------------------------------

struct DevBuf {
  void* p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
};

struct Act {  // an activation: fp32 copy and (reduced-precision mode) 16-bit copy
  float* f = nullptr;
  uint16_t* l = nullptr;
};

struct TowerWS {
  Act X, A, H1;
  // xLSTM
  float *XN = nullptr, *XCA = nullptr, *GIN = nullptr, *SY = nullptr, *X1 = nullptr,
        *XMG = nullptr, *XMC = nullptr, *QKV = nullptr, *KS = nullptr, *IF = nullptr,
        *IG = nullptr, *FG = nullptr, *DEN = nullptr, *NUM = nullptr, *X2 = nullptr;
  Act XN2, HS;
  // Mamba2
  float *PROJ = nullptr, *DTS = nullptr, *DEC = nullptr, *MXC = nullptr,
        *YS = nullptr;
  Act YN;
  // RetNet
  float *QKVG = nullptr, *KR = nullptr, *QS = nullptr, *O = nullptr;
  Act YO;
  // Hawk
  float *GRP = nullptr, *KXC = nullptr, *GATES = nullptr;
  Act GH;
  GemmWorkspace gemm_ws;
};

// Host threads that enqueue the side streams' share of a tick. A kernel
// launch costs the calling thread ~2.6 us in the HIP runtime, so one thread
// spends ~2 ms on a tick's ~700 launches, longer than a small tick runs on
// the GPU; launches to different streams from different threads go through
// the runtime concurrently (four threads: ~0.9 us per launch in all).
// Worker i runs the task posted for it; wait() returns once every posted
// task has finished, with each task's status and error text.
class EnqueuePool {
 public:
  EnqueuePool(int device, int n) : w_(n) {
    try {
      for (int i = 0; i < n; ++i) w_[i].th = std::thread([this, device, i] { loop(device, i); });
    } catch (...) {
      shutdown();  // the threads already started end before the error goes on
      throw;
    }
  }
  ~EnqueuePool() { shutdown(); }
  void post(int i, std::function<int()> fn) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      w_[i].fn = std::move(fn);
      w_[i].has = true;
      w_[i].st = HK_OK;
      w_[i].err.clear();
      ++pending_;
    }
    cv_.notify_all();
  }
  // The first failing task's status (its error text in *err), else HK_OK.
  int wait(std::string* err) {
    std::unique_lock<std::mutex> lk(mu_);
    done_.wait(lk, [this] { return pending_ == 0; });
    for (auto& w : w_)
      if (w.st != HK_OK) {
        *err = w.err;
        return w.st;
      }
    return HK_OK;
  }

 private:
  struct Worker {
    std::thread th;
    std::function<int()> fn;
    bool has = false;
    int st = HK_OK;
    std::string err;
  };
  void shutdown() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& w : w_)
      if (w.th.joinable()) w.th.join();
  }
  void loop(int device, int i) {
    const hipError_t dev_st = hipSetDevice(device);
    for (;;) {
      std::function<int()> fn;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return stop_ || w_[i].has; });
        if (!w_[i].has) return;  // stop_ with nothing posted
        fn = std::move(w_[i].fn);
        w_[i].has = false;
      }
      int st;
      std::string err;
      if (dev_st != hipSuccess) {
        st = HK_ERR_HIP;
        err = std::string("enqueue thread: hipSetDevice: ") + hipGetErrorString(dev_st);
      } else {
        try {
          st = fn();
          if (st != HK_OK) err = hk_last_error();
        } catch (const std::exception& ex) {
          st = HK_ERR_HIP;
          err = std::string("enqueue thread: ") + ex.what();
        }
      }
      {
        std::lock_guard<std::mutex> lk(mu_);
        w_[i].st = st;
        w_[i].err = std::move(err);
        if (--pending_ == 0) done_.notify_all();
      }
    }
  }
  std::vector<Worker> w_;
  std::mutex mu_;
  std::condition_variable cv_, done_;
  int pending_ = 0;
  bool stop_ = false;
};

}  // namespace

struct Engine {
  Dims d{};
  int capacity = 0, max_rows = 0, max_runs = 0;
  int device = -1;            // the device current at creation (owns every buffer)
  float* scratch = nullptr;   // that device's address of `scratch`
  // CastLinear mode (example_model.py:150-157): lowp = the converted
  // linears store and compute in lp_fmt (bf16 or fp16), else all fp32.
  bool lowp = false;
  int lp_fmt = kLpBF16;
  std::vector<std::unique_ptr<DevBuf>> bufs;
  // slots[tower][layer+1][slot]; layer index 0 holds the tower-level slots.
  std::vector<std::vector<std::vector<Slot>>> slots;
  std::vector<Slot> gslots;
  // state[tower][layer][leaf] -> device base, per-slot elements
  std::vector<std::vector<std::vector<float*>>> state;
  std::vector<std::vector<int64_t>> leaf_elems;
  // Write-back logs of the matrix-state leaves, [tower][layer] (null for
  // Hawk): see MatScanDesc.
  struct MatLog {
    float* hdr = nullptr;
    float* b = nullptr;
    float* g = nullptr;
  };
  std::vector<std::vector<MatLog>> mlog;
  TowerWS ws[kTowers];
  TowerWS ws_x2;             // xLSTM workspace of the second run group
  Act FE;
  // Tick descriptors, one device block (layout of stage_ints()): slot ids,
  // run offsets and active-run counts of the whole tick, run offsets of the
  // second xLSTM group (relative to its first row), per-group counts, and
  // each row's position in its run and slot.
  int* d_desc = nullptr;
  int* d_slots = nullptr;
  int* d_off = nullptr;
  int* d_act = nullptr;      // [max_rows]: runs active at each step
  int* d_off2 = nullptr;     // [max_runs + 1]
  int* d_act1 = nullptr;     // [max_rows]
  int* d_act2 = nullptr;     // [max_rows]
  int* d_pos = nullptr;      // [max_rows]: position of each row in its run
  int* d_rslot = nullptr;    // [max_rows]: slot of each row's run
  unsigned long long* d_xch = nullptr;   // [max_rows][H]: sLSTM h exchange words
  unsigned long long* d_xch2 = nullptr;  // the same for the second xLSTM group
  // Exchange tags: eager launches count up from 1 per buffer below
  // kGraphTag0; captured launches take tags from kGraphTag0 up, each used by
  // one captured launch only (see GraphEntry).
  unsigned int xch_tag[2] = {0, 0};      // tag of the last eager sLSTM launch on d_xch / d_xch2
  unsigned int graph_tag_next = 0x80000000u;
  bool sl_overlap = false;  // the two groups' persistent launches can be co-resident together
  double x_weight_us = 0.0;  // one xLSTM layer's weights read at 5 TB/s (the split rule's cost)
  int* d_err = nullptr;      // [1]: set by a kernel whose barrier timed out
  uint64_t* d_trace = nullptr;  // HK_TRACE_SLSTM: per-step stamps of layer 0's sLSTM
  int* h_stage = nullptr;    // pinned [2][stage_ints()]
  int* h_err = nullptr;      // pinned [1]: d_err read back by hk_engine_check
  int stage_ints() const { return 3 * max_runs + 2 + 5 * max_rows; }
  hipEvent_t stage_done[2] = {nullptr, nullptr};
  int stage_idx = 0;
  // The towers are independent and run concurrently, forked from and joined
  // back to the caller's stream per tick (all streams at default priority).
  // Four streams in all, one per hardware queue of a default HIP process:
  // the caller's stream runs the xLSTM tower's first run group (the longest
  // runs), side[0] its second group, side[1] Mamba2, side[2] RetNet then
  // Hawk.
  static constexpr int kSide = 3;
  hipStream_t side[kSide] = {nullptr, nullptr, nullptr};
  // hipGraph replay of small ticks (the reference captures its whole step
  // once and replays it per round, example_model.py:444-492). A tick's work
  // depends on its run lengths alone (the descriptors, features and
  // predictions sit in fixed device buffers), so graphs are cached by that
  // key. Each entry holds two executables that differ only in the tags of
  // their persistent sLSTM launches, replayed alternately: between two
  // replays of one executable the other one rewrote every exchange word the
  // first polls, with other tags, so a poll never accepts a word left over
  // from the previous replay of its own executable.
  struct GraphEntry {
    hipGraphExec_t exec[2] = {nullptr, nullptr};
    int next = 0;
    uint64_t last_use = 0;
  };
  int graph_rows = 0;   // ticks of at most this many rows replay graphs (0: never)
  int graph_cap = 0;    // shapes cached at most (least recently used evicted)
  std::map<std::vector<int>, GraphEntry> graphs;
  uint64_t graph_clock = 0;
  int64_t graph_captures = 0, graph_replays = 0;
  bool capturing = false;
  hipStream_t cap_s = nullptr;   // capture origin
  float* g_feat = nullptr;       // [max_rows][F] a replayed tick's features
  float* g_pred = nullptr;       // [max_rows][4] its predictions
  hipEvent_t fork_ev = nullptr;
  hipEvent_t join_ev[kSide] = {nullptr, nullptr, nullptr};
  // Where two persistent sLSTM launches cannot be co-resident at once, the
  // two xLSTM groups' launches alternate per layer (group 2 then group 1).
  std::vector<hipEvent_t> sl_ev[2];
  std::vector<char> seen;
  // Optional per-launch timing of the matrix-state scans (kind 0 mLSTM,
  // 1 Mamba2, 2 RetNet): event pairs recorded on the launch stream.
  int prof = 0;  // bit k: time launches of kind k
  std::vector<std::pair<hipEvent_t, hipEvent_t>> prof_ev[5];
  size_t prof_used[5] = {0, 0, 0, 0, 0};
  // Threads enqueueing the side streams' launches (created on the first
  // tick that uses them).
  std::unique_ptr<EnqueuePool> pool;

  ~Engine() {
    pool.reset();
    for (auto& kv : graphs)
      for (auto& x : kv.second.exec)
        if (x) (void)hipGraphExecDestroy(x);
    if (cap_s) (void)hipStreamDestroy(cap_s);
    for (auto& st : side)
      if (st) (void)hipStreamDestroy(st);
    if (fork_ev) (void)hipEventDestroy(fork_ev);
    for (auto& ev : join_ev)
      if (ev) (void)hipEventDestroy(ev);
    for (auto& v : sl_ev)
      for (auto& ev : v)
        if (ev) (void)hipEventDestroy(ev);

    for (auto& v : prof_ev)
      for (auto& pr : v) {
        (void)hipEventDestroy(pr.first);
        (void)hipEventDestroy(pr.second);
      }
    for (auto& e : stage_done)
      if (e) (void)hipEventDestroy(e);
    if (h_stage) (void)hipHostFree(h_stage);
    if (h_err) (void)hipHostFree(h_err);
  }

  void* alloc_bytes(size_t bytes) {
    auto b = std::make_unique<DevBuf>();
    if (hipMalloc(&b->p, std::max<size_t>(bytes, 256)) != hipSuccess) {
      b->p = nullptr;
      return nullptr;
    }
    void* p = b->p;
    bufs.push_back(std::move(b));
    return p;
  }
  float* alloc_f(int64_t n) { return static_cast<float*>(alloc_bytes((size_t)n * 4)); }
  uint16_t* alloc_l(int64_t n) { return static_cast<uint16_t*>(alloc_bytes((size_t)n * 2)); }
  Act alloc_act(int64_t n, bool need_f32) {
    Act a;
    if (need_f32 || !lowp) a.f = alloc_f(n);
    if (lowp) a.l = alloc_l(n);
    return a;
  }
};

namespace {

bool any_null(const Act& a, bool need_f32, bool lowp) {
  return ((need_f32 || !lowp) && !a.f) || (lowp && !a.l);
}

int build_workspace(Engine& e) {
  const Dims& d = e.d;
  const int64_t R = e.max_rows;
  for (int t = 0; t <= kTowers; ++t) {
    // t == kTowers: the second xLSTM group's workspace
    TowerWS& w = t < kTowers ? e.ws[t] : e.ws_x2;
    w.X.f = e.alloc_f(R * d.H);
    w.A = e.alloc_act(R * d.H, true);
    w.H1 = e.alloc_act(R * d.P, false);
    if (!w.X.f || any_null(w.A, true, e.lowp) || any_null(w.H1, false, e.lowp)) return HK_ERR_HIP;
    int64_t max_n = std::max<int64_t>(d.P, d.H);
    switch (t < kTowers ? t : (int)kXLSTM) {
      case kXLSTM:
        w.XN = e.alloc_f(R * d.H);
        w.XCA = e.alloc_f(R * d.H);
        w.GIN = e.alloc_f(R * 4 * d.H);
        w.SY = e.alloc_f(R * d.H);
        w.X1 = e.alloc_f(R * d.H);
        w.XN2 = e.alloc_act(R * d.H, false);
        w.XMG = e.alloc_f(R * 2 * d.I);
        w.XMC = e.alloc_f(R * d.I);
        w.QKV = e.alloc_f(R * 3 * d.I);
        w.KS = e.alloc_f(R * d.I);
        w.IF = e.alloc_f(R * 2 * d.nh * kMaxIfSegments);
        w.IG = e.alloc_f(R * d.nh);
        w.FG = e.alloc_f(R * d.nh);
        w.DEN = e.alloc_f(R * d.nh);
        w.NUM = e.alloc_f(R * d.I * kMaxRowParts);
        w.HS = e.alloc_act(R * d.I, false);
        w.X2 = e.alloc_f(R * d.H);
        if (!w.XN || !w.XCA || !w.GIN || !w.SY || !w.X1 || any_null(w.XN2, false, e.lowp) ||
            !w.XMG || !w.XMC || !w.QKV || !w.KS || !w.IF || !w.IG || !w.FG || !w.DEN || !w.NUM ||
            any_null(w.HS, false, e.lowp) || !w.X2)
          return HK_ERR_HIP;
        max_n = std::max<int64_t>(max_n, 2 * d.I);
        break;
      case kMamba2: {
        const int64_t C = d.Im + 2LL * d.bc;
        w.PROJ = e.alloc_f(R * (C + d.Im));
        w.DTS = e.alloc_f(R * d.nhm);
        w.DEC = e.alloc_f(R * d.nhm);
        w.MXC = e.alloc_f(R * C);
        w.YS = e.alloc_f(R * d.Im * kMaxRowParts);
        w.YN = e.alloc_act(R * d.Im, false);
        if (!w.PROJ || !w.DTS || !w.DEC || !w.MXC || !w.YS ||
            any_null(w.YN, false, e.lowp))
          return HK_ERR_HIP;
        max_n = std::max<int64_t>(max_n, C + d.Im);
        break;
      }
      case kRetNet:
        w.QKVG = e.alloc_f(R * 4 * d.H);
        w.KR = e.alloc_f(R * d.H);
        w.QS = e.alloc_f(R * d.H);
        w.O = e.alloc_f(R * d.H * kMaxRowParts);
        w.YO = e.alloc_act(R * d.H, false);
        if (!w.QKVG || !w.KR || !w.QS || !w.O || any_null(w.YO, false, e.lowp)) return HK_ERR_HIP;
        max_n = std::max<int64_t>(max_n, 4 * d.H);
        break;
      case kHawk:
        w.GRP = e.alloc_f(R * 2 * d.H);
        w.KXC = e.alloc_f(R * d.H);
        w.GATES = e.alloc_f(R * 2 * d.H);
        w.GH = e.alloc_act(R * d.H, false);
        if (!w.GRP || !w.KXC || !w.GATES || any_null(w.GH, false, e.lowp)) return HK_ERR_HIP;
        max_n = std::max<int64_t>(max_n, 2 * d.H);
        break;
    }
    // Split-K partial sums: up to 8 splits of the widest projection.
    w.gemm_ws.partial_elems = std::min<int64_t>(8 * R * max_n, 1LL << 26);
    w.gemm_ws.partial = e.alloc_f(w.gemm_ws.partial_elems);
    // One arrival counter per output tile of a split GEMM (a GEMM with more
    // tiles than this runs unsplit).
    w.gemm_ws.arrival_elems = 1 << 16;
    w.gemm_ws.arrivals = static_cast<int*>(e.alloc_bytes((size_t)w.gemm_ws.arrival_elems * 4));
    if (!w.gemm_ws.partial || !w.gemm_ws.arrivals) return HK_ERR_HIP;
    HK_CHECK_HIP(hipMemset(w.gemm_ws.arrivals, 0, (size_t)w.gemm_ws.arrival_elems * 4));
  }
  e.FE = e.alloc_act(R * d.Fpad, false);
  e.g_feat = e.alloc_f(R * d.F);
  e.g_pred = e.alloc_f(R * kTowers);
  if (!e.g_feat || !e.g_pred) return HK_ERR_HIP;
  if (any_null(e.FE, false, e.lowp)) return HK_ERR_HIP;
  e.d_desc = static_cast<int*>(e.alloc_bytes((size_t)e.stage_ints() * 4));
  e.d_xch = static_cast<unsigned long long*>(e.alloc_bytes((size_t)e.max_rows * d.H * 8));
  e.d_xch2 = static_cast<unsigned long long*>(e.alloc_bytes((size_t)e.max_rows * d.H * 8));
  e.d_err = static_cast<int*>(e.alloc_bytes(4));
  if (!e.d_desc || !e.d_xch || !e.d_xch2 || !e.d_err) return HK_ERR_HIP;
  e.d_slots = e.d_desc;
  e.d_off = e.d_slots + e.max_runs;
  e.d_act = e.d_off + e.max_runs + 1;
  e.d_off2 = e.d_act + e.max_rows;
  e.d_act1 = e.d_off2 + e.max_runs + 1;
  e.d_act2 = e.d_act1 + e.max_rows;
  e.d_pos = e.d_act2 + e.max_rows;
  e.d_rslot = e.d_pos + e.max_rows;
  HK_CHECK_HIP(hipMemset(e.d_err, 0, 4));
  if (std::getenv("HK_TRACE_SLSTM")) {
    e.d_trace = static_cast<uint64_t*>(e.alloc_bytes((size_t)e.max_rows * 8 * 8));
    if (!e.d_trace) return HK_ERR_HIP;
  }
  HK_CHECK_HIP(hipMemset(e.d_xch, 0, (size_t)e.max_rows * d.H * 8));
  HK_CHECK_HIP(hipMemset(e.d_xch2, 0, (size_t)e.max_rows * d.H * 8));
  HK_CHECK_HIP(hipHostMalloc((void**)&e.h_err, 4, hipHostMallocDefault));
  HK_CHECK_HIP(hipHostMalloc((void**)&e.h_stage, (size_t)2 * e.stage_ints() * 4,
                             hipHostMallocDefault));
  for (auto& ev : e.stage_done) HK_CHECK_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  for (int i = 0; i < Engine::kSide; ++i) {
    HK_CHECK_HIP(hipStreamCreateWithFlags(&e.side[i], hipStreamNonBlocking));
    HK_CHECK_HIP(hipEventCreateWithFlags(&e.join_ev[i], hipEventDisableTiming));
  }
  HK_CHECK_HIP(hipEventCreateWithFlags(&e.fork_ev, hipEventDisableTiming));
  HK_CHECK_HIP(hipStreamCreateWithFlags(&e.cap_s, hipStreamNonBlocking));
  for (auto& v : e.sl_ev) {
    v.assign(d.D, nullptr);
    for (auto& ev : v) HK_CHECK_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  }
  {
    const int st =
        slstm_persist_pair_fits(d.H, d.nh_s, e.max_runs, e.max_rows, e.lowp, &e.sl_overlap);
    if (st != HK_OK) return st;
  }

  return HK_OK;
}

// Runs `fn` bracketed by timing events of `kind` when profiling of that kind
// is on (0 mLSTM scan, 1 Mamba2 scan, 2 RetNet scan, 3 sLSTM recurrence,
// 4 GEMM).
template <typename Fn>
int timed(Engine& e, int kind, hipStream_t s, Fn&& fn) {
  if (!(e.prof & (1 << kind))) return fn();
  auto& v = e.prof_ev[kind];
  if (e.prof_used[kind] == v.size()) {
    std::pair<hipEvent_t, hipEvent_t> pr;
    HK_CHECK_HIP(hipEventCreate(&pr.first));
    HK_CHECK_HIP(hipEventCreate(&pr.second));
    v.push_back(pr);
  }
  auto& pr = v[e.prof_used[kind]++];
  HK_CHECK_HIP(hipEventRecord(pr.first, s));
  int st = fn();
  HK_CHECK_HIP(hipEventRecord(pr.second, s));
  return st;
}

// ---- one linear layer --------------------------------------------------------

struct Lin {
  const Slot* w;
  const Slot* b;  // may be null
};

// y = x . W^T (+ b); CastLinear semantics when W is a reduced-precision slot.
int linear(Engine& e, TowerWS& w, const Act& x, int64_t ldx, const Lin& lin, int M, int N, int K,
           int act, const float* residual, int64_t ldr, float* out, int64_t ldo, uint16_t* out_lp,
           int64_t ldl, hipStream_t s, const float* dt_a = nullptr, float* dt_decay = nullptr) {
  GemmArgs g;
  const bool lp = lin.w->def.lp && e.lowp;
  g.type = !lp ? GemmType::kF32 : e.lp_fmt == kLpF16 ? GemmType::kF16 : GemmType::kBF16;
  g.A = lp ? (const void*)x.l : (const void*)x.f;
  HK_REQUIRE(g.A != nullptr, "linear %s: missing %s input", lin.w->def.name, lp ? "16-bit" : "fp32");
  g.lda = ldx;
  g.W = lin.w->ptr;
  g.ldw = K;
  g.w_packed = lp && lin.w->packed;
  // In the reduced-precision modes the kept-fp32 linears that run here
  // (Mamba2's dt_proj, whose input is an RMSNorm output; the mLSTM gate
  // projections over q, k, v on shapes mlstm_qkv_if does not cover) run as
  // split f16 like the BlockLinear products (fp32-level error); the fp32
  // mode keeps fp32 arithmetic here.
  if (!lp && e.lowp) g.split_wscale = lin.w->split_scale;
  // A tick's four streams share the device: above 64 rows the larger tiles
  // of the shared rule measure faster in the tick (C4: 9.21-9.24 against
  // 9.34-9.37 ms); at 64 rows (the B=64 latency tick) the lone rule's
  // smaller tiles do (p50 5.09 against 5.17 ms). The xLSTM run groups'
  // GEMMs, on the tick's two critical chains, keep the lone rule's tiles at
  // any row count (C4 8.60-8.62 against 8.64-8.66 ms, four alternating
  // pairs; 200 or 256 work-groups for them: 8.67-8.74 ms).
  const bool xlstm_group = &w == &e.ws[kXLSTM] || &w == &e.ws_x2;
  g.min_tiles = M > 64 && !xlstm_group ? kMinTilesShared : kMinTilesAlone;
  g.M = M;
  g.N = N;
  g.K = K;
  g.ep.bias = lin.b ? static_cast<const float*>(lin.b->ptr) : nullptr;
  g.ep.round_lp = lp;
  g.ep.lp_fmt = e.lp_fmt;
  g.ep.act = act;
  g.ep.residual = residual;
  g.ep.ldr = ldr;
  g.ep.out = out;
  g.ep.ldo = ldo;
  g.ep.out_lp = out_lp;
  g.ep.ldl = ldl;
  g.ep.dt_a = dt_a;
  g.ep.dt_decay = dt_decay;
  g.ep.ldd = N;
  return timed(e, 4, s, [&] { return gemm(g, w.gemm_ws, s); });
}

// Block-diagonal fp32 products (BlockLinear, model/modules.py:71-79), several
// in one launch: batch b = j * blocks + k is block k of product j, reading x
// (or x2 for j >= x2_from) and W[b] = W + b*bs*bs, writing out columns
// b*bs .. b*bs + bs - 1:
//   out[:, b*bs + o] = sum_h src[:, k*bs + h] * W[b][o][h].
// In the reduced-precision modes the BlockLinear products of the sLSTM gate
// inputs and the RG-LRU gates run as split f16 on matrix cores
// (GemmArgs::split_wscale; `wscale` is the weight slot's split_scale):
// fp32-level error (each operand as an f16 value plus its f16 remainder), a
// fifth of the fp32 matrix-core time per product. Their inputs (LayerNorm
// outputs, silu(conv) and conv outputs of normalised rows) stay far below the
// f16 range the split needs (65504). The fp32 mode keeps fp32 arithmetic.
int block_linear(Engine& e, TowerWS& w, const float* x, const float* x2, int x2_from, int64_t ldx,
                 const float* W, float wscale, int products, int blocks, int bs, int M, float* out,
                 int64_t ldo, hipStream_t s) {
  GemmArgs g;
  g.type = GemmType::kF32;
  g.split_wscale = e.lowp ? wscale : 0.0f;
  g.A = x;
  g.A2 = x2;
  g.a2_from = x2 ? x2_from * blocks : 0;
  g.a_period = blocks;
  g.lda = ldx;
  g.W = W;
  g.ldw = bs;
  g.M = M;
  g.N = bs;
  g.K = bs;
  g.batch = products * blocks;
  g.a_bstride = bs;
  g.w_bstride = (int64_t)bs * bs;
  g.c_bstride = bs;
  g.ep.out = out;
  g.ep.ldo = ldo;
  return timed(e, 4, s, [&] { return gemm(g, w.gemm_ws, s); });
}

#define HK_TRY(expr)          \
  do {                        \
    int st_ = (expr);         \
    if (st_ != HK_OK) return st_; \
  } while (0)

const Slot* S(Engine& e, int t, int l, int i) { return &e.slots[t][l + 1][i]; }

// Column segments of the fused q/k/v + gate projection launch: about 256
// four-column blocks (one per thread) per work-group, at most
// kMaxIfSegments partial planes.
int if_segments(int inner) {
  const int nb = inner / 4;
  int sg = std::min(kMaxIfSegments, std::max(1, nb / 256));
  while (sg > 1 && nb % sg != 0) --sg;
  return sg;
}

// The matrix-state leaf of tower t (-1: none).
int matrix_leaf(int t) {
  return t == kXLSTM ? XS_L_C : t == kMamba2 ? MS_SSM : t == kRetNet ? RS_S : -1;
}

// Layout and write-back log of tower t's matrix state at layer l (the scan
// operands are the caller's).
MatScanDesc mat_state_desc(const Engine& e, int t, int l) {
  const Dims& d = e.d;
  const int leaf = matrix_leaf(t);
  MatScanDesc m;
  m.state = e.state[t][l][leaf];
  m.slot_stride = e.leaf_elems[t][leaf];
  if (t == kXLSTM) {
    m.rows = m.cols = d.hs_m;
    m.heads = d.nh;
  } else if (t == kMamba2) {
    // SSM state stored [head][c][h]: tile rows are the contracted bc axis.
    m.rows = d.bc;
    m.cols = d.hm;
    m.heads = d.nhm;
  } else {
    m.rows = m.cols = d.hs_r;
    m.heads = d.nh;
  }
  m.row_stride = m.cols;
  m.col_stride = 1;
  m.head_stride = (int64_t)m.rows * m.cols;
  const Engine::MatLog& lg = e.mlog[t][l];
  m.log_hdr = lg.hdr;
  m.log_b = lg.b;
  m.log_g = lg.g;
  m.log_cap = lg.hdr ? kLogCap : 0;
  return m;
}

int row_parts(const Runs& r, int rows) {
  if (r.max_len < kRowSplitMinLen) return 1;
  int p = kMaxRowParts;
  while (p > 1 && rows % (4 * p) != 0) p /= 2;
  return p;
}

int timed_mat_scan(Engine& e, int kind, const MatScanDesc& m, hipStream_t s) {
  return timed(e, kind, s, [&] { return launch_mat_scan(m, s); });
}
const float* F32(Engine& e, int t, int l, int i) {
  return static_cast<const float*>(e.slots[t][l + 1][i].ptr);
}

// A group of consecutive runs of the tick handled as a batch of its own: its
// rows are rows row0 .. row0 + r.n_rows - 1 of the tick, and r.run_off,
// act_dev and act count from its first row and run.
struct Group {
  Runs r;
  const int* act_dev = nullptr;  // [steps] runs of the group active per step
  std::vector<int> act;          // host copy
  int row0 = 0;
};

// Ordering of a persistent sLSTM launch against another group's: wait for
// `wait` (if any) before it, record `rec` (if any) after it.
struct SlOrder {
  hipEvent_t wait = nullptr;
  hipEvent_t rec = nullptr;
};

int run_xlstm(Engine& e, TowerWS& w, int l, const Group& g, unsigned long long* xch,
              const SlOrder& ord, hipStream_t s) {
  const Dims& d = e.d;
  const Runs& r = g.r;
  const std::vector<int>& act = g.act;
  const int n = r.n_rows;
  const int H = d.H, I = d.I;
  float** st = e.state[kXLSTM][l].data();
  const int64_t* le = e.leaf_elems[kXLSTM].data();
  // sLSTM block (model/xlstm.py:400-424); its input and skip is A = norm1(x).
  // (XN = LayerNorm(A) * slstm.norm was computed with A by tower_layer.)
  HK_TRY(conv_scan(r, w.XN, H, H, st[XS_S_CONV], le[XS_S_CONV], F32(e, kXLSTM, l, X_S_CONV_W),
                   F32(e, kXLSTM, l, X_S_CONV_B), 1, w.XCA, H, s));
  // i, f from the conv path, z, o from LN(x): one launch of 4 x nh_s blocks
  HK_TRY(block_linear(e, w, w.XCA, w.XN, 2, H, F32(e, kXLSTM, l, X_S_IN_W),
                      S(e, kXLSTM, l, X_S_IN_W)->split_scale, 4, d.nh_s, d.bs_s, n,
                      w.GIN, 4 * H, s));
  if (slstm_persist_supported(H, d.nh_s)) {
    if (ord.wait) HK_CHECK_HIP(hipStreamWaitEvent(s, ord.wait, 0));
    // Each exchange buffer has its own eager tag sequence and is used by
    // one group, on one stream; a launch being captured takes a tag no other
    // launch uses.
    unsigned int tag;
    if (e.capturing) {
      tag = e.graph_tag_next++;
    } else {
      unsigned int& t = e.xch_tag[xch == e.d_xch2 ? 1 : 0];
      if (++t >= 0x80000000u) {
        // Eager tags wrapped: clear this buffer (words that could carry a
        // reused tag). Every earlier launch on it is ordered before this
        // point by stream order.
        HK_CHECK_HIP(hipMemsetAsync(xch, 0, (size_t)e.max_rows * H * 8, s));
        t = 1;
      }
      tag = t;
    }
    HK_TRY(timed(e, 3, s, [&] {
      return slstm_persist(r, g.act_dev, (int)act.size(), w.GIN, H, d.nh_s,
                           F32(e, kXLSTM, l, X_S_ST_W), F32(e, kXLSTM, l, X_S_ST_B), st[XS_S_H],
                           st[XS_S_C], st[XS_S_N], st[XS_S_M], w.SY, xch, tag, e.d_err,
                           (l == 0 && xch == e.d_xch) ? e.d_trace : nullptr, e.lowp, s);
    }));
    if (ord.rec) HK_CHECK_HIP(hipEventRecord(ord.rec, s));
  } else {
    for (size_t t = 0; t < act.size(); ++t) {
      HK_TRY(slstm_round(r, (int)t, act[t], w.GIN, H, d.nh_s, F32(e, kXLSTM, l, X_S_ST_W),
                         F32(e, kXLSTM, l, X_S_ST_B), st[XS_S_H], st[XS_S_C], st[XS_S_N],
                         st[XS_S_M], w.SY, s));
    }
    HK_TRY(slstm_final(r, w.SY, H, st[XS_S_H], s));
  }
  HK_TRY(slstm_post(w.SY, w.A.f, F32(e, kXLSTM, l, X_S_GN_W), F32(e, kXLSTM, l, X_S_GN_B), d.nh_s,
                    F32(e, kXLSTM, l, X_L_NORM), n, H, w.X1, w.XN2.f, w.XN2.l, e.lp_fmt, s));
  // mLSTM block (model/xlstm.py:298-325).
  HK_TRY(linear(e, w, w.XN2, H, {S(e, kXLSTM, l, X_L_XG_W), nullptr}, n, 2 * I, H, 0, nullptr, 0,
                w.XMG, 2 * I, nullptr, 0, s));
  const float* wqkv = F32(e, kXLSTM, l, X_L_QKV_W);
  const float k_div = (float)std::sqrt((double)d.hs_m);
  const int n_if = 2 * d.nh;
  const int segs = if_segments(I);
  ConvCommit conv_commit;
  if (mlstm_qkv_if_supported(I, n_if, segs)) {
    // the conv, q, k, v and the gate pre-activations in one launch (segment
    // partials); mlstm_post writes the conv state the runs leave
    const ConvIn conv{st[XS_L_CONV], le[XS_L_CONV], F32(e, kXLSTM, l, X_L_CONV_W),
                      F32(e, kXLSTM, l, X_L_CONV_B), r.row_pos, r.row_slot, w.XMC};
    HK_TRY(mlstm_qkv_if(conv, w.XMG, 2 * I, wqkv, wqkv + (int64_t)I * 4, wqkv + (int64_t)2 * I * 4,
                        n, I, k_div, F32(e, kXLSTM, l, X_L_IF_W), F32(e, kXLSTM, l, X_L_IF_B), n_if,
                        w.QKV, w.KS, w.IF, segs, s));
    conv_commit = ConvCommit{st[XS_L_CONV], le[XS_L_CONV], r.row_pos, r.row_slot, w.XMG, 2 * I};
    HK_TRY(mlstm_gates(r, w.IF, segs, (int64_t)n * n_if, d.nh, w.QKV, I, w.KS, st[XS_L_N],
                       st[XS_L_M], w.IG, w.FG, w.DEN, s));
  } else {
    HK_TRY(conv_scan(r, w.XMG, 2 * I, I, st[XS_L_CONV], le[XS_L_CONV],
                     F32(e, kXLSTM, l, X_L_CONV_W), F32(e, kXLSTM, l, X_L_CONV_B), 1, w.XMC, I, s));
    HK_TRY(mlstm_qkv(w.XMC, w.XMG, 2 * I, wqkv, wqkv + (int64_t)I * 4, wqkv + (int64_t)2 * I * 4,
                     n, I, 4, k_div, w.QKV, w.KS, s));
    HK_TRY(linear(e, w, Act{w.QKV, nullptr}, 3 * I,
                  {S(e, kXLSTM, l, X_L_IF_W), S(e, kXLSTM, l, X_L_IF_B)}, n, n_if, 3 * I, 0,
                  nullptr, 0, w.IF, n_if, nullptr, 0, s));
    HK_TRY(mlstm_gates(r, w.IF, 1, 0, d.nh, w.QKV, I, w.KS, st[XS_L_N], st[XS_L_M], w.IG, w.FG,
                       w.DEN, s));
  }
  MatScanDesc m = mat_state_desc(e, kXLSTM, l);
  m.slot_ids = r.slot_ids;
  m.run_off = r.run_off;
  m.n_runs = r.n_runs;
  m.alpha = {w.FG, d.nh, 1};
  m.scale = {w.IG, d.nh, 1};
  m.beta = {w.KS, I, d.hs_m};
  m.gamma = {w.QKV + 2 * I, 3 * I, d.hs_m};
  m.w = {w.QKV, 3 * I, d.hs_m};
  m.out = w.NUM;
  m.out_row_stride = I;
  m.out_head_stride = d.hs_m;
  m.row_parts = row_parts(r, d.hs_m);
  m.out_part_stride = (int64_t)n * I;
  HK_TRY(timed_mat_scan(e, 0, m, s));
  HK_TRY(mlstm_post(w.NUM, m.row_parts, m.out_part_stride, w.DEN, d.nh, F32(e, kXLSTM, l, X_L_GN_W), F32(e, kXLSTM, l, X_L_GN_B),
                    F32(e, kXLSTM, l, X_L_SKIP), w.XMC, w.XMG + I, 2 * I, n, I, d.nh, w.HS.f,
                    w.HS.l, e.lp_fmt, log_commit_of(m), conv_commit, s));
  HK_TRY(linear(e, w, w.HS, I, {S(e, kXLSTM, l, X_L_DOWN_W), nullptr}, n, H, I, 0, w.X1, H, w.X2,
                H, nullptr, 0, s));
  // final_norm and the Block's residual (x = final_norm(x2) + x) are applied
  // by tower_layer together with the next RMSNorm.
  return HK_OK;
}

int run_mamba2(Engine& e, int l, const Runs& r, hipStream_t s) {
  const Dims& d = e.d;
  TowerWS& w = e.ws[kMamba2];
  const int n = r.n_rows;
  const int H = d.H, I = d.Im;
  const int C = I + 2 * d.bc;
  const int W = C + I;
  float** st = e.state[kMamba2][l].data();
  const int64_t* le = e.leaf_elems[kMamba2].data();
  // model/mamba2.py:77-97
  HK_TRY(linear(e, w, w.A, H, {S(e, kMamba2, l, M_PROJ_W), nullptr}, n, W, H, 0, nullptr, 0,
                w.PROJ, W, nullptr, 0, s));
  // dt = softplus(dt_proj(x)) and decay = exp(A dt) in the GEMM's epilogue
  HK_TRY(linear(e, w, Act{w.A.f, nullptr}, H, {S(e, kMamba2, l, M_DT_W), S(e, kMamba2, l, M_DT_B)},
                n, d.nhm, H, 0, nullptr, 0, w.DTS, d.nhm, nullptr, 0, s,
                F32(e, kMamba2, l, M_A), w.DEC));
  HK_TRY(conv_scan(r, w.PROJ, W, C, st[MS_CONV], le[MS_CONV], F32(e, kMamba2, l, M_CONV_W),
                   F32(e, kMamba2, l, M_CONV_B), 1, w.MXC, C, s));
  MatScanDesc m = mat_state_desc(e, kMamba2, l);
  m.slot_ids = r.slot_ids;
  m.run_off = r.run_off;
  m.n_runs = r.n_runs;
  m.alpha = {w.DEC, d.nhm, 1};
  m.scale = {w.DTS, d.nhm, 1};
  m.beta = {w.MXC + I, C, 0};
  m.gamma = {w.MXC, C, d.hm};
  m.w = {w.MXC + I + d.bc, C, 0};
  m.out = w.YS;
  m.out_row_stride = I;
  m.out_head_stride = d.hm;
  // (not split: the 128-row tile leaves too little work per part, and this
  // tower's stream is not the one that ends the tick)
  m.out_part_stride = (int64_t)n * I;
  HK_TRY(timed_mat_scan(e, 1, m, s));
  HK_TRY(mamba2_post(w.YS, m.row_parts, m.out_part_stride, w.MXC, C, w.PROJ + C, W, F32(e, kMamba2, l, M_D),
                     F32(e, kMamba2, l, M_NORM), n, I, d.hm, w.YN.f, w.YN.l, e.lp_fmt,
                     log_commit_of(m), s));
  HK_TRY(linear(e, w, w.YN, I, {S(e, kMamba2, l, M_OUT_W), nullptr}, n, H, I, 0, w.X.f, H, w.X.f,
                H, nullptr, 0, s));
  return HK_OK;
}

int run_retnet(Engine& e, int l, const Runs& r, hipStream_t s) {
  const Dims& d = e.d;
  TowerWS& w = e.ws[kRetNet];
  const int n = r.n_rows;
  const int H = d.H;
  float** st = e.state[kRetNet][l].data();
  const int64_t* le = e.leaf_elems[kRetNet].data();
  // model/retnet.py:234-269
  HK_TRY(linear(e, w, w.A, H, {S(e, kRetNet, l, R_QKVG_W), nullptr}, n, 4 * H, H, 0, nullptr, 0,
                w.QKVG, 4 * H, nullptr, 0, s));
  const float scaling = (float)std::pow((double)d.hs_r, -0.5);
  HK_TRY(retnet_prep(r, w.QKVG, 4 * H, H, d.nh, scaling, F32(e, kRetNet, l, R_ANGLE),
                     F32(e, kRetNet, l, R_DECAY), reinterpret_cast<int*>(st[RS_OFF]),
                     st[RS_SCALE], w.KR, w.QS, s));
  MatScanDesc m = mat_state_desc(e, kRetNet, l);
  m.slot_ids = r.slot_ids;
  m.run_off = r.run_off;
  m.n_runs = r.n_runs;
  m.alpha = {F32(e, kRetNet, l, R_DECAY), 0, 1};
  m.beta = {w.KR, H, d.hs_r};
  m.gamma = {w.QKVG + 2 * H, 4 * H, d.hs_r};
  m.w = {w.QS, H, d.hs_r};
  m.out = w.O;
  m.out_row_stride = H;
  m.out_head_stride = d.hs_r;
  m.row_parts = row_parts(r, d.hs_r);
  m.out_part_stride = (int64_t)n * H;
  HK_TRY(timed_mat_scan(e, 2, m, s));
  // the slots' offsets and scales advance after every reader (retnet_prep)
  const RetnetAdvance adv{r.slot_ids, r.run_off, r.n_runs, d.nh, F32(e, kRetNet, l, R_DECAY),
                          reinterpret_cast<int*>(st[RS_OFF]), st[RS_SCALE]};
  HK_TRY(retnet_post(w.O, m.row_parts, m.out_part_stride, w.QKVG + 3 * H, 4 * H, n, H, d.hs_r,
                     w.YO.f, w.YO.l, e.lp_fmt, log_commit_of(m), adv, s));
  HK_TRY(linear(e, w, w.YO, H, {S(e, kRetNet, l, R_OUT_W), nullptr}, n, H, H, 0, w.X.f, H, w.X.f,
                H, nullptr, 0, s));
  return HK_OK;
}

int run_hawk(Engine& e, int l, const Runs& r, hipStream_t s) {
  const Dims& d = e.d;
  TowerWS& w = e.ws[kHawk];
  const int n = r.n_rows;
  const int H = d.H;
  float** st = e.state[kHawk][l].data();
  const int64_t* le = e.leaf_elems[kHawk].data();
  // model/hawk.py:77-84; GRP = [gate | recurrent]
  HK_TRY(linear(e, w, w.A, H, {S(e, kHawk, l, K_PROJ_W), nullptr}, n, 2 * H, H, 0, nullptr, 0,
                w.GRP, 2 * H, nullptr, 0, s));
  HK_TRY(conv_scan(r, w.GRP + H, 2 * H, H, st[KS_CONV], le[KS_CONV], F32(e, kHawk, l, K_CONV_W),
                   F32(e, kHawk, l, K_CONV_B), 0, w.KXC, H, s));
  // input and recurrence gates of the RG-LRU, one launch of 2 x nb_h blocks
  HK_TRY(block_linear(e, w, w.KXC, nullptr, 0, H, F32(e, kHawk, l, K_GATES_W),
                      S(e, kHawk, l, K_GATES_W)->split_scale, 2, d.nb_h, d.bs_h,
                      n, w.GATES, 2 * H, s));
  HK_TRY(rglru_scan(r, w.KXC, w.GATES, w.GATES + H, 2 * H, w.GRP, 2 * H, F32(e, kHawk, l, K_A),
                    8.0f, H, st[KS_H], w.GH.f, w.GH.l, e.lp_fmt, s));
  HK_TRY(linear(e, w, w.GH, H, {S(e, kHawk, l, K_OUT_W), nullptr}, n, H, H, 0, w.X.f, H, w.X.f, H,
                nullptr, 0, s));
  return HK_OK;
}

// input_up -> relu -> input_down (model/inference_model.py:88-90)
int tower_head(Engine& e, int t, TowerWS& w, const Group& g, hipStream_t s) {
  const Dims& d = e.d;
  const int n = g.r.n_rows;
  const int64_t off = (int64_t)g.row0 * d.Fpad;
  const Act fe{e.FE.f ? e.FE.f + off : nullptr, e.FE.l ? e.FE.l + off : nullptr};
  HK_TRY(linear(e, w, fe, d.Fpad, {S(e, t, -1, T_UP_W), S(e, t, -1, T_UP_B)}, n, d.P, d.Fpad, 1,
                nullptr, 0, w.H1.f, d.P, w.H1.l, d.P, s));
  return linear(e, w, w.H1, d.P, {S(e, t, -1, T_DOWN_W), S(e, t, -1, T_DOWN_B)}, n, d.H, d.P, 0,
                nullptr, 0, w.X.f, d.H, nullptr, 0, s);
}

// Block l (model/inference_model.py:63-68).
int tower_layer(Engine& e, int t, TowerWS& w, const Group& g, int l, unsigned long long* xch,
                const SlOrder& ord, hipStream_t s) {
  const Dims& d = e.d;
  const int n = g.r.n_rows;
  const int H = d.H, P = d.P;
  constexpr float kRmsEps = 1.1920928955078125e-07f;  // torch.finfo(float32).eps
  if (t == kXLSTM) {
    // A = RMSNorm(x); XN = slstm.norm(A) (model/xlstm.py:314)
    HK_TRY(rms_ln_rows(w.X.f, F32(e, t, l, B_NORM1), kRmsEps, F32(e, t, l, X_S_NORM), n, H, w.A.f,
                       w.A.l, e.lp_fmt, w.XN, s));
  } else {
    HK_TRY(rmsnorm_rows(w.X.f, H, F32(e, t, l, B_NORM1), kRmsEps, n, H, w.A.f, H, w.A.l, e.lp_fmt, H, s));
  }
  switch (t) {
    case kXLSTM: HK_TRY(run_xlstm(e, w, l, g, xch, ord, s)); break;
    case kMamba2: HK_TRY(run_mamba2(e, l, g.r, s)); break;
    case kRetNet: HK_TRY(run_retnet(e, l, g.r, s)); break;
    default: HK_TRY(run_hawk(e, l, g.r, s)); break;
  }
  if (t == kXLSTM) {
    // x = final_norm(x2) + x (model/xlstm.py:365, inference_model.py:66); A = RMSNorm(x)
    HK_TRY(ln_res_rms_rows(w.X2, F32(e, t, l, X_F_NORM), w.X.f, F32(e, t, l, B_NORM2), kRmsEps, n,
                           H, w.A.f, w.A.l, e.lp_fmt, s));
  } else {
    HK_TRY(rmsnorm_rows(w.X.f, H, F32(e, t, l, B_NORM2), kRmsEps, n, H, w.A.f, H, w.A.l, e.lp_fmt, H, s));
  }
  HK_TRY(linear(e, w, w.A, H, {S(e, t, l, B_FC1_W), S(e, t, l, B_FC1_B)}, n, P, H, 1, nullptr, 0,
                w.H1.f, P, w.H1.l, P, s));
  return linear(e, w, w.H1, P, {S(e, t, l, B_FC2_W), S(e, t, l, B_FC2_B)}, n, H, P, 0, w.X.f, H,
                w.X.f, H, nullptr, 0, s);
}

// Shared output_proj into column t of preds (model/inference_model.py:142).
int tower_tail(Engine& e, int t, TowerWS& w, const Group& g, float* preds, hipStream_t s) {
  return output_proj(w.X.f, static_cast<const float*>(e.gslots[G_OUT_W].ptr),
                     static_cast<const float*>(e.gslots[G_OUT_B].ptr), g.r.n_rows, e.d.H,
                     preds + (int64_t)g.row0 * kTowers, kTowers, t, s);
}

// Every tower of the tick, enqueued layer by layer: the xLSTM on the caller's
// stream s (run group g1) and, when split, side[0] (group g2); Mamba2 on
// side[1]; RetNet and Hawk on side[2].
// - The two xLSTM groups' persistent sLSTM launches alternate (g2 layer l
//   after g1 layer l-1, g1 layer l after g2 layer l), so two persistent
//   launches never compete for co-residency.
// (Pacing the side towers' layers to the xLSTM's, so that their HBM traffic
// spreads over the whole tick, measured no faster: the sLSTM chain then
// meets the same traffic later.)
int run_towers(Engine& e, const Group& all, const Group& g1, const Group* g2, hipStream_t s,
                     float* preds) {
  TowerWS& w1 = e.ws[kXLSTM];
  TowerWS& w2 = e.ws_x2;
  HK_TRY(tower_head(e, kMamba2, e.ws[kMamba2], all, e.side[1]));
  HK_TRY(tower_head(e, kRetNet, e.ws[kRetNet], all, e.side[2]));
  HK_TRY(tower_head(e, kHawk, e.ws[kHawk], all, e.side[2]));
  HK_TRY(tower_head(e, kXLSTM, w1, g1, s));
  if (g2) HK_TRY(tower_head(e, kXLSTM, w2, *g2, e.side[0]));
  for (int l = 0; l < e.d.D; ++l) {
    if (g2) {
      // The groups' persistent sLSTM launches run side by side when two fit
      // on the device at once, else they alternate layer by layer.
      const bool alt = !e.sl_overlap;
      SlOrder o2{alt && l > 0 ? e.sl_ev[0][l - 1] : nullptr, alt ? e.sl_ev[1][l] : nullptr};
      HK_TRY(tower_layer(e, kXLSTM, w2, *g2, l, e.d_xch2, o2, e.side[0]));
      SlOrder o1{alt ? e.sl_ev[1][l] : nullptr, alt ? e.sl_ev[0][l] : nullptr};
      HK_TRY(tower_layer(e, kXLSTM, w1, g1, l, e.d_xch, o1, s));
    } else {
      HK_TRY(tower_layer(e, kXLSTM, w1, g1, l, e.d_xch, SlOrder{}, s));
    }
    HK_TRY(tower_layer(e, kMamba2, e.ws[kMamba2], all, l, nullptr, SlOrder{}, e.side[1]));
    HK_TRY(tower_layer(e, kRetNet, e.ws[kRetNet], all, l, nullptr, SlOrder{}, e.side[2]));
    HK_TRY(tower_layer(e, kHawk, e.ws[kHawk], all, l, nullptr, SlOrder{}, e.side[2]));
  }
  HK_TRY(tower_tail(e, kMamba2, e.ws[kMamba2], all, preds, e.side[1]));
  HK_TRY(tower_tail(e, kRetNet, e.ws[kRetNet], all, preds, e.side[2]));
  HK_TRY(tower_tail(e, kHawk, e.ws[kHawk], all, preds, e.side[2]));
  HK_TRY(tower_tail(e, kXLSTM, w1, g1, preds, s));
  if (g2) HK_TRY(tower_tail(e, kXLSTM, w2, *g2, preds, e.side[0]));
  return HK_OK;
}

// One xLSTM run group's tower on stream s.
int xlstm_stream(Engine& e, TowerWS& w, const Group& g, unsigned long long* xch, float* preds,
                 hipStream_t s) {
  HK_TRY(tower_head(e, kXLSTM, w, g, s));
  for (int l = 0; l < e.d.D; ++l) HK_TRY(tower_layer(e, kXLSTM, w, g, l, xch, SlOrder{}, s));
  return tower_tail(e, kXLSTM, w, g, preds, s);
}

// Mamba2 on side[1].
int mamba2_stream(Engine& e, const Group& all, float* preds) {
  hipStream_t s = e.side[1];
  TowerWS& w = e.ws[kMamba2];
  HK_TRY(tower_head(e, kMamba2, w, all, s));
  for (int l = 0; l < e.d.D; ++l) HK_TRY(tower_layer(e, kMamba2, w, all, l, nullptr, SlOrder{}, s));
  return tower_tail(e, kMamba2, w, all, preds, s);
}

// RetNet and Hawk, layer by layer, on side[2].
int retnet_hawk_stream(Engine& e, const Group& all, float* preds) {
  hipStream_t s = e.side[2];
  HK_TRY(tower_head(e, kRetNet, e.ws[kRetNet], all, s));
  HK_TRY(tower_head(e, kHawk, e.ws[kHawk], all, s));
  for (int l = 0; l < e.d.D; ++l) {
    HK_TRY(tower_layer(e, kRetNet, e.ws[kRetNet], all, l, nullptr, SlOrder{}, s));
    HK_TRY(tower_layer(e, kHawk, e.ws[kHawk], all, l, nullptr, SlOrder{}, s));
  }
  HK_TRY(tower_tail(e, kRetNet, e.ws[kRetNet], all, preds, s));
  return tower_tail(e, kHawk, e.ws[kHawk], all, preds, s);
}

// The work of run_towers with each side stream's launches enqueued by a
// thread of its own while this thread enqueues the first xLSTM group's. Only
// for ticks whose streams need no cross-stream order inside the tick (the
// two groups' persistent sLSTM launches fit side by side); the enqueue order
// within each stream is run_towers'. Returns 1 (nothing enqueued) when the
// threads cannot be started.
int run_towers_mt(Engine& e, const Group& all, const Group& g1, const Group* g2, hipStream_t s,
                  float* preds) {
  if (!e.pool) {
    try {
      e.pool = std::make_unique<EnqueuePool>(e.device, Engine::kSide);
    } catch (...) {
      return 1;
    }
  }
  EnqueuePool& p = *e.pool;
  if (g2) p.post(0, [&] { return xlstm_stream(e, e.ws_x2, *g2, e.d_xch2, preds, e.side[0]); });
  p.post(1, [&] { return mamba2_stream(e, all, preds); });
  p.post(2, [&] { return retnet_hawk_stream(e, all, preds); });
  const int st = xlstm_stream(e, e.ws[kXLSTM], g1, e.d_xch, preds, s);
  std::string err;
  const int wst = p.wait(&err);  // the threads use e, all, g1, g2 until here
  if (st != HK_OK) return st;
  if (wst != HK_OK) set_error("%s", err.c_str());
  return wst;
}

// Where to split the length-sorted runs into two xLSTM groups (returns
// n_runs for no split). Per layer a group costs about kStepUs per sLSTM step
// of its longest run plus kSymbolUs per symbol for the mLSTM state traffic;
// the two groups run concurrently, but each reads every weight of the layer
// (weight_us, the layer's weight bytes at 5 TB/s), so a split pays when the
// larger of the two costs plus that second read is well below the unsplit
// cost. (Four one-request symbols in fp32 (C1): unsplit 23 us against 13 +
// 41 split, measured 3.90 against 4.10 ms per step; 256 Zipf requests in
// bf16 (C4): about 1000 against 500 + 24.)
int xlstm_split_point(const int* run_off, int n_runs, double weight_us) {
  constexpr double kStepUs = 3.0, kSymbolUs = 5.0, kGain = 0.8;
  if (n_runs < 2) return n_runs;
  const int len0 = run_off[1] - run_off[0];
  const double whole = kStepUs * len0 + kSymbolUs * n_runs;
  double best = whole;
  int best_k = n_runs;
  for (int k = 1; k < n_runs; ++k) {
    const int lenk = run_off[k + 1] - run_off[k];
    const double c = std::max(kStepUs * len0 + kSymbolUs * k,
                              kStepUs * lenk + kSymbolUs * (n_runs - k)) +
                     weight_us;
    if (c < best) {
      best = c;
      best_k = k;
    }
  }
  return best < kGain * whole ? best_k : n_runs;
}

// What a tick's device work depends on besides its buffers: the run
// layout (counts, the xLSTM groups) and the per-step active-run counts.
struct TickShape {
  int n_runs = 0, n_rows = 0, steps = 0;
  int split = 0, row_split = 0, steps2 = 0;
  std::vector<int> act, act1, act2;
};

// The device work of one tick on stream s, descriptors already in d_desc:
// feature staging, every tower (forked to the side streams and joined back),
// predictions into preds_dev.
int enqueue_tick(Engine& e, const TickShape& sh, const float* features_dev, float* preds_dev,
                 hipStream_t s) {
  Group all;
  all.r = Runs{e.d_slots, e.d_off, sh.n_runs, sh.n_rows, sh.steps, e.d_pos, e.d_rslot};
  all.act_dev = e.d_act;
  all.act = sh.act;
  HK_TRY(stage_features(features_dev, sh.n_rows, e.d.F, e.d.Fpad, e.FE.f, e.FE.l, e.lp_fmt, s));
  HK_CHECK_HIP(hipEventRecord(e.fork_ev, s));
  for (int i = 0; i < Engine::kSide; ++i) HK_CHECK_HIP(hipStreamWaitEvent(e.side[i], e.fork_ev, 0));
  const bool split = sh.split < sh.n_runs;
  Group g1, g2;
  if (split) {
    g1.r = Runs{e.d_slots, e.d_off, sh.split, sh.row_split, sh.steps, e.d_pos, e.d_rslot};
    g1.act_dev = e.d_act1;
    g1.act = sh.act1;
    g2.r = Runs{e.d_slots + sh.split, e.d_off2, sh.n_runs - sh.split, sh.n_rows - sh.row_split,
                sh.steps2, e.d_pos + sh.row_split, e.d_rslot + sh.row_split};
    g2.act_dev = e.d_act2;
    g2.act = sh.act2;
    g2.row0 = sh.row_split;
  }
  const Group& first = split ? g1 : all;
  const Group* second = split ? &g2 : nullptr;
  // Threads enqueue the streams' launches unless the tick is being captured
  // or profiled, or the groups' sLSTM launches alternate across streams.
  int st = 1;
  if (!e.capturing && e.prof == 0 && e.d_trace == nullptr && (!split || e.sl_overlap))
    st = run_towers_mt(e, all, first, second, s, preds_dev);
  if (st == 1) st = run_towers(e, all, first, second, s, preds_dev);
  HK_TRY(st);
  for (int i = 0; i < Engine::kSide; ++i) {
    HK_CHECK_HIP(hipEventRecord(e.join_ev[i], e.side[i]));
    HK_CHECK_HIP(hipStreamWaitEvent(s, e.join_ev[i], 0));
  }
  return HK_OK;
}

// Captures one tick of shape sh (features from g_feat, predictions to
// g_pred) into an executable graph.
int capture_tick(Engine& e, const TickShape& sh, hipGraphExec_t* out) {
  *out = nullptr;
  HK_CHECK_HIP(hipStreamBeginCapture(e.cap_s, hipStreamCaptureModeRelaxed));
  e.capturing = true;
  const int st = enqueue_tick(e, sh, e.g_feat, e.g_pred, e.cap_s);
  e.capturing = false;
  hipGraph_t graph = nullptr;
  const hipError_t end = hipStreamEndCapture(e.cap_s, &graph);
  if (st != HK_OK) {
    if (graph) (void)hipGraphDestroy(graph);
    return st;
  }
  if (end != hipSuccess) {
    set_error("capture_tick: hipStreamEndCapture: %s", hipGetErrorString(end));
    return HK_ERR_HIP;
  }
  const hipError_t inst = hipGraphInstantiate(out, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (inst != hipSuccess) {
    set_error("capture_tick: hipGraphInstantiate: %s", hipGetErrorString(inst));
    return HK_ERR_HIP;
  }
  return HK_OK;
}

// A tick through the graph cache: features into g_feat, one graph launch
// (captured on first sight of the shape), predictions out of g_pred, all on
// stream s.
int tick_replay(Engine& e, const std::vector<int>& key, const TickShape& sh,
                const float* features_dev, float* preds_dev, hipStream_t s) {
  auto it = e.graphs.find(key);
  if (it == e.graphs.end()) {
    // Two captures consume at most 2 * 2 * depth tags.
    if (e.graph_tag_next > 0xFFFFFFFFu - 4u * (unsigned)e.d.D - 4u)
      return enqueue_tick(e, sh, features_dev, preds_dev, s);  // tags exhausted: eager
    if ((int)e.graphs.size() >= e.graph_cap) {
      auto lru = e.graphs.begin();
      for (auto j = e.graphs.begin(); j != e.graphs.end(); ++j)
        if (j->second.last_use < lru->second.last_use) lru = j;
      // its last replay must be done before the executable goes
      HK_CHECK_HIP(hipStreamSynchronize(s));
      for (auto& x : lru->second.exec)
        if (x) HK_CHECK_HIP(hipGraphExecDestroy(x));
      e.graphs.erase(lru);
    }
    Engine::GraphEntry g;
    for (int p = 0; p < 2; ++p) {
      const int st = capture_tick(e, sh, &g.exec[p]);
      if (st != HK_OK) {
        for (auto& x : g.exec)
          if (x) (void)hipGraphExecDestroy(x);
        return st;
      }
      ++e.graph_captures;
    }
    it = e.graphs.emplace(key, g).first;
  }
  Engine::GraphEntry& g = it->second;
  g.last_use = ++e.graph_clock;
  HK_CHECK_HIP(hipMemcpyAsync(e.g_feat, features_dev, (size_t)sh.n_rows * e.d.F * 4,
                              hipMemcpyDeviceToDevice, s));
  HK_CHECK_HIP(hipGraphLaunch(g.exec[g.next], s));
  g.next ^= 1;
  ++e.graph_replays;
  HK_CHECK_HIP(hipMemcpyAsync(preds_dev, e.g_pred, (size_t)sh.n_rows * kTowers * 4,
                              hipMemcpyDeviceToDevice, s));
  return HK_OK;
}

Slot* find_slot(Engine& e, int tower, int layer, int slot) {
  if (tower == -1) {
    if (layer != -1 || slot < 0 || slot >= (int)e.gslots.size()) return nullptr;
    return &e.gslots[slot];
  }
  if (tower < 0 || tower >= kTowers || layer < -1 || layer >= e.d.D) return nullptr;
  auto& v = e.slots[tower][layer + 1];
  if (slot < 0 || slot >= (int)v.size()) return nullptr;
  return &v[slot];
}

}  // namespace
}  // namespace hk

using hk::Engine;

extern "C" {

// cfg: hidden, proj, depth, heads, features, mamba_head, mamba_bc, capacity,
//      max_rows, max_runs, lp (0 fp32, 1 bf16, 2 fp16 CastLinear)
int hk_engine_create(const int* cfg, int n_cfg, void** out) {
  HK_REQUIRE(cfg && out && n_cfg == 11, "hk_engine_create: expected 11 config ints");
  *out = nullptr;
  auto e = std::make_unique<Engine>();
  hk::Dims& d = e->d;
  d.H = cfg[0];
  d.P = cfg[1];
  d.D = cfg[2];
  d.nh = cfg[3];
  d.F = cfg[4];
  d.hm = cfg[5];
  d.bc = cfg[6];
  e->capacity = cfg[7];
  e->max_rows = cfg[8];
  e->max_runs = cfg[9];
  HK_REQUIRE(cfg[10] >= 0 && cfg[10] <= 2, "hk_engine_create: lp must be 0 (fp32), 1 (bf16) or 2 (fp16)");
  e->lowp = cfg[10] != 0;
  e->lp_fmt = cfg[10] == 2 ? hk::kLpF16 : hk::kLpBF16;
  HK_REQUIRE(d.H > 0 && d.P > 0 && d.D > 0 && d.nh > 0 && d.F > 0 && d.hm > 0 && d.bc > 0,
             "hk_engine_create: non-positive dimension");
  HK_REQUIRE(e->capacity > 0 && e->max_rows > 0 && e->max_runs > 0,
             "hk_engine_create: capacity, max_rows and max_runs must be positive");
  d.Fpad = (int)hk::round_up(d.F, 64);
  d.nh_s = d.nh / 2;
  HK_REQUIRE(d.nh_s >= 1 && d.H % d.nh_s == 0, "sLSTM heads (heads/2) must divide hidden");
  d.bs_s = d.H / d.nh_s;
  d.I = 2 * d.H;
  HK_REQUIRE(d.I % d.nh == 0, "heads must divide 2*hidden");
  d.hs_m = d.I / d.nh;
  d.Im = 2 * d.H;
  HK_REQUIRE(d.Im % d.hm == 0, "mamba head size must divide 2*hidden");
  d.nhm = d.Im / d.hm;
  HK_REQUIRE(d.H % d.nh == 0 && (d.H / d.nh) % 2 == 0, "heads must divide hidden evenly");
  d.hs_r = d.H / d.nh;
  d.nb_h = 4;
  HK_REQUIRE(d.H % 4 == 0, "hidden must be a multiple of 4");
  d.bs_h = d.H / 4;
  HK_REQUIRE(d.bs_s % 16 == 0 && d.bs_h % 16 == 0 && d.H % 16 == 0,
             "block sizes must be multiples of 16 (fp32 MFMA K tile)");
  HK_REQUIRE(d.hs_m <= 512 && d.hs_r <= 512 && d.bc <= 512 && d.nh <= 16 && d.nh_s <= 16,
             "head sizes above 512 or more than 16 heads are not supported");
  HK_REQUIRE(d.bs_s <= 1008, "sLSTM head size too large for LDS staging");

  // weights
  e->slots.resize(hk::kTowers);
  for (int t = 0; t < hk::kTowers; ++t) {
    e->slots[t].resize(d.D + 1);
    for (auto& def : hk::tower_slots(d)) e->slots[t][0].push_back(hk::Slot{def});
    for (int l = 0; l < d.D; ++l)
      for (auto& def : hk::block_slots(d, t)) e->slots[t][l + 1].push_back(hk::Slot{def});
  }
  for (auto& def : hk::global_slots(d)) e->gslots.push_back(hk::Slot{def});
  auto alloc_slot = [&](hk::Slot& s) -> bool {
    const bool lp = s.def.lp && e->lowp;
    const size_t bytes = (size_t)s.def.numel * (lp ? 2 : 4);
    // CastLinear weights of a packable shape are stored packed for the
    // matrix cores (every engine shape is; the checks keep odd widths on the
    // row-major path).
    s.packed = lp && s.def.k > 0 && s.def.numel % s.def.k == 0 &&
               hk::packable((int)(s.def.numel / s.def.k), s.def.k);
    s.ptr = e->alloc_bytes(bytes);
    return s.ptr != nullptr;
  };
  for (auto& tv : e->slots)
    for (auto& lv : tv)
      for (auto& s : lv)
        if (!alloc_slot(s)) {
          hk::set_error("hk_engine_create: out of device memory for weights");
          return HK_ERR_HIP;
        }
  {
    double bytes = 0.0;
    for (const auto& s : e->slots[hk::kXLSTM][1])
      bytes += (double)s.def.numel * (s.def.lp && e->lowp ? 2 : 4);
    e->x_weight_us = bytes / 5.0e6;
  }
  for (auto& s : e->gslots)
    if (!alloc_slot(s)) {
      hk::set_error("hk_engine_create: out of device memory for weights");
      return HK_ERR_HIP;
    }

  // state store
  e->state.resize(hk::kTowers);
  e->leaf_elems.resize(hk::kTowers);
  for (int t = 0; t < hk::kTowers; ++t) {
    e->leaf_elems[t] = hk::state_leaves(d, t);
    e->state[t].resize(d.D);
    for (int l = 0; l < d.D; ++l) {
      for (int64_t per : e->leaf_elems[t]) {
        float* p = e->alloc_f(per * e->capacity);
        if (!p) {
          hk::set_error("hk_engine_create: out of device memory for the state store "
                        "(%d slots)", e->capacity);
          return HK_ERR_HIP;
        }
        e->state[t][l].push_back(p);
      }
    }
  }
  // write-back logs of the matrix states, empty
  e->mlog.assign(hk::kTowers, std::vector<Engine::MatLog>(d.D));
  for (int t = 0; t < hk::kTowers; ++t) {
    if (hk::matrix_leaf(t) < 0) continue;
    for (int l = 0; l < d.D; ++l) {
      hk::MatScanDesc m = hk::mat_state_desc(*e, t, l);  // layout (no log yet)
      const int64_t per_head = (int64_t)e->capacity * m.heads;
      Engine::MatLog& lg = e->mlog[t][l];
      lg.hdr = e->alloc_f(per_head * hk::kLogHdr);
      lg.b = e->alloc_f(per_head * hk::kLogCap * m.rows);
      lg.g = e->alloc_f(per_head * hk::kLogCap * m.cols);
      if (!lg.hdr || !lg.b || !lg.g) {
        hk::set_error("hk_engine_create: out of device memory for the write-back logs");
        return HK_ERR_HIP;
      }
      m = hk::mat_state_desc(*e, t, l);
      HK_TRY(hk::mat_log_clear(m, nullptr, 0, e->capacity, nullptr));
    }
  }
  HK_CHECK_HIP(hipDeviceSynchronize());
  int st = hk::build_workspace(*e);
  if (st != HK_OK) {
    hk::set_error("hk_engine_create: out of device memory for the workspace (%d rows)",
                  e->max_rows);
    return st;
  }
  e->seen.assign(e->capacity, 0);
  HK_CHECK_HIP(hipGetDevice(&e->device));
  HK_TRY(hk::scratch_on_current_device(&e->scratch));
  *out = e.release();
  return HK_OK;
}

int hk_engine_destroy(void* h) {
  if (!h) return HK_OK;
  (void)hipDeviceSynchronize();
  delete static_cast<Engine*>(h);
  return HK_OK;
}

int hk_engine_param_numel(void* h, int tower, int layer, int slot, int64_t* numel) {
  HK_REQUIRE(h && numel, "hk_engine_param_numel: null argument");
  hk::Slot* s = hk::find_slot(*static_cast<Engine*>(h), tower, layer, slot);
  HK_REQUIRE(s, "hk_engine_param_numel: no slot (%d, %d, %d)", tower, layer, slot);
  *numel = s->def.numel;
  return HK_OK;
}

// Synchronous: copies `numel` fp32 values from host memory into the slot,
// converting to the engine's 16-bit format (weights) or rounding through it
// (biases) when the slot is a reduced-precision linear and the engine runs
// in that mode.
int hk_engine_load_param(void* h, int tower, int layer, int slot, const float* host,
                         int64_t numel) {
  HK_REQUIRE(h && host, "hk_engine_load_param: null argument");
  Engine& e = *static_cast<Engine*>(h);
  hk::Slot* s = hk::find_slot(e, tower, layer, slot);
  HK_REQUIRE(s, "hk_engine_load_param: no slot (%d, %d, %d)", tower, layer, slot);
  HK_REQUIRE(numel == s->def.numel, "hk_engine_load_param: %s expects %lld values, got %lld",
             s->def.name, (long long)s->def.numel, (long long)numel);
  if (s->def.lp && e.lowp) {
    float* tmp = nullptr;
    HK_CHECK_HIP(hipMalloc(&tmp, (size_t)numel * 4));
    hipError_t err = hipMemcpy(tmp, host, (size_t)numel * 4, hipMemcpyHostToDevice);
    uint16_t* dst = static_cast<uint16_t*>(s->ptr);
    int st = err != hipSuccess ? HK_ERR_HIP
             : s->packed       ? hk::pack_f32_to_lp(tmp, dst, (int)(numel / s->def.k), s->def.k,
                                                    e.lp_fmt, nullptr)
                               : hk::to_lp(tmp, dst, numel, e.lp_fmt, nullptr);
    if (st == HK_OK) err = hipDeviceSynchronize();
    (void)hipFree(tmp);
    if (err != hipSuccess) {
      hk::set_error("hk_engine_load_param: %s", hipGetErrorString(err));
      return HK_ERR_HIP;
    }
    if (st != HK_OK) return st;
  } else if (s->def.lp_bias && e.lowp) {
    std::vector<float> v(host, host + numel);
    for (auto& x : v) x = hk::round_lp(x, e.lp_fmt);
    HK_CHECK_HIP(hipMemcpy(s->ptr, v.data(), (size_t)numel * 4, hipMemcpyHostToDevice));
  } else {
    HK_CHECK_HIP(hipMemcpy(s->ptr, host, (size_t)numel * 4, hipMemcpyHostToDevice));
    s->split_scale = hk::split_scale_of(host, numel);
  }
  s->bound = true;
  return HK_OK;
}

// hk_engine_load_param with no device allocation: CastLinear weights travel
// through this device's `scratch` array, kScratchFloats values at a time
// (copy in, convert into the slot, wait, next chunk), so a slot of any size
// binds through the 16 MiB array; biases are rounded in place in the slot and
// fp32 slots copied straight in. Calls on one device share its array; a lock
// per device serialises their staging within the process.
int hk_engine_load_param_noalloc(void* h, int tower, int layer, int slot, const float* host,
                                 int64_t numel) {
  HK_REQUIRE(h && host, "hk_engine_load_param_noalloc: null argument");
  Engine& e = *static_cast<Engine*>(h);
  hk::Slot* s = hk::find_slot(e, tower, layer, slot);
  HK_REQUIRE(s, "hk_engine_load_param_noalloc: no slot (%d, %d, %d)", tower, layer, slot);
  HK_REQUIRE(numel == s->def.numel,
             "hk_engine_load_param_noalloc: %s expects %lld values, got %lld", s->def.name,
             (long long)s->def.numel, (long long)numel);
  int dev = -1;
  HK_CHECK_HIP(hipGetDevice(&dev));
  HK_REQUIRE(dev == e.device && e.scratch != nullptr,
             "hk_engine_load_param_noalloc: the engine lives on device %d, device %d is current",
             e.device, dev);
  if (s->def.lp && e.lowp) {
    uint16_t* dst = static_cast<uint16_t*>(s->ptr);
    // A packed slot moves in whole 32-row blocks: rows r .. r + n of W fill
    // packed elements r*K .. (r + n)*K, so each chunk packs on its own.
    const int64_t K = s->def.k;
    const int64_t step = s->packed ? (hk::kScratchFloats / K) / 32 * 32 * K : hk::kScratchFloats;
    HK_REQUIRE(step > 0, "hk_engine_load_param_noalloc: %s rows do not fit the staging array",
               s->def.name);
    std::lock_guard<std::mutex> lock(hk::g_scratch_use_mu[dev]);
    auto chunks = [&]() -> int {
      for (int64_t off = 0; off < numel; off += step) {
        const int64_t n = std::min(step, numel - off);
        HK_CHECK_HIP(hipMemcpy(e.scratch, host + off, (size_t)n * 4, hipMemcpyHostToDevice));
        if (s->packed) {
          HK_TRY(hk::pack_f32_to_lp(e.scratch, dst + off, (int)(n / K), (int)K, e.lp_fmt, nullptr));
        } else {
          HK_TRY(hk::to_lp(e.scratch, dst + off, n, e.lp_fmt, nullptr));
        }
        HK_CHECK_HIP(hipStreamSynchronize(nullptr));  // the next chunk overwrites the array
      }
      return HK_OK;
    };
    const int st = chunks();
    if (st != HK_OK) {
      // a failed chunk may have left a conversion reading the array: wait
      // for it before the lock lets another binding overwrite the array
      (void)hipStreamSynchronize(nullptr);
      return st;
    }
  } else if (s->def.lp_bias && e.lowp) {
    HK_CHECK_HIP(hipMemcpy(s->ptr, host, (size_t)numel * 4, hipMemcpyHostToDevice));
    HK_TRY(hk::round_lp_inplace(static_cast<float*>(s->ptr), numel, e.lp_fmt, nullptr));
    HK_CHECK_HIP(hipStreamSynchronize(nullptr));
  } else {
    HK_CHECK_HIP(hipMemcpy(s->ptr, host, (size_t)numel * 4, hipMemcpyHostToDevice));
    s->split_scale = hk::split_scale_of(host, numel);
  }
  s->bound = true;
  return HK_OK;
}

int hk_engine_state_numel(void* h, int tower, int leaf, int64_t* per_slot) {
  HK_REQUIRE(h && per_slot, "hk_engine_state_numel: null argument");
  Engine& e = *static_cast<Engine*>(h);
  HK_REQUIRE(tower >= 0 && tower < hk::kTowers, "bad tower %d", tower);
  HK_REQUIRE(leaf >= 0 && leaf < (int)e.leaf_elems[tower].size(), "bad leaf %d", leaf);
  *per_slot = e.leaf_elems[tower][leaf];
  return HK_OK;
}

// Copies leaf `leaf` of slots [slot0, slot0+nslots) between the store and a
// device buffer (to_engine != 0: buffer -> store). Stream-ordered.
int hk_engine_state_copy(void* h, int tower, int layer, int leaf, int slot0, int nslots,
                         void* buf, int to_engine, void* stream) {
  HK_REQUIRE(h && buf, "hk_engine_state_copy: null argument");
  Engine& e = *static_cast<Engine*>(h);
  HK_REQUIRE(tower >= 0 && tower < hk::kTowers && layer >= 0 && layer < e.d.D,
             "hk_engine_state_copy: bad tower/layer");
  HK_REQUIRE(leaf >= 0 && leaf < (int)e.leaf_elems[tower].size(), "bad leaf %d", leaf);
  HK_REQUIRE(slot0 >= 0 && nslots >= 0 && slot0 + nslots <= e.capacity,
             "hk_engine_state_copy: slots out of range");
  const int64_t per = e.leaf_elems[tower][leaf];
  float* base = e.state[tower][layer][leaf] + (int64_t)slot0 * per;
  const size_t bytes = (size_t)nslots * per * 4;
  hipStream_t s = (hipStream_t)stream;
  // A matrix-state leaf with pending write-back updates is materialised
  // before it is read, and its log emptied once it is overwritten.
  const bool logged = leaf == hk::matrix_leaf(tower) && nslots > 0;
  if (to_engine) {
    HK_CHECK_HIP(hipMemcpyAsync(base, buf, bytes, hipMemcpyDeviceToDevice, s));
    if (logged) HK_TRY(hk::mat_log_clear(hk::mat_state_desc(e, tower, layer), nullptr, slot0, nslots, s));
  } else {
    if (logged) HK_TRY(hk::mat_log_flush(hk::mat_state_desc(e, tower, layer), slot0, nslots, s));
    HK_CHECK_HIP(hipMemcpyAsync(buf, base, bytes, hipMemcpyDeviceToDevice, s));
  }
  return HK_OK;
}

// Resets slots to the reference's init_state values (zeros; the sLSTM
// running max starts at -inf, model/xlstm.py:375). n < 0 resets every slot.
int hk_engine_reset_slots(void* h, const int* slots_host, int n, void* stream) {
  HK_REQUIRE(h, "hk_engine_reset_slots: null handle");
  Engine& e = *static_cast<Engine*>(h);
  hipStream_t s = (hipStream_t)stream;
  for (int t = 0; t < hk::kTowers; ++t) {
    for (int l = 0; l < e.d.D; ++l) {
      for (size_t leaf = 0; leaf < e.leaf_elems[t].size(); ++leaf) {
        const float v = (t == hk::kXLSTM && leaf == hk::XS_S_M) ? -INFINITY : 0.0f;
        const int64_t per = e.leaf_elems[t][leaf];
        float* base = e.state[t][l][leaf];
        const bool logged = (int)leaf == hk::matrix_leaf(t);
        if (n < 0) {
          HK_TRY(hk::fill_f32(base, per * e.capacity, v, s));
          if (logged) HK_TRY(hk::mat_log_clear(hk::mat_state_desc(e, t, l), nullptr, 0, e.capacity, s));
        } else {
          for (int i = 0; i < n; ++i) {
            const int slot = slots_host[i];
            HK_REQUIRE(slot >= 0 && slot < e.capacity, "reset: slot %d out of range", slot);
            HK_TRY(hk::fill_f32(base + (int64_t)slot * per, per, v, s));
            if (logged) HK_TRY(hk::mat_log_clear(hk::mat_state_desc(e, t, l), nullptr, slot, 1, s));
          }
        }
      }
    }
  }
  return HK_OK;
}

// Appends counts_host[i] zero-valued pending-update entries to every
// matrix-state log of slot slots_host[i] (up to the log capacity): the state
// the slots stand for is unchanged, while the next ticks read and write the
// log as they would after a long run of ticks. Synchronous.
int hk_engine_log_fill(void* h, const int* slots_host, const int* counts_host, int n,
                       void* stream) {
  HK_REQUIRE(h, "hk_engine_log_fill: null handle");
  Engine& e = *static_cast<Engine*>(h);
  HK_REQUIRE(n >= 0 && (n == 0 || (slots_host && counts_host)), "hk_engine_log_fill: bad arguments");
  if (n == 0) return HK_OK;
  for (int i = 0; i < n; ++i) {
    HK_REQUIRE(slots_host[i] >= 0 && slots_host[i] < e.capacity,
               "hk_engine_log_fill: slot %d out of range", slots_host[i]);
    HK_REQUIRE(counts_host[i] >= 0, "hk_engine_log_fill: negative count");
  }
  hipStream_t s = (hipStream_t)stream;
  int* buf = nullptr;
  HK_CHECK_HIP(hipMalloc(&buf, 2 * sizeof(int) * (size_t)n));
  int st = HK_OK;
  if (hipMemcpyAsync(buf, slots_host, sizeof(int) * n, hipMemcpyHostToDevice, s) != hipSuccess ||
      hipMemcpyAsync(buf + n, counts_host, sizeof(int) * n, hipMemcpyHostToDevice, s) !=
          hipSuccess) {
    hk::set_error("hk_engine_log_fill: copy failed");
    st = HK_ERR_HIP;
  }
  for (int t = 0; t < hk::kTowers && st == HK_OK; ++t) {
    if (hk::matrix_leaf(t) < 0) continue;
    for (int l = 0; l < e.d.D && st == HK_OK; ++l)
      st = hk::mat_log_fill(hk::mat_state_desc(e, t, l), buf, buf + n, n, s);
  }
  // the copies read host memory and the kernels read buf: wait before both go
  if (hipStreamSynchronize(s) != hipSuccess && st == HK_OK) {
    hk::set_error("hk_engine_log_fill: %s", hipGetErrorString(hipGetLastError()));
    st = HK_ERR_HIP;
  }
  HK_CHECK_HIP(hipFree(buf));
  return st;
}

// Waits for the work enqueued on `stream` so far (a tick ends with every side
// stream joined back into its stream, so waiting for the tick's stream waits
// for the whole tick; nothing else on the device is waited for) and reports a
// step barrier that timed out in any earlier tick (then returns -2 and clears
// the flag). The flag travels with the stream's work: one copy into pinned
// host memory, then one stream synchronisation.
int hk_engine_check(void* h, void* stream) {
  HK_REQUIRE(h, "hk_engine_check: null handle");
  Engine& e = *static_cast<Engine*>(h);
  hipStream_t s = (hipStream_t)stream;
  HK_CHECK_HIP(hipMemcpyAsync(e.h_err, e.d_err, 4, hipMemcpyDeviceToHost, s));
  HK_CHECK_HIP(hipStreamSynchronize(s));
  const int flag = *e.h_err;
  if (e.d_trace) {
    // Phases of the last tick's layer-0 sLSTM steps in microseconds
    // (s_memrealtime runs at 100 MHz), work-group 0, first chunk: poll for
    // h_{t-1}, staging barrier, product, cell update, later chunks, and the
    // gap to the next step.
    std::vector<uint64_t> tr((size_t)e.max_rows * 8);
    HK_CHECK_HIP(hipMemcpyAsync(tr.data(), e.d_trace, tr.size() * 8, hipMemcpyDeviceToHost, s));
    HK_CHECK_HIP(hipStreamSynchronize(s));
    static const char* names[6] = {"poll", "stage", "dot", "cell", "rest-chunks", "next"};
    double tot[6] = {0, 0, 0, 0, 0, 0};
    int n = 0;
    for (int t = 0; t < e.max_rows && tr[t * 8 + 5] > tr[t * 8 + 0]; ++t, ++n) {
      double ph[6];
      for (int k = 0; k < 5; ++k)
        ph[k] = tr[t * 8 + k + 1] > tr[t * 8 + k] ? (double)(tr[t * 8 + k + 1] - tr[t * 8 + k]) * 0.01 : 0.0;
      ph[5] = (t + 1 < e.max_rows && tr[(t + 1) * 8] > tr[t * 8 + 5])
                  ? (double)(tr[(t + 1) * 8] - tr[t * 8 + 5]) * 0.01 : 0.0;
      for (int k = 0; k < 6; ++k) tot[k] += ph[k];
      if (t < 3 || t % 10 == 0) {
        fprintf(stderr, "slstm step %d:", t);
        for (int k = 0; k < 6; ++k) fprintf(stderr, " %s %.2f", names[k], ph[k]);
        const uint64_t* q = &tr[t * 8];
        if (q[2] <= q[6] && q[6] <= q[7] && q[7] <= q[3])  // VALU product sub-phases
          fprintf(stderr, " [fma %.2f xbuf %.2f gsum %.2f]", (q[6] - q[2]) * 0.01,
                  (q[7] - q[6]) * 0.01, (q[3] - q[7]) * 0.01);
        fprintf(stderr, " us\n");
      }
    }
    fprintf(stderr, "slstm %d steps:", n);
    for (int k = 0; k < 6; ++k) fprintf(stderr, " %s %.1f", names[k], tot[k]);
    fprintf(stderr, " us\n");
    HK_CHECK_HIP(hipMemsetAsync(e.d_trace, 0, tr.size() * 8, s));
  }
  if (flag) {
    HK_CHECK_HIP(hipMemsetAsync(e.d_err, 0, 4, s));
    HK_CHECK_HIP(hipStreamSynchronize(s));
    hk::set_error("hk_engine_check: a kernel step barrier timed out (results invalid)");
    return HK_ERR_HIP;
  }
  return HK_OK;
}

// Per-launch timing (kind 0 mLSTM scan, 1 Mamba2 scan, 2 RetNet scan,
// 3 sLSTM recurrence, 4 GEMM): bit k of `kinds` records kind k; 0 stops.
// Clears earlier records.
int hk_engine_profile(void* h, int kinds) {
  HK_REQUIRE(h, "hk_engine_profile: null handle");
  HK_REQUIRE(kinds >= 0 && kinds < 32, "hk_engine_profile: bad kind mask %d", kinds);
  Engine& e = *static_cast<Engine*>(h);
  e.prof = kinds;
  for (auto& u : e.prof_used) u = 0;
  return HK_OK;
}

// Waits for the recorded launches of `kind` and returns their count and
// summed duration (ms); clears the records.
int hk_engine_profile_read(void* h, int kind, int* count, double* total_ms) {
  HK_REQUIRE(h && count && total_ms, "hk_engine_profile_read: null argument");
  Engine& e = *static_cast<Engine*>(h);
  HK_REQUIRE(kind >= 0 && kind < 5, "hk_engine_profile_read: bad kind %d", kind);
  double tot = 0.0;
  for (size_t i = 0; i < e.prof_used[kind]; ++i) {
    auto& pr = e.prof_ev[kind][i];
    HK_CHECK_HIP(hipEventSynchronize(pr.second));
    float ms = 0.0f;
    HK_CHECK_HIP(hipEventElapsedTime(&ms, pr.first, pr.second));
    tot += ms;
  }
  *count = (int)e.prof_used[kind];
  *total_ms = tot;
  e.prof_used[kind] = 0;
  return HK_OK;
}

// One tick. slot_ids_host[n_runs] and run_off_host[n_runs+1] describe runs
// sorted by non-increasing length; features_dev is [n_rows, features] fp32
// and preds_dev receives [n_rows, 4] (one column per tower), in row order.
int hk_engine_tick(void* h, const int* slot_ids_host, const int* run_off_host, int n_runs,
                   const float* features_dev, float* preds_dev, void* stream) {
  HK_REQUIRE(h, "hk_engine_tick: null handle");
  Engine& e = *static_cast<Engine*>(h);
  hipStream_t s = (hipStream_t)stream;
  if (n_runs == 0) return HK_OK;
  HK_REQUIRE(slot_ids_host && run_off_host && features_dev && preds_dev,
             "hk_engine_tick: null argument");
  if (n_runs < 0 || n_runs > e.max_runs) {
    hk::set_error("hk_engine_tick: %d runs exceeds max_runs %d", n_runs, e.max_runs);
    return HK_ERR_CAPACITY;
  }
  for (auto& tv : e.slots)
    for (auto& lv : tv)
      for (auto& sl : lv) HK_REQUIRE(sl.bound, "hk_engine_tick: weight %s not loaded", sl.def.name);
  for (auto& sl : e.gslots) HK_REQUIRE(sl.bound, "hk_engine_tick: weight %s not loaded", sl.def.name);
  HK_REQUIRE(run_off_host[0] == 0, "hk_engine_tick: run_off[0] must be 0");
  const int n_rows = run_off_host[n_runs];
  if (n_rows > e.max_rows) {
    hk::set_error("hk_engine_tick: %d rows exceeds max_rows %d", n_rows, e.max_rows);
    return HK_ERR_CAPACITY;
  }
  int prev = INT32_MAX;
  for (int i = 0; i < n_runs; ++i) {
    const int len = run_off_host[i + 1] - run_off_host[i];
    HK_REQUIRE(len >= 1, "hk_engine_tick: run %d is empty", i);
    HK_REQUIRE(len <= prev, "hk_engine_tick: runs must be sorted by non-increasing length");
    prev = len;
    const int slot = slot_ids_host[i];
    HK_REQUIRE(slot >= 0 && slot < e.capacity, "hk_engine_tick: slot %d out of range", slot);
  }
  for (int i = 0; i < n_runs; ++i) {
    char& seen = e.seen[slot_ids_host[i]];
    if (seen) {
      for (int j = 0; j < i; ++j) e.seen[slot_ids_host[j]] = 0;
      hk::set_error("hk_engine_tick: slot %d appears in two runs", slot_ids_host[i]);
      return HK_ERR_ARG;
    }
    seen = 1;
  }
  for (int i = 0; i < n_runs; ++i) e.seen[slot_ids_host[i]] = 0;

  // Descriptors through a two-deep pinned ring (the copy of tick k-2 must be
  // done before its staging area is rewritten), one copy per tick.
  const int k = e.stage_idx;
  e.stage_idx ^= 1;
  HK_CHECK_HIP(hipEventSynchronize(e.stage_done[k]));
  const int steps = run_off_host[1] - run_off_host[0];
  // xLSTM run groups: runs [0, split) and [split, n_runs).
  const int split = hk::xlstm_split_point(run_off_host, n_runs, e.x_weight_us);
  const int row_split = run_off_host[split];
  const int steps2 = split < n_runs ? run_off_host[split + 1] - run_off_host[split] : 0;
  int* stage = e.h_stage + (size_t)k * e.stage_ints();
  int* h_slots = stage;
  int* h_off = h_slots + e.max_runs;
  int* h_act = h_off + e.max_runs + 1;
  int* h_off2 = h_act + e.max_rows;
  int* h_act1 = h_off2 + e.max_runs + 1;
  int* h_act2 = h_act1 + e.max_rows;
  int* h_pos = h_act2 + e.max_rows;
  int* h_rslot = h_pos + e.max_rows;
  std::memcpy(h_slots, slot_ids_host, (size_t)n_runs * 4);
  for (int i = 0; i < n_runs; ++i)
    for (int r = run_off_host[i]; r < run_off_host[i + 1]; ++r) {
      h_pos[r] = r - run_off_host[i];
      h_rslot[r] = slot_ids_host[i];
    }
  std::memcpy(h_off, run_off_host, (size_t)(n_runs + 1) * 4);
  {
    int c = n_runs;
    for (int t = 0; t < steps; ++t) {
      while (c > 0 && run_off_host[c] - run_off_host[c - 1] <= t) --c;
      h_act[t] = c;
      h_act1[t] = std::min(c, split);
      if (t < steps2) h_act2[t] = c - split;
    }
  }
  for (int i = split; i <= n_runs; ++i) h_off2[i - split] = run_off_host[i] - row_split;
  HK_CHECK_HIP(hipMemcpyAsync(e.d_desc, stage, (size_t)e.stage_ints() * 4, hipMemcpyHostToDevice,
                              s));
  HK_CHECK_HIP(hipEventRecord(e.stage_done[k], s));

  hk::TickShape sh;
  sh.n_runs = n_runs;
  sh.n_rows = n_rows;
  sh.steps = steps;
  sh.split = split;
  sh.row_split = row_split;
  sh.steps2 = steps2;
  sh.act.assign(h_act, h_act + steps);
  sh.act1.assign(h_act1, h_act1 + steps);
  sh.act2.assign(h_act2, h_act2 + steps2);
  if (e.graph_rows > 0 && n_rows <= e.graph_rows && e.prof == 0 && e.d_trace == nullptr) {
    std::vector<int> key(n_runs);
    for (int i = 0; i < n_runs; ++i) key[i] = run_off_host[i + 1] - run_off_host[i];
    return hk::tick_replay(e, key, sh, features_dev, preds_dev, s);
  }
  return hk::enqueue_tick(e, sh, features_dev, preds_dev, s);
}

// Replay small ticks through cached hipGraphs: ticks of at most max_rows
// rows, at most max_graphs tick shapes cached (least recently used evicted);
// max_rows 0 turns replay off and frees the cache.
int hk_engine_graphs(void* h, int max_rows, int max_graphs) {
  HK_REQUIRE(h, "hk_engine_graphs: null handle");
  Engine& e = *static_cast<Engine*>(h);
  HK_REQUIRE(max_rows >= 0 && max_graphs >= 0, "hk_engine_graphs: negative limit");
  HK_REQUIRE(max_rows == 0 || max_graphs > 0, "hk_engine_graphs: replay needs a cache");
  e.graph_rows = std::min(max_rows, e.max_rows);
  e.graph_cap = max_graphs;
  if (max_rows == 0 || (int)e.graphs.size() > max_graphs) {
    HK_CHECK_HIP(hipDeviceSynchronize());
    for (auto& kv : e.graphs)
      for (auto& x : kv.second.exec)
        if (x) HK_CHECK_HIP(hipGraphExecDestroy(x));
    e.graphs.clear();
  }
  return HK_OK;
}

int hk_engine_graph_info(void* h, int64_t* cached, int64_t* captures, int64_t* replays) {
  HK_REQUIRE(h && cached && captures && replays, "hk_engine_graph_info: null argument");
  Engine& e = *static_cast<Engine*>(h);
  *cached = (int64_t)e.graphs.size();
  *captures = e.graph_captures;
  *replays = e.graph_replays;
  return HK_OK;
}

}  // extern "C"
