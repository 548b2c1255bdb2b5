// Matrix-state scan kernel for gfx950 (see scan_mat.h for the recurrence).
//
// One 256-thread work-group (4 wave64s) owns one (run, head, 64-column tile).
// Lane = column, so every state row is one coalesced 256-byte access per wave;
// wave w holds rows [w*RPW, (w+1)*RPW) of the tile in VGPRs for the whole run,
// so the state crosses HBM exactly twice per tick however long the run is.
// The contraction over rows is in-lane (RPW FMAs into 4 accumulators), then a
// 4-way cross-wave sum through LDS. Per-step row vectors (scale*beta, w) are
// staged once into LDS and read back as broadcasts.
#include "scan_mat.h"

namespace hk {
namespace {

template <int RPW>
__global__ __launch_bounds__(256) void mat_scan_kernel(MatScanDesc d) {
  constexpr int kRows = 4 * RPW;
  __shared__ __align__(16) float sb[kRows];
  __shared__ __align__(16) float sw[kRows];
  __shared__ float red[4][64];

  const int run = blockIdx.x;
  const int head = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = blockIdx.z * 64 + lane;
  const bool col_ok = col < d.cols;

  int slot, r0, len;
  if (d.per_row) {
    slot = run;
    r0 = run;
    len = (d.mask == nullptr || d.mask[run]) ? 1 : 0;
  } else {
    slot = d.slot_ids[run];
    r0 = d.run_off[run];
    len = d.run_off[run + 1] - r0;
  }
  float* out_base = d.out + (int64_t)head * d.out_head_stride;
  if (len == 0) {
    // Idle row (reference API): state untouched, output defined as zero.
    if (wave == 0 && col_ok) out_base[(int64_t)r0 * d.out_row_stride + col] = 0.0f;
    return;
  }

  // Rows past d.rows hold zero in LDS and in the tile, so they contribute
  // nothing and need no branch in the inner loop.
  for (int i = d.rows + threadIdx.x; i < kRows; i += 256) {
    sb[i] = 0.0f;
    sw[i] = 0.0f;
  }

  float* base = d.state + (int64_t)slot * d.slot_stride + (int64_t)head * d.head_stride +
                (int64_t)col * d.col_stride;
  const int rbase = wave * RPW;
  float s[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = rbase + i;
    s[i] = (col_ok && r < d.rows) ? base[(int64_t)r * d.row_stride] : 0.0f;
  }

  for (int t = 0; t < len; ++t) {
    const int64_t row = r0 + t;
    const float a = d.alpha.ptr[row * d.alpha.row_stride + head * d.alpha.head_stride];
    const float sc =
        d.scale.ptr ? d.scale.ptr[row * d.scale.row_stride + head * d.scale.head_stride] : 1.0f;
    const float g =
        col_ok ? d.gamma.ptr[row * d.gamma.row_stride + head * d.gamma.head_stride + col] : 0.0f;
    const float* bsrc = d.beta.ptr + row * d.beta.row_stride + head * d.beta.head_stride;
    const float* wsrc = d.w.ptr + row * d.w.row_stride + head * d.w.head_stride;
    for (int i = threadIdx.x; i < d.rows; i += 256) {
      sb[i] = sc * bsrc[i];  // (i*k), (dt*b): the association the reference uses
      sw[i] = wsrc[i];
    }
    __syncthreads();

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < RPW; i += 4) {
      const float4 bv = *reinterpret_cast<const float4*>(&sb[rbase + i]);
      const float4 wv = *reinterpret_cast<const float4*>(&sw[rbase + i]);
      s[i + 0] = a * s[i + 0] + bv.x * g;
      s[i + 1] = a * s[i + 1] + bv.y * g;
      s[i + 2] = a * s[i + 2] + bv.z * g;
      s[i + 3] = a * s[i + 3] + bv.w * g;
      acc[0] += wv.x * s[i + 0];
      acc[1] += wv.y * s[i + 1];
      acc[2] += wv.z * s[i + 2];
      acc[3] += wv.w * s[i + 3];
    }
    red[wave][lane] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    __syncthreads();
    if (wave == 0 && col_ok) {
      out_base[row * d.out_row_stride + col] =
          (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
    }
  }

#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = rbase + i;
    if (col_ok && r < d.rows) base[(int64_t)r * d.row_stride] = s[i];
  }
}

}  // namespace

int launch_mat_scan(const MatScanDesc& d, hipStream_t stream) {
  HK_REQUIRE(d.state && d.out && d.alpha.ptr && d.beta.ptr && d.gamma.ptr && d.w.ptr,
             "mat_scan: null operand");
  HK_REQUIRE(d.rows > 0 && d.cols > 0 && d.heads > 0, "mat_scan: empty tile %dx%d heads %d",
             d.rows, d.cols, d.heads);
  HK_REQUIRE(d.per_row || (d.slot_ids && d.run_off), "mat_scan: need run descriptors");
  HK_REQUIRE(d.heads <= 65535, "mat_scan: too many heads");
  if (d.n_runs == 0) return HK_OK;
  dim3 grid(d.n_runs, d.heads, (d.cols + 63) / 64);
  dim3 block(256);
  if (d.rows <= 32) {
    hipLaunchKernelGGL(mat_scan_kernel<8>, grid, block, 0, stream, d);
  } else if (d.rows <= 64) {
    hipLaunchKernelGGL(mat_scan_kernel<16>, grid, block, 0, stream, d);
  } else if (d.rows <= 128) {
    hipLaunchKernelGGL(mat_scan_kernel<32>, grid, block, 0, stream, d);
  } else if (d.rows <= 256) {
    hipLaunchKernelGGL(mat_scan_kernel<64>, grid, block, 0, stream, d);
  } else if (d.rows <= 512) {
    hipLaunchKernelGGL(mat_scan_kernel<128>, grid, block, 0, stream, d);
  } else {
    HK_REQUIRE(false, "mat_scan: %d rows exceeds the 512-row tile", d.rows);
  }
  HK_LAUNCH_CHECK();
  return HK_OK;
}

}  // namespace hk
