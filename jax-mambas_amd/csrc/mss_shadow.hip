// Low-precision copies of the float32 master weights, refreshed once per training step: for
// every weight in a table, dst = bf16(src) and, where asked, dst_t = bf16(src)^T (the layout
// the input-gradient GEMMs W^T dY read fastest: a contiguous A operand instead of a transposed
// view, 44 vs 53 us for the config-5 out-projection, 64 vs 72 us for the in-projection). One
// launch for the whole table: a workgroup per 64 x 64 tile, its entry found by binary search
// over the entries' first-tile indices; the tile goes through LDS (row 65 floats wide, so the
// column reads of the transposed store hit distinct banks) and both stores are coalesced.
// Rounding: round to nearest even (v_cvt_pk_bf16_f32), as a cast of the master.
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

namespace {

constexpr int kShTile = 64;
constexpr int kShThreads = 256;

__global__ __launch_bounds__(kShThreads) void shadow_refresh_kernel(ShadowParams p) {
  __shared__ float tile[kShTile][kShTile + 1];
  const int tid = threadIdx.x;
  const int tx = tid & 63, ty = tid >> 6;  // column in the tile, first row
  for (long long t = blockIdx.x; t < p.n_tiles; t += gridDim.x) {
    int lo = 0, hi = p.n_entries - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.entries[mid].tile0 <= t) lo = mid;
      else hi = mid - 1;
    }
    const ShadowEntry e = p.entries[lo];
    const long long lt = t - e.tile0;
    const int tiles_c = (e.cols + kShTile - 1) / kShTile;
    const int r0 = static_cast<int>(lt / tiles_c) * kShTile;
    const int c0 = static_cast<int>(lt % tiles_c) * kShTile;
    const int c = c0 + tx;
#pragma unroll
    for (int i = 0; i < kShTile / 4; ++i) {
      const int rr = ty + 4 * i;
      const int r = r0 + rr;
      float v = 0.f;
      if (r < e.rows && c < e.cols) {
        v = e.src[static_cast<size_t>(r) * e.cols + c];
        if (e.dst) store_as(e.dst + static_cast<size_t>(r) * e.cols + c, v);
      }
      tile[rr][tx] = v;
    }
    if (e.dst_t) {
      __syncthreads();
      const int r = r0 + tx;
#pragma unroll
      for (int i = 0; i < kShTile / 4; ++i) {
        const int cc = ty + 4 * i;
        if (r < e.rows && c0 + cc < e.cols) store_as(e.dst_t + static_cast<size_t>(c0 + cc) * e.ld_t + r, tile[tx][cc]);
      }
    }
    __syncthreads();  // the tile is rewritten by the next iteration
  }
}

}  // namespace

hipError_t launch_shadow_refresh(const ShadowParams& p, hipStream_t stream) {
  const long long blocks = p.n_tiles < 8192 ? p.n_tiles : 8192;
  hipLaunchKernelGGL(shadow_refresh_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kShThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mss
