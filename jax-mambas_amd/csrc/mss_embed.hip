// Token embedding into the channel-major residual stream and its gradient, for the LM's
// input (reference mamba/mamba1.py:378-380: nnx.Embed, whose table the output head shares).
//
//   forward   h[f][t] = E[tok[t]][f]            (E [V][D] float32, h [D][T], row stride ldh)
//   backward  dE[v][:] += sum over t with tok[t] == v, in increasing t, of dh[:][t]
//
// Forward: one workgroup per 64 tokens x 64 features; the tokens' 256-byte row pieces are read
// into LDS (rows 65 floats wide) and written out as 64-token rows of h, both coalesced. A
// token outside [0, V) gives a row of NaN (nothing is read for it).
// Backward, given the tokens sorted stably (sorted values and their positions): dh is first
// transposed through LDS into a token-major workspace (rows of D floats), then one workgroup
// per sorted index: the first index of each run of equal tokens sums the run's rows (a fixed
// association) and adds the sum to dE's row, so every row of dE is written by one workgroup
// and the result does not depend on timing. Out-of-range tokens are skipped. D a multiple
// of 4, at most kEmbedMaxD.
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

namespace {

constexpr int kEmTile = 64;
constexpr int kEmThreads = 256;
constexpr int kEmPerWg = 4;  // sorted indices per workgroup of the gradient's run sums

__global__ __launch_bounds__(kEmThreads) void embed_cm_kernel(EmbedParams p) {
  __shared__ float tile[kEmTile][kEmTile + 1];  // [token][feature]
  const int tid = threadIdx.x;
  // Feature blocks fastest in the 1-D grid: the pieces of one token block's rows are read by
  // neighbouring workgroups, close in time.
  const int n_fb = (p.D + kEmTile - 1) / kEmTile;
  const long long t0 = static_cast<long long>(blockIdx.x / n_fb) * kEmTile;
  const int f0 = static_cast<int>(blockIdx.x % n_fb) * kEmTile;
  const int c = tid & 63, r = tid >> 6;
#pragma unroll 4
  for (int i = 0; i < kEmTile / 4; ++i) {  // token t0 + r + 4 i, feature f0 + c
    const int tt = r + 4 * i;
    const long long t = t0 + tt;
    float v = 0.f;
    if (t < p.T && f0 + c < p.D) {
      const long long tok = p.tokens[t];
      v = (tok >= 0 && tok < p.V) ? p.E[tok * p.D + f0 + c] : __builtin_nanf("");
    }
    tile[tt][c] = v;
  }
  __syncthreads();
#pragma unroll 4
  for (int i = 0; i < kEmTile / 4; ++i) {  // feature f0 + r + 4 i, token t0 + c
    const int ff = r + 4 * i;
    if (f0 + ff < p.D && t0 + c < p.T) p.h[static_cast<size_t>(f0 + ff) * p.ldh + t0 + c] = tile[c][ff];
  }
}

// dh [D][T] (row stride ldh) -> work [T][D].
__global__ __launch_bounds__(kEmThreads) void embed_transpose_kernel(EmbedParams p) {
  __shared__ float tile[kEmTile][kEmTile + 1];  // [feature][token]
  const int tid = threadIdx.x;
  const long long t0 = static_cast<long long>(blockIdx.x) * kEmTile;
  const int f0 = blockIdx.y * kEmTile;
  const int c = tid & 63, r = tid >> 6;
#pragma unroll 4
  for (int i = 0; i < kEmTile / 4; ++i) {
    const int ff = r + 4 * i;
    tile[ff][c] = (f0 + ff < p.D && t0 + c < p.T) ? p.dh[static_cast<size_t>(f0 + ff) * p.ldh + t0 + c] : 0.f;
  }
  __syncthreads();
#pragma unroll 4
  for (int i = 0; i < kEmTile / 4; ++i) {
    const int tt = r + 4 * i;
    if (t0 + tt < p.T && f0 + c < p.D) p.work[(t0 + tt) * p.D + f0 + c] = tile[c][tt];
  }
}

// Run sum of sorted index j when it is the first of its run of equal tokens. The run's end: a
// short linear probe, then a binary search over the sorted tokens for long runs. Its rows are
// summed by 4 groups of 64 threads (group g: rows j + g, j + g + 4, ..., 16-byte pieces, 4
// rows of a group in flight), the 4 partial rows added in group order through LDS (a fixed
// association: the result does not depend on timing), then added to dE's row.
__device__ __forceinline__ void embed_run_add(const EmbedParams& p, long long j, f32x4 (*part)[kEmbedMaxD / 4]) {
  const long long* __restrict__ st = p.sorted_tokens;
  const long long tok = st[j];
  if (tok < 0 || tok >= p.V) return;
  if (j > 0 && st[j - 1] == tok) return;  // not the first of its run
  long long end = j + 1;
  while (end < p.T && end < j + 8 && st[end] == tok) ++end;
  if (end == j + 8 && end < p.T && st[end] == tok) {  // long run: first index past it
    long long lo = end, hi = p.T;  // st[lo] == tok; the answer is in (lo, hi]
    while (hi - lo > 1) {
      const long long mid = (lo + hi) >> 1;
      if (st[mid] == tok) lo = mid;
      else hi = mid;
    }
    end = hi;
  }
  const int tid = threadIdx.x;
  const int g = tid >> 6, l = tid & 63;
  const int d4 = p.D / 4;
  const f32x4* __restrict__ work = reinterpret_cast<const f32x4*>(p.work);
  for (int f4 = l; f4 < d4; f4 += 64) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    long long k = j + g;
    for (; k + 12 < end; k += 16) {  // 4 rows of this group in flight
      const f32x4 v0 = work[p.order[k] * d4 + f4];
      const f32x4 v1 = work[p.order[k + 4] * d4 + f4];
      const f32x4 v2 = work[p.order[k + 8] * d4 + f4];
      const f32x4 v3 = work[p.order[k + 12] * d4 + f4];
      acc += v0;
      acc += v1;
      acc += v2;
      acc += v3;
    }
    for (; k < end; k += 4) acc += work[p.order[k] * d4 + f4];
    part[g][f4] = acc;
  }
  __syncthreads();
  f32x4* __restrict__ row = reinterpret_cast<f32x4*>(p.dE + tok * p.D);
  for (int f4 = tid; f4 < d4; f4 += kEmThreads) {
    f32x4 s = part[0][f4];
    s += part[1][f4];
    s += part[2][f4];
    s += part[3][f4];
    row[f4] += s;
  }
  __syncthreads();  // part is rewritten by the next run
}

// kEmPerWg consecutive sorted indices per workgroup, in turn (fewer, longer-lived workgroups
// than one per index: most indices are not the first of a run and need no work).
__global__ __launch_bounds__(kEmThreads) void embed_segment_add_kernel(EmbedParams p) {
  __shared__ f32x4 part[4][kEmbedMaxD / 4];
  for (int q = 0; q < kEmPerWg; ++q) {
    const long long j = static_cast<long long>(blockIdx.x) * kEmPerWg + q;  // workgroup-uniform
    if (j >= p.T) break;
    embed_run_add(p, j, part);
  }
}

}  // namespace

hipError_t launch_embed_cm(const EmbedParams& p, hipStream_t stream) {
  const long long blocks = ((p.T + kEmTile - 1) / kEmTile) * ((p.D + kEmTile - 1) / kEmTile);
  hipLaunchKernelGGL(embed_cm_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kEmThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_embed_cm_backward(const EmbedParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((p.T + kEmTile - 1) / kEmTile), (p.D + kEmTile - 1) / kEmTile);
  hipLaunchKernelGGL(embed_transpose_kernel, grid, dim3(kEmThreads), 0, stream, p);
  hipLaunchKernelGGL(embed_segment_add_kernel, dim3(static_cast<unsigned>((p.T + kEmPerWg - 1) / kEmPerWg)),
                     dim3(kEmThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mss
