// AdamW over float32 master weights in one launch per training step, writing the bf16
// shadows of the updated weights on the way out (the copies the next step's GEMMs read), so
// no separate refresh pass re-reads the masters. Per element, in float32 (decoupled weight
// decay, Loshchilov & Hutter, "Decoupled Weight Decay Regularization", Algorithm 2, with the
// bias-corrected moments of Kingma & Ba):
//   p  <- p * (1 - lr * wd)
//   m  <- m + (1 - beta1) (g - m)
//   v  <- beta2 v + (1 - beta2) g^2
//   p  <- p - (lr / (1 - beta1^t)) m / (sqrt(v) / sqrt(1 - beta2^t) + eps)
// t read from device memory (the caller advances it before the launch, so a captured step
// replays with the right count). Work units of 4096 elements: flat runs of an entry (16-byte
// vector accesses, scalar tails), or 64 x 64 tiles for an entry whose transposed shadow is
// kept (the updated tile goes through LDS, row 65 floats wide, so both shadow stores are
// coalesced). A launch takes up to 40 entries by value (kernel arguments: nothing to build in
// device memory, so the launch can be captured as it is); a workgroup per unit finds its
// entry by a binary search over the entries' first units, uniform across the workgroup.
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

namespace {

constexpr int kAwThreads = 256;
constexpr int kAwTile = 64;

struct AwCoef {
  float decay, b1c, b2, b2c, step_size, bc2_sqrt, eps;  // b1c = 1 - beta1, b2c = 1 - beta2
};

__device__ __forceinline__ void adamw_elem(const AwCoef& k, float& p, float g, float& m, float& v) {
  p *= k.decay;
  m = __builtin_fmaf(k.b1c, g - m, m);
  v = __builtin_fmaf(k.b2, v, k.b2c * g * g);
  const float denom = sqrtf(v) / k.bc2_sqrt + k.eps;
  p -= k.step_size * (m / denom);
}

__device__ __forceinline__ void adamw_vec(const AwCoef& k, f32x4& p, const f32x4& g, f32x4& m, f32x4& v) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float pc = p[c], mc = m[c], vc = v[c];
    adamw_elem(k, pc, g[c], mc, vc);
    p[c] = pc;
    m[c] = mc;
    v[c] = vc;
  }
}

__global__ __launch_bounds__(kAwThreads) void adamw_kernel(AdamWParams prm) {
  __shared__ float tile[kAwTile][kAwTile + 1];
  const int tid = threadIdx.x;
  const long long u = blockIdx.x;
  int lo = 0, hi = prm.n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (prm.unit0[mid] <= u) lo = mid;
    else hi = mid - 1;
  }
  const AdamWEntry& e = prm.e[lo];
  const long long lu = u - prm.unit0[lo];
  AwCoef k;
  {
    const float t = *e.step;
    k.decay = 1.f - prm.lr * prm.weight_decay;
    k.b1c = 1.f - prm.beta1;
    k.b2 = prm.beta2;
    k.b2c = 1.f - prm.beta2;
    k.step_size = prm.lr / (1.f - powf(prm.beta1, t));
    k.bc2_sqrt = sqrtf(1.f - powf(prm.beta2, t));
    k.eps = prm.eps;
  }
  if (!e.shadow_t) {
    // Flat run [4096 lu, 4096 lu + 4096) of the entry: thread tid takes elements
    // 4 (256 i + tid) .. +3, i = 0..3, as one 16-byte access per array where whole.
    const long long base = lu * kAdamWUnit;
    f32x4 pv[4], gv[4], mv[4], vv[4];
    bool whole[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const long long idx = base + 4LL * (i * kAwThreads + tid);
      whole[i] = idx + 4 <= e.numel;
      if (whole[i]) {
        pv[i] = *reinterpret_cast<const f32x4*>(e.param + idx);
        gv[i] = *reinterpret_cast<const f32x4*>(e.grad + idx);
        mv[i] = *reinterpret_cast<const f32x4*>(e.exp_avg + idx);
        vv[i] = *reinterpret_cast<const f32x4*>(e.exp_avg_sq + idx);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const long long idx = base + 4LL * (i * kAwThreads + tid);
      if (whole[i]) {
        adamw_vec(k, pv[i], gv[i], mv[i], vv[i]);
        *reinterpret_cast<f32x4*>(e.param + idx) = pv[i];
        *reinterpret_cast<f32x4*>(e.exp_avg + idx) = mv[i];
        *reinterpret_cast<f32x4*>(e.exp_avg_sq + idx) = vv[i];
        if (e.shadow) {
          const uint2 o = {pack_bf16x2(pv[i][0], pv[i][1]), pack_bf16x2(pv[i][2], pv[i][3])};
          *reinterpret_cast<uint2*>(e.shadow + idx) = o;
        }
      } else {
        for (long long x = idx; x < e.numel && x < idx + 4; ++x) {
          float p = e.param[x], m = e.exp_avg[x], v = e.exp_avg_sq[x];
          adamw_elem(k, p, e.grad[x], m, v);
          e.param[x] = p;
          e.exp_avg[x] = m;
          e.exp_avg_sq[x] = v;
          if (e.shadow) store_as(e.shadow + x, p);
        }
      }
    }
    return;
  }
  // 64 x 64 tile (r0, c0) of the entry as [rows][cols] (cols a multiple of 4): thread tid
  // updates rows r0 + tid / 16 + 16 i, columns c0 + 4 (tid % 16) .. +3.
  const int tiles_c = (e.cols + kAwTile - 1) / kAwTile;
  const int r0 = static_cast<int>(lu / tiles_c) * kAwTile;
  const int c0 = static_cast<int>(lu % tiles_c) * kAwTile;
  const int cc = 4 * (tid & 15);
  const int c = c0 + cc;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rr = (tid >> 4) + 16 * i;
    const int r = r0 + rr;
    f32x4 pv = {0.f, 0.f, 0.f, 0.f};
    if (r < e.rows && c < e.cols) {
      const size_t idx = static_cast<size_t>(r) * e.cols + c;
      pv = *reinterpret_cast<const f32x4*>(e.param + idx);
      const f32x4 gv = *reinterpret_cast<const f32x4*>(e.grad + idx);
      f32x4 mv = *reinterpret_cast<const f32x4*>(e.exp_avg + idx);
      f32x4 vv = *reinterpret_cast<const f32x4*>(e.exp_avg_sq + idx);
      adamw_vec(k, pv, gv, mv, vv);
      *reinterpret_cast<f32x4*>(e.param + idx) = pv;
      *reinterpret_cast<f32x4*>(e.exp_avg + idx) = mv;
      *reinterpret_cast<f32x4*>(e.exp_avg_sq + idx) = vv;
      if (e.shadow) {
        const uint2 o = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
        *reinterpret_cast<uint2*>(e.shadow + idx) = o;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) tile[rr][cc + q] = pv[q];
  }
  __syncthreads();
  // Transposed: thread tid writes column c0 + tid / 4, rows r0 + 16 (tid % 4) .. +15, i.e. 16
  // consecutive bf16 of shadow_t's row (two 16-byte stores when whole).
  const int ct = tid >> 2;
  const int rt = 16 * (tid & 3);
  if (c0 + ct >= e.cols) return;
  bf16_t* dst = e.shadow_t + static_cast<size_t>(c0 + ct) * e.ld_t + r0 + rt;
  if (r0 + rt + 16 <= e.rows) {
    u32x4 o[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      o[h].x = pack_bf16x2(tile[rt + 8 * h][ct], tile[rt + 8 * h + 1][ct]);
      o[h].y = pack_bf16x2(tile[rt + 8 * h + 2][ct], tile[rt + 8 * h + 3][ct]);
      o[h].z = pack_bf16x2(tile[rt + 8 * h + 4][ct], tile[rt + 8 * h + 5][ct]);
      o[h].w = pack_bf16x2(tile[rt + 8 * h + 6][ct], tile[rt + 8 * h + 7][ct]);
    }
    reinterpret_cast<u32x4*>(dst)[0] = o[0];
    reinterpret_cast<u32x4*>(dst)[1] = o[1];
  } else {
    for (int q = 0; q < 16 && r0 + rt + q < e.rows; ++q) store_as(dst + q, tile[rt + q][ct]);
  }
}

}  // namespace

hipError_t launch_adamw(const AdamWParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(adamw_kernel, dim3(static_cast<unsigned>(p.unit0[p.n])), dim3(kAwThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mss
