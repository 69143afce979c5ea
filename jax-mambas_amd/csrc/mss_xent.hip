// Cross-entropy over bf16 logits with fp32 math, forward and backward.
//
// The language-model loss of the training step (the reference trains with
// optax softmax cross-entropy on the head's logits, experiments/mamba_inductionheads.py:
// 129-136), for a [rows][vocab] bf16 logits matrix and int64 targets:
//   forward   lse[r] = log sum_v exp(z[r][v]);  loss[r] = lse[r] - z[r][target[r]]
//   backward  dz[r][v] = scale * (exp(z[r][v] - lse[r]) - [v == target[r]]),
//             scale = *grad_scale (device scalar: the upstream gradient / rows)
// One workgroup per row; 16-byte loads when rows are aligned. Reads the logits once per
// direction (the backward recomputes the softmax from lse) and writes dz once, in bf16; or,
// for a loss that will be differentiated, both directions in one pass (xent_fused_kernel),
// the gradient formed for the mean's scale and multiplied later by the upstream gradient
// only when that is not 1.
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

constexpr int kXentThreads = 256;


__device__ __forceinline__ void unpack8(const u32x4 a, float (&v)[8]) {
  const unsigned w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// Online (max, sum of exp(x - max)) merge.
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mx = m > m2 ? m : m2;
  if (mx == -INFINITY) return;
  s = s * fast_exp2((m - mx) * kLog2e) + s2 * fast_exp2((m2 - mx) * kLog2e);
  m = mx;
}

template <bool kVec>
__global__ __launch_bounds__(kXentThreads) void xent_fwd_kernel(XentParams p) {
  __shared__ float s_m[kXentThreads / 64], s_s[kXentThreads / 64];
  const int r = blockIdx.x;
  const bf16_t* row = p.z + static_cast<size_t>(r) * p.vocab;
  float m = -INFINITY, s = 0.f;
  if constexpr (kVec) {
    const int nv = p.vocab / 8;
    for (int i = threadIdx.x; i < nv; i += kXentThreads) {
      float v[8];
      unpack8(reinterpret_cast<const u32x4*>(row)[i], v);
      float lm = v[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) lm = lm > v[j] ? lm : v[j];
      float ls = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ls += fast_exp2((v[j] - lm) * kLog2e);
      lse_merge(m, s, lm, ls);
    }
  } else {
    for (int i = threadIdx.x; i < p.vocab; i += kXentThreads) lse_merge(m, s, to_f32(row[i]), 1.f);
  }
  // wave merge (xor butterfly through LDS-free lane shuffles)
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off);
    const float s2 = __shfl_xor(s, off);
    lse_merge(m, s, m2, s2);
  }
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_m[wv] = m;
    s_s[wv] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = s_m[0], S = s_s[0];
    for (int i = 1; i < kXentThreads / 64; ++i) lse_merge(M, S, s_m[i], s_s[i]);
    const float l = M + fast_log2(S) * (1.f / kLog2e);
    p.lse[r] = l;
    const long long tg = p.target[r];  // an out-of-range label gives a NaN loss, no read
    p.loss[r] = (tg >= 0 && tg < p.vocab) ? l - to_f32(row[tg]) : __builtin_nanf("");
  }
}

template <bool kVec>
__global__ __launch_bounds__(kXentThreads) void xent_bwd_kernel(XentParams p) {
  const int r = blockIdx.x;
  const size_t base = static_cast<size_t>(r) * p.vocab;
  const bf16_t* row = p.z + base;
  bf16_t* drow = p.dz + base;
  const float l = p.lse[r];
  const long long tgt = p.target[r];
  const float scale = *p.grad_scale;
  if constexpr (kVec) {
    const int nv = p.vocab / 8;
    for (int i = threadIdx.x; i < nv; i += kXentThreads) {
      float v[8];
      unpack8(reinterpret_cast<const u32x4*>(row)[i], v);
      unsigned w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float g0 = fast_exp2((v[2 * j] - l) * kLog2e) - (8LL * i + 2 * j == tgt ? 1.f : 0.f);
        float g1 = fast_exp2((v[2 * j + 1] - l) * kLog2e) - (8LL * i + 2 * j + 1 == tgt ? 1.f : 0.f);
        w[j] = pack_bf16x2(g0 * scale, g1 * scale);
      }
      u32x4 o;
      o.x = w[0]; o.y = w[1]; o.z = w[2]; o.w = w[3];
      reinterpret_cast<u32x4*>(drow)[i] = o;
    }
  } else {
    for (int i = threadIdx.x; i < p.vocab; i += kXentThreads) {
      const float g = fast_exp2((to_f32(row[i]) - l) * kLog2e) - (i == tgt ? 1.f : 0.f);
      store_as(drow + i, g * scale);
    }
  }
}

// Forward and gradient in one pass over the logits, for training steps whose loss is then
// differentiated: the row (vocab % 8 == 0, 16-byte aligned, vocab <= kXentFusedMaxVocab) is
// held in registers, 16-byte vectors of 8 bf16 strided over 1024 threads, so it is read from
// HBM once; lse and loss as xent_fwd_kernel's arithmetic (the row's partial sums merged in
// another fixed order: 1024 threads instead of 256, so lse may differ from that kernel's in
// the last bits), then dz = scale * (softmax - onehot) from this lse as xent_bwd_kernel.
constexpr int kXentFusedThreads = 1024;
constexpr int kXentFusedVecs = kXentFusedMaxVocab / 8 / kXentFusedThreads;  // vectors per thread
static_assert(kXentFusedMaxVocab % (8 * kXentFusedThreads) == 0, "whole vectors per thread");

__global__ __launch_bounds__(kXentFusedThreads) void xent_fused_kernel(XentParams p) {
  __shared__ float s_m[kXentFusedThreads / 64], s_s[kXentFusedThreads / 64], s_l;
  const int r = blockIdx.x;
  const size_t base = static_cast<size_t>(r) * p.vocab;
  const u32x4* row = reinterpret_cast<const u32x4*>(p.z + base);
  const int nv = p.vocab / 8;
  u32x4 reg[kXentFusedVecs];
#pragma unroll
  for (int k = 0; k < kXentFusedVecs; ++k) {
    const int i = threadIdx.x + k * kXentFusedThreads;
    if (i < nv) reg[k] = row[i];
  }
  float m = -INFINITY, s = 0.f;
#pragma unroll
  for (int k = 0; k < kXentFusedVecs; ++k) {
    const int i = threadIdx.x + k * kXentFusedThreads;
    if (i < nv) {
      float v[8];
      unpack8(reg[k], v);
      float lm = v[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) lm = lm > v[j] ? lm : v[j];
      float ls = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ls += fast_exp2((v[j] - lm) * kLog2e);
      lse_merge(m, s, lm, ls);
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off);
    const float s2 = __shfl_xor(s, off);
    lse_merge(m, s, m2, s2);
  }
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_m[wv] = m;
    s_s[wv] = s;
  }
  __syncthreads();
  const long long tgt = p.target[r];
  if (threadIdx.x == 0) {
    float M = s_m[0], S = s_s[0];
    for (int i = 1; i < kXentFusedThreads / 64; ++i) lse_merge(M, S, s_m[i], s_s[i]);
    const float l = M + fast_log2(S) * (1.f / kLog2e);
    p.lse[r] = l;
    p.loss[r] = (tgt >= 0 && tgt < p.vocab) ? l - to_f32(p.z[base + tgt]) : __builtin_nanf("");
    s_l = l;
  }
  __syncthreads();
  const float l = s_l;
  const float scale = *p.grad_scale;
  u32x4* drow = reinterpret_cast<u32x4*>(p.dz + base);
#pragma unroll
  for (int k = 0; k < kXentFusedVecs; ++k) {
    const int i = threadIdx.x + k * kXentFusedThreads;
    if (i < nv) {
      float v[8];
      unpack8(reg[k], v);
      unsigned w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float g0 = fast_exp2((v[2 * j] - l) * kLog2e) - (8LL * i + 2 * j == tgt ? 1.f : 0.f);
        float g1 = fast_exp2((v[2 * j + 1] - l) * kLog2e) - (8LL * i + 2 * j + 1 == tgt ? 1.f : 0.f);
        w[j] = pack_bf16x2(g0 * scale, g1 * scale);
      }
      u32x4 o;
      o.x = w[0]; o.y = w[1]; o.z = w[2]; o.w = w[3];
      drow[i] = o;
    }
  }
}

// dz *= *factor (bf16, rounded once), skipped entirely when *factor == 1 (the usual upstream
// gradient of a loss): every workgroup reads the factor and leaves at once.
__global__ __launch_bounds__(256) void xent_rescale_kernel(bf16_t* dz, long long n, const float* factor) {
  const float f = *factor;
  if (f == 1.f) return;
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += static_cast<long long>(gridDim.x) * 256)
    store_as(dz + i, to_f32(dz[i]) * f);
}

hipError_t launch_xent_fused(const XentParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(xent_fused_kernel, dim3(p.rows), dim3(kXentFusedThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_xent_rescale(bf16_t* dz, long long n, const float* factor, hipStream_t stream) {
  const long long blocks = (n + 255) / 256;
  hipLaunchKernelGGL(xent_rescale_kernel, dim3(static_cast<unsigned>(blocks < 1024 ? blocks : 1024)), dim3(256), 0,
                     stream, dz, n, factor);
  return hipGetLastError();
}

hipError_t launch_xent(const XentParams& p, bool bwd, bool vec, hipStream_t stream) {
  const dim3 grid(p.rows), block(kXentThreads);
  if (bwd) {
    if (vec) hipLaunchKernelGGL(xent_bwd_kernel<true>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(xent_bwd_kernel<false>, grid, block, 0, stream, p);
  } else {
    if (vec) hipLaunchKernelGGL(xent_fwd_kernel<true>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(xent_fwd_kernel<false>, grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace mss
