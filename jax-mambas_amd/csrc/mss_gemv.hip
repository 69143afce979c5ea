// Decode-shaped GEMM for gfx950: Y = W X with W [M][K] bf16 (a weight matrix), X [K][N]
// bf16 (N = the decode batch, 1, 2, 4 or 8 tokens, rows of N contiguous values) and
// Y [M][N] bf16, float32 accumulation.
//
// No counterpart kernel in the reference: its decode step (mamba/mamba1.py:200-214,
// 339-363) runs the projections through XLA dot products. At decode shapes the products
// read each weight once and the activations are a few KB, so a general GEMM's tiling
// leaves the launch dominated by fixed costs; here a wave reads kR weight rows in 16-byte
// slices (lanes split K) and sums over its lanes with DPP, one pass over W at full width.
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

// N values of one X row (16-bit each) from LDS, as one 2N-byte access.
template <int kN>
__device__ __forceinline__ void load_xrow(const bf16_t* x, float (&v)[kN]) {
  if constexpr (kN == 8) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(x);
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(a[i] << 16);
      v[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
    }
  } else if constexpr (kN == 4) {
    const uint2 w = *reinterpret_cast<const uint2*>(x);
    v[0] = __uint_as_float(w.x << 16);
    v[1] = __uint_as_float(w.x & 0xffff0000u);
    v[2] = __uint_as_float(w.y << 16);
    v[3] = __uint_as_float(w.y & 0xffff0000u);
  } else if constexpr (kN == 2) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(x);
    v[0] = __uint_as_float(w << 16);
    v[1] = __uint_as_float(w & 0xffff0000u);
  } else {
    v[0] = __uint_as_float(static_cast<uint32_t>(x[0].bits) << 16);
  }
}

// A workgroup of 4 waves stages X (K x N bf16, at most 64 KB) in LDS once; each
// wave then produces kR consecutive rows of Y: lane l covers K elements 8l + 512 s
// (s = 0, 1, ..), reading 16 bytes of each of its kR weight rows per step, and the wave
// sums over its lanes. Rows past M are clamped to M - 1 for the reads and never stored.
template <int kN, int kR>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
  extern __shared__ u32x4 s_x[];
  const int tid = threadIdx.x;
  const int n_q = p.K * kN / 8;  // 16-byte words of X (K % 8 == 0)
  const u32x4* __restrict__ xg = static_cast<const u32x4*>(p.X);
  for (int i = tid; i < n_q; i += 256) s_x[i] = xg[i];
  __syncthreads();
  const int lane = tid & 63;
  const int m0 = (blockIdx.x * 4 + (tid >> 6)) * kR;
  if (m0 >= p.M) return;  // wave-uniform, after the only barrier
  const bf16_t* __restrict__ W = static_cast<const bf16_t*>(p.W);
  const bf16_t* X = reinterpret_cast<const bf16_t*>(s_x);
  float acc[kR][kN];
#pragma unroll
  for (int r = 0; r < kR; ++r)
#pragma unroll
    for (int c = 0; c < kN; ++c) acc[r][c] = 0.f;
  for (int k0 = lane * 8; k0 < p.K; k0 += 512) {
    float w[kR][8];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const int m = min(m0 + r, p.M - 1);
      const u32x4 q = *reinterpret_cast<const u32x4*>(W + static_cast<size_t>(m) * p.ldw + k0);
      const uint32_t a[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[r][2 * i] = __uint_as_float(a[i] << 16);
        w[r][2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x[kN];
      load_xrow<kN>(X + (k0 + e) * kN, x);
#pragma unroll
      for (int r = 0; r < kR; ++r)
#pragma unroll
        for (int c = 0; c < kN; ++c) acc[r][c] = __builtin_fmaf(w[r][e], x[c], acc[r][c]);
    }
  }
  bf16_t* __restrict__ Y = static_cast<bf16_t*>(p.Y);
#pragma unroll
  for (int r = 0; r < kR; ++r) {
#pragma unroll
    for (int c = 0; c < kN; ++c) {
      const float s = wave_sum(acc[r][c]);
      if (lane == 0 && m0 + r < p.M) Y[static_cast<size_t>(m0 + r) * kN + c] = f32_to_bf16(s);
    }
  }
}

template <int kN>
static hipError_t launch_gemv_n(const GemvParams& p, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(p.K) * kN * sizeof(bf16_t);
  // 4 rows per wave (X staged once per 16 rows) when that still gives >= 256 workgroups.
  if (p.M >= 4096) {
    const int waves = (p.M + 3) / 4;
    hipLaunchKernelGGL((gemv_kernel<kN, 4>), dim3((waves + 3) / 4), dim3(256), lds, stream, p);
  } else {
    hipLaunchKernelGGL((gemv_kernel<kN, 1>), dim3((p.M + 3) / 4), dim3(256), lds, stream, p);
  }
  return hipGetLastError();
}

hipError_t launch_gemv(const GemvParams& p, hipStream_t stream) {
  switch (p.N) {
    case 1: return launch_gemv_n<1>(p, stream);
    case 2: return launch_gemv_n<2>(p, stream);
    case 4: return launch_gemv_n<4>(p, stream);
    case 8: return launch_gemv_n<8>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mss
