// Residual add + RMSNorm over the feature axis of channel-major activations.
//
// The Mamba-1 block's pre-norm and residual (reference mamba/mamba1.py:300-337:
// x = norm(h); ...; out = proj_down(...) + h, nnx.RMSNorm(epsilon=1e-5)), on a residual
// stream kept as a (features, tokens) fp32 matrix h[f][t]:
//
//   forward   hn = h + delta (delta: the previous block's output, bf16, optional)
//             rstd[t] = 1 / sqrt(mean_f hn[f][t]^2 + eps);  x[f][t] = hn[f][t] * rstd[t] * w[f]
//   backward  given dx (grad of x) and dhn_in (grad of hn from the stream, fp32), with h
//             the forward's normalised input (its hn when a delta was added):
//             xhat = hn * rstd;  c[t] = mean_f w[f] dx[f][t] xhat[f][t]
//             dhn = dhn_in + rstd * (w * dx - xhat * c);  dw[f] = sum_t dx xhat
//             (dh = ddelta = dhn; ddelta is also written in the activation dtype for the
//             producing GEMM). delta, x, dx and ddelta are fp32 or bf16 (template).
//
// Mapping: a workgroup owns 64 consecutive tokens (one per lane; loads of a feature row
// are 256 contiguous bytes per wave) and its kW waves split the features; per-token sums
// meet in LDS. dw is summed per workgroup (wave sums, fixed order) into partials that a
// second kernel adds in a fixed order.
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

constexpr int kNormW = 16;  // waves per workgroup (features split 16 ways)


template <typename io_t>
__global__ __launch_bounds__(kNormW * 64) void add_rmsnorm_fwd_kernel(NormParams p) {
  const io_t* __restrict__ delta = static_cast<const io_t*>(p.delta);
  io_t* __restrict__ xo = static_cast<io_t*>(p.x);
  __shared__ float s_ss[kNormW][64];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int t = blockIdx.x * 64 + lane;
  const bool ok = t < p.tokens;
  const size_t T = p.tokens;
  float ss = 0.f;
  if (ok) {
#pragma unroll 4
    for (int f = wv; f < p.features; f += kNormW) {
      float v = p.h[f * T + t];
      if (delta) {
        v += to_f32(delta[f * T + t]);
        p.hn[f * T + t] = v;
      }
      ss = __builtin_fmaf(v, v, ss);
    }
  }
  s_ss[wv][lane] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormW; ++i) tot += s_ss[i][lane];
  const float r = 1.f / __builtin_sqrtf(tot / p.features + p.eps);
  if (!ok) return;
  if (wv == 0) p.rstd[t] = r;
  const float* src = delta ? p.hn : p.h;
#pragma unroll 4
  for (int f = wv; f < p.features; f += kNormW) {
    store_as(xo + f * T + t, src[f * T + t] * r * p.w[f]);
  }
}

template <typename io_t>
__global__ __launch_bounds__(kNormW * 64) void add_rmsnorm_bwd_kernel(NormParams p) {
  const io_t* __restrict__ dx = static_cast<const io_t*>(p.dx);
  io_t* __restrict__ ddelta = static_cast<io_t*>(p.ddelta);
  __shared__ float s_c[kNormW][64];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int t = blockIdx.x * 64 + lane;
  const bool ok = t < p.tokens;
  const size_t T = p.tokens;
  const float* hn = p.h;  // the forward's normalised input (hn when a delta was added)
  const float r = ok ? p.rstd[t] : 0.f;
  float c = 0.f;
  if (ok) {
#pragma unroll 4
    for (int f = wv; f < p.features; f += kNormW) {
      const float xh = hn[f * T + t] * r;
      c = __builtin_fmaf(p.w[f] * to_f32(dx[f * T + t]), xh, c);
    }
  }
  s_c[wv][lane] = c;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormW; ++i) tot += s_c[i][lane];
  const float cm = tot / p.features;
  for (int f = wv; f < p.features; f += kNormW) {
    float dwv = 0.f;
    if (ok) {
      const float xh = hn[f * T + t] * r;
      const float g = to_f32(dx[f * T + t]);
      float d = r * (p.w[f] * g - xh * cm);
      if (p.dhn_in) d += p.dhn_in[f * T + t];
      p.dhn[f * T + t] = d;
      if (ddelta) store_as(ddelta + f * T + t, d);
      dwv = g * xh;
    }
    dwv = wave_sum(dwv);  // every lane of the wave takes part
    if (lane == 0) p.dw_part[static_cast<size_t>(blockIdx.x) * p.features + f] = dwv;
  }
}

// dw[f] = sum over workgroup partials, fixed order: a workgroup owns 64 features (lanes);
// its 16 waves take every 16th partial and meet in LDS.
__global__ __launch_bounds__(1024) void norm_dw_reduce_kernel(const float* __restrict__ part, int n_blk,
                                                              int features, float* dw) {
  __shared__ float s_sum[16][64];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int f = blockIdx.x * 64 + lane;
  float s = 0.f;
  if (f < features) {
    for (int i = wv; i < n_blk; i += 16) s += part[static_cast<size_t>(i) * features + f];
  }
  s_sum[wv][lane] = s;
  __syncthreads();
  if (wv == 0 && f < features) {
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) tot += s_sum[i][lane];
    dw[f] = tot;
  }
}

// Few tokens (decode): one workgroup per token, threads over the features, so the work
// spreads over `tokens` workgroups instead of one. Same arithmetic as the wide kernel.
template <typename io_t>
__global__ __launch_bounds__(256) void add_rmsnorm_fwd_rows_kernel(NormParams p) {
  __shared__ float s_part[4];
  const io_t* __restrict__ delta = static_cast<const io_t*>(p.delta);
  io_t* __restrict__ xo = static_cast<io_t*>(p.x);
  const int t = blockIdx.x;
  const size_t T = p.tokens;
  float ss = 0.f;
  for (int f = threadIdx.x; f < p.features; f += 256) {
    float v = p.h[f * T + t];
    if (delta) {
      v += to_f32(delta[f * T + t]);
      p.hn[f * T + t] = v;
    }
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = s_part[0] + s_part[1] + s_part[2] + s_part[3];
  const float r = 1.f / __builtin_sqrtf(tot / p.features + p.eps);
  if (threadIdx.x == 0) p.rstd[t] = r;
  const float* src = delta ? p.hn : p.h;
  for (int f = threadIdx.x; f < p.features; f += 256) store_as(xo + f * T + t, src[f * T + t] * r * p.w[f]);
}

constexpr int kNormRowsMaxTokens = 256;

int norm_blocks(int tokens) { return (tokens + 63) / 64; }

hipError_t launch_norm_fwd(const NormParams& p, bool io_bf16, hipStream_t stream) {
  if (p.tokens <= kNormRowsMaxTokens) {
    if (io_bf16) hipLaunchKernelGGL(add_rmsnorm_fwd_rows_kernel<bf16_t>, dim3(p.tokens), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(add_rmsnorm_fwd_rows_kernel<float>, dim3(p.tokens), dim3(256), 0, stream, p);
    return hipGetLastError();
  }
  const dim3 grid(norm_blocks(p.tokens)), block(kNormW * 64);
  if (io_bf16) hipLaunchKernelGGL(add_rmsnorm_fwd_kernel<bf16_t>, grid, block, 0, stream, p);
  else hipLaunchKernelGGL(add_rmsnorm_fwd_kernel<float>, grid, block, 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_norm_bwd(const NormParams& p, bool io_bf16, float* dw, hipStream_t stream) {
  const int nb = norm_blocks(p.tokens);
  if (io_bf16) hipLaunchKernelGGL(add_rmsnorm_bwd_kernel<bf16_t>, dim3(nb), dim3(kNormW * 64), 0, stream, p);
  else hipLaunchKernelGGL(add_rmsnorm_bwd_kernel<float>, dim3(nb), dim3(kNormW * 64), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(norm_dw_reduce_kernel, dim3((p.features + 63) / 64), dim3(1024), 0, stream,
                     p.dw_part, nb, p.features, dw);
  return hipGetLastError();
}

}  // namespace mss
