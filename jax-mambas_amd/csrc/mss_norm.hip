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
// second kernel adds in a fixed order. Up to kNormW * kNormRegs features (a 768-wide
// model), each thread keeps its features in registers between the sum and the output pass
// (one read of every input); wider streams re-read them.
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

constexpr int kNormW = 16;     // waves per workgroup (features split 16 ways)
constexpr int kNormRegs = 48;  // features per thread held in registers (<= 768 features)

// Forward, features <= kNormW * kNormRegs. Loads take clamped (valid) addresses and the
// values are masked, with no branch between them, so a batch of loads is in flight at once.
// Two batches of 24 features (measured on MI355X at 768 features x 16384 tokens: 30-34 us
// against 42 with three batches of 16 and 45 with one of 48, which reaches 128 VGPRs).
template <typename io_t, bool kDelta>
__device__ __forceinline__ float norm_fwd_load(const NormParams& p, const io_t* __restrict__ delta,
                                               int wv, size_t tc, float (&v)[kNormRegs]) {
  constexpr int kBatch = 24;
  const size_t T = p.tokens;
  const int F = p.features;
  float ss = 0.f;
#pragma unroll
  for (int i0 = 0; i0 < kNormRegs; i0 += kBatch) {
    float hv[kBatch], dv[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int f = wv + (i0 + k) * kNormW;
      const size_t o = static_cast<size_t>(f < F ? f : F - 1) * T + tc;
      hv[k] = p.h[o];
      if constexpr (kDelta) dv[k] = to_f32(delta[o]);
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int f = wv + (i0 + k) * kNormW;
      const float x = kDelta ? hv[k] + dv[k] : hv[k];
      v[i0 + k] = f < F ? x : 0.f;
      ss = __builtin_fmaf(v[i0 + k], v[i0 + k], ss);
    }
  }
  return ss;
}

template <typename io_t>
__global__ __launch_bounds__(kNormW * 64) void add_rmsnorm_fwd_reg_kernel(NormParams p) {
  const io_t* __restrict__ delta = static_cast<const io_t*>(p.delta);
  io_t* __restrict__ xo = static_cast<io_t*>(p.x);
  __shared__ float s_ss[kNormW][64];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int t = blockIdx.x * 64 + lane;
  const bool ok = t < p.tokens;
  const size_t T = p.tokens;
  const size_t tc = ok ? t : p.tokens - 1;
  const int F = p.features;
  float v[kNormRegs];
  const float ss = delta ? norm_fwd_load<io_t, true>(p, delta, wv, tc, v)
                         : norm_fwd_load<io_t, false>(p, delta, wv, tc, v);
  s_ss[wv][lane] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormW; ++i) tot += s_ss[i][lane];
  const float r = 1.f / __builtin_sqrtf(tot / F + p.eps);
  if (!ok) return;
  if (wv == 0) p.rstd[t] = r;
#pragma unroll
  for (int i = 0; i < kNormRegs; ++i) {
    const int f = wv + i * kNormW;
    if (f < F) {
      const size_t o = static_cast<size_t>(f) * T + t;
      if (delta) p.hn[o] = v[i];
      store_as(xo + o, v[i] * r * p.w[f]);
    }
  }
}

// Backward, features a multiple of 2 * kNormW and at most kNormW * kNormRegs. A workgroup
// owns kNormBwdTiles tiles of 32 tokens, walked in turn: each wave covers two feature rows
// at a time (lanes 0-31 and 32-63, 128 contiguous bytes each), so a thread keeps xhat and
// dx of kNormRegs / 2 features in registers; feature slot i of a thread is
// f0 + 2 * kNormW * i, valid for i < F / 32 in the whole workgroup. Loads go out in batches;
// the stream gradient dhn_in is read per batch just before the matching writes (each
// element is read before it is written, so dhn may alias dhn_in). dw sums over the
// workgroup's tokens collect in LDS (each feature has one owning half-wave) until one
// partial row is written.
constexpr int kNormBwdTiles = 2;
constexpr int kNormBwdTok = 32 * kNormBwdTiles;  // tokens per workgroup
template <typename io_t>
__global__ __launch_bounds__(kNormW * 64) void add_rmsnorm_bwd_reg_kernel(NormParams p) {
  constexpr int kR = kNormRegs / 2;
  constexpr int kBatch = 8;
  __shared__ float s_c[kNormW][64];
  __shared__ float s_w[kNormW * kNormRegs];
  __shared__ float s_dw[kNormW * kNormRegs];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const size_t T = p.tokens;
  const int F = p.features;
  const int n_slots = F / (2 * kNormW);
  const int f0 = 2 * wv + (lane >> 5);
  const size_t stride = 2 * kNormW * T;  // elements between a thread's feature slots
  const size_t base = static_cast<size_t>(f0) * T;
  const bool has_din = p.dhn_in != nullptr;
  for (int f = threadIdx.x; f < F; f += kNormW * 64) {
    s_w[f] = p.w[f];
    s_dw[f] = 0.f;
  }
  for (int tile = 0; tile < kNormBwdTiles; ++tile) {
    const int t = (blockIdx.x * kNormBwdTiles + tile) * 32 + (lane & 31);
    const bool ok = t < p.tokens;
    const size_t tc = ok ? t : p.tokens - 1;
    const float* __restrict__ hn = p.h + base + tc;  // the forward's normalised input
    const io_t* __restrict__ dx = static_cast<const io_t*>(p.dx) + base + tc;
    const float r = p.rstd[tc];
    __syncthreads();  // s_w written; the previous tile's s_c reads are done
    float xh[kR], g[kR];
    float c = 0.f;
#pragma unroll
    for (int i0 = 0; i0 < kR; i0 += kBatch) {
      float hv[kBatch], gv[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int sl = i0 + k < n_slots ? i0 + k : n_slots - 1;  // clamped: no branch
        hv[k] = hn[sl * stride];
        gv[k] = to_f32(dx[sl * stride]);
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int i = i0 + k;
        const bool valid = ok && i < n_slots;
        xh[i] = valid ? hv[k] * r : 0.f;
        g[i] = valid ? gv[k] : 0.f;
        c = __builtin_fmaf(s_w[i < n_slots ? f0 + 2 * kNormW * i : 0] * g[i], xh[i], c);
      }
    }
    s_c[wv][lane] = c;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kNormW; ++i) tot += s_c[i][lane & 31] + s_c[i][(lane & 31) + 32];
    const float cm = tot / F;
    // Without a stream gradient the loads below read hn (valid memory) and are masked.
    const float* __restrict__ din_p = (has_din ? p.dhn_in : p.h) + base + tc;
    float* dhn = p.dhn + base + t;
    io_t* ddelta = p.ddelta ? static_cast<io_t*>(p.ddelta) + base + t : nullptr;
#pragma unroll
    for (int i0 = 0; i0 < kR; i0 += kBatch) {
      if (i0 >= n_slots) break;
      float din[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int sl = i0 + k < n_slots ? i0 + k : n_slots - 1;
        const float x = din_p[sl * stride];
        din[k] = has_din ? x : 0.f;
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int i = i0 + k;
        if (i >= n_slots) break;  // workgroup-uniform
        const int f = f0 + 2 * kNormW * i;
        const float d = __builtin_fmaf(r, __builtin_fmaf(s_w[f], g[i], -xh[i] * cm), din[k]);
        if (ok) {
          dhn[i * stride] = d;
          if (ddelta) store_as(ddelta + i * stride, d);
        }
        // dw of feature f over this half-wave's 32 tokens (zero past the last token): row
        // sums, then rows 0+1 into lane 31 and rows 2+3 into lane 63.
        float v = g[i] * xh[i];
        v += dpp_mov<kRowShr1, 0xF>(0.f, v);
        v += dpp_mov<kRowShr2, 0xF>(0.f, v);
        v += dpp_mov<kRowShr4, 0xF>(0.f, v);
        v += dpp_mov<kRowShr8, 0xF>(0.f, v);
        v += dpp_mov<kRowBcast15, 0xA>(0.f, v);
        if ((lane & 31) == 31) s_dw[f] += v;
      }
    }
  }
  __syncthreads();
  for (int f = threadIdx.x; f < F; f += kNormW * 64) p.dw_part[static_cast<size_t>(blockIdx.x) * F + f] = s_dw[f];
}

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
    // Four independent partial sums keep four loads in flight (fixed order throughout).
    float s4[4] = {0.f, 0.f, 0.f, 0.f};
    int i = wv;
    for (; i + 48 < n_blk; i += 64) {
#pragma unroll
      for (int k = 0; k < 4; ++k) s4[k] += part[static_cast<size_t>(i + 16 * k) * features + f];
    }
    for (; i < n_blk; i += 16) s4[0] += part[static_cast<size_t>(i) * features + f];
    s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
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

// Workgroups of the backward (also the dw partial rows the workspace holds): the register
// kernel's 32-token workgroups, which bound the 64-token ones of the wide-stream kernel.
int norm_blocks(int tokens) { return (tokens + kNormBwdTok - 1) / kNormBwdTok; }

hipError_t launch_norm_fwd(const NormParams& p, bool io_bf16, hipStream_t stream) {
  if (p.tokens <= kNormRowsMaxTokens) {
    if (io_bf16) hipLaunchKernelGGL(add_rmsnorm_fwd_rows_kernel<bf16_t>, dim3(p.tokens), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(add_rmsnorm_fwd_rows_kernel<float>, dim3(p.tokens), dim3(256), 0, stream, p);
    return hipGetLastError();
  }
  const dim3 grid((p.tokens + 63) / 64), block(kNormW * 64);
  if (p.features <= kNormW * kNormRegs) {
    if (io_bf16) hipLaunchKernelGGL(add_rmsnorm_fwd_reg_kernel<bf16_t>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(add_rmsnorm_fwd_reg_kernel<float>, grid, block, 0, stream, p);
  } else {
    if (io_bf16) hipLaunchKernelGGL(add_rmsnorm_fwd_kernel<bf16_t>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(add_rmsnorm_fwd_kernel<float>, grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

hipError_t launch_norm_bwd(const NormParams& p, bool io_bf16, float* dw, hipStream_t stream) {
  const bool regs = p.features <= kNormW * kNormRegs && p.features % (2 * kNormW) == 0;
  const int nb = regs ? norm_blocks(p.tokens) : (p.tokens + 63) / 64;
  if (regs) {
    if (io_bf16) hipLaunchKernelGGL(add_rmsnorm_bwd_reg_kernel<bf16_t>, dim3(nb), dim3(kNormW * 64), 0, stream, p);
    else hipLaunchKernelGGL(add_rmsnorm_bwd_reg_kernel<float>, dim3(nb), dim3(kNormW * 64), 0, stream, p);
  } else {
    if (io_bf16) hipLaunchKernelGGL(add_rmsnorm_bwd_kernel<bf16_t>, dim3(nb), dim3(kNormW * 64), 0, stream, p);
    else hipLaunchKernelGGL(add_rmsnorm_bwd_kernel<float>, dim3(nb), dim3(kNormW * 64), 0, stream, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(norm_dw_reduce_kernel, dim3((p.features + 63) / 64), dim3(1024), 0, stream,
                     p.dw_part, nb, p.features, dw);
  return hipGetLastError();
}

}  // namespace mss
