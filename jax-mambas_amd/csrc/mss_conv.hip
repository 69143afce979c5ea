// Causal depthwise conv1d (+ optional SiLU) over channel rows, forward and backward.
//
// The Mamba-1 block's short convolution (reference mamba/mamba1.py:250-255, 313-329:
// nnx.Conv with feature_group_count = channels, padding "CAUSAL", then silu), on the row
// layouts of the scan: each (b, d) row holds `seqlen` contiguous steps at
// b * sb + d * sd, so an (channels, B*L) activation matrix is read in place.
//
//   pre[t] = bias[d] + sum_{k<K} w[d][k] * x[t - (K-1) + k]      (x[t<0] = 0)
//   y[t]   = act(pre[t]),  y[t] = 0 for t >= seq_lens[b]
//
// Mapping: one thread = kE consecutive steps of one row (a 16-byte vector when rows are
// aligned, else kE = 1); grid (step tiles, channels, batch). On the vector path the K-1
// halo steps around a thread's vector come from its neighbours through LDS.
// Backward recomputes pre from x (no residual), forms g = dy * act'(pre), and writes
//   dx[t] = sum_k w[k] * g[t + (K-1) - k],   and per-block partials of
//   dw[k] = sum_t g[t] * x[t - (K-1) + k],   dbias = sum_t g[t]
// reduced in a fixed order by a second kernel (deterministic).
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

constexpr int kConvThreads = 256;

__device__ __forceinline__ float silu_grad(float p) {
  const float s = sigmoid(p);
  return s * (1.f + p * (1.f - s));
}

template <int kE, typename io_t>
__device__ __forceinline__ void load_vec(const io_t* __restrict__ p, float (&v)[kE]) {
  if constexpr (kE == 1) {
    v[0] = to_f32(p[0]);
  } else if constexpr (sizeof(io_t) == 4) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4*>(p);
    const unsigned w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
}

template <int kE, typename io_t>
__device__ __forceinline__ void store_vec(io_t* __restrict__ p, const float (&v)[kE]) {
  if constexpr (kE == 1) {
    store_as(p, v[0]);
  } else if constexpr (sizeof(io_t) == 4) {
    f32x4 a = {v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p) = a;
  } else {
    u32x4 a;
    unsigned w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    a.x = w[0]; a.y = w[1]; a.z = w[2]; a.w = w[3];
    *reinterpret_cast<u32x4*>(p) = a;
  }
}

// Scalar read of row element t (0 outside [0, L)).
template <typename io_t>
__device__ __forceinline__ float at(const io_t* __restrict__ row, int t, int L) {
  return (t >= 0 && t < L) ? to_f32(row[t]) : 0.f;
}

// Vector path (kE >= K-1): the K-1 steps before a thread's vector are the previous
// thread's last ones and, in the backward, the K-1 gradient terms after it are the next
// thread's first ones; they are exchanged through LDS, so only the first (last) thread of a
// workgroup reads its halo from global memory. Scalar path (kE = 1): halos are read.
template <int kK, int kE>
struct ConvShare {
  static constexpr bool kOn = kE > 1 && kK > 1;
  static constexpr int kRows = kOn ? kConvThreads : 1;
  static constexpr int kH = kK > 1 ? kK - 1 : 1;
};

template <int kK, int kE, bool kSilu, typename io_t>
__global__ __launch_bounds__(kConvThreads) void conv_fwd_kernel(ConvParams p) {
  using Sh = ConvShare<kK, kE>;
  __shared__ float s_tail[Sh::kRows][Sh::kH];
  const int L = p.seqlen;
  const int d = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int t0 = (blockIdx.x * kConvThreads + tid) * kE;
  const bool live = t0 < L;
  if (!Sh::kOn && !live) return;  // no barrier on the scalar path
  const long long row = b * p.sb + d * p.sd;
  const io_t* __restrict__ xr = static_cast<const io_t*>(p.x) + row;
  io_t* __restrict__ yr = static_cast<io_t*>(p.y) + row;
  const int len = p.seq_lens ? min(max(p.seq_lens[b], 0), L) : L;
  float w[kK];
#pragma unroll
  for (int k = 0; k < kK; ++k) w[k] = p.w[d * kK + k];
  const float bias = p.bias ? p.bias[d] : 0.f;

  float xe[kE + kK - 1];  // x[t0 - (K-1) .. t0 + kE)
  float v[kE];
  const bool full = kE > 1 && t0 + kE <= L;
  if (full) {
    load_vec<kE>(xr + t0, v);
  } else {
#pragma unroll
    for (int j = 0; j < kE; ++j) v[j] = at(xr, t0 + j, L);
  }
  if constexpr (Sh::kOn) {
#pragma unroll
    for (int k = 0; k < kK - 1; ++k) s_tail[tid][k] = v[kE - (kK - 1) + k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kK - 1; ++k)
      xe[k] = tid > 0 ? s_tail[tid - 1][k] : at(xr, t0 - (kK - 1) + k, L);
    if (!live) return;
  } else {
#pragma unroll
    for (int k = 0; k < kK - 1; ++k) xe[k] = at(xr, t0 - (kK - 1) + k, L);
  }
#pragma unroll
  for (int j = 0; j < kE; ++j) xe[kK - 1 + j] = v[j];
  float out[kE];
#pragma unroll
  for (int j = 0; j < kE; ++j) {
    float pre = bias;
#pragma unroll
    for (int k = 0; k < kK; ++k) pre = __builtin_fmaf(w[k], xe[j + k], pre);
    out[j] = (t0 + j < len) ? (kSilu ? pre * sigmoid(pre) : pre) : 0.f;
  }
  if (full) {
    store_vec<kE>(yr + t0, out);
  } else {
#pragma unroll
    for (int j = 0; j < kE; ++j)
      if (t0 + j < L) store_as(yr + t0 + j, out[j]);
  }
}

template <int kK, int kE, bool kSilu, typename io_t>
__global__ __launch_bounds__(kConvThreads) void conv_bwd_kernel(ConvParams p) {
  using Sh = ConvShare<kK, kE>;
  __shared__ float s_red[kConvThreads / 64][kK + 1];
  __shared__ float s_xt[Sh::kRows][Sh::kH];  // last K-1 x of each thread's vector
  __shared__ float s_gh[Sh::kRows][Sh::kH];  // first K-1 gradient terms g of each thread
  const int L = p.seqlen;
  const int d = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int t0 = (blockIdx.x * kConvThreads + tid) * kE;
  const long long row = b * p.sb + d * p.sd;
  const io_t* __restrict__ xr = static_cast<const io_t*>(p.x) + row;
  const io_t* __restrict__ gr = static_cast<const io_t*>(p.dy) + row;
  io_t* __restrict__ dxr = static_cast<io_t*>(p.dx) + row;
  const int len = p.seq_lens ? min(max(p.seq_lens[b], 0), L) : L;
  float w[kK];
#pragma unroll
  for (int k = 0; k < kK; ++k) w[k] = p.w[d * kK + k];
  const float bias = p.bias ? p.bias[d] : 0.f;

  float dw[kK + 1];  // [0, K): dw, K: dbias
#pragma unroll
  for (int k = 0; k <= kK; ++k) dw[k] = 0.f;

  // Threads past the row's end (t0 >= L) hold zeros and take part in the barriers.
  // x[t0 - (K-1) .. t0 + kE + K - 1) and g[t0 .. t0 + kE + K - 1)
  constexpr int kX = kE + 2 * (kK - 1);
  constexpr int kG = kE + kK - 1;
  float xe[kX];
  float ge[kG];
  const bool full = kE > 1 && t0 + kE <= L;
  float v[kE], dv[kE];
  if (full) {
    load_vec<kE>(xr + t0, v);
    load_vec<kE>(gr + t0, dv);
  } else {
#pragma unroll
    for (int j = 0; j < kE; ++j) {
      v[j] = at(xr, t0 + j, L);
      dv[j] = at(gr, t0 + j, L);
    }
  }
#pragma unroll
  for (int j = 0; j < kE; ++j) {
    xe[kK - 1 + j] = v[j];
    ge[j] = dv[j];
  }
  // The last thread of the workgroup (or every thread on the scalar path) reads the halo
  // after its vector; the others take the next thread's gradient terms below.
  const bool own_after = !Sh::kOn || tid == kConvThreads - 1;
  if constexpr (Sh::kOn) {
#pragma unroll
    for (int k = 0; k < kK - 1; ++k) s_xt[tid][k] = v[kE - (kK - 1) + k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kK - 1; ++k)
      xe[k] = tid > 0 ? s_xt[tid - 1][k] : at(xr, t0 - (kK - 1) + k, L);
  } else {
#pragma unroll
    for (int k = 0; k < kK - 1; ++k) xe[k] = at(xr, t0 - (kK - 1) + k, L);
  }
#pragma unroll
  for (int k = 0; k < kK - 1; ++k) {
    xe[kK - 1 + kE + k] = own_after ? at(xr, t0 + kE + k, L) : 0.f;
    ge[kE + k] = own_after ? at(gr, t0 + kE + k, L) : 0.f;
  }
  // g[t] = dy[t] * act'(pre[t]) for own steps (and the after-halo when read here); 0 past
  // the length.
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    if (j >= kE && !own_after) continue;
    float pre = bias;
#pragma unroll
    for (int k = 0; k < kK; ++k) pre = __builtin_fmaf(w[k], xe[j + k], pre);
    const float gj = kSilu ? ge[j] * silu_grad(pre) : ge[j];
    ge[j] = (t0 + j < len) ? gj : 0.f;
  }
  if constexpr (Sh::kOn) {
#pragma unroll
    for (int k = 0; k < kK - 1; ++k) s_gh[tid][k] = ge[k];
    __syncthreads();
    if (!own_after) {
#pragma unroll
      for (int k = 0; k < kK - 1; ++k) ge[kE + k] = s_gh[tid + 1][k];
    }
  }
  if (t0 < L) {
    float dx[kE];
#pragma unroll
    for (int j = 0; j < kE; ++j) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < kK; ++k) s = __builtin_fmaf(w[k], ge[j + kK - 1 - k], s);
      dx[j] = s;
      // own steps only for the weight sums
#pragma unroll
      for (int k = 0; k < kK; ++k) dw[k] = __builtin_fmaf(ge[j], xe[j + k], dw[k]);
      dw[kK] += ge[j];
    }
    if (full) {
      store_vec<kE>(dxr + t0, dx);
    } else {
#pragma unroll
      for (int j = 0; j < kE; ++j)
        if (t0 + j < L) store_as(dxr + t0 + j, dx[j]);
    }
  }
  // block sums of dw / dbias -> partial slot (d, b, blockIdx.x)
#pragma unroll
  for (int k = 0; k <= kK; ++k) dw[k] = wave_sum(dw[k]);
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int k = 0; k <= kK; ++k) s_red[wv][k] = dw[k];
  }
  __syncthreads();
  if (threadIdx.x <= kK) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kConvThreads / 64; ++i) s += s_red[i][threadIdx.x];
    const size_t slot = (static_cast<size_t>(d) * p.batch + b) * gridDim.x + blockIdx.x;
    p.part[slot * (kK + 1) + threadIdx.x] = s;
  }
}

// dw[d][k] = sum over (b, tile) partials, fixed order; dbias likewise.
__global__ __launch_bounds__(256) void conv_reduce_kernel(const float* __restrict__ part, int n_slot,
                                                          int dim, int width, float* dw, float* dbias) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= dim * (width + 1)) return;
  const int d = i / (width + 1);
  const int k = i - d * (width + 1);
  const float* src = part + static_cast<size_t>(d) * n_slot * (width + 1) + k;
  float s = 0.f;
  for (int j = 0; j < n_slot; ++j) s += src[static_cast<size_t>(j) * (width + 1)];
  if (k < width) {
    dw[d * width + k] = s;
  } else if (dbias) {
    dbias[d] = s;
  }
}

int conv_tile_steps(int vec, int io_bf16) { return kConvThreads * (vec ? (io_bf16 ? 8 : 4) : 1); }

template <int kK, bool kSilu, typename io_t>
static hipError_t launch_conv_t(const ConvParams& p, bool bwd, bool vec, hipStream_t stream) {
  constexpr int kV = sizeof(io_t) == 2 ? 8 : 4;
  const int per = vec ? kV : 1;
  const dim3 grid((p.seqlen + kConvThreads * per - 1) / (kConvThreads * per), p.dim, p.batch);
  if (bwd) {
    if (vec) hipLaunchKernelGGL((conv_bwd_kernel<kK, kV, kSilu, io_t>), grid, dim3(kConvThreads), 0, stream, p);
    else hipLaunchKernelGGL((conv_bwd_kernel<kK, 1, kSilu, io_t>), grid, dim3(kConvThreads), 0, stream, p);
  } else {
    if (vec) hipLaunchKernelGGL((conv_fwd_kernel<kK, kV, kSilu, io_t>), grid, dim3(kConvThreads), 0, stream, p);
    else hipLaunchKernelGGL((conv_fwd_kernel<kK, 1, kSilu, io_t>), grid, dim3(kConvThreads), 0, stream, p);
  }
  return hipGetLastError();
}

template <int kK, typename io_t>
static hipError_t launch_conv_k(const ConvParams& p, bool bwd, bool vec, bool silu, hipStream_t stream) {
  return silu ? launch_conv_t<kK, true, io_t>(p, bwd, vec, stream)
              : launch_conv_t<kK, false, io_t>(p, bwd, vec, stream);
}

template <typename io_t>
static hipError_t launch_conv_io(const ConvParams& p, bool bwd, bool vec, bool silu, hipStream_t stream) {
  switch (p.width) {
    case 1: return launch_conv_k<1, io_t>(p, bwd, vec, silu, stream);
    case 2: return launch_conv_k<2, io_t>(p, bwd, vec, silu, stream);
    case 3: return launch_conv_k<3, io_t>(p, bwd, vec, silu, stream);
    default: return launch_conv_k<4, io_t>(p, bwd, vec, silu, stream);
  }
}

hipError_t launch_conv(const ConvParams& p, bool bwd, bool vec, bool silu, bool io_bf16,
                       hipStream_t stream) {
  return io_bf16 ? launch_conv_io<bf16_t>(p, bwd, vec, silu, stream)
                 : launch_conv_io<float>(p, bwd, vec, silu, stream);
}

hipError_t launch_conv_reduce(const ConvParams& p, int n_tiles, float* dw, float* dbias,
                              hipStream_t stream) {
  const int n = p.dim * (p.width + 1);
  hipLaunchKernelGGL(conv_reduce_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, p.part,
                     p.batch * n_tiles, p.dim, p.width, dw, dbias);
  return hipGetLastError();
}

}  // namespace mss
