// Single-token recurrent step (decode): selective-state update and causal-conv window update.
//
// Reference behaviour: S6.step (mamba/mamba1.py:200-214: a_bar = exp(delta*A), Euler or ZOH
// b_bar, x = a_bar * state + b_bar * u, y = C . x + D * u) and Mamba.step (:339-363: the
// conv cache holds the last K-1 inputs; the step convolves [cache, x] and shifts the
// cache; silu; the block gates the SSM output by silu(z)), with the scan's fused extras:
//   delta = softplus(delta_raw + bias) (optional), D skip, out = y * silu(z) (optional).
// A 16-lane DPP row per (b, d) channel, one lane per state. Inputs use the scan's row
// strides (elements): u/delta/z/out at b*io_sb + d*io_sd, B/C at b*bc_sb + n*bc_sn, so a
// (features, batch) activation matrix is read in place. The state is [B][D][N] float32,
// updated in place (the layout of the scan's last_state, so a prefill hands over directly).
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

// Lane = state n, a 16-lane DPP row = one (b, d) channel (N <= 16; lanes n >= N idle
// but take part in the row sum).
template <bool kZOH, typename io_t, typename bc_t>
__global__ __launch_bounds__(256) void ssm_step_kernel(StepParams p) {
  const long long idx = (static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x) >> 4;
  const int n = threadIdx.x & 15;
  const bool ch_ok = idx < static_cast<long long>(p.batch) * p.dim;
  const int b = ch_ok ? static_cast<int>(idx % p.batch) : 0;  // batch fastest: coalesced for (D, B)
  const int d = ch_ok ? static_cast<int>(idx / p.batch) : 0;
  const int N = p.dstate;
  const bool on = ch_ok && n < N;
  const long long io = b * p.io_sb + d * p.io_sd;
  float yv = 0.f, u = 0.f;
  if (ch_ok) {
    u = to_f32(static_cast<const io_t*>(p.u)[io]);
    float dt = to_f32(static_cast<const io_t*>(p.delta)[io]) + (p.delta_bias ? p.delta_bias[d] : 0.f);
    if (p.delta_softplus) dt = softplus(dt);
    if (on) {
      const float an = p.A[static_cast<size_t>(d) * N + n];
      const float a = fast_exp2(dt * an * kLog2e);
      const float bn = to_f32(static_cast<const bc_t*>(p.B)[b * p.bc_sb + n * p.bc_sn]);
      const float bu = kZOH ? (expm1f(dt * an) / an) * bn * u : dt * bn * u;
      float* st = p.state + (static_cast<size_t>(b) * p.dim + d) * N + n;
      const float h = __builtin_fmaf(a, *st, bu);
      *st = h;
      yv = to_f32(static_cast<const bc_t*>(p.C)[b * p.bc_sb + n * p.bc_sn]) * h;
    }
  }
  // sum over the row's 16 lanes: lane 15 ends with the total
  yv += dpp_mov<kRowShr1, 0xF>(0.f, yv);
  yv += dpp_mov<kRowShr2, 0xF>(0.f, yv);
  yv += dpp_mov<kRowShr4, 0xF>(0.f, yv);
  yv += dpp_mov<kRowShr8, 0xF>(0.f, yv);
  if (ch_ok && n == 15) {
    float y = yv;
    if (p.D) y = __builtin_fmaf(p.D[d], u, y);
    if (p.z) {
      const float z = to_f32(static_cast<const io_t*>(p.z)[io]);
      y *= z * sigmoid(z);
    }
    store_as(static_cast<io_t*>(p.out) + io, y);
  }
}

template <typename io_t>
__global__ __launch_bounds__(256) void conv_step_kernel(ConvStepParams p) {
  const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<long long>(p.batch) * p.dim) return;
  const int b = static_cast<int>(idx % p.batch);
  const int d = static_cast<int>(idx / p.batch);
  const int K = p.width;
  const long long io = b * p.sb + d * p.sd;
  io_t* cache = static_cast<io_t*>(p.state) + (static_cast<size_t>(b) * p.dim + d) * (K - 1);
  const float x = to_f32(static_cast<const io_t*>(p.x)[io]);
  const float* w = p.w + static_cast<size_t>(d) * K;
  float pre = p.bias ? p.bias[d] : 0.f;
  // window = [cache[0], ..., cache[K-2], x]; the cache shifts left by one.
  for (int k = 0; k < K - 1; ++k) {
    const float v = to_f32(cache[k]);
    pre = __builtin_fmaf(w[k], v, pre);
    if (k > 0) cache[k - 1] = cache[k];
  }
  pre = __builtin_fmaf(w[K - 1], x, pre);
  if (K > 1) store_as(cache + K - 2, x);
  const float y = p.act ? pre * sigmoid(pre) : pre;
  store_as(static_cast<io_t*>(p.y) + io, y);
}

hipError_t launch_ssm_step(const StepParams& p, bool zoh, bool io_bf16, bool bc_bf16, hipStream_t stream) {
  const long long n = static_cast<long long>(p.batch) * p.dim * 16;  // 16 lanes per channel
  const dim3 grid(static_cast<unsigned>((n + 255) / 256)), block(256);
#define MSS_STEP(Z, IO, BC) hipLaunchKernelGGL((ssm_step_kernel<Z, IO, BC>), grid, block, 0, stream, p)
  if (zoh) {
    if (io_bf16) { if (bc_bf16) MSS_STEP(true, bf16_t, bf16_t); else MSS_STEP(true, bf16_t, float); }
    else { if (bc_bf16) MSS_STEP(true, float, bf16_t); else MSS_STEP(true, float, float); }
  } else {
    if (io_bf16) { if (bc_bf16) MSS_STEP(false, bf16_t, bf16_t); else MSS_STEP(false, bf16_t, float); }
    else { if (bc_bf16) MSS_STEP(false, float, bf16_t); else MSS_STEP(false, float, float); }
  }
#undef MSS_STEP
  return hipGetLastError();
}

hipError_t launch_conv_step(const ConvStepParams& p, bool io_bf16, hipStream_t stream) {
  const long long n = static_cast<long long>(p.batch) * p.dim;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256)), block(256);
  if (io_bf16) hipLaunchKernelGGL(conv_step_kernel<bf16_t>, grid, block, 0, stream, p);
  else hipLaunchKernelGGL(conv_step_kernel<float>, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace mss
