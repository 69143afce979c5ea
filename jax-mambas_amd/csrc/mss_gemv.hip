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

// s[i] of a register array as a chain of selects. Each candidate goes through an empty
// asm so that the chain is not folded back into one indexed load, which the compiler
// would serve from scratch memory.
template <int kN>
__device__ __forceinline__ float pick(const float (&s)[kN], int i) {
  float v = s[0];
#pragma unroll
  for (int c = 1; c < kN; ++c) {
    float sc = s[c];
    asm("; pick %1" : "+v"(sc) : "n"(c));
    v = i == c ? sc : v;
  }
  return v;
}

// Totals over the wave of 8 values per lane (a row's 8 token sums), returned transposed:
// every lane holds the total of value (lane & 7). Three in-row exchange steps each keep half
// of a lane's values and add its partner's matching half (partners: the row_half_mirror
// pair i <-> 7-i of each 8 lanes, then XOR 2, then XOR 1 within quads; each pairs lanes that
// hold the same set of values), which leaves value 4*bit2 + 2*bit1 + bit0 = lane & 7 in
// every lane; then the lanes holding the same value are summed: row_ror:8 within the row,
// a swizzle across rows (XOR 16), a permute across halves (XOR 32). 26 instructions against
// 8 full-wave sums of 7; a fixed order, so the result is deterministic.
constexpr int kRowHalfMirror = 0x141, kQuadXor2 = 0x4E, kQuadXor1 = 0xB1, kRowRor8 = 0x128;

__device__ __forceinline__ float wave_sum8(const float (&x)[8]) {
  const int lane = threadIdx.x & 63;
  float y[4], z[2];
  const bool lo4 = (lane & 4) == 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float keep = lo4 ? x[i] : x[i + 4];
    const float send = lo4 ? x[i + 4] : x[i];
    y[i] = keep + dpp_mov<kRowHalfMirror, 0xF>(0.f, send);
  }
  const bool lo2 = (lane & 2) == 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float keep = lo2 ? y[i] : y[i + 2];
    const float send = lo2 ? y[i + 2] : y[i];
    z[i] = keep + dpp_mov<kQuadXor2, 0xF>(0.f, send);
  }
  const bool lo1 = (lane & 1) == 0;
  float v = (lo1 ? z[0] : z[1]) + dpp_mov<kQuadXor1, 0xF>(0.f, lo1 ? z[1] : z[0]);
  v += dpp_mov<kRowRor8, 0xF>(0.f, v);
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, v)));
  return v;
}

// Offsets into the step operands are int: the entry points reject calls whose operands
// span 2^31 elements or more.
//
// Raw bits of the fused epilogues' operands, loaded before the products so their latency
// overlaps the weight reads. The loads are unconditional (indexes clamped into range,
// absent optional operands read from a present one) and the bf16 values stay as bits
// until after the barrier, so no load waits on its own inside a branch: the vector
// memory counter is in order, and any such wait would also wait for the weights.
__device__ __forceinline__ float bits_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

// Conv-window step of channel m for token `lane` (lanes < kN): weights, bias, window.
struct ConvOperands {
  float w[4], bias;
  uint32_t c[3];
};

__device__ __forceinline__ void load_conv(const ConvStepParams& p, int m, int lane, int n_tok, ConvOperands& o) {
  const int K = p.width;
  const int mm = m < p.dim ? m : 0;
  const int b = lane < n_tok ? lane : 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) o.w[k] = p.w[mm * K + min(k, K - 1)];
  o.bias = p.bias ? p.bias[mm] : 0.f;
  // width 1 has no window state (the pointer may be null): read the weights instead, unused
  const uint16_t* cache = K > 1 ? static_cast<const uint16_t*>(p.state) + (b * p.dim + mm) * (K - 1)
                                : reinterpret_cast<const uint16_t*>(p.w);
#pragma unroll
  for (int k = 0; k < 3; ++k) o.c[k] = cache[min(k, max(K - 2, 0))];
}

// Conv-window step of channel m for token `lane` on x (rounded to bf16): the arithmetic
// of conv_step_kernel (mss_step.hip): pre = bias + sum_k w[k] window[k] over
// window = [state, x], y = act(pre), the state shifts left and takes x.
__device__ __forceinline__ void conv_step_core(const ConvStepParams& p, int m, int b, float x, const ConvOperands& o) {
  const int K = p.width;
  bf16_t* cache = static_cast<bf16_t*>(p.state) + (b * p.dim + m) * (K - 1);
  float pre = o.bias;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    if (k < K - 1) {
      pre = __builtin_fmaf(o.w[k], bits_f32(o.c[k]), pre);
      if (k > 0) cache[k - 1].bits = static_cast<uint16_t>(o.c[k]);
    }
  }
  pre = __builtin_fmaf(pick<4>(o.w, K - 1), x, pre);
  if (K > 1) cache[K - 2] = f32_to_bf16(x);
  const float y = p.act ? pre * sigmoid(pre) : pre;
  static_cast<bf16_t*>(p.y)[b * static_cast<int>(p.sb) + m * static_cast<int>(p.sd)] = f32_to_bf16(y);
}

template <int kN>
__device__ __forceinline__ void conv_epilogue(const ConvStepParams& p, int m, const float (&s)[kN], int lane,
                                              const ConvOperands& o) {
  if (lane >= kN) return;
  conv_step_core(p, m, lane, pick<kN>(s, lane), o);
}

// Selective-state step of channel d: lanes are (token, state) pairs, 16 lanes (one DPP
// row) per token, four tokens per pass.
template <int kP>
struct SsmOperands {
  float a[kP], h[kP];
  uint32_t u[kP], b[kP], c[kP], z[kP];
  float bias, D;
};

template <int kN>
__device__ __forceinline__ void load_ssm(const StepParams& p, int d, int lane, SsmOperands<(kN + 3) / 4>& o) {
  const int N = p.dstate;
  const int n = min(lane & 15, N - 1);
  const uint16_t* U = static_cast<const uint16_t*>(p.u);
  const uint16_t* Z = static_cast<const uint16_t*>(p.z ? p.z : p.u);
  const uint16_t* Bm = static_cast<const uint16_t*>(p.B);
  const uint16_t* Cm = static_cast<const uint16_t*>(p.C);
  o.bias = p.delta_bias ? p.delta_bias[d] : 0.f;
  o.D = p.D ? p.D[d] : 0.f;
#pragma unroll
  for (int pass = 0; pass < (kN + 3) / 4; ++pass) {
    const int tok = pass * 4 + (lane >> 4);
    const int b = tok < kN ? tok : 0;
    const int io = b * static_cast<int>(p.io_sb) + d * static_cast<int>(p.io_sd);
    const int bc = b * static_cast<int>(p.bc_sb) + n * static_cast<int>(p.bc_sn);
    o.u[pass] = U[io];
    o.z[pass] = Z[io];
    o.a[pass] = p.A[d * N + n];
    o.b[pass] = Bm[bc];
    o.c[pass] = Cm[bc];
    o.h[pass] = p.state[(b * p.dim + d) * N + n];
  }
}

// Selective-state step of channel d on the raw delta (rounded to bf16): the arithmetic of
// ssm_step_kernel (mss_step.hip): delta = softplus(raw + bias), h = exp(delta A) h +
// b_bar u, y = sum_n C h + D u, out = y silu(z).
template <int kN>
__device__ __forceinline__ void ssm_epilogue(const StepParams& p, bool zoh, int d, const float (&s)[kN], int lane,
                                             const SsmOperands<(kN + 3) / 4>& o) {
  const int n = lane & 15;
  const int N = p.dstate;
#pragma unroll
  for (int pass = 0; pass < (kN + 3) / 4; ++pass) {
    const int tok = pass * 4 + (lane >> 4);
    const bool ok = tok < kN;
    const int b = ok ? tok : 0;
    const float u = bits_f32(o.u[pass]);
    float dt = pick<kN>(s, b) + o.bias;
    if (p.delta_softplus) dt = softplus(dt);
    float yv = 0.f;
    if (ok && n < N) {
      const float an = o.a[pass];
      const float a = fast_exp2(dt * an * kLog2e);
      const float bn = bits_f32(o.b[pass]);
      const float bu = zoh ? (expm1f(dt * an) / an) * bn * u : dt * bn * u;
      const float h = __builtin_fmaf(a, o.h[pass], bu);
      p.state[(b * p.dim + d) * N + n] = h;
      yv = bits_f32(o.c[pass]) * h;
    }
    yv += dpp_mov<kRowShr1, 0xF>(0.f, yv);
    yv += dpp_mov<kRowShr2, 0xF>(0.f, yv);
    yv += dpp_mov<kRowShr4, 0xF>(0.f, yv);
    yv += dpp_mov<kRowShr8, 0xF>(0.f, yv);
    if (ok && n == 15) {
      float y = yv;
      if (p.D) y = __builtin_fmaf(o.D, u, y);
      if (p.z) {
        const float z = bits_f32(o.z[pass]);
        y *= z * sigmoid(z);
      }
      static_cast<bf16_t*>(p.out)[b * static_cast<int>(p.io_sb) + d * static_cast<int>(p.io_sd)] = f32_to_bf16(y);
    }
  }
}


// Features of the residual stream one thread holds in the norm prologue.
constexpr int kNormFeat = kNormGemvMaxFeatures / 256;

// kN float32 values of one stream row (16-byte aligned when kN >= 4).
template <int kN>
__device__ __forceinline__ void load_hrow(const float* h, float (&v)[kN]) {
  if constexpr (kN >= 4) {
#pragma unroll
    for (int q = 0; q < kN / 4; ++q) {
      const f32x4 a = reinterpret_cast<const f32x4*>(h)[q];
      v[4 * q] = a.x;
      v[4 * q + 1] = a.y;
      v[4 * q + 2] = a.z;
      v[4 * q + 3] = a.w;
    }
  } else if constexpr (kN == 2) {
    const float2 a = *reinterpret_cast<const float2*>(h);
    v[0] = a.x;
    v[1] = a.y;
  } else {
    v[0] = h[0];
  }
}

template <int kN>
__device__ __forceinline__ void store_hrow(float* h, const float (&v)[kN]) {
  if constexpr (kN >= 4) {
#pragma unroll
    for (int q = 0; q < kN / 4; ++q)
      reinterpret_cast<f32x4*>(h)[q] = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
  } else if constexpr (kN == 2) {
    *reinterpret_cast<float2*>(h) = float2{v[0], v[1]};
  } else {
    h[0] = v[0];
  }
}

// kN bf16 values as one 2kN-byte store (LDS).
template <int kN>
__device__ __forceinline__ void store_xrow(bf16_t* x, const float (&v)[kN]) {
  uint32_t b[kN];
#pragma unroll
  for (int c = 0; c < kN; ++c) b[c] = f32_to_bf16(v[c]).bits;
  if constexpr (kN == 8) {
    *reinterpret_cast<u32x4*>(x) = u32x4{b[0] | b[1] << 16, b[2] | b[3] << 16, b[4] | b[5] << 16, b[6] | b[7] << 16};
  } else if constexpr (kN == 4) {
    *reinterpret_cast<uint2*>(x) = uint2{b[0] | b[1] << 16, b[2] | b[3] << 16};
  } else if constexpr (kN == 2) {
    *reinterpret_cast<uint32_t*>(x) = b[0] | b[1] << 16;
  } else {
    x[0].bits = static_cast<uint16_t>(b[0]);
  }
}

// X = RMSNorm(h + delta) * w of the kN tokens into LDS: the arithmetic of
// add_rmsnorm_fwd_rows_kernel (mss_norm.hip) for each token, in the same order (thread t
// sums its features t, t + 256, .. by fma, the waves by wave_sum, then waves 0..3 in
// order; x = (hn * rstd) * w rounded to bf16), so X equals that kernel's output bit for
// bit. Every workgroup computes X (a few KB from the L2); workgroup 0 also stores hn and
// rstd. The stream loads are issued before any use, behind the weights already in flight.
template <int kN, bool kTransposed = false>
__device__ __forceinline__ void norm_prologue(const NormParams& q, int K, bf16_t* X, float (*s_ss)[4]) {
  const int tid = threadIdx.x;
  const bf16_t* __restrict__ delta = static_cast<const bf16_t*>(q.delta);
  float v[kNormFeat][kN], w[kNormFeat];
#pragma unroll
  for (int j = 0; j < kNormFeat; ++j) {
    const int f = min(tid + 256 * j, K - 1);
    load_hrow<kN>(q.h + f * kN, v[j]);
    w[j] = q.w[f];
  }
  if (delta) {
    float dv[kNormFeat][kN];
#pragma unroll
    for (int j = 0; j < kNormFeat; ++j) load_xrow<kN>(delta + min(tid + 256 * j, K - 1) * kN, dv[j]);
#pragma unroll
    for (int j = 0; j < kNormFeat; ++j)
#pragma unroll
      for (int c = 0; c < kN; ++c) v[j][c] += dv[j][c];
  }
  float ss[kN];
#pragma unroll
  for (int c = 0; c < kN; ++c) ss[c] = 0.f;
#pragma unroll
  for (int j = 0; j < kNormFeat; ++j) {
    if (tid + 256 * j < K) {
#pragma unroll
      for (int c = 0; c < kN; ++c) ss[c] = __builtin_fmaf(v[j][c], v[j][c], ss[c]);
    }
  }
#pragma unroll
  for (int c = 0; c < kN; ++c) {
    const float t = wave_sum(ss[c]);
    if ((tid & 63) == 0) s_ss[c][tid >> 6] = t;
  }
  __syncthreads();
  float r[kN];
#pragma unroll
  for (int c = 0; c < kN; ++c) {
    const float tot = s_ss[c][0] + s_ss[c][1] + s_ss[c][2] + s_ss[c][3];
    r[c] = 1.f / __builtin_sqrtf(tot / K + q.eps);
  }
  const bool first = blockIdx.x == 0;
#pragma unroll
  for (int j = 0; j < kNormFeat; ++j) {
    const int f = tid + 256 * j;
    if (f < K) {
      if (first && delta) store_hrow<kN>(q.hn + f * kN, v[j]);
      float x[kN];
#pragma unroll
      for (int c = 0; c < kN; ++c) x[c] = v[j][c] * r[c] * w[j];
      if constexpr (kTransposed) {
#pragma unroll
        for (int c = 0; c < kN; ++c) X[c * K + f] = f32_to_bf16(x[c]);  // [kN][K]
      } else {
        store_xrow<kN>(X + f * kN, x);
      }
    }
  }
  if (first && q.rstd && tid == 0) {
#pragma unroll
    for (int c = 0; c < kN; ++c) q.rstd[c] = r[c];
  }
}

// A workgroup of 4 waves stages X (K x N bf16, at most 64 KB) in LDS once; each wave
// produces kR consecutive rows of Y: lane l covers K elements 8l + 512 s (s = 0, 1, ..),
// reading 16 bytes of each of its kR weight rows per step, and the wave sums over its
// lanes. The first kPre steps of weights, and a fused epilogue's operands, are loaded
// before X is staged, so one memory latency covers them all. Rows past M are clamped to
// M - 1 for the reads and never stored. The row's sums are rounded to bf16 before the
// epilogue (kEpi, as GemvParams::epi), so a fused epilogue sees the values the separate
// step kernel would read back from Y. kNorm: X is the norm prologue's (norm_prologue).
// kS 4 (plain GEMMs with one row per wave only): the workgroup's 4 waves share a row, wave
// ws taking the 512-element K steps ws, ws + 4, .. (their X rows read straight into
// registers); their per-token totals are added through LDS in wave order, so launches of
// few rows fill more of the chip.
template <int kN, int kR, int kEpi, int kPre, bool kNorm, int kS = 1>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
  static_assert(kEpi == 0 || kR == 1, "fused epilogues take one row per wave");
  static_assert(kS == 1 || (kS == 4 && kR == 1 && kEpi == 0 && !kNorm), "K split: plain GEMMs, one row");
  extern __shared__ u32x4 s_x[];
  __shared__ float s_ss[kNorm ? kN : 1][4];
  __shared__ float s_red[kS > 1 ? kS : 1][kN];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int ws = kS > 1 ? tid >> 6 : 0;  // this wave's share of the K steps
  // wave-uniform row index in a scalar register (the per-channel operands then come
  // through scalar loads)
  const int m0 = __builtin_amdgcn_readfirstlane(kS > 1 ? blockIdx.x : (blockIdx.x * 4 + (tid >> 6)) * kR);
  const bool wave_on = m0 < p.M;
  const int mc = min(m0, p.M - 1);  // rows past M read row M - 1 (no branch around loads)
  const bf16_t* __restrict__ W = static_cast<const bf16_t*>(p.W);
  u32x4 wq[kPre][kR];
  ConvOperands co;
  SsmOperands<(kN + 3) / 4> so;
  if constexpr (kEpi == 1) load_conv(p.cs, mc, lane, kN, co);
  if constexpr (kEpi == 2) load_ssm<kN>(p.ss, mc, lane, so);
#pragma unroll
  for (int st = 0; st < kPre; ++st) {
    const int k0 = lane * 8 + 512 * (st * kS + ws);
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const int m = min(mc + r, p.M - 1);
      // steps past K re-read the row's first slice (unused)
      wq[st][r] = *reinterpret_cast<const u32x4*>(W + static_cast<size_t>(m) * p.ldw + (k0 < p.K ? k0 : 0));
    }
  }
  // K split over the waves (kRegX): each lane reads only its own K slices of X (8 k x kN
  // tokens = kN 16-byte words per step), straight from global memory into registers, issued
  // with the weight slices: no LDS stage and no barrier before the products (130M decode
  // step: 0.533 -> 0.500 ms). Otherwise X is staged once per workgroup in LDS (reading it
  // into registers there too, with one row per wave, measured 0.513 ms).
  constexpr bool kRegX = kS > 1;
  const u32x4* __restrict__ xg = static_cast<const u32x4*>(p.X);
  u32x4 xq[kRegX ? kPre : 1][kN];
  if constexpr (kRegX) {
#pragma unroll
    for (int st = 0; st < kPre; ++st) {
      const int k0 = lane * 8 + 512 * (st * kS + ws);
      const int kk = k0 < p.K ? k0 : 0;  // steps past K re-read the first slice (unused)
#pragma unroll
      for (int j = 0; j < kN; ++j) xq[st][j] = xg[kk * kN / 8 + j];
    }
  } else {
    if constexpr (kNorm) {
      norm_prologue<kN>(p.nm, p.K, reinterpret_cast<bf16_t*>(s_x), s_ss);
    } else {
      const int n_q = p.K * kN / 8;  // 16-byte words of X (K % 8 == 0)
      for (int i = tid; i < n_q; i += 256) s_x[i] = xg[i];
    }
    __syncthreads();
  }
  if (!wave_on) return;  // (kS > 1: every wave has a row; its later barrier is reached by all)
  const bf16_t* X = reinterpret_cast<const bf16_t*>(s_x);
  float acc[kR][kN];
#pragma unroll
  for (int r = 0; r < kR; ++r)
#pragma unroll
    for (int c = 0; c < kN; ++c) acc[r][c] = 0.f;
  if constexpr (kRegX) {
    // products of one step from registers: weight slice q, X words x
    auto reg_step = [&](const u32x4& q, const u32x4 (&x)[kN]) {
      const uint32_t a[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float w = e & 1 ? __uint_as_float(a[e / 2] & 0xffff0000u) : __uint_as_float(a[e / 2] << 16);
#pragma unroll
        for (int c = 0; c < kN; ++c) {
          const int i = e * kN + c;  // bf16 element i of the step's kN words
          const uint32_t v[4] = {x[i / 8].x, x[i / 8].y, x[i / 8].z, x[i / 8].w};
          const float xv = i & 1 ? __uint_as_float(v[(i % 8) / 2] & 0xffff0000u) : __uint_as_float(v[(i % 8) / 2] << 16);
          acc[0][c] = __builtin_fmaf(w, xv, acc[0][c]);
        }
      }
    };
#pragma unroll
    for (int st = 0; st < kPre; ++st) {
      if (lane * 8 + 512 * (st * kS + ws) < p.K) reg_step(wq[st][0], xq[st]);
    }
    for (int k0 = lane * 8 + 512 * (kPre * kS + ws); k0 < p.K; k0 += 512 * kS) {
      const u32x4 q = *reinterpret_cast<const u32x4*>(W + static_cast<size_t>(mc) * p.ldw + k0);
      u32x4 x[kN];
#pragma unroll
      for (int j = 0; j < kN; ++j) x[j] = xg[k0 * kN / 8 + j];
      reg_step(q, x);
    }
  } else {
    auto step = [&](int k0, const u32x4 (&q)[kR]) {
      float w[kR][8];
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        const uint32_t a[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
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
    };
#pragma unroll
    for (int st = 0; st < kPre; ++st) {
      const int k0 = lane * 8 + 512 * st;
      if (k0 < p.K) step(k0, wq[st]);
    }
    for (int k0 = lane * 8 + 512 * kPre; k0 < p.K; k0 += 512) {
      u32x4 q[kR];
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        const int m = min(mc + r, p.M - 1);
        q[r] = *reinterpret_cast<const u32x4*>(W + static_cast<size_t>(m) * p.ldw + k0);
      }
      step(k0, q);
    }
  }
  if constexpr (kS > 1) {
    float t;  // this wave's partial total of token lane (lanes < kN)
    if constexpr (kN == 8) {
      t = wave_sum8(acc[0]);  // token lane & 7
    } else {
      float s[kN];
#pragma unroll
      for (int c = 0; c < kN; ++c) s[c] = wave_sum(acc[0][c]);
      t = pick<kN>(s, lane);
    }
    if (lane < kN) s_red[ws][lane] = t;
    __syncthreads();
    if (ws != 0 || lane >= kN) return;
    float v = s_red[0][lane];
#pragma unroll
    for (int w = 1; w < kS; ++w) v += s_red[w][lane];
    static_cast<bf16_t*>(p.Y)[static_cast<size_t>(m0) * kN + lane] = f32_to_bf16(v);
    return;
  }
  bf16_t* __restrict__ Y = static_cast<bf16_t*>(p.Y);
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int m = m0 + r;
    float s[kN];  // row m's value for each token, rounded to bf16 (uniform over the wave)
    if constexpr (kN == 8) {
      const float t = to_f32(f32_to_bf16(wave_sum8(acc[r])));  // token lane & 7
#pragma unroll
      for (int c = 0; c < kN; ++c) s[c] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), c));
    } else {
#pragma unroll
      for (int c = 0; c < kN; ++c) s[c] = to_f32(f32_to_bf16(wave_sum(acc[r][c])));
    }
    if (m >= p.M) continue;
    if constexpr (kEpi == 1) {
      if (m < p.cs.dim) {
        conv_epilogue<kN>(p.cs, m, s, lane, co);
        continue;
      }
    }
    if constexpr (kEpi == 2) {
      ssm_epilogue<kN>(p.ss, p.zoh, m, s, lane, so);
      continue;
    }
    if (lane < kN) Y[static_cast<size_t>(m) * kN + lane] = f32_to_bf16(pick<kN>(s, lane));
  }
}

// Plain decode GEMM of a tall matrix (M >= 4096: the tied head, M = 50280, K = 768) on the
// matrix cores: each wave computes a 16-row tile Y[r0..r0+15][0..kN-1] with
// v_mfma_f32_16x16x16_bf16 (bf16 products, float32 sums), token columns kN..15 of the B
// operand zero. Operand layout of the instruction (lane l, element e of its 4): A[i][k] at
// l = i + 16 (k / 4), e = k % 4; B[k][j] at l = j + 16 (k / 4), e = k % 4; D[i][j] at
// l = j + 16 (i / 4), e = i % 4. A permutation of k applied to both A and B leaves the
// product unchanged, so a lane's 32-byte slice of its row (16 consecutive k; the 4 lanes of
// a row read one whole 128-byte line) feeds four instructions, 4 values each as k-group
// l / 16. X is
// staged in LDS transposed ([kN][K]), so a lane's B operand is 16 contiguous bytes too;
// lanes of the token columns kN..15, whose outputs are never stored (column j of D depends
// on column j of B only), read token row j % kN. The first kMfmaPf weight slices are loaded
// before X is staged.
// K % 64 == 0; rows past M read row M - 1 and are not stored. The VALU kernel spends most
// of its time on the 309 M multiply-adds of the head (float32 VALU, no packed forms); here
// the matrix cores take them and the weight stream sets the pace.
typedef short mfma_bf16x4 __attribute__((ext_vector_type(4)));
typedef float mfma_f32x4 __attribute__((ext_vector_type(4)));
constexpr int kMfmaPf = 4;  // weight slices (64 k, two 16-byte loads each) in flight per lane
// the same for the one-tile-per-wave tall GEMMs (the tied head: 6 or all 12 slices of
// K = 768 in flight measured 0.504 / 0.505 ms per 130M decode step against 0.503 with 4)
#ifndef MSS_MFMA_PF_TALL
#define MSS_MFMA_PF_TALL 4
#endif
// Plain GEMMs take the matrix cores from this many rows (the 768-row out-projection of the
// 130M decode step with K split 4 ways on them: 0.616 ms per token step against 0.571 on the
// VALU kernel, its 48 workgroups too few).
#ifndef MSS_MFMA_MIN_M
#define MSS_MFMA_MIN_M 4096
#endif
constexpr int kMfmaMaxK = 4096;  // the same X bytes as the VALU kernel stages (<= 64 KB)

__device__ __forceinline__ mfma_bf16x4 bf16x4_of(uint32_t lo, uint32_t hi) {
  const uint2 v = {lo, hi};
  return __builtin_bit_cast(mfma_bf16x4, v);
}

// kEpi 1: the conv-window step on rows [0, cs.dim) (each lane: its token column, four rows),
// operands loaded before the X barrier; kNorm: X is the norm prologue's, stored transposed.
// kSplit 1: each wave owns a 16-row tile (4 tiles per workgroup); kSplit 4: the workgroup's
// 4 waves share one tile, each taking a quarter of the K steps, and the partial tiles are
// added in wave order through LDS (more, shorter workgroups for the in-projection's 3072
// rows).
template <int kN, int kEpi, bool kNorm, int kSplit>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(GemvParams p) {
  constexpr int kPf = kSplit == 1 ? MSS_MFMA_PF_TALL : kMfmaPf;
  static_assert(kEpi == 0 || kEpi == 1, "plain store or conv-window step");
  static_assert(kSplit == 1 || kSplit == 4, "one tile per wave or one per workgroup");
  extern __shared__ u32x4 s_xt[];  // [kN][K] bf16: X transposed
  __shared__ float s_ss[kNorm ? kN : 1][4];
  __shared__ mfma_f32x4 s_acc[kSplit > 1 ? kSplit : 1][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = p.K;
  const int steps = K / 64;
  // the wave's tile and its range of K steps [s_lo, s_hi)
  const int r0 = kSplit == 1 ? (blockIdx.x * 4 + wv) * 16 : blockIdx.x * 16;
  const int per = (steps + kSplit - 1) / kSplit;
  const int s_lo = kSplit == 1 ? 0 : min(wv * per, steps);
  const int s_hi = kSplit == 1 ? steps : min(s_lo + per, steps);
  const int g = lane >> 4;  // k-group of the lane
  const int row = min(r0 + (lane & 15), p.M - 1);
  const bf16_t* __restrict__ wrow = static_cast<const bf16_t*>(p.W) + static_cast<size_t>(row) * p.ldw + g * 16;
  u32x4 wq[kPf][2];
#pragma unroll
  for (int j = 0; j < kPf; ++j) {  // steps past the range re-read the row's last slice
    const bf16_t* src = wrow + min(s_lo + j, steps - 1) * 64;
    wq[j][0] = *reinterpret_cast<const u32x4*>(src);
    wq[j][1] = *reinterpret_cast<const u32x4*>(src + 8);
  }
  const int col = lane & 15;  // the lane's token column of D
  ConvOperands co[4];
  if constexpr (kEpi == 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) load_conv(p.cs, min(r0 + 4 * g + e, p.M - 1), col, kN, co[e]);
  }
  bf16_t* __restrict__ xt = reinterpret_cast<bf16_t*>(s_xt);
  if constexpr (kNorm) {
    norm_prologue<kN, true>(p.nm, K, xt, s_ss);
  } else {
    const bf16_t* __restrict__ X = static_cast<const bf16_t*>(p.X);
    for (int kk = tid; kk < K; kk += 256) {
      float xv[kN];
      load_xrow<kN>(X + kk * kN, xv);  // X row kk: kN tokens, one 2kN-byte load
#pragma unroll
      for (int c = 0; c < kN; ++c) xt[c * K + kk] = f32_to_bf16(xv[c]);  // exact: bf16 values
    }
  }
  __syncthreads();
  if (r0 >= p.M) return;  // after the last barrier every wave of a kSplit tile shares
  const bf16_t* __restrict__ xrow = xt + ((lane & 15) % kN) * K + g * 16;
  mfma_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = s_lo; s0 < s_hi; s0 += kPf) {
#pragma unroll
    for (int j = 0; j < kPf; ++j) {
      const int s = s0 + j;
      if (s < s_hi) {
        const u32x4 a0 = wq[j][0], a1 = wq[j][1];
        if (s + kPf < s_hi) {
          const bf16_t* src = wrow + (s + kPf) * 64;
          wq[j][0] = *reinterpret_cast<const u32x4*>(src);
          wq[j][1] = *reinterpret_cast<const u32x4*>(src + 8);
        }
        const u32x4 b0 = *reinterpret_cast<const u32x4*>(xrow + s * 64);
        const u32x4 b1 = *reinterpret_cast<const u32x4*>(xrow + s * 64 + 8);
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bf16x4_of(a0.x, a0.y), bf16x4_of(b0.x, b0.y), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bf16x4_of(a0.z, a0.w), bf16x4_of(b0.z, b0.w), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bf16x4_of(a1.x, a1.y), bf16x4_of(b1.x, b1.y), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bf16x4_of(a1.z, a1.w), bf16x4_of(b1.z, b1.w), acc, 0, 0, 0);
      }
    }
  }
  if constexpr (kSplit > 1) {
    s_acc[wv][lane] = acc;
    __syncthreads();
    if (wv != 0) return;
    acc = s_acc[0][lane];
#pragma unroll
    for (int w = 1; w < kSplit; ++w) acc += s_acc[w][lane];
  }
  if (col < kN) {
    bf16_t* __restrict__ Y = static_cast<bf16_t*>(p.Y);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = r0 + 4 * g + e;
      if (m >= p.M) continue;
      if constexpr (kEpi == 1) {
        if (m < p.cs.dim) {  // rounded to bf16 first, as the separate step would read it
          conv_step_core(p.cs, m, col, to_f32(f32_to_bf16(acc[e])), co[e]);
          continue;
        }
      }
      Y[static_cast<size_t>(m) * kN + col] = f32_to_bf16(acc[e]);
    }
  }
}

// Plain GEMMs of at most this many rows (and K > 512) split K over the workgroup's 4 waves,
// one row per workgroup: the 130M decode step's x projection (80 rows, K 1536; 20
// workgroups unsplit) and out-projection (768 rows; 192) take it, 0.571 -> 0.534 ms per
// token step on MI355X with X staged in LDS (0.544 with the out-projection split 2 ways, 2
// rows per workgroup), 0.500 with X read into registers.
#ifndef MSS_GEMV_SPLIT_MAX_M
#define MSS_GEMV_SPLIT_MAX_M 1024
#endif

template <int kN, int kS>
static hipError_t launch_gemv_split(const GemvParams& p, int steps, hipStream_t stream) {
  const dim3 grid(p.M);
  const size_t lds = 0;  // X is read into registers
  switch (min((steps + kS - 1) / kS, 4)) {  // K steps each wave loads before the X barrier
    case 1: hipLaunchKernelGGL((gemv_kernel<kN, 1, 0, 1, false, kS>), grid, dim3(256), lds, stream, p); break;
    case 2: hipLaunchKernelGGL((gemv_kernel<kN, 1, 0, 2, false, kS>), grid, dim3(256), lds, stream, p); break;
    case 3: hipLaunchKernelGGL((gemv_kernel<kN, 1, 0, 3, false, kS>), grid, dim3(256), lds, stream, p); break;
    default: hipLaunchKernelGGL((gemv_kernel<kN, 1, 0, 4, false, kS>), grid, dim3(256), lds, stream, p); break;
  }
  return hipGetLastError();
}

template <int kN, int kEpi, int kPre>
static hipError_t launch_gemv_p(const GemvParams& p, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(p.K) * kN * sizeof(bf16_t);
  // On the matrix cores (X transposed in LDS, K % 64 == 0): tall plain GEMMs, and every
  // in-projection with the conv-window step fused (with or without the norm prologue, so
  // the two fused entry points give the same bits).
  if constexpr (kEpi == 0 || kEpi == 1) {
    const bool mfma = p.K % 64 == 0 && p.K <= kMfmaMaxK && (kEpi == 1 || (p.M >= MSS_MFMA_MIN_M && !p.norm));
    if (mfma) {
      if (p.norm && p.K > kNormGemvMaxFeatures) return hipErrorInvalidValue;
      if (kEpi == 0 && p.M >= 4096) {
        hipLaunchKernelGGL((gemv_mfma_kernel<kN, kEpi, false, 1>), dim3((p.M + 63) / 64), dim3(256), lds, stream, p);
      } else if (p.norm) {
        hipLaunchKernelGGL((gemv_mfma_kernel<kN, kEpi, true, 4>), dim3((p.M + 15) / 16), dim3(256), lds, stream, p);
      } else {
        hipLaunchKernelGGL((gemv_mfma_kernel<kN, kEpi, false, 4>), dim3((p.M + 15) / 16), dim3(256), lds, stream, p);
      }
      return hipGetLastError();
    }
  }
  // 4 rows per wave (X staged once per 16 rows) when that still gives >= 256 workgroups.
  if constexpr (kEpi == 0) {
    if (p.M >= 4096) {
      const int waves = (p.M + 3) / 4;
      hipLaunchKernelGGL((gemv_kernel<kN, 4, kEpi, kPre, false>), dim3((waves + 3) / 4), dim3(256), lds, stream, p);
      return hipGetLastError();
    }
  }
  // the norm prologue is fused only in front of the conv-window step (the in-projection)
  if constexpr (kEpi == 1) {
    if (p.norm) {
      if (p.K > kNormGemvMaxFeatures) return hipErrorInvalidValue;
      // (workgroups of 8 or 16 waves, each normalising a share of the tokens and so
      // re-reading the stream 2x or 4x less, measured slower on MI355X: 0.629 and 0.634 ms
      // per 130M decode step against 0.625 with 4 waves)
      hipLaunchKernelGGL((gemv_kernel<kN, 1, kEpi, kPre, true>), dim3((p.M + 3) / 4), dim3(256), lds, stream, p);
      return hipGetLastError();
    }
  }
  if (p.norm) return hipErrorInvalidValue;
  if constexpr (kEpi == 0) {
    const int steps = (p.K + 511) / 512;
    if (steps >= 2 && steps <= 16 && p.M <= MSS_GEMV_SPLIT_MAX_M) return launch_gemv_split<kN, 4>(p, steps, stream);
  }
  hipLaunchKernelGGL((gemv_kernel<kN, 1, kEpi, kPre, false>), dim3((p.M + 3) / 4), dim3(256), lds, stream, p);
  return hipGetLastError();
}

// Weight steps (512 elements of K each) loaded into registers before the X barrier: all
// of them up to K = 2048, the rest streamed after it.
template <int kN, int kEpi>
static hipError_t launch_gemv_n(const GemvParams& p, hipStream_t stream) {
  switch (min((p.K + 511) / 512, 4)) {
    case 1: return launch_gemv_p<kN, kEpi, 1>(p, stream);
    case 2: return launch_gemv_p<kN, kEpi, 2>(p, stream);
    case 3: return launch_gemv_p<kN, kEpi, 3>(p, stream);
    default: return launch_gemv_p<kN, kEpi, 4>(p, stream);
  }
}

template <int kEpi>
static hipError_t launch_gemv_e(const GemvParams& p, hipStream_t stream) {
  switch (p.N) {
    case 1: return launch_gemv_n<1, kEpi>(p, stream);
    case 2: return launch_gemv_n<2, kEpi>(p, stream);
    case 4: return launch_gemv_n<4, kEpi>(p, stream);
    case 8: return launch_gemv_n<8, kEpi>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv(const GemvParams& p, hipStream_t stream) {
  switch (p.epi) {
    case 0: return launch_gemv_e<0>(p, stream);
    case 1: return launch_gemv_e<1>(p, stream);
    case 2: return launch_gemv_e<2>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mss
