// Device-side helpers shared by the forward and backward selective-scan kernels.
//
// Work mapping used by both kernels: one wavefront (64 lanes) owns one (batch, channel)
// row; its 64 lanes own 64 consecutive segments of kT steps each, so one wave covers a
// chunk of 64*kT steps and walks the sequence chunk by chunk. Inside a segment a lane
// runs the recurrence sequentially; segments are joined with a 64-lane affine scan on
// DPP lane shifts. The state loop (n) is outermost inside a chunk so only one state's
// per-step coefficients live in registers at a time.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mss {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kMaxN = 16;
// Float32 scans with more states: the forward keeps this many per wave; the backward runs
// over groups of at most kMaxN states.
constexpr int kMaxNWide = 256;
// Step granularity of the `carries` residual: the state before every kSegSteps-step segment.
constexpr int kSegSteps = 8;
// Steps per chunk of the backward scans (a wave pass: 64 lanes of kSegSteps steps). Of a row
// with a length, the scans write dB/dC partial sums only for chunks holding a valid step; the
// reduction takes the steps of later chunks as zero.
constexpr int kPartChunk = 64 * kSegSteps;
__host__ __device__ constexpr int live_part_end(int len, int L) {
  const int e = (len + kPartChunk - 1) / kPartChunk * kPartChunk;
  return e < L ? e : L;
}
constexpr int kRefChunk = 2048;

struct bf16_t {
  uint16_t bits;
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}
__device__ __forceinline__ void store_as(float* p, float v) { *p = v; }
// float32 -> bf16, round to nearest even (NaN stays NaN): gfx950's v_cvt_pk_bf16_f32, one
// instruction per two values (the compiler selects it for these conversions).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  bf16_t r;
  r.bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  return r;
}
// Two values as one bf16 pair, `lo` in bits 0..15.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ void store_as(bf16_t* p, float v) { *p = f32_to_bf16(v); }

// ---------------------------------------------------------------------------------
// Cross-lane moves (gfx9 DPP). Lanes whose source is outside the pattern keep `old`.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_mov(float old, float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                         kCtrl, kRowMask, 0xF, false));
}
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowShl1 = 0x101, kRowShl2 = 0x102, kRowShl4 = 0x104, kRowShl8 = 0x108;
constexpr int kWaveShr1 = 0x138, kWaveShl1 = 0x130;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Inclusive scan over the 64 lanes (lane order = time order) of affine maps
// h -> P*h + H. Combining an earlier element (Pl, Hl) with a later one (Pr, Hr) gives
// (Pl*Pr, Pr*Hl + Hr): the operator of reference native/selective_scan_cuda.cu:58-63.
// Each Hillis-Steele step fuses the lane shift into the ALU ops:
//   H = P * H[src] + H ;  P = P[src] * P      (lanes without a source keep their values)
// A DPP read needs two wait states after a VALU write of its source: each step's reads
// come after the previous step's write of that register, one VALU instruction and an
// `s_nop 0`; `s_nop 1` pads the first and the last step. One asm statement, so the
// compiler neither places a write between a pad and the read it guards nor pads between
// steps itself.
#define MSS_FWD_SCAN_STEP(CTRL, RM)                               \
  "v_fmac_f32_dpp %0, %0, %1 " CTRL " row_mask:" RM " bank_mask:0xf\n\t" \
  "v_mul_f32_dpp %1, %1, %1 " CTRL " row_mask:" RM " bank_mask:0xf\n\t"  \
  "s_nop 0\n\t"
__device__ __forceinline__ void wave_scan_affine_fwd(float& P, float& H) {
  asm volatile("s_nop 1\n\t"                                   //
               MSS_FWD_SCAN_STEP("row_shr:1", "0xf")            //
               MSS_FWD_SCAN_STEP("row_shr:2", "0xf")            //
               MSS_FWD_SCAN_STEP("row_shr:4", "0xf")            //
               MSS_FWD_SCAN_STEP("row_shr:8", "0xf")            //
               MSS_FWD_SCAN_STEP("row_bcast:15", "0xa")         //
               MSS_FWD_SCAN_STEP("row_bcast:31", "0xc")         //
               "s_nop 1"
               : "+v"(H), "+v"(P));
}
#undef MSS_FWD_SCAN_STEP

// Sum over the 64 lanes; the result is returned uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<kRowShr1, 0xF>(0.f, v);
  v += dpp_mov<kRowShr2, 0xF>(0.f, v);
  v += dpp_mov<kRowShr4, 0xF>(0.f, v);
  v += dpp_mov<kRowShr8, 0xF>(0.f, v);
  v += dpp_mov<kRowBcast15, 0xA>(0.f, v);
  v += dpp_mov<kRowBcast31, 0xC>(0.f, v);
  return readlane(v, 63);
}

// Batch row of the workgroups whose grid y index is `rank`, for scans with variable
// lengths: the rows in order of decreasing length (equal lengths by index). The dispatcher
// hands out workgroups in grid order, so the longest rows start first and the shortest
// ones form the tail. Without lengths, or with more than 64 rows, rows keep their order.
// Each wave computes it alone (no barrier); the result is uniform.
constexpr int kMaxSortedRows = 64;
__device__ __forceinline__ int row_longest_first(const int* __restrict__ seq_lens, int batch, int L,
                                                 int rank) {
  if (seq_lens == nullptr || batch > kMaxSortedRows) return rank;
  const int lane = threadIdx.x & 63;
  const int mine = lane < batch ? min(max(seq_lens[lane], 0), L) : -1;
  int r = 0;  // rows ordered before this lane's row
  for (int j = 0; j < batch; ++j) {
    const int o = __builtin_amdgcn_readlane(mine, j);
    r += (o > mine) || (o == mine && j < lane);
  }
  // The ranks of the rows are a permutation of [0, batch): one lane matches any rank the grid
  // holds (the fallback only guards a rank outside it).
  const unsigned long long hit = __ballot(lane < batch && r == rank);
  return hit ? __builtin_amdgcn_readfirstlane(__ffsll(static_cast<long long>(hit)) - 1) : rank;
}

// ---------------------------------------------------------------------------------
// Scalar math.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// 1 - exp(-x) for x >= 0 (= sigmoid(y) when x = softplus(y)); series below 1/64 keeps
// the relative error near one ulp where 1 - exp(-x) would cancel.
__device__ __forceinline__ float one_minus_exp_neg(float x) {
  const float e = fast_exp2(-x * kLog2e);
  const float series = x * __builtin_fmaf(x, __builtin_fmaf(x, __builtin_fmaf(x, -1.f / 24.f, 1.f / 6.f), -0.5f), 1.f);
  return x < 0.015625f ? series : 1.f - e;
}

// softplus(x) = max(x, 0) + log1p(exp(-|x|)), branch-free. With w = exp(-|x|) in (0, 1] and
// u = fl(1 + w), the rounding error e = w - (u - 1) is exact (Fast2Sum), and
// log1p(w) = log(u) + log1p(e / u) = log(u) + e * (1 - w) to well below an ulp, so small
// results keep their relative accuracy (for x << 0, u = 1 and the result is w itself).
// Above x = 20 the correction is below half an ulp of x: the result is x, the reference
// kernel's identity branch (native/upstream_mamba/selective_scan_bwd_kernel.cuh:157).
__device__ __forceinline__ float softplus(float x) {
  const float w = fast_exp2(-fabsf(x) * kLog2e);
  const float u = 1.f + w;
  const float e = w - (u - 1.f);
  const float l = __builtin_fmaf(fast_log2(u), kLn2, __builtin_fmaf(-e, w, e));
  return fmaxf(x, 0.f) + l;
}

__device__ __forceinline__ float sigmoid(float x) {
  return fast_rcp(1.f + fast_exp2(-x * kLog2e));
}

// ---------------------------------------------------------------------------------
// Segment loads/stores. `row` points at element 0 of a [..][L] row; the segment is
// elements [t, t+N). `fast` must be wave-uniform: true when 16-byte vector access is
// legal for the row and the whole wave's chunk lies inside [0, L); otherwise elements at
// or beyond `L` read as 0 and are not written.
template <int N>
__device__ __forceinline__ void load_seg(const float* __restrict__ row, int t, int L, bool fast,
                                         float (&v)[N]) {
  if (fast) {
    const f32x4* p = reinterpret_cast<const f32x4*>(row + t);
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const f32x4 x = p[q];
      v[4 * q + 0] = x.x;
      v[4 * q + 1] = x.y;
      v[4 * q + 2] = x.z;
      v[4 * q + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = (t + j < L) ? row[t + j] : 0.f;
  }
}

template <int N>
__device__ __forceinline__ void load_seg(const bf16_t* __restrict__ row, int t, int L, bool fast,
                                         float (&v)[N]) {
  if (fast) {
    const u32x4* p = reinterpret_cast<const u32x4*>(row + t);
#pragma unroll
    for (int q = 0; q < N / 8; ++q) {
      const u32x4 x = p[q];
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[8 * q + 2 * k + 0] = __uint_as_float(w[k] << 16);
        v[8 * q + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = (t + j < L) ? to_f32(row[t + j]) : 0.f;
  }
}

template <int N>
__device__ __forceinline__ void store_seg(float* __restrict__ row, int t, int L, bool fast,
                                          const float (&v)[N]) {
  if (fast) {
    f32x4* p = reinterpret_cast<f32x4*>(row + t);
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const f32x4 x = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
      p[q] = x;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (t + j < L) row[t + j] = v[j];
  }
}

template <int N>
__device__ __forceinline__ void store_seg(bf16_t* __restrict__ row, int t, int L, bool fast,
                                          const float (&v)[N]) {
  if (fast) {
    u32x4* p = reinterpret_cast<u32x4*>(row + t);
#pragma unroll
    for (int q = 0; q < N / 8; ++q) {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = pack_bf16x2(v[8 * q + 2 * k], v[8 * q + 2 * k + 1]);
      const u32x4 x = {w[0], w[1], w[2], w[3]};
      p[q] = x;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (t + j < L) store_as(row + t + j, v[j]);
  }
}

// ---------------------------------------------------------------------------------
// LDS staging of B/C rows with gfx950 direct-to-LDS loads (global_load_lds, 16 bytes per
// lane). A staged row holds 64 segments of kT steps.
typedef __attribute__((address_space(3))) void* lds_void_t;
typedef __attribute__((address_space(1))) void* gbl_void_t;

// Staging layout of one chunk row: 16-byte slots; segment i (lane i) owns slots
// [kQ*i, kQ*i + kQ) with its q-th slot stored at kQ*i + (q ^ swz(i)) so that 16
// consecutive lanes reading their q-th slot hit 16 distinct 4-bank groups.
template <int kQ>
__device__ __forceinline__ int slot_swz(int i) {
  static_assert(kQ >= 1 && kQ <= 16 && (kQ & (kQ - 1)) == 0, "kQ must be a power of two <= 16");
  constexpr int kShift = kQ == 16 ? 0 : (kQ == 8 ? 1 : (kQ == 4 ? 2 : (kQ == 2 ? 3 : 4)));
  return (i >> kShift) & (kQ - 1);
}

template <typename bc_t>
struct BcStage {
  static constexpr int kElemsPerSlot = 16 / static_cast<int>(sizeof(bc_t));
};

// Read lane `lane`'s kT staged values of one row (fp32 or bf16 in LDS) as floats.
template <int kT, typename bc_t>
__device__ __forceinline__ void read_staged(const uint4* __restrict__ row, int lane, float (&v)[kT]) {
  constexpr int kE = BcStage<bc_t>::kElemsPerSlot;
  constexpr int kQ = kT / kE;
  const int sw = slot_swz<kQ>(lane);
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const uint4 x = row[kQ * lane + (q ^ sw)];
    if constexpr (sizeof(bc_t) == 4) {
      v[4 * q + 0] = __uint_as_float(x.x);
      v[4 * q + 1] = __uint_as_float(x.y);
      v[4 * q + 2] = __uint_as_float(x.z);
      v[4 * q + 3] = __uint_as_float(x.w);
    } else {
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[8 * q + 2 * k + 0] = __uint_as_float(w[k] << 16);
        v[8 * q + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      }
    }
  }
}

__device__ __forceinline__ void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---------------------------------------------------------------------------------
// Kernel parameter blocks (host fills them after validation).
struct NormParams {
  int features, tokens;
  float eps;
  const float* h;
  const void* delta;    // optional, activation dtype
  const float* w;
  float* hn;            // written when delta is given
  void* x;              // activation dtype
  float* rstd;
  // backward
  const void* dx;       // activation dtype
  const float* dhn_in;  // optional
  float* dhn;
  void* ddelta;         // optional, activation dtype
  float* dw_part;       // [n_blocks][features]
};

constexpr int kXentFusedMaxVocab = 65536;  // rows the fused forward + gradient holds in registers
struct XentParams {
  int rows, vocab;
  const bf16_t* z;
  const long long* target;
  float* loss;  // [rows]
  float* lse;   // [rows]
  const float* grad_scale;
  bf16_t* dz;
};

constexpr int kCUs = 256;  // MI355X compute units

// Skinny projection GEMM C[M][T] (+)= W[M][K] X[K][T], bf16 with float32 sums: K <= 128
// takes the expand kernel (M % 16 == 0), else the reduce kernel (M <= 128, M % 16 == 0,
// K % 64 == 0); T % 64 == 0.
constexpr int kProjExpandMaxK = 128;
constexpr int kProjReduceMaxM = 128;
struct ProjParams {
  int M, K, T, accumulate;
  int w_trans;  // W given as W^T [K][M] (row stride ldw)
  long long ldw, ldx, ldc;
  const void* W;
  const void* X;
  void* C;
};

// Weight-gradient GEMM C[M][N] (+)= A[M][K] B[N][K]^T, bf16 operands with K-contiguous rows,
// float32 output; K split over `splits` workgroups per kWgradTile-square output tile (partial
// at the edges), whose partial tiles ([splits][M][N] float32 in `workspace`) a second kernel
// adds in order. N a multiple of 4, K a multiple of 64.
constexpr int kWgradTile = 192;
struct WgradParams {
  int M, N, K, splits, accumulate;
  long long lda, ldb, ldc;
  const void* A;
  const void* B;
  float* C;
  float* workspace;
};
int wgrad_splits(int M, int N, int K);  // the split count launch_wgrad expects

// bf16 shadows of float32 weights (layout of mss_shadow_entry in the public header).
struct ShadowEntry {
  const float* src;
  bf16_t* dst;
  bf16_t* dst_t;
  int rows, cols;
  long long ld_t;
  long long tile0;
};
struct ShadowParams {
  const ShadowEntry* entries;  // device memory
  int n_entries;
  long long n_tiles;
};

// AdamW over float32 masters with bf16 shadows (layout of mss_adamw_entry in the public
// header). A launch takes up to kAdamWMaxEntries entries by value in its arguments (so a
// captured launch needs no table in device memory); unit0[i] is entry i's first work unit.
struct AdamWEntry {
  float* param;
  const float* grad;
  float* exp_avg;
  float* exp_avg_sq;
  const float* step;  // the step number of this update (1 on the first)
  bf16_t* shadow;     // may be null
  bf16_t* shadow_t;   // may be null: then flat 4096-element units, else 64 x 64 tiles
  int rows, cols;
  long long ld_t;
  long long numel;
};
constexpr int kAdamWMaxEntries = 40;
constexpr int kAdamWUnit = 4096;
struct AdamWParams {
  AdamWEntry e[kAdamWMaxEntries];
  long long unit0[kAdamWMaxEntries + 1];
  int n;
  float lr, beta1, beta2, eps, weight_decay;
};

// Token embedding into a channel-major stream and its gradient (mss_embed_cm*).
constexpr int kEmbedMaxD = 1024;  // backward: model width limit (16 KB of LDS partial rows)
struct EmbedParams {
  long long T;
  int V, D;
  long long ldh;                    // row stride of h / dh (>= T)
  const long long* tokens;          // [T]
  const float* E;                   // [V][D]
  float* h;                         // [D][ldh]
  const float* dh;                  // [D][ldh]
  const long long* sorted_tokens;   // [T], ascending (stable sort of tokens)
  const long long* order;           // [T], positions of sorted_tokens
  float* work;                      // [T][D]
  float* dE;                        // [V][D], accumulated
};

struct StepParams {
  int batch, dim, dstate, delta_softplus;
  long long io_sb, io_sd, bc_sb, bc_sn;
  float* state;  // [B][D][N], updated in place
  const void* u;
  const void* delta;
  const void* z;  // optional
  const void* B;
  const void* C;
  const float* A;
  const float* D;           // optional
  const float* delta_bias;  // optional
  void* out;
};


struct ConvStepParams {
  int batch, dim, width, act;
  long long sb, sd;  // strides of x and y
  void* state;       // [B][D][width-1], activation dtype, updated in place
  const void* x;
  const float* w;
  const float* bias;  // optional
  void* y;
};

// Largest feature count of the RMSNorm prologue fused in front of the decode GEMM.
constexpr int kNormGemvMaxFeatures = 1024;

struct GemvParams {
  int M, K, N;      // Y [M][N] = W [M][K] X [K][N]
  long long ldw;    // W row stride (elements)
  const void* W;    // bf16
  const void* X;    // bf16, rows of N contiguous values
  void* Y;          // bf16, rows of N contiguous values
  // Epilogue over the N tokens of each row (a channel). 0: store Y. 1: rows [0, cs.dim) are
  // the conv input x of their channel: the conv-window step (cs, x bf16) replaces the store.
  // 2: row m is the raw delta of channel m: the selective-state step (ss, Euler or ZOH,
  // bf16 io and B/C) replaces the store.
  int epi, zoh;
  ConvStepParams cs;
  StepParams ss;
  // norm != 0: X is not read; each workgroup computes it as the residual add + RMSNorm of
  // nm (features K, tokens N, bf16 delta and x) and workgroup 0 writes nm.hn (when delta)
  // and nm.rstd (when not null); nm.x is not written.
  int norm;
  NormParams nm;
};

struct ConvParams {
  int batch, dim, seqlen, width;
  long long sb, sd;  // row strides (elements) of x, y, dy, dx: batch, channel
  const void* x;
  const float* w;     // [dim][width]
  const float* bias;  // [dim] or null
  const int* seq_lens;
  void* y;
  const void* dy;
  void* dx;
  float* part;  // backward: per-(d, b, tile) partials of dw / dbias, (width + 1) floats each
};

struct FwdParams {
  int batch, dim, seqlen, dstate;
  int delta_softplus;
  int vec_io;  // 16-byte vector access legal for u/delta/z/out rows
  int vec_bc;  // ... for B/C rows
  int n_seg;  // ceil(L / kSegSteps): carries row length
  int n_ref;    // ceil(L / 2048)
  long long io_sb, io_sd;  // row strides (elements) of u/delta/z/out/y_pre: batch, channel
  long long bc_sb, bc_sn;  // row strides of B/C: batch, state
  const void* u;
  const void* delta;
  const float* A;
  const void* B;
  const void* C;
  const float* D;
  const void* z;
  const float* delta_bias;
  const float* x0;
  const int* seq_lens;
  void* out;
  float* last;
  float* carries;  // [B][D][N][n_seg]: state before each kSegSteps-step segment
  float* ref_states;
  void* y_pre;
};

// The silu(z) gate's backward needs y sigma(z); out = y z sigma(z) gives it as out / z wherever
// z is not tiny, so the real-A forward keeps y itself (y_pre) only where |z| < kZTiny.
constexpr float kZTiny = 1e-20f;

// Backward launch shape: waves per workgroup and channels per workgroup.
struct BwdPlan {
  int waves, chan_per_block;
};

struct BwdParams {
  int batch, dim, seqlen, dstate;
  int delta_softplus;
  int vec_io, vec_bc;
  int n_seg;
  int waves;           // waves per backward workgroup (12 or 16)
  int chan_per_block;  // channels one workgroup walks (multiple of the wave count)
  int n_blocks_d;      // ceil(dim / chan_per_block)
  long long io_sb, io_sd;  // row strides of u/delta/z/y_pre/dout/du/ddelta/dz
  long long bc_sb, bc_sn;  // row strides of B/C and dB/dC
  const void* u;
  const void* delta;
  const float* A;
  const void* B;
  const void* C;
  const float* D;
  const void* z;
  const float* delta_bias;
  const float* x0;
  const int* seq_lens;
  const float* carries;  // [B][D][N][n_seg] from the forward
  const void* y_pre;     // real A: y where |z| < kZTiny (elsewhere unwritten); complex A: y
  const void* out;       // real A with z: the forward's gated output
  const void* dout;
  const float* dlast;
  void* du;
  void* ddelta;
  void* dz;
  float* dinit;
  // A state group of a wider scan (dstate here is the group's size): row strides of the
  // full tensors, in elements. a_ld: A rows; state_ld: x0/dlast/dinit rows (per (b, d));
  // carry_cs: carries per (b, d). acc_out: du/ddelta add to what the buffers hold (the
  // other groups' terms) instead of overwriting them.
  int a_ld, state_ld;
  long long carry_cs;
  int acc_out;
  // workspace partials
  float* part_dBC;   // [n_blocks_d][part_stride]; block = [batch][2][dstate][L] (+ padding)
  size_t part_stride;  // floats per channel block, a multiple of 64
  float* part_dA;    // [batch][dim][dstate]
  float* part_dD;    // [batch][dim]
  float* part_dbias; // [batch][dim]
};

}  // namespace mss
