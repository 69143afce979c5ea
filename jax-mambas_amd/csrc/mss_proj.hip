// Skinny projection GEMMs of the training step on the matrix cores (bf16 operands, float32
// sums), for the selective scan's input projections: the reference's s_B / s_C / Linear_R
// (d_inner -> R + 2N, stacked here as one x-projection) and Linear_Delta (R -> d_inner),
// mamba/mamba1.py:52-67, 107-124, whose products XLA runs as dot products. Activations are
// channel-major [features][tokens] (tokens contiguous), the layout the scan reads in place.
// Each of these GEMMs moves one 50 MB activation matrix past a weight of at most 128 rows or
// columns, so they are HBM-bound; the kernels stream the big operand once.
//
//   proj_reduce_kernel  C[M][T] (+)= W[M][K] X[K][T], M <= 128, long K (the x-projection,
//                       and the dt-rank gradient W_dt^T dDelta)
//   proj_expand_kernel  C[M][T] (+)= W[M][K] X[K][T], K <= 128 (the dt-projection, and the
//                       x-projection's input gradient W_x^T dx_dbl added into du)
// (These projections' weight gradients, A B^T over the tokens with an 80- or 48-wide side,
// stay with the library GEMM: a kernel of this family that split the tokens over workgroups
// and summed partial tiles in a fixed order measured 23.4 / 28.8 us against the library's
// 22.4 / 21.7 at the config-5 shapes, the short operand re-read by every output block. The
// block's wide projections' weight gradients run on mss_wgrad.hip.)
//
// Instruction: v_mfma_f32_16x16x16_bf16. Operand layout (lane l, element e of its 4):
// A[i][k] at l = i + 16 (k / 4), e = k % 4; B[k][j] at l = j + 16 (k / 4), e = k % 4;
// D[i][j] at l = j + 16 (i / 4), e = i % 4. Any permutation of k applied to A and B alike
// leaves the product unchanged.
//
// With tokens contiguous, a B operand over the feature dimension (4 features of one token
// per lane) is a transpose: lane (j, g) loads 4 feature rows x 4 consecutive tokens
// (8 bytes per row, 16 lanes per 128-byte line) and v_perm_b32 regroups them into the B
// operands of four 16-token column tiles whose column j is token 4j + c (c = the tile). The
// D tiles then hold, per lane and output row, tokens 4j..4j+3: one 8-byte store per row.
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

typedef short pbf16x4 __attribute__((ext_vector_type(4)));
typedef float pf32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ pbf16x4 pbf16x4_of(uint32_t lo, uint32_t hi) {
  const uint2 v = {lo, hi};
  return __builtin_bit_cast(pbf16x4, v);
}

__device__ __forceinline__ pf32x4 mfma16(pbf16x4 a, pbf16x4 b, pf32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// r[i] holds tokens t..t+3 of feature row i (two bf16 pairs); b[c] gets (r0[t+c], r1[t+c],
// r2[t+c], r3[t+c]), the 4 features of token t+c.
__device__ __forceinline__ void transpose_4x4(const uint2 (&r)[4], pbf16x4 (&b)[4]) {
  constexpr uint32_t kLo = 0x05040100u, kHi = 0x07060302u;  // low / high halves of two dwords
  b[0] = pbf16x4_of(__builtin_amdgcn_perm(r[1].x, r[0].x, kLo), __builtin_amdgcn_perm(r[3].x, r[2].x, kLo));
  b[1] = pbf16x4_of(__builtin_amdgcn_perm(r[1].x, r[0].x, kHi), __builtin_amdgcn_perm(r[3].x, r[2].x, kHi));
  b[2] = pbf16x4_of(__builtin_amdgcn_perm(r[1].y, r[0].y, kLo), __builtin_amdgcn_perm(r[3].y, r[2].y, kLo));
  b[3] = pbf16x4_of(__builtin_amdgcn_perm(r[1].y, r[0].y, kHi), __builtin_amdgcn_perm(r[3].y, r[2].y, kHi));
}

// Output row m, tokens [t, t+4) from the four column tiles' element e: bf16, optionally
// added to the values already there (float32 sum, rounded once).
__device__ __forceinline__ void store_row4(bf16_t* __restrict__ crow, const pf32x4 (&acc)[4], int e, bool accumulate) {
  float v[4] = {acc[0][e], acc[1][e], acc[2][e], acc[3][e]};
  if (accumulate) {
    const uint2 old = *reinterpret_cast<const uint2*>(crow);
    v[0] += __uint_as_float(old.x << 16);
    v[1] += __uint_as_float(old.x & 0xffff0000u);
    v[2] += __uint_as_float(old.y << 16);
    v[3] += __uint_as_float(old.y & 0xffff0000u);
  }
  const uint2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  *reinterpret_cast<uint2*>(crow) = o;
}

template <int kN>
__device__ __forceinline__ void wait_vmem_n() {
  static_assert(kN >= 0 && kN < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kN) : "memory");
}

// ---------------------------------------------------------------------------------------
// C[M][T] (+)= W[M][K] X[K][T] for M = 16 kMB rows and K % 64 == 0. One workgroup per 64
// tokens: kMB compute waves (one per 16-row tile, each over all of K) and two copy waves.
// X and W travel in 64-k blocks (X: 64 rows x 64 tokens, 8 KB; W: M rows x 64 k, or for a
// weight given transposed, kTrans, W^T's 64 k x M) through an LDS ring by direct-to-LDS
// copies: copy wave 0 issues X's, copy wave 1 W's, each tracking its own copies with vmcnt
// so the ring can hold as many blocks in flight as the larger count allows (the compute
// waves issue no global loads: the compiler waits for every outstanding load before an
// LDS read of a ring it cannot index statically). The waves meet at a bare s_barrier per
// block (__syncthreads' fence would drain every copy in flight): before it the copy waves
// wait, by count, for the current block's copies only, and the compute waves for their LDS
// reads, so a stage is refilled only after its last reader is done. B operands: four
// 8-byte X reads per 4 features, transposed in registers; A operands: 32 bytes of a W row
// (16 k feeding the block's four instructions as k-groups), or four 2-byte W^T reads per
// 4 k.
template <int kMB>
constexpr int red_stages() { return 2 + 63 / (2 * kMB > 8 ? 2 * kMB : 8) < 8 ? 2 + 63 / (2 * kMB > 8 ? 2 * kMB : 8) : 8; }

template <int kMB, bool kTrans>
__global__ __launch_bounds__((kMB + 2) * 64) void proj_reduce_kernel(ProjParams p) {
  constexpr int kStages = red_stages<kMB>();
  constexpr int kXSlots = 64 * 64 * 2 / 16;  // 16-byte slots of an X block
  constexpr int kWSlots = kMB * 16 * 8;      // of a W block
  constexpr int kXCopies = kXSlots / 64, kWCopies = kWSlots / 64;  // copy instructions per block
  static_assert((kStages - 2) * kXCopies < 64 && (kStages - 2) * kWCopies < 64, "vmcnt range");
  __shared__ u32x4 s_x[kStages][kXSlots];  // slot = row * 8 + 8-token group
  __shared__ u32x4 s_w[kStages][kWSlots];  // slot = row * 8 + 8-k group (kTrans: k * 2kMB + 8-row group)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool copy_x = w == kMB, copy_w = w == kMB + 1, compute = w < kMB;
  const int j = lane & 15, g = lane >> 4;
  const int T0 = blockIdx.x * 64;
  const int nblk = p.K / 64;
  const bf16_t* __restrict__ X = static_cast<const bf16_t*>(p.X);
  const bf16_t* __restrict__ W = static_cast<const bf16_t*>(p.W);

  auto issue = [&](int b) {  // this copy wave's copies of block b into stage b % kStages
    const int st = b % kStages;
    if (copy_x) {
#pragma unroll
      for (int i = 0; i < kXCopies; ++i) {
        const int slot = i * 64 + lane;
        const bf16_t* src = X + static_cast<size_t>(64 * b + (slot >> 3)) * p.ldx + T0 + (slot & 7) * 8;
        __builtin_amdgcn_global_load_lds((gbl_void_t)src, (lds_void_t)(&s_x[st][i * 64]), 16, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kWCopies; ++i) {
        const int slot = i * 64 + lane;
        const bf16_t* src = kTrans ? W + static_cast<size_t>(64 * b + slot / (2 * kMB)) * p.ldw + (slot % (2 * kMB)) * 8
                                   : W + static_cast<size_t>(slot >> 3) * p.ldw + 64 * b + (slot & 7) * 8;
        __builtin_amdgcn_global_load_lds((gbl_void_t)src, (lds_void_t)(&s_w[st][i * 64]), 16, 0, 0);
      }
    }
  };
  if (!compute) {
#pragma unroll
    for (int b = 0; b < kStages - 1; ++b)
      if (b < nblk) issue(b);
  }

  pf32x4 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = pf32x4{0.f, 0.f, 0.f, 0.f};
  for (int b = 0; b < nblk; ++b) {
    if (copy_x || copy_w) {  // block b landed; the later blocks issued so far may stay in flight
      if (b + kStages - 2 >= nblk) wait_vmem_all();
      else if (copy_x) wait_vmem_n<(kStages - 2) * kXCopies>();
      else wait_vmem_n<(kStages - 2) * kWCopies>();
    } else {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // block b - 1's reads are done
    }
    __builtin_amdgcn_s_barrier();  // every wave sees block b; block b - 1's stage is free
    if (!compute) {
      if (b + kStages - 1 < nblk) issue(b + kStages - 1);
      continue;
    }
    const int st = b % kStages;
    uint32_t av[8];
    if constexpr (kTrans) {  // W^T stage [64 k][16 kMB m]: row m = 16 w + j, k = 16 g + 2 i (+1)
      const uint16_t* __restrict__ ws = reinterpret_cast<const uint16_t*>(&s_w[st][0]) + 16 * w + j;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        av[i] = static_cast<uint32_t>(ws[(16 * g + 2 * i) * 16 * kMB]) |
                (static_cast<uint32_t>(ws[(16 * g + 2 * i + 1) * 16 * kMB]) << 16);
    } else {
      const u32x4 a0 = s_w[st][(16 * w + j) * 8 + 2 * g];
      const u32x4 a1 = s_w[st][(16 * w + j) * 8 + 2 * g + 1];
      av[0] = a0.x; av[1] = a0.y; av[2] = a0.z; av[3] = a0.w;
      av[4] = a1.x; av[5] = a1.y; av[6] = a1.z; av[7] = a1.w;
    }
    const uint2* __restrict__ xs = reinterpret_cast<const uint2*>(&s_x[st][0]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // k = 64 b + 16 g + 4 q + e
      uint2 r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = xs[(16 * g + 4 * q + e) * 16 + j];
      pbf16x4 bo[4];
      transpose_4x4(r, bo);
      const pbf16x4 ao = pbf16x4_of(av[2 * q], av[2 * q + 1]);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = mfma16(ao, bo[c], acc[c]);
    }
  }
  if (!compute) return;
  bf16_t* __restrict__ C = static_cast<bf16_t*>(p.C);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    store_row4(C + static_cast<size_t>(16 * w + 4 * g + e) * p.ldc + T0 + 4 * j, acc, e, p.accumulate != 0);
}

// ---------------------------------------------------------------------------------------
// C[M][T] (+)= W[M][K] X[K][T] for K = 16 kKB <= 128 and M % 16 == 0. A workgroup of 4 waves
// covers 64 tokens x kExpandTiles 16-row tiles: each wave loads the 64-token X block once
// (transposed in registers into the B operands of all of K) and walks the workgroup's tiles
// w, w + 4, ..., loading the next tile's W rows (and, accumulating, the C values to add to)
// while it computes and stores the current one, so the output streams out without a wait
// on a fresh X block per tile. kTrans: the weight given as W^T [K][M], its 4 k of a row
// read as four 2-byte loads (the weight is small and cached).
constexpr int kExpandWaveTiles = 6;  // 16-row tiles per wave
constexpr int kExpandCAhead = 6;     // accumulating: tiles whose C values are loaded ahead
constexpr int kExpandTiles = 4 * kExpandWaveTiles;

template <int kKB, bool kTrans>
__device__ __forceinline__ void expand_load_w(const bf16_t* __restrict__ W, long long ldw, int row, int g,
                                              uint2 (&wr)[kKB]) {
#pragma unroll
  for (int kb = 0; kb < kKB; ++kb) {
    if constexpr (kTrans) {
      const uint16_t* src = reinterpret_cast<const uint16_t*>(W) + static_cast<size_t>(16 * kb + 4 * g) * ldw + row;
      wr[kb].x = static_cast<uint32_t>(src[0]) | (static_cast<uint32_t>(src[ldw]) << 16);
      wr[kb].y = static_cast<uint32_t>(src[2 * ldw]) | (static_cast<uint32_t>(src[3 * ldw]) << 16);
    } else {
      wr[kb] = *reinterpret_cast<const uint2*>(W + static_cast<size_t>(row) * ldw + 16 * kb + 4 * g);
    }
  }
}

template <int kKB, bool kTrans, bool kAcc>
__global__ __launch_bounds__(256) void proj_expand_kernel(ProjParams p) {
  constexpr int kWT = kExpandWaveTiles;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int T0 = blockIdx.x * 64;
  const int n_mt = p.M / 16;
  const int mt0 = blockIdx.y * kExpandTiles + w;  // the wave's tiles: mt0 + 4 i
  if (mt0 >= n_mt) return;
  const int n_t = min(kWT, (n_mt - mt0 + 3) / 4);  // wave-uniform
  const bf16_t* __restrict__ X = static_cast<const bf16_t*>(p.X);
  const bf16_t* __restrict__ W = static_cast<const bf16_t*>(p.W);
  bf16_t* __restrict__ C = static_cast<bf16_t*>(p.C) + T0 + 4 * j;
  auto crow = [&](int i, int e) { return C + static_cast<size_t>(16 * (mt0 + 4 * i) + 4 * g + e) * p.ldc; };
  uint2 cr[kAcc ? kWT : 1][4];
  if constexpr (kAcc) {
#pragma unroll
    for (int i = 0; i < kExpandCAhead && i < kWT; ++i)
      if (i < n_t)
#pragma unroll
        for (int e = 0; e < 4; ++e) cr[i][e] = *reinterpret_cast<const uint2*>(crow(i, e));
  }
  pbf16x4 bo[kKB][4];
  {
    uint2 xr[kKB][4];
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        xr[kb][e] = *reinterpret_cast<const uint2*>(X + static_cast<size_t>(16 * kb + 4 * g + e) * p.ldx + T0 + 4 * j);
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) transpose_4x4(xr[kb], bo[kb]);
  }
  uint2 wr[2][kKB];
  expand_load_w<kKB, kTrans>(W, p.ldw, 16 * mt0 + j, g, wr[0]);
#pragma unroll
  for (int i = 0; i < kWT; ++i) {
    if (i >= n_t) break;
    if (i + 1 < n_t) expand_load_w<kKB, kTrans>(W, p.ldw, 16 * (mt0 + 4 * (i + 1)) + j, g, wr[(i + 1) & 1]);
    if (kAcc && i + kExpandCAhead < kWT && i + kExpandCAhead < n_t) {
#pragma unroll
      for (int e = 0; e < 4; ++e) cr[i + kExpandCAhead][e] = *reinterpret_cast<const uint2*>(crow(i + kExpandCAhead, e));
    }
    pf32x4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = pf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb) {
      const pbf16x4 ao = pbf16x4_of(wr[i & 1][kb].x, wr[i & 1][kb].y);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = mfma16(ao, bo[kb][c], acc[c]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {  // row 16 (mt0 + 4 i) + 4 g + e, tokens 4 j .. 4 j + 3
      float v[4] = {acc[0][e], acc[1][e], acc[2][e], acc[3][e]};
      if constexpr (kAcc) {
        v[0] += __uint_as_float(cr[i][e].x << 16);
        v[1] += __uint_as_float(cr[i][e].x & 0xffff0000u);
        v[2] += __uint_as_float(cr[i][e].y << 16);
        v[3] += __uint_as_float(cr[i][e].y & 0xffff0000u);
      }
      const uint2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      *reinterpret_cast<uint2*>(crow(i, e)) = o;
    }
  }
}

// ---------------------------------------------------------------------------------------
template <int kMB>
static void launch_reduce_t(const ProjParams& p, hipStream_t stream) {
  if (p.w_trans)
    hipLaunchKernelGGL((proj_reduce_kernel<kMB, true>), dim3(p.T / 64), dim3((kMB + 2) * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((proj_reduce_kernel<kMB, false>), dim3(p.T / 64), dim3((kMB + 2) * 64), 0, stream, p);
}

template <int kKB>
static void launch_expand_t(const ProjParams& p, hipStream_t stream) {
  const dim3 grid(p.T / 64, (p.M / 16 + kExpandTiles - 1) / kExpandTiles);
  const bool acc = p.accumulate != 0;
  if (p.w_trans && acc)
    hipLaunchKernelGGL((proj_expand_kernel<kKB, true, true>), grid, dim3(256), 0, stream, p);
  else if (p.w_trans)
    hipLaunchKernelGGL((proj_expand_kernel<kKB, true, false>), grid, dim3(256), 0, stream, p);
  else if (acc)
    hipLaunchKernelGGL((proj_expand_kernel<kKB, false, true>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((proj_expand_kernel<kKB, false, false>), grid, dim3(256), 0, stream, p);
}

hipError_t launch_proj(const ProjParams& p, hipStream_t stream) {
  if (p.K <= kProjExpandMaxK) {
    switch (p.K / 16) {
      case 1: launch_expand_t<1>(p, stream); break;
      case 2: launch_expand_t<2>(p, stream); break;
      case 3: launch_expand_t<3>(p, stream); break;
      case 4: launch_expand_t<4>(p, stream); break;
      case 5: launch_expand_t<5>(p, stream); break;
      case 6: launch_expand_t<6>(p, stream); break;
      case 7: launch_expand_t<7>(p, stream); break;
      default: launch_expand_t<8>(p, stream); break;
    }
  } else {
    switch (p.M / 16) {
      case 1: launch_reduce_t<1>(p, stream); break;
      case 2: launch_reduce_t<2>(p, stream); break;
      case 3: launch_reduce_t<3>(p, stream); break;
      case 4: launch_reduce_t<4>(p, stream); break;
      case 5: launch_reduce_t<5>(p, stream); break;
      case 6: launch_reduce_t<6>(p, stream); break;
      case 7: launch_reduce_t<7>(p, stream); break;
      default: launch_reduce_t<8>(p, stream); break;
    }
  }
  return hipGetLastError();
}

}  // namespace mss
