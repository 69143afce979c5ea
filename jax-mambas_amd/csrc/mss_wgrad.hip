// Weight-gradient GEMMs of the training step on the matrix cores: C[M][N] (+)= A[M][K] B[N][K]^T
// with bf16 operands whose rows are contiguous along K (the tokens) and float32 output, i.e.
// dW = dY X^T for a linear layer over channel-major activations [features][tokens]. In the
// reference these are the gradients XLA forms for the Mamba block's dense projections
// (mamba/mamba1.py:272-276, 330-337: in_proj over [x; z], out_proj) and for the S6 input
// projections (s_B / s_C / Linear_R stacked as one x-projection, Linear_Delta; :52-67,
// 107-124). Tiles at the M / N edges are partial (rows past the edge read the last row and
// their outputs are dropped).
//
// The output is small (at the 130M shape 3072 x 768 and 768 x 1536) and the contraction long
// (16384 tokens), so a library tiling that gives one workgroup per output tile leaves most of
// the GPU idle or re-streams the operands through small tiles (measured on MI355X: 105-115 us
// and 65-68 us with float32 output). Here the tokens are split over workgroups (split-K): each
// workgroup computes one 192 x 192 float32 partial tile over K / S tokens, S chosen so that
// tiles x S fills the 256 CUs once; a second kernel adds the S partial planes in a fixed order
// (deterministic), plus C when accumulating.
//
// Workgroup: 8 waves. Waves w and w + 4 own the same 96 x 96 sub-tile (3 x 3 tiles of
// v_mfma_f32_32x32x16_bf16) and split each 64-k stage's four 16-k steps between them, two
// waves per SIMD; their accumulators are added through LDS at the end. Operands travel by
// direct-to-LDS copies (16 bytes per lane) through a 3-stage ring of static buffers, each
// stage 192 rows x 64 k of A and of B (48 KB), with a counted vmcnt wait and a bare s_barrier
// per stage (__syncthreads would drain the copies in flight). A row's eight 16-byte k-chunks
// sit at chunk ^ ((row >> 1) & 7): the 16 lanes of one LDS read phase (16 rows, one chunk)
// then cover all 64 banks. XCD-aware order: consecutive workgroup ids go to different XCDs,
// so each XCD gets a contiguous range of (split, tile) numbers, tiles ordered so the ones an
// XCD holds share the larger operand's rows.
//
// 32x32x16 operand layout (lane l, its 8 bf16): A[i][k] at l = i + 32 (k / 8), element k % 8;
// B[k][j] at l = j + 32 (k / 8), element k % 8; D[i][j] at l = j + 32 ((i / 4) % 2),
// register 4 (i / 8) + i % 4.
#include <hip/hip_runtime.h>

#include "mss_common.h"

namespace mss {

namespace {

typedef __bf16 wbf16x8 __attribute__((ext_vector_type(8)));
typedef float wf32x16 __attribute__((ext_vector_type(16)));

constexpr int kWgTile = kWgradTile;  // 192
constexpr int kWgSub = kWgTile / 2;  // 96: a wave pair's sub-tile
constexpr int kWgMT = kWgSub / 32;   // 3 MFMA tiles per side
constexpr int kWgWaves = 8;
constexpr int kWgThreads = 64 * kWgWaves;
constexpr int kWgSlots = kWgTile * 8;                // 16-byte slots of one operand stage
constexpr int kWgCopies = 2 * kWgSlots / kWgThreads;  // copy instructions per thread per stage
static_assert(kWgSlots % kWgThreads == 0, "whole copy rounds");

template <int kN>
__device__ __forceinline__ void wg_wait_vm() {
  static_assert(kN >= 0 && kN < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kN) : "memory");
}

__device__ __forceinline__ int wg_swz(int row) { return (row >> 1) & 7; }

__global__ __launch_bounds__(kWgThreads) void wgrad_kernel(WgradParams p) {
  __shared__ u32x4 sA0[kWgSlots], sB0[kWgSlots], sA1[kWgSlots], sB1[kWgSlots], sA2[kWgSlots], sB2[kWgSlots];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wt = w & 3, wk = w >> 2;  // sub-tile, half of the k steps
  const int wm = wt & 1, wn = wt >> 1;
  const int j = lane & 31, g = lane >> 5;
  const int tiles_m = (p.M + kWgTile - 1) / kWgTile, tiles_n = (p.N + kWgTile - 1) / kWgTile;
  const int tiles = tiles_m * tiles_n;
  const int nwg = tiles * p.splits;
  const int id = blockIdx.x;
  const int lin = nwg % 8 == 0 ? (id & 7) * (nwg / 8) + (id >> 3) : id;
  const int s = lin / tiles;
  const int rem = lin - s * tiles;
  int mb, nb;
  if (p.M >= p.N) {
    mb = rem / tiles_n;
    nb = rem - mb * tiles_n;
  } else {
    nb = rem / tiles_m;
    mb = rem - nb * tiles_m;
  }
  const int m0 = mb * kWgTile, n0 = nb * kWgTile;
  const int ks_total = p.K / 64;
  const int kb = static_cast<int>(static_cast<long long>(s) * ks_total / p.splits);
  const int nk = static_cast<int>(static_cast<long long>(s + 1) * ks_total / p.splits) - kb;
  const bf16_t* __restrict__ A = static_cast<const bf16_t*>(p.A);
  const bf16_t* __restrict__ B = static_cast<const bf16_t*>(p.B);

  // Stage kk: slot i * 64 + lane of each operand = row slot / 8, stored chunk slot % 8. Rows
  // past M (N) re-read the last row: finite values whose products land in discarded outputs.
  auto issue = [&](int kk, u32x4* dA, u32x4* dB) {
    const int k0 = kk * 64;
#pragma unroll
    for (int t = 0; t < kWgCopies / 2; ++t) {
      const int i = w + kWgWaves * t;
      const int slot = i * 64 + lane;
      const int row = slot >> 3, c = (slot & 7) ^ wg_swz(row);
      const bf16_t* src = A + static_cast<size_t>(min(m0 + row, p.M - 1)) * p.lda + k0 + 8 * c;
      __builtin_amdgcn_global_load_lds((gbl_void_t)src, (lds_void_t)(dA + i * 64), 16, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < kWgCopies / 2; ++t) {
      const int i = w + kWgWaves * t;
      const int slot = i * 64 + lane;
      const int row = slot >> 3, c = (slot & 7) ^ wg_swz(row);
      const bf16_t* src = B + static_cast<size_t>(min(n0 + row, p.N - 1)) * p.ldb + k0 + 8 * c;
      __builtin_amdgcn_global_load_lds((gbl_void_t)src, (lds_void_t)(dB + i * 64), 16, 0, 0);
    }
  };

  wf32x16 acc[kWgMT][kWgMT];
#pragma unroll
  for (int a = 0; a < kWgMT; ++a)
#pragma unroll
    for (int b = 0; b < kWgMT; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  struct Ops {
    wbf16x8 a[kWgMT], b[kWgMT];
  };
  auto load_ops = [&](const u32x4* bufA, const u32x4* bufB, int ks, Ops& o) {
    const int ck = 2 * ks + g;
#pragma unroll
    for (int t = 0; t < kWgMT; ++t) {
      const int ra = wm * kWgSub + 32 * t + j;
      o.a[t] = __builtin_bit_cast(wbf16x8, bufA[ra * 8 + (ck ^ wg_swz(ra))]);
      const int rb = wn * kWgSub + 32 * t + j;
      o.b[t] = __builtin_bit_cast(wbf16x8, bufB[rb * 8 + (ck ^ wg_swz(rb))]);
    }
  };
  auto mma = [&](const Ops& o) {
#pragma unroll
    for (int mt = 0; mt < kWgMT; ++mt)
#pragma unroll
      for (int nt = 0; nt < kWgMT; ++nt)
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(o.a[mt], o.b[nt], acc[mt][nt], 0, 0, 0);
  };
  auto compute = [&](const u32x4* bufA, const u32x4* bufB) {
    __builtin_amdgcn_iglp_opt(0);  // interleave the operand reads with the products
    Ops o0, o1;
    load_ops(bufA, bufB, 2 * wk, o0);
    load_ops(bufA, bufB, 2 * wk + 1, o1);
    mma(o0);
    mma(o1);
  };

  // Ring of three stages: stage st + 2 is copied while stage st is multiplied.
  if (nk > 0) issue(kb, sA0, sB0);
  if (nk > 1) issue(kb + 1, sA1, sB1);
#define MSS_WGRAD_STEP(O, CA, CB, NA, NB)                  \
  {                                                        \
    const int st = gg + O;                                 \
    if (st < nk) {                                         \
      if (st + 1 < nk)                                     \
        wg_wait_vm<kWgCopies>();                           \
      else                                                 \
        wg_wait_vm<0>();                                   \
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   \
      __builtin_amdgcn_s_barrier();                        \
      if (st + 2 < nk) issue(kb + st + 2, NA, NB);         \
      compute(CA, CB);                                     \
    }                                                      \
  }
  for (int gg = 0; gg < nk; gg += 3) {
    MSS_WGRAD_STEP(0, sA0, sB0, sA2, sB2)
    MSS_WGRAD_STEP(1, sA1, sB1, sA0, sB0)
    MSS_WGRAD_STEP(2, sA2, sB2, sA1, sB1)
  }
#undef MSS_WGRAD_STEP

  // Wave w + 4 hands its accumulators to wave w, one row of MFMA tiles at a time, through the
  // idle stage buffers (sub-tiles 0, 1 in sA0, 2, 3 in sB0: 3 tiles x 16 x 64 floats each).
  float* xs = reinterpret_cast<float*>(wt < 2 ? sA0 : sB0) + (wt & 1) * kWgMT * 16 * 64;
  static_assert(2 * kWgMT * 16 * 64 * 4 <= kWgSlots * 16, "hand-over fits a stage buffer");
#pragma unroll
  for (int mt = 0; mt < kWgMT; ++mt) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();
    if (wk == 1) {
#pragma unroll
      for (int nt = 0; nt < kWgMT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) xs[(nt * 16 + r) * 64 + lane] = acc[mt][nt][r];
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int nt = 0; nt < kWgMT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mt][nt][r] += xs[(nt * 16 + r) * 64 + lane];
    }
  }
  if (wk == 1) return;

  // One split: the tile goes to C (added to it when accumulating); else to partial plane s.
  const bool direct = p.splits == 1;
  float* __restrict__ out = direct ? p.C : p.workspace + static_cast<size_t>(s) * p.M * p.N;
  const long long ldo = direct ? p.ldc : p.N;
#pragma unroll
  for (int mt = 0; mt < kWgMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kWgMT; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * kWgSub + 32 * mt + 8 * (r >> 2) + 4 * g + (r & 3);
        const int col = n0 + wn * kWgSub + 32 * nt + j;
        if (row >= p.M || col >= p.N) continue;
        float* dst = out + static_cast<size_t>(row) * ldo + col;
        float v = acc[mt][nt][r];
        if (direct && p.accumulate) v += *dst;
        *dst = v;
      }
}

// C = (C +) sum over s of partial plane s, in order s = 0, 1, ..., 4 columns per thread.
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(WgradParams p) {
  const int n4 = p.N / 4;
  const long long total = static_cast<long long>(p.M) * n4;
  const size_t plane = static_cast<size_t>(p.M) * p.N;
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < total; i += static_cast<long long>(gridDim.x) * 256) {
    const int row = static_cast<int>(i / n4);
    const int c4 = static_cast<int>(i - static_cast<long long>(row) * n4);
    const float* src = p.workspace + static_cast<size_t>(row) * p.N + 4 * c4;
    float4* dst = reinterpret_cast<float4*>(p.C + static_cast<size_t>(row) * p.ldc + 4 * c4);
    float4 acc = p.accumulate ? *dst : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < p.splits; ++s) {
      const float4 v = *reinterpret_cast<const float4*>(src + s * plane);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    *dst = acc;
  }
}

}  // namespace

int wgrad_splits(int M, int N, int K) {
  const int tiles = ((M + kWgTile - 1) / kWgTile) * ((N + kWgTile - 1) / kWgTile);
  const int ks = K / 64;
  int s = (kCUs + tiles / 2) / tiles;  // one pass of one workgroup per CU (144 KB of LDS each)
  s = s < ks / 4 ? s : ks / 4;         // at least 4 stages per split
  return s < 1 ? 1 : s;
}

hipError_t launch_wgrad(const WgradParams& p, hipStream_t stream) {
  const int nwg = ((p.M + kWgTile - 1) / kWgTile) * ((p.N + kWgTile - 1) / kWgTile) * p.splits;
  hipLaunchKernelGGL(wgrad_kernel, dim3(nwg), dim3(kWgThreads), 0, stream, p);
  if (p.splits > 1) {
    const long long total = static_cast<long long>(p.M) * (p.N / 4);
    const long long blocks = (total + 255) / 256;
    hipLaunchKernelGGL(wgrad_reduce_kernel, dim3(static_cast<unsigned>(blocks < 2048 ? blocks : 2048)), dim3(256), 0,
                       stream, p);
  }
  return hipGetLastError();
}

}  // namespace mss
