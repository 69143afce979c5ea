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
// waves per SIMD; their accumulators are added through LDS at the end. Shapes with a side
// below 192 (the S6 projections' 80- and 48-wide gradients) take 96 x 96 tiles instead: 4
// waves per workgroup, one 16-k step of each stage apiece, two workgroups per CU. Operands travel by
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

constexpr int kWgSub = 96;          // a sub-tile: 3 x 3 MFMA tiles of 32 x 32
constexpr int kWgMT = kWgSub / 32;   // 3 MFMA tiles per side

// Launch shapes: kTile x kTile output tiles of (kTile / 96)^2 sub-tiles, each owned by kKW
// waves that split the 16-k steps of every kBK-deep stage; kNS stages in the ring.
template <int kTile, int kKW, int kNS, int kBK>
struct WgShape {
  static constexpr int kSubs = kTile / kWgSub;
  static constexpr int kWaves = kSubs * kSubs * kKW;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kChunks = kBK / 8;           // 16-byte chunks of a row in a stage
  static constexpr int kSlots = kTile * kChunks;    // 16-byte slots of one operand stage
  static constexpr int kCopies = 2 * kSlots / kThreads;  // copy instructions per thread per stage
  static constexpr int kSteps = kBK / 16 / kKW;     // 16-k steps per wave per stage
  static_assert(2 * kSlots % kThreads == 0 && kCopies % 2 == 0, "copy rounds per stage");
  static_assert(kBK == 64 || kBK == 128, "8 or 16 chunks per row");
  static_assert(kSteps >= 1 && kSteps * kKW * 16 == kBK, "k steps split evenly");
  static_assert((kNS == 3 || kNS == 6) && (kNS - 2) * kCopies < 64, "ring depth within the buffers and vmcnt");
};

template <int kN>
__device__ __forceinline__ void wg_wait_vm() {
  static_assert(kN >= 0 && kN < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kN) : "memory");
}

// Position of a row's chunk c in LDS: the 16 lanes of one read phase (16 consecutive rows,
// one chunk) land on 16 distinct 16-byte bank groups, i.e. all 64 banks.
template <int kChunks>
__device__ __forceinline__ int wg_pos(int row, int c) {
  return kChunks == 8 ? c ^ ((row >> 1) & 7) : c ^ (row & 15);
}

template <int kTile, int kKW, int kNS, int kBK>
__global__ __launch_bounds__(64 * (kTile / kWgSub) * (kTile / kWgSub) * kKW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void wgrad_kernel(WgradParams p) {
  using Sh = WgShape<kTile, kKW, kNS, kBK>;
  constexpr int kSlots = Sh::kSlots, kWaves = Sh::kWaves, kSubs = Sh::kSubs, kSubTiles = kSubs * kSubs;
  constexpr int kChunks = Sh::kChunks, kWgCopies = Sh::kCopies;
  constexpr int kS3 = kNS > 3 ? kSlots : 1, kS4 = kNS > 4 ? kSlots : 1, kS5 = kNS > 5 ? kSlots : 1;
  // The ring's stages as distinct objects, each selected by a constant: the compiler then
  // tells the copies in flight into one from the reads of another (it would wait for every
  // copy before reading a stage it cannot identify).
  __shared__ u32x4 sA0[kSlots], sB0[kSlots], sA1[kSlots], sB1[kSlots], sA2[kSlots], sB2[kSlots];
  __shared__ u32x4 sA3[kS3], sB3[kS3], sA4[kS4], sB4[kS4], sA5[kS5], sB5[kS5];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wt = w % kSubTiles, wk = w / kSubTiles;  // sub-tile, share of the k steps
  const int wm = wt % kSubs, wn = wt / kSubs;
  const int j = lane & 31, g = lane >> 5;
  const int tiles_m = (p.M + kTile - 1) / kTile, tiles_n = (p.N + kTile - 1) / kTile;
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
  const int m0 = mb * kTile, n0 = nb * kTile;
  const int ks_total = p.K / kBK;
  const int kb = static_cast<int>(static_cast<long long>(s) * ks_total / p.splits);
  const int nk = static_cast<int>(static_cast<long long>(s + 1) * ks_total / p.splits) - kb;
  const bf16_t* __restrict__ A = static_cast<const bf16_t*>(p.A);
  const bf16_t* __restrict__ B = static_cast<const bf16_t*>(p.B);

  // Stage kk: slot i * 64 + lane of each operand = row slot / 8, stored chunk slot % 8. Rows
  // past M (N) re-read the last row: finite values whose products land in discarded outputs.
  auto issue = [&](int kk, u32x4* dA, u32x4* dB) {
    const int k0 = kk * kBK;
#pragma unroll
    for (int t = 0; t < kWgCopies / 2; ++t) {
      const int i = w + kWaves * t;
      const int slot = i * 64 + lane;
      const int row = slot / kChunks, c = wg_pos<kChunks>(row, slot % kChunks);
      const bf16_t* src = A + static_cast<size_t>(min(m0 + row, p.M - 1)) * p.lda + k0 + 8 * c;
      __builtin_amdgcn_global_load_lds((gbl_void_t)src, (lds_void_t)(dA + i * 64), 16, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < kWgCopies / 2; ++t) {
      const int i = w + kWaves * t;
      const int slot = i * 64 + lane;
      const int row = slot / kChunks, c = wg_pos<kChunks>(row, slot % kChunks);
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
      o.a[t] = __builtin_bit_cast(wbf16x8, bufA[ra * kChunks + wg_pos<kChunks>(ra, ck)]);
      const int rb = wn * kWgSub + 32 * t + j;
      o.b[t] = __builtin_bit_cast(wbf16x8, bufB[rb * kChunks + wg_pos<kChunks>(rb, ck)]);
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
    constexpr int kSteps = Sh::kSteps;
    const int ks0 = kSteps * wk;
    Ops o0, o1;
    load_ops(bufA, bufB, ks0, o0);
    if constexpr (kSteps == 1) {
      mma(o0);
    } else {
#pragma unroll
      for (int q = 0; q < kSteps; q += 2) {  // operands of step q + 1 read under step q's products
        load_ops(bufA, bufB, ks0 + q + 1, o1);
        mma(o0);
        if (q + 2 < kSteps) load_ops(bufA, bufB, ks0 + q + 2, o0);
        mma(o1);
      }
    }
  };

  // Ring of kNS stages: stages st + 1 .. st + kNS - 1 are in flight while stage st is
  // multiplied. Stage st has landed once at most (the number of stages issued after it) x
  // kWgCopies of this thread's copies are outstanding. Each step names its buffers
  // explicitly (the copies' destinations must be evident to the compiler).
#define MSS_WGRAD_STEP(O, CA, CB, NA, NB)                                          \
  {                                                                                \
    const int st = gg + O;                                                         \
    if (st < nk) {                                                                 \
      const int later = min(kNS - 2, nk - 1 - st);                                 \
      if (later >= 4) wg_wait_vm<4 * kWgCopies>();                                 \
      else if (later == 3) wg_wait_vm<3 * kWgCopies>();                            \
      else if (later == 2) wg_wait_vm<2 * kWgCopies>();                            \
      else if (later == 1) wg_wait_vm<kWgCopies>();                                \
      else wg_wait_vm<0>();                                                        \
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                           \
      __builtin_amdgcn_s_barrier();                                                \
      if (st + kNS - 1 < nk) issue(kb + st + kNS - 1, NA, NB);                     \
      compute(CA, CB);                                                             \
    }                                                                              \
  }
  static_assert(kNS == 3 || kNS == 6, "rings of 3 or 6 stages");
  if constexpr (kNS == 3) {
    if (nk > 0) issue(kb, sA0, sB0);
    if (nk > 1) issue(kb + 1, sA1, sB1);
    for (int gg = 0; gg < nk; gg += 3) {
      MSS_WGRAD_STEP(0, sA0, sB0, sA2, sB2)
      MSS_WGRAD_STEP(1, sA1, sB1, sA0, sB0)
      MSS_WGRAD_STEP(2, sA2, sB2, sA1, sB1)
    }
  } else {
    if (nk > 0) issue(kb, sA0, sB0);
    if (nk > 1) issue(kb + 1, sA1, sB1);
    if (nk > 2) issue(kb + 2, sA2, sB2);
    if (nk > 3) issue(kb + 3, sA3, sB3);
    if (nk > 4) issue(kb + 4, sA4, sB4);
    for (int gg = 0; gg < nk; gg += 6) {
      MSS_WGRAD_STEP(0, sA0, sB0, sA5, sB5)
      MSS_WGRAD_STEP(1, sA1, sB1, sA0, sB0)
      MSS_WGRAD_STEP(2, sA2, sB2, sA1, sB1)
      MSS_WGRAD_STEP(3, sA3, sB3, sA2, sB2)
      MSS_WGRAD_STEP(4, sA4, sB4, sA3, sB3)
      MSS_WGRAD_STEP(5, sA5, sB5, sA4, sB4)
    }
  }
#undef MSS_WGRAD_STEP

  // The other waves of a sub-tile hand their accumulators to its first wave (wk == 0), in
  // order wk = 1, 2, ..., one row of MFMA tiles at a time, through the idle stage buffers
  // (3 tiles x 16 x 64 floats per sub-tile: sub-tiles 0, 1 in sA0, 2, 3 in sB0).
  constexpr int kHalf = (kSubTiles + 1) / 2;
  float* xs = reinterpret_cast<float*>(wt < kHalf ? sA0 : sB0) + (wt % kHalf) * kWgMT * 16 * 64;
  static_assert(kHalf * kWgMT * 16 * 64 * 4 <= kSlots * 16, "hand-over fits a stage buffer");
#pragma unroll
  for (int mt = 0; mt < kWgMT; ++mt) {
#pragma unroll
    for (int src = 1; src < kKW; ++src) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __syncthreads();
      if (wk == src) {
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
  }
  if (wk != 0) return;

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

static int wgrad_tile(int M, int N) { return M >= kWgradTile && N >= kWgradTile ? kWgradTile : kWgSub; }
// Stage depth: 128 k (256-byte row pieces, fewer DRAM page visits) for the 96 x 96 tiles of the
// skinny, memory-bound shapes when K allows, else 64.
static int wgrad_bk(int M, int N, int K) { return wgrad_tile(M, N) == kWgSub && K % 128 == 0 ? 128 : 64; }

int wgrad_splits(int M, int N, int K) {
  const int t = wgrad_tile(M, N);
  const int tiles = ((M + t - 1) / t) * ((N + t - 1) / t);
  const int ks = K / wgrad_bk(M, N, K);
  int s = (kCUs + tiles / 2) / tiles;  // one pass over the CUs
  s = s < ks / 4 ? s : ks / 4;         // at least 4 stages per split
  return s < 1 ? 1 : s;
}

hipError_t launch_wgrad(const WgradParams& p, hipStream_t stream) {
  const int t = wgrad_tile(p.M, p.N);
  const int nwg = ((p.M + t - 1) / t) * ((p.N + t - 1) / t) * p.splits;
  if (t == kWgradTile)
    hipLaunchKernelGGL((wgrad_kernel<kWgradTile, 2, 3, 64>), dim3(nwg), dim3(WgShape<kWgradTile, 2, 3, 64>::kThreads), 0,
                       stream, p);
  else if (wgrad_bk(p.M, p.N, p.K) == 128)
    hipLaunchKernelGGL((wgrad_kernel<kWgSub, 4, 3, 128>), dim3(nwg), dim3(WgShape<kWgSub, 4, 3, 128>::kThreads), 0,
                       stream, p);
  else
    hipLaunchKernelGGL((wgrad_kernel<kWgSub, 4, 6, 64>), dim3(nwg), dim3(WgShape<kWgSub, 4, 6, 64>::kThreads), 0,
                       stream, p);
  if (p.splits > 1) {
    const long long total = static_cast<long long>(p.M) * (p.N / 4);
    const long long blocks = (total + 255) / 256;
    hipLaunchKernelGGL(wgrad_reduce_kernel, dim3(static_cast<unsigned>(blocks < 2048 ? blocks : 2048)), dim3(256), 0,
                       stream, p);
  }
  return hipGetLastError();
}

}  // namespace mss
