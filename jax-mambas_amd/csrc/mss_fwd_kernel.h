// Forward selective-scan kernel for gfx950 (MI355X): the kernel template and its launch
// shapes, shared by the translation units that instantiate it (mss_fwd.hip: float32 I/O and
// the dispatcher; mss_fwd_bf16.hip: bf16 I/O, compiled with another machine-scheduler
// strategy). Algorithm and mapping: see the comment at the top of mss_fwd.hip.
#pragma once
#include "mss_common.h"


// Launch shapes. A "wide" shape (16 steps per lane, 4 waves per SIMD) for bf16 grids that
// fill the GPU several times over, and a "narrow" one (8 steps per lane, 6 waves per SIMD:
// 50% more resident workgroups) for float32 rows and for grids that fit in one pass of it,
// where the wide shape would leave a half-occupied tail pass. Waves per workgroup and states per staging round
// are shared; all are overridable at build time for tuning sweeps.
#ifndef MSS_FWD_W
#define MSS_FWD_W 8
#endif
#ifndef MSS_FWD_NB
#define MSS_FWD_NB 4
#endif
#ifndef MSS_FWD_T_WIDE
#define MSS_FWD_T_WIDE 16
#endif
#ifndef MSS_FWD_OCC_WIDE
#define MSS_FWD_OCC_WIDE 4
#endif
#ifndef MSS_FWD_T_NARROW
#define MSS_FWD_T_NARROW 8
#endif
#ifndef MSS_FWD_OCC_NARROW
#define MSS_FWD_OCC_NARROW 6
#endif

namespace mss {

// Stage elements [t0, t0 + 64*kT) of `nrows` rows (B rows of states n0.., then C rows)
// into dst[row][slot] (64*kT elements of bc_t per row), spread over all threads.
// Row k of B (C) starts at Bb (Cb) + (n0 + k) * sn.
// dma: rows are 16-byte aligned and L is a multiple of the slot width, so each slot is
// either fully inside [0, L) or fully past it; past-the-end slots re-read the last valid
// slot (finite values; they only meet zero coefficients).
template <int kT, int kW, int kNB, typename bc_t>
__device__ __forceinline__ void stage_round(const bc_t* __restrict__ Bb, const bc_t* __restrict__ Cb,
                                            int n0, int nb, int t0, int L, long long sn, bool dma,
                                            uint4 (*dst)[2][64 * kT * sizeof(bc_t) / 16], int tid) {
  constexpr int kE = BcStage<bc_t>::kElemsPerSlot;
  constexpr int kQ = kT / kE;
  constexpr int kSlots = 64 * kQ;  // per row
  const int total = nb * 2 * kSlots;
  if (dma) {
    const int lane = tid & 63;
    const int w = tid >> 6;
    // Lane's source offset inside a row for slot s0 + lane: the same for every row.
    for (int f0 = w * 64; f0 < total; f0 += kW * 64) {
      const int rowi = f0 / kSlots;  // uniform: kSlots is a multiple of 64
      const int k = rowi >> 1;
      const int which = rowi & 1;
      const int s0 = f0 - rowi * kSlots;
      const int s = s0 + lane;
      const int i = s / kQ;  // kQ is a power of two
      const int q = (s % kQ) ^ slot_swz<kQ>(i);
      int e = t0 + i * kT + q * kE;
      e = e < L ? e : L - kE;
      const bc_t* src = (which ? Cb : Bb) + (n0 + k) * sn + e;
      __builtin_amdgcn_global_load_lds((gbl_void_t)src, (lds_void_t)(&dst[k][which][s0]), 16, 0, 0);
    }
  } else {
    for (int f = tid; f < nb * 2 * 64 * kT; f += kW * 64) {
      const int rowi = f / (64 * kT);
      const int k = rowi >> 1;
      const int which = rowi & 1;
      const int e = f - rowi * 64 * kT;
      const int i = e / kT;
      const int r = e % kT;
      const int q = r / kE;
      const int sl = kQ * i + (q ^ slot_swz<kQ>(i));
      const int t = t0 + e;
      const bc_t* src = (which ? Cb : Bb) + (n0 + k) * sn;
      bc_t v;
      if (t < L) {
        v = src[t];
      } else {
        store_as(&v, 0.f);
      }
      reinterpret_cast<bc_t*>(&dst[k][which][0])[sl * kE + (r % kE)] = v;
    }
  }
}

// kMaxS: the per-wave state tables' size (kMaxN, or kMaxNWide for float32 scans with more
// states).
template <int kT, int kW, int kNB, int kOcc, bool kZOH, typename io_t, typename bc_t, int kMaxS = kMaxN>
__global__ __launch_bounds__(kW * 64) __attribute__((amdgpu_waves_per_eu(kOcc, kOcc)))
void fwd_kernel(FwdParams p) {
  constexpr int kChunk = 64 * kT;
  static_assert(kT % kSegSteps == 0, "lane segments must hold whole carry segments");
  constexpr int kRowSlots = kChunk * static_cast<int>(sizeof(bc_t)) / 16;
  // Two stage buffers as distinct objects, selected statically (rounds run in pairs), so
  // the compiler can tell the in-flight copy into one from the reads of the other.
  __shared__ uint4 stage0[kNB][2][kRowSlots];  // [state][B|C][slot]
  __shared__ uint4 stage1[kNB][2][kRowSlots];
  __shared__ float s_run[kW][kMaxS];
  __shared__ float s_a2[kW][kMaxS];
  __shared__ float s_a[kW][kMaxS];
  // 16-step lanes: each wave's z row for the current chunk, copied from global memory at the
  // chunk start (direct-to-LDS) so its latency passes under the state loop instead of after
  // it; lane i's q-th 16-byte slot at [q * 64 + i]. (Measured on MI355X, c3 forward 414 ->
  // 406 us, a c5 layer's 162 -> 158; with the 8-step float32 shape, whose three workgroups
  // per CU it would take 16 KB of LDS each, c2 102 -> 111, so that shape keeps the load.)
  constexpr bool kZLds = kT == 16;
  constexpr int kZq = kT * static_cast<int>(sizeof(io_t)) / 16;
  __shared__ uint4 s_z[kW][kZLds ? kZq * 64 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = row_longest_first(p.seq_lens, p.batch, p.seqlen, blockIdx.y);
  const int d_raw = blockIdx.x * kW + w;
  const bool active = d_raw < p.dim;
  const int d = active ? d_raw : p.dim - 1;
  const int L = p.seqlen;
  const int N = p.dstate;
  const int len = p.seq_lens ? min(max(p.seq_lens[b], 0), L) : L;
  const size_t chan = static_cast<size_t>(b) * p.dim + d;
  const long long row = b * p.io_sb + d * p.io_sd;

  const io_t* __restrict__ u_row = static_cast<const io_t*>(p.u) + row;
  const io_t* __restrict__ dl_row = static_cast<const io_t*>(p.delta) + row;
  io_t* __restrict__ out_row = static_cast<io_t*>(p.out) + row;
  const bc_t* __restrict__ Bb = static_cast<const bc_t*>(p.B) + b * p.bc_sb;
  const bc_t* __restrict__ Cb = static_cast<const bc_t*>(p.C) + b * p.bc_sb;

  for (int n = lane; n < N; n += 64) {
    s_run[w][n] = p.x0 ? p.x0[chan * N + n] : 0.f;
    const float an = p.A[static_cast<size_t>(d) * N + n];
    s_a[w][n] = an;
    s_a2[w][n] = an * kLog2e;
  }
  const float Dv = p.D ? p.D[d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
  const bool vec_io = p.vec_io != 0;
  const bool dma = p.vec_bc != 0;
  float dsum_total = 0.f;  // sum of delta over all finished steps (reference residual)

  const int n_chunks = (L + kChunk - 1) / kChunk;
  const int n_active_chunks = (len + kChunk - 1) / kChunk;
  // Rounds of kNB states per chunk, padded to an even count so round g of every chunk
  // uses buffer g & 1.
  const int rounds = ((N + kNB - 1) / kNB + 1) & ~1;
  auto issue_round = [&](int r, uint4 (*buf)[2][kRowSlots]) {
    const int c = r / rounds;
    const int n0 = (r - c * rounds) * kNB;
    const int nb = min(kNB, N - n0);
    if (nb > 0) stage_round<kT, kW, kNB, bc_t>(Bb, Cb, n0, nb, c * kChunk, L, p.bc_sn, dma, buf, tid);
  };
  if (n_active_chunks > 0) issue_round(0, stage0);

  for (int c = 0; c < n_chunks; ++c) {
    const int t0 = c * kChunk;
    const int tl = t0 + lane * kT;
    const bool fast = vec_io && (t0 + kChunk <= L);  // wave-uniform
    // Reference residual slot written at this chunk's end (2048-step boundary or end of
    // the sequence), -1 if none.
    const int chunk_end = t0 + kChunk;
    const int ref_idx = (chunk_end % kRefChunk == 0 || c == n_chunks - 1)
                            ? min((chunk_end + kRefChunk - 1) / kRefChunk, p.n_ref) - 1
                            : -1;

    if (c >= n_active_chunks) {
      // Entire chunk is past this row's length: state frozen, output zero. The backward's
      // residuals (carries, y_pre) are not written here: it never reads them.
      if (active) {
        float zero[kT];
#pragma unroll
        for (int j = 0; j < kT; ++j) zero[j] = 0.f;
        if (p.out) store_seg<kT>(out_row, tl, L, fast, zero);
        if (p.ref_states && lane == 63 && ref_idx >= 0) {
          for (int n = 0; n < N; ++n) {
            float* rs = p.ref_states + ((chan * p.n_ref + ref_idx) * N + n) * 2;
            rs[0] = fast_exp2(s_a2[w][n] * dsum_total);
            rs[1] = s_run[w][n];
          }
        }
        if (p.last && c == n_chunks - 1)
          for (int n = lane; n < N; n += 64) p.last[chan * N + n] = s_run[w][n];
      }
      continue;
    }

    float dlt[kT], dlu[kT], y[kT];
    float ssum = 0.f;
    // z through LDS for whole vectorisable chunks (wave-uniform); the first round barrier's
    // wait covers the copies.
    const bool z_lds = kZLds && active && fast && p.z != nullptr && p.out != nullptr;
    if (active) {
      load_seg<kT>(dl_row, tl, L, fast, dlt);
      load_seg<kT>(u_row, tl, L, fast, y);
      if (kZLds && z_lds) {
        const io_t* zsrc = static_cast<const io_t*>(p.z) + row + tl;
#pragma unroll
        for (int q = 0; q < kZq; ++q)
          __builtin_amdgcn_global_load_lds((gbl_void_t)(zsrc + q * (16 / static_cast<int>(sizeof(io_t)))),
                                           (lds_void_t)(&s_z[w][q * 64]), 16, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < kT; ++j) {
        const bool valid = tl + j < len;
        const float x = dlt[j] + bias;
        float dv = p.delta_softplus ? softplus(x) : x;
        dv = valid ? dv : 0.f;
        const float uu = valid ? y[j] : 0.f;
        dlt[j] = dv;
        dlu[j] = kZOH ? uu : dv * uu;  // ZOH keeps u; Euler keeps delta*u
        y[j] = Dv * uu;
        ssum += dv;
      }
    } else {
#pragma unroll
      for (int j = 0; j < kT; ++j) dlt[j] = dlu[j] = y[j] = 0.f;
    }
    if (p.ref_states) dsum_total += wave_sum(ssum);

    auto compute_round = [&](int g, uint4 (*buf)[2][kRowSlots]) {
      const int n0 = g * kNB;
      const int nb = min(kNB, N - n0);
      for (int k = 0; k < nb; ++k) {
        const int n = n0 + k;
        const float a2 = s_a2[w][n];
        const float run = s_run[w][n];  // read early: its wait would otherwise follow the scan
        float a[kT], bu[kT];
        float H = 0.f;
        {
          float bv[kT];
          read_staged<kT, bc_t>(buf[k][0], lane, bv);
#pragma unroll
          for (int j = 0; j < kT; ++j) {
            a[j] = fast_exp2(dlt[j] * a2);
            if constexpr (kZOH) {
              const float An = s_a[w][n];
              bu[j] = (expm1f(dlt[j] * An) * fast_rcp(An)) * bv[j] * dlu[j];
            } else {
              bu[j] = dlu[j] * bv[j];
            }
            H = __builtin_fmaf(a[j], H, bu[j]);
          }
        }
        float P = fast_exp2(a2 * ssum);
        wave_scan_affine_fwd(P, H);
        const float hend = __builtin_fmaf(P, run, H);  // true state at the lane's last step
        float h = dpp_mov<kWaveShr1, 0xF>(run, hend);   // carry-in (lane 0: running state)
        {
          float cv[kT];
          float hseg[kT / kSegSteps];  // state before each kSegSteps-step sub-segment
          read_staged<kT, bc_t>(buf[k][1], lane, cv);
#pragma unroll
          for (int j = 0; j < kT; ++j) {
            if (j % kSegSteps == 0) hseg[j / kSegSteps] = h;
            h = __builtin_fmaf(a[j], h, bu[j]);
            y[j] = __builtin_fmaf(cv[j], h, y[j]);
          }
          // Residual for the backward: the state entering every kSegSteps-step segment.
          if (p.carries) {
            float* crow = p.carries + (chan * N + n) * p.n_seg + tl / kSegSteps;
#pragma unroll
            for (int q = 0; q < kT / kSegSteps; ++q)
              if (tl / kSegSteps + q < p.n_seg) crow[q] = hseg[q];
          }
        }
        const float run_new = readlane(hend, 63);
        if (lane == 0) s_run[w][n] = run_new;
        // Reference residual: (prod, h) at 2048-step chunk ends.
        if (p.ref_states && lane == 63 && ref_idx >= 0) {
          float* rs = p.ref_states + ((chan * p.n_ref + ref_idx) * N + n) * 2;
          rs[0] = fast_exp2(a2 * dsum_total);
          rs[1] = hend;
        }
        if (p.last && c == n_chunks - 1 && lane == 63) p.last[chan * N + n] = hend;
      }
    };
    const int last_round = n_active_chunks * rounds;
    for (int g = 0; g < rounds; g += 2) {
      const int r = c * rounds + g;
      wait_vmem_all();   // this thread's copies for round r have landed in LDS
      __syncthreads();   // ... and everyone's; round r-1's readers are done
      if (r + 1 < last_round) issue_round(r + 1, stage1);
      if (active) compute_round(g, stage0);
      wait_vmem_all();
      __syncthreads();
      if (r + 2 < last_round) issue_round(r + 2, stage0);
      if (active) compute_round(g + 1, stage1);
    }

    if (active && p.out) {
      if (p.z) {
        float zv[kT];
        if (kZLds && z_lds) {
          // the wave's own copies, completed at the first round barrier
          if constexpr (sizeof(io_t) == 4) {
#pragma unroll
            for (int q = 0; q < kZq; ++q) {
              const uint4 x = s_z[w][q * 64 + lane];
              zv[4 * q + 0] = __uint_as_float(x.x);
              zv[4 * q + 1] = __uint_as_float(x.y);
              zv[4 * q + 2] = __uint_as_float(x.z);
              zv[4 * q + 3] = __uint_as_float(x.w);
            }
          } else {
#pragma unroll
            for (int q = 0; q < kZq; ++q) {
              const uint4 x = s_z[w][q * 64 + lane];
              const uint32_t wd[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                zv[8 * q + 2 * k + 0] = __uint_as_float(wd[k] << 16);
                zv[8 * q + 2 * k + 1] = __uint_as_float(wd[k] & 0xffff0000u);
              }
            }
          }
        } else {
          load_seg<kT>(static_cast<const io_t*>(p.z) + row, tl, L, fast, zv);
        }
        if (p.y_pre) {
          // The backward takes y sigma(z) from out / z; y itself is kept only where z is too
          // small for that (rare: nothing else of the row is written).
          io_t* __restrict__ yrow = static_cast<io_t*>(p.y_pre) + row;
#pragma unroll
          for (int j = 0; j < kT; ++j)
            if (tl + j < len && __builtin_fabsf(zv[j]) < kZTiny) store_as(yrow + tl + j, y[j]);
        }
#pragma unroll
        for (int j = 0; j < kT; ++j) y[j] *= zv[j] * sigmoid(zv[j]);
      }
#pragma unroll
      for (int j = 0; j < kT; ++j) y[j] = (tl + j < len) ? y[j] : 0.f;
      store_seg<kT>(out_row, tl, L, fast, y);
    }
  }
}

template <int kT, int kW, int kNB, int kOcc, bool kZOH, typename io_t, typename bc_t, int kMaxS = kMaxN>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  dim3 grid((p.dim + kW - 1) / kW, p.batch);
  hipLaunchKernelGGL((fwd_kernel<kT, kW, kNB, kOcc, kZOH, io_t, bc_t, kMaxS>), grid, dim3(kW * 64), 0, stream, p);
  return hipGetLastError();
}

template <bool kZOH, typename io_t, typename bc_t>
static hipError_t launch_fwd_z(const FwdParams& p, hipStream_t stream) {
  if (p.dstate > kMaxN) {
    // Wider state (float32 only): 24 KB of state tables per workgroup, two workgroups of
    // the narrow shape per CU (4 waves per SIMD).
    if constexpr (sizeof(io_t) == 4 && sizeof(bc_t) == 4) {
      if (p.dstate > kMaxNWide) return hipErrorInvalidValue;
      return launch_fwd_t<MSS_FWD_T_NARROW, MSS_FWD_W, MSS_FWD_NB, 4, kZOH, io_t, bc_t, kMaxNWide>(p, stream);
    } else {
      return hipErrorInvalidValue;
    }
  }
  // Resident workgroups of the narrow shape: 256 CUs * kOcc waves per SIMD * 4 SIMDs / kW.
  // Float32 rows take the narrow shape at every grid size (measured on MI355X: B=16 D=2560
  // L=8192 with variable lengths 1.69 -> 1.39 ms, B=8 D=2048 L=4096 0.54 -> 0.48 ms); bf16
  // rows take it only when the grid fits one pass of it (B=8 D=2048 L=4096 428 vs 436 us,
  // B=8 D=1536 L=2048 167 vs 175 us wide vs narrow).
  constexpr long long kNarrowSlots = 256LL * MSS_FWD_OCC_NARROW * 4 / MSS_FWD_W;
  const long long groups = static_cast<long long>(p.batch) * ((p.dim + MSS_FWD_W - 1) / MSS_FWD_W);
  if (sizeof(io_t) == 4 || groups <= kNarrowSlots)
    return launch_fwd_t<MSS_FWD_T_NARROW, MSS_FWD_W, MSS_FWD_NB, MSS_FWD_OCC_NARROW, kZOH, io_t, bc_t>(p, stream);
  return launch_fwd_t<MSS_FWD_T_WIDE, MSS_FWD_W, MSS_FWD_NB, MSS_FWD_OCC_WIDE, kZOH, io_t, bc_t>(p, stream);
}

}  // namespace mss
