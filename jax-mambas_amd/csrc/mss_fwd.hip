// Forward selective scan for gfx950 (MI355X).
//
// Reference behaviour followed (not its structure): native/selective_scan_cuda.cu:205-332
// (per (batch, channel) recurrence with cross-chunk carry, exp2 form of exp(delta*A),
// identity padding past the sequence end, chunk residual at 2048-step ends) plus the
// fusions the reference model performs around the scan (mamba/mamba1.py:160-198, 300-337).
//
// Mapping: workgroup = kW waves = kW consecutive channels of one batch row; wave = one
// channel; lane = one segment of kT consecutive steps; one wave pass covers a chunk of
// 64*kT steps. Per chunk and per state n:
//   phase A  lane-local: a_t = exp2(delta_t * A_n * log2e), bu_t; aggregate (P, H) of the
//            segment with zero carry (P = exp2(A_n * log2e * sum delta), one exp per lane)
//   scan     64-lane inclusive affine scan of (P, H) on DPP; the lane's carry-in is the
//            previous lane's end state (the chunk's running state for lane 0)
//   phase C  lane-local re-run from the true carry; y_t += C_t * h_t
// B and C rows of the chunk are staged in LDS once per workgroup and shared by its waves:
// rounds of kNB states are copied global->LDS with gfx950's direct-to-LDS loads into one
// of two buffers while the previous round is computed (one barrier per round).
#include "mss_fwd_kernel.h"

namespace mss {

// bf16-I/O instantiations live in mss_fwd_bf16.hip.
hipError_t launch_fwd_bf16(const FwdParams& p, int zoh, int bc_bf16, hipStream_t stream);

hipError_t launch_fwd(const FwdParams& p, int zoh, int io_bf16, int bc_bf16, hipStream_t stream) {
  if (io_bf16) return launch_fwd_bf16(p, zoh, bc_bf16, stream);
  if (zoh) return bc_bf16 ? launch_fwd_z<true, float, bf16_t>(p, stream) : launch_fwd_z<true, float, float>(p, stream);
  return bc_bf16 ? launch_fwd_z<false, float, bf16_t>(p, stream) : launch_fwd_z<false, float, float>(p, stream);
}

// ---------------------------------------------------------------------------------
// Carry rebuild for the reference-signature backward (mss_scan_bwd): the state entering
// every 8-step segment, recomputed from the reference's chunk residual, which holds the
// state only at 2048-step block ends (native/selective_scan_cuda.cu:306-320; the reference
// backward likewise re-runs each block's recurrence from it,
// native/upstream_mamba/selective_scan_bwd_kernel.cuh:254-264). Real A, Euler, float32, no
// fused extras (the reference contract). Blocks are independent, so the grid is (channel
// groups, batch, 2048-step blocks): one wave per (channel, block), lane = an 8-step segment of
// a 512-step chunk. Per chunk and state: the segment's zero-carry aggregate (P, H), the
// 64-lane affine scan, the lane's carry-in stored; no C, no output.
constexpr int kRebuildW = 8;

template <int kMaxS>
__global__ __launch_bounds__(kRebuildW * 64) void carry_rebuild_kernel(FwdParams p) {
  constexpr int kT = kSegSteps;
  constexpr int kChunk = 64 * kT;
  constexpr int kChunksPerBlock = kRefChunk / kChunk;
  __shared__ float s_run[kRebuildW][kMaxS];
  __shared__ float s_a2[kRebuildW][kMaxS];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int blk = blockIdx.z;
  const int d = blockIdx.x * kRebuildW + w;
  if (d >= p.dim) return;  // no barrier in this kernel: idle waves may leave
  const int L = p.seqlen;
  const int N = p.dstate;
  const size_t chan = static_cast<size_t>(b) * p.dim + d;
  for (int n = lane; n < N; n += 64) {
    // state entering the block: the initial state, or h at the previous block's end
    s_run[w][n] = blk == 0 ? (p.x0 ? p.x0[chan * N + n] : 0.f)
                           : p.ref_states[((chan * p.n_ref + blk - 1) * N + n) * 2 + 1];
    s_a2[w][n] = p.A[static_cast<size_t>(d) * N + n] * kLog2e;
  }
  const float* __restrict__ u_row = static_cast<const float*>(p.u) + chan * L;
  const float* __restrict__ dl_row = static_cast<const float*>(p.delta) + chan * L;
  const float* __restrict__ Bb = static_cast<const float*>(p.B) + static_cast<size_t>(b) * N * L;
  const int c_end = min((L + kChunk - 1) / kChunk, (blk + 1) * kChunksPerBlock);
  for (int c = blk * kChunksPerBlock; c < c_end; ++c) {
    const int tl = c * kChunk + lane * kT;
    const bool fast = p.vec_io && c * kChunk + kChunk <= L;
    float dlt[kT], dlu[kT];
    load_seg<kT>(dl_row, tl, L, fast, dlt);
    load_seg<kT>(u_row, tl, L, fast, dlu);
    float ssum = 0.f;
#pragma unroll
    for (int j = 0; j < kT; ++j) {
      dlu[j] *= dlt[j];
      ssum += dlt[j];
    }
    const int seg_idx = tl / kT;
    const bool fast_b = fast && p.vec_bc;
    // B rows one state ahead: the next state's load is in flight while this one computes.
    float bv[kT];
    load_seg<kT>(Bb, tl, L, fast_b, bv);
    for (int n = 0; n < N; ++n) {
      const float a2 = s_a2[w][n];
      const float run = s_run[w][n];
      float bn[kT];
      if (n + 1 < N) load_seg<kT>(Bb + static_cast<size_t>(n + 1) * L, tl, L, fast_b, bn);
      float H = 0.f;
#pragma unroll
      for (int j = 0; j < kT; ++j) H = __builtin_fmaf(fast_exp2(dlt[j] * a2), H, dlu[j] * bv[j]);
      float P = fast_exp2(a2 * ssum);
      wave_scan_affine_fwd(P, H);
      const float hend = __builtin_fmaf(P, run, H);       // state after the lane's segment
      const float hin = dpp_mov<kWaveShr1, 0xF>(run, hend);  // state entering it
      if (seg_idx < p.n_seg) p.carries[(chan * N + n) * p.n_seg + seg_idx] = hin;
      const float run_new = readlane(hend, 63);
      if (lane == 0) s_run[w][n] = run_new;
      if (n + 1 < N) {
#pragma unroll
        for (int j = 0; j < kT; ++j) bv[j] = bn[j];
      }
    }
  }
}

hipError_t launch_carry_rebuild(const FwdParams& p, hipStream_t stream) {
  const dim3 grid((p.dim + kRebuildW - 1) / kRebuildW, p.batch, p.n_ref);
  if (p.dstate > kMaxNWide) return hipErrorInvalidValue;
  if (p.dstate > kMaxN)
    hipLaunchKernelGGL(carry_rebuild_kernel<kMaxNWide>, grid, dim3(kRebuildW * 64), 0, stream, p);
  else
    hipLaunchKernelGGL(carry_rebuild_kernel<kMaxN>, grid, dim3(kRebuildW * 64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mss
