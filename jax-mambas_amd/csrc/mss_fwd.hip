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
// B and C rows of the chunk are staged in LDS once per workgroup and shared by its waves.
#include "mss_common.h"

namespace mss {

template <int kT, int kW, bool kZOH, typename io_t, typename bc_t>
__global__ __launch_bounds__(kW * 64) void fwd_kernel(FwdParams p) {
  constexpr int kChunk = 64 * kT;
  constexpr int kStride = kT + 4;
  constexpr int kNB = 4;  // states staged per LDS round
  __shared__ __attribute__((aligned(16))) float sB[kNB][64 * kStride];
  __shared__ __attribute__((aligned(16))) float sC[kNB][64 * kStride];
  __shared__ float s_run[kW][kMaxN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.y;
  const int d_raw = blockIdx.x * kW + w;
  const bool active = d_raw < p.dim;
  const int d = active ? d_raw : p.dim - 1;
  const int L = p.seqlen;
  const int N = p.dstate;
  const int len = p.seq_lens ? min(max(p.seq_lens[b], 0), L) : L;
  const size_t chan = static_cast<size_t>(b) * p.dim + d;
  const size_t row = chan * L;

  const io_t* __restrict__ u_row = static_cast<const io_t*>(p.u) + row;
  const io_t* __restrict__ dl_row = static_cast<const io_t*>(p.delta) + row;
  io_t* __restrict__ out_row = static_cast<io_t*>(p.out) + row;
  const bc_t* __restrict__ Bb = static_cast<const bc_t*>(p.B) + static_cast<size_t>(b) * N * L;
  const bc_t* __restrict__ Cb = static_cast<const bc_t*>(p.C) + static_cast<size_t>(b) * N * L;

  if (lane < N) s_run[w][lane] = p.x0 ? p.x0[chan * N + lane] : 0.f;
  const float Dv = p.D ? p.D[d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
  const bool vec_io = p.vec_io != 0;
  const bool vec_bc = p.vec_bc != 0;
  float dsum_total = 0.f;  // sum of delta over all finished steps (reference residual)

  const int n_chunks = (L + kChunk - 1) / kChunk;
  for (int c = 0; c < n_chunks; ++c) {
    const int t0 = c * kChunk;
    const int tl = t0 + lane * kT;

    if (t0 >= len) {
      // Entire chunk is past this row's length: state frozen, output zero.
      if (active) {
        float zero[kT];
#pragma unroll
        for (int j = 0; j < kT; ++j) zero[j] = 0.f;
        if (p.out) store_seg<kT>(out_row, tl, L, vec_io, zero);
        const int cidx = (tl + kT) / kCarryChunk - 1;
        if (p.carries && ((tl + kT) % kCarryChunk == 0) && cidx < p.n_carry) {
          for (int n = 0; n < N; ++n)
            p.carries[(chan * p.n_carry + cidx) * N + n] = s_run[w][n];
        }
        if (p.ref_states && lane == 63 && c < p.n_ref) {
          for (int n = 0; n < N; ++n) {
            const float a2 = p.A[d * N + n] * kLog2e;
            float* rs = p.ref_states + ((chan * p.n_ref + c) * N + n) * 2;
            rs[0] = fast_exp2(a2 * dsum_total);
            rs[1] = s_run[w][n];
          }
        }
        if (p.last && c == n_chunks - 1 && lane < N) p.last[chan * N + lane] = s_run[w][lane];
      }
      continue;
    }

    float dlt[kT], dlu[kT], y[kT];
    float ssum = 0.f;
    if (active) {
      load_seg<kT>(dl_row, tl, L, vec_io, dlt);
      load_seg<kT>(u_row, tl, L, vec_io, y);
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

    for (int n0 = 0; n0 < N; n0 += kNB) {
      const int nb = min(kNB, N - n0);
      __syncthreads();  // previous round's LDS readers are done
      for (int k = 0; k < nb; ++k) {
        stage_row<kT>(Bb + static_cast<size_t>(n0 + k) * L, t0, L, vec_bc, sB[k], tid, kW * 64);
        stage_row<kT>(Cb + static_cast<size_t>(n0 + k) * L, t0, L, vec_bc, sC[k], tid, kW * 64);
      }
      __syncthreads();
      if (!active) continue;
      for (int k = 0; k < nb; ++k) {
        const int n = n0 + k;
        const float An = p.A[d * N + n];
        const float a2 = An * kLog2e;
        float a[kT], bu[kT];
        float H = 0.f;
        {
          float bv[kT];
          lds_read_seg<kT>(sB[k], lane, bv);
#pragma unroll
          for (int j = 0; j < kT; ++j) {
            a[j] = fast_exp2(dlt[j] * a2);
            if constexpr (kZOH) {
              bu[j] = (expm1f(dlt[j] * An) / An) * bv[j] * dlu[j];
            } else {
              bu[j] = dlu[j] * bv[j];
            }
            H = __builtin_fmaf(a[j], H, bu[j]);
          }
        }
        float P = fast_exp2(a2 * ssum);
        wave_scan_affine_fwd(P, H);
        const float run = s_run[w][n];
        const float hend = __builtin_fmaf(P, run, H);  // true state at the lane's last step
        float h = dpp_mov<kWaveShr1, 0xF>(run, hend);   // carry-in (lane 0: running state)
        {
          float cv[kT];
          lds_read_seg<kT>(sC[k], lane, cv);
#pragma unroll
          for (int j = 0; j < kT; ++j) {
            h = __builtin_fmaf(a[j], h, bu[j]);
            y[j] = __builtin_fmaf(cv[j], h, y[j]);
          }
        }
        const float run_new = readlane(hend, 63);
        if (lane == 0) s_run[w][n] = run_new;
        // Residuals: state at each 1024-step boundary; reference (prod, h) at 2048 ends.
        if (p.carries && ((tl + kT) % kCarryChunk == 0)) {
          const int cidx = (tl + kT) / kCarryChunk - 1;
          if (cidx < p.n_carry) p.carries[(chan * p.n_carry + cidx) * N + n] = hend;
        }
        if (p.ref_states && lane == 63 && (tl + kT) % kRefChunk == 0) {
          float* rs = p.ref_states + ((chan * p.n_ref + (tl + kT) / kRefChunk - 1) * N + n) * 2;
          rs[0] = fast_exp2(a2 * dsum_total);
          rs[1] = hend;
        }
        if (p.last && c == n_chunks - 1 && lane == 63) p.last[chan * N + n] = hend;
      }
    }

    if (active && p.out) {
      if (p.z) {
        float zv[kT];
        load_seg<kT>(static_cast<const io_t*>(p.z) + row, tl, L, vec_io, zv);
#pragma unroll
        for (int j = 0; j < kT; ++j) y[j] *= zv[j] * sigmoid(zv[j]);
      }
#pragma unroll
      for (int j = 0; j < kT; ++j) y[j] = (tl + j < len) ? y[j] : 0.f;
      store_seg<kT>(out_row, tl, L, vec_io, y);
    }
  }
}

template <int kT, int kW, bool kZOH, typename io_t, typename bc_t>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  dim3 grid((p.dim + kW - 1) / kW, p.batch);
  hipLaunchKernelGGL((fwd_kernel<kT, kW, kZOH, io_t, bc_t>), grid, dim3(kW * 64), 0, stream, p);
  return hipGetLastError();
}

template <bool kZOH, typename io_t, typename bc_t>
static hipError_t launch_fwd_z(const FwdParams& p, hipStream_t stream) {
  return launch_fwd_t<32, 4, kZOH, io_t, bc_t>(p, stream);
}

hipError_t launch_fwd(const FwdParams& p, int zoh, int io_bf16, int bc_bf16, hipStream_t stream) {
  if (zoh) {
    if (io_bf16) return bc_bf16 ? launch_fwd_z<true, bf16_t, bf16_t>(p, stream)
                                : launch_fwd_z<true, bf16_t, float>(p, stream);
    return bc_bf16 ? launch_fwd_z<true, float, bf16_t>(p, stream)
                   : launch_fwd_z<true, float, float>(p, stream);
  }
  if (io_bf16) return bc_bf16 ? launch_fwd_z<false, bf16_t, bf16_t>(p, stream)
                              : launch_fwd_z<false, bf16_t, float>(p, stream);
  return bc_bf16 ? launch_fwd_z<false, float, bf16_t>(p, stream)
                 : launch_fwd_z<false, float, float>(p, stream);
}

}  // namespace mss
