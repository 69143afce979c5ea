// Backward selective scan for gfx950 (MI355X).
//
// Reference behaviour followed (not its structure):
// native/upstream_mamba/selective_scan_bwd_kernel.cuh:136-299 (reverse chunk loop, forward
// recompute from chunk-start states, reverse adjoint scan seeded by the final-state
// cotangent, du/ddelta/dA/dB/dC formulas) and its dormant fused branches :151-203,
// :442-485 (softplus, z gate, D, delta bias, initial-state gradient).
//
// Mapping: one wave per channel, lane = segment of kT steps, chunk = 64*kT = 512 steps
// (the granularity of the forward's `carries` residual, so no forward recompute across
// chunks is needed). A workgroup of kW waves walks K rounds of kW channels of one batch
// row ("channel block") and every chunk from last to first. Per chunk, per state n:
//   forward  local aggregate + 64-lane DPP scan from the stored chunk-start state, then a
//            re-run that keeps h_t and a_bar*h_{t-1} in registers
//   reverse  local aggregate of the adjoint + 64-lane reverse scan seeded by the carry from
//            the chunk to the right (or dlast), then a re-run producing lambda_t and all
//            per-step gradient terms
// dB/dC are sums over channels: each wave adds its per-(n, t) terms into an LDS
// accumulator shared by the workgroup (rows owned in rotation, plain read-add-write),
// flushed once per chunk to a per-channel-block partial; a second kernel sums the
// partials in a fixed order.
// This replaces the reference's one-global-atomic-per-(b,d,n,t) scheme
// (selective_scan_bwd_kernel.cuh:295-318).
#include <type_traits>

#include "mss_common.h"

namespace mss {

constexpr int kBwdT = 8;
constexpr int kBwdW = 12;
constexpr int kMaxChanPerBlock = 240;  // 20 rounds of 12 waves
constexpr int kCUs = 256;               // MI355X compute units

template <int kT, int kW, bool kZOH, bool kHasZ, typename io_t, typename bc_t>
__global__ __launch_bounds__(kW * 64) void bwd_kernel(BwdParams p) {
  constexpr int kChunk = 64 * kT;
  static_assert(kChunk == kCarryChunk, "backward chunk must match the carry residual");
  // dB/dC partial sums of the workgroup's channels for one chunk: [copy][n][j][which][lane]
  // (step j of lane `lane`'s segment): conflict-free for the 64 lanes of a wave, and every
  // access of a state is a constant offset from one per-lane base, so the read-add-writes
  // batch freely. At state iteration i wave w owns row n = (i + w) mod N of
  // copy w / N, so rows are updated with plain read-add-write in a fixed order
  // (LDS float atomics run ~40x slower than stores on gfx950 and are avoided).
  __shared__ float acc[2 * kMaxN * kChunk];
  __shared__ float s_mu[kMaxChanPerBlock][kMaxN];
  __shared__ float s_dA[kMaxChanPerBlock][kMaxN];
  __shared__ float s_dD[kMaxChanPerBlock];
  __shared__ float s_db[kMaxChanPerBlock];
  __shared__ float s_a[kW][kMaxN];
  __shared__ float s_h0[kW][kMaxN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.y;
  const int blk = blockIdx.x;
  const int L = p.seqlen;
  const int N = p.dstate;
  const int K = p.chan_per_block / kW;
  const int len = p.seq_lens ? min(max(p.seq_lens[b], 0), L) : L;
  const bool vec_io = p.vec_io != 0;
  const bool vec_bc = p.vec_bc != 0;
  const bc_t* __restrict__ Bb = static_cast<const bc_t*>(p.B) + b * p.bc_sb;
  const bc_t* __restrict__ Cb = static_cast<const bc_t*>(p.C) + b * p.bc_sb;

  const int n_copy = (kW + N - 1) / N;  // n_copy * N <= 2 * kMaxN for N <= kMaxN
  const int w_mod_n = w % N;
  float* const acc_w = acc + (w / N) * 2 * N * kChunk;
  for (int i = tid; i < 2 * kMaxN * kChunk; i += kW * 64) acc[i] = 0.f;
  for (int k = 0; k < K; ++k) {
    const int cl = k * kW + w;
    const int d = blk * p.chan_per_block + cl;
    if (lane < kMaxN) {
      float mu0 = 0.f;
      if (d < p.dim && lane < N && p.dlast) mu0 = p.dlast[(static_cast<size_t>(b) * p.dim + d) * N + lane];
      s_mu[cl][lane] = mu0;
      s_dA[cl][lane] = 0.f;
    }
    if (lane == 0) {
      s_dD[cl] = 0.f;
      s_db[cl] = 0.f;
    }
  }
  __syncthreads();

  const int n_chunks = (L + kChunk - 1) / kChunk;
  for (int c = n_chunks - 1; c >= 0; --c) {
    const int t0 = c * kChunk;
    const int tl = t0 + lane * kT;
    // A chunk wholly inside the row's length, with vector-aligned rows, runs a specialised
    // body without bounds checks or validity masks (every chunk but a ragged last one).
    const bool full = vec_io && vec_bc && (t0 + kChunk <= len);  // wave-uniform
    auto chunk_body = [&](auto full_tag) {
    constexpr bool kFull = decltype(full_tag)::value;
    const bool fast = kFull || (vec_io && (t0 + kChunk <= L));     // wave-uniform
    const bool fast_bc = kFull || (vec_bc && (t0 + kChunk <= L));  // wave-uniform
    for (int k = 0; k < K; ++k) {
      const int cl = k * kW + w;
      const int d_raw = blk * p.chan_per_block + cl;
      const bool active = d_raw < p.dim;
      const int d = active ? d_raw : p.dim - 1;
      const size_t chan = static_cast<size_t>(b) * p.dim + d;
      const long long row = b * p.io_sb + d * p.io_sd;
      io_t* __restrict__ du_row = static_cast<io_t*>(p.du) + row;
      io_t* __restrict__ dd_row = static_cast<io_t*>(p.ddelta) + row;

      if (!kFull && t0 >= len) {  // whole chunk past this row's length: zero gradients, carry passes
        if (!active) continue;
        float zero[kT];
#pragma unroll
        for (int j = 0; j < kT; ++j) zero[j] = 0.f;
        store_seg<kT>(du_row, tl, L, fast, zero);
        store_seg<kT>(dd_row, tl, L, fast, zero);
        if constexpr (kHasZ) store_seg<kT>(static_cast<io_t*>(p.dz) + row, tl, L, fast, zero);
        if (c == 0 && p.dinit && lane < N) {
          // len == 0: x0 flows through identity steps to the last state.
          p.dinit[chan * N + lane] = s_mu[cl][lane];
        }
        continue;
      }

      if (lane < N) {
        s_a[w][lane] = p.A[static_cast<size_t>(d) * N + lane];
        s_h0[w][lane] = c == 0 ? (p.x0 ? p.x0[chan * N + lane] : 0.f)
                               : p.carries[(chan * p.n_carry + (c - 1)) * N + lane];
      }
      const float Dv = p.D ? p.D[d] : 0.f;
      const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
      float dlt[kT], dlu[kT], uu[kT], g[kT], s1[kT], s2[kT];
      float ssum = 0.f;
      load_seg<kT>(static_cast<const io_t*>(p.delta) + row, tl, L, fast, dlt);
      load_seg<kT>(static_cast<const io_t*>(p.u) + row, tl, L, fast, uu);
      load_seg<kT>(static_cast<const io_t*>(p.dout) + row, tl, L, fast, g);
      if constexpr (kHasZ) {
        // Gate: g = dout * silu(z); dz = dout * y * sigmoid(z) * (1 + z * (1 - sigmoid(z)))
        // with y the pre-gate output kept by the forward.
        float zr[kT], yp[kT];
        load_seg<kT>(static_cast<const io_t*>(p.z) + row, tl, L, fast, zr);
        load_seg<kT>(static_cast<const io_t*>(p.y_pre) + row, tl, L, fast, yp);
#pragma unroll
        for (int j = 0; j < kT; ++j) {
          const bool valid = kFull || tl + j < len;
          const float go = valid ? g[j] : 0.f;
          const float sz = sigmoid(zr[j]);
          yp[j] = go * yp[j] * sz * __builtin_fmaf(zr[j], 1.f - sz, 1.f);
          g[j] = go * zr[j] * sz;
        }
        store_seg<kT>(static_cast<io_t*>(p.dz) + row, tl, L, fast, yp);
      }
#pragma unroll
      for (int j = 0; j < kT; ++j) {
        const bool valid = kFull || tl + j < len;
        const float x = dlt[j] + bias;
        float dv = p.delta_softplus ? softplus(x) : x;
        dv = valid ? dv : 0.f;
        const float uv = valid ? uu[j] : 0.f;
        dlt[j] = dv;
        uu[j] = uv;
        dlu[j] = dv * uv;
        if constexpr (!kHasZ) g[j] = valid ? g[j] : 0.f;
        s1[j] = 0.f;
        s2[j] = 0.f;
        ssum += dv;
      }

      // States in a per-wave rotated order (see the accumulator above); the barrier per
      // iteration keeps every wave inside the same iteration. B/C rows of the next state are
      // requested at the end of each iteration, into the registers of the current ones.
      float bv[kT], cv[kT];
      if (active) {
        load_seg<kT>(Bb + w_mod_n * p.bc_sn, tl, L, fast_bc, bv);
        load_seg<kT>(Cb + w_mod_n * p.bc_sn, tl, L, fast_bc, cv);
      }
      for (int i = 0; i < N; ++i) {
        int n = i + w_mod_n;
        n = n >= N ? n - N : n;
        __syncthreads();
        if (!active) continue;
        // This wave owns accumulator row n until the next barrier. Its dC half is fetched
        // now and updated by the forward re-run (where h_t is produced), its dB half is
        // fetched after that and updated by the reverse pass: half a row of registers live.
        float* accn = acc_w + n * 2 * kChunk + lane;
        float accC[kT];
#pragma unroll
        for (int j = 0; j < kT; ++j) accC[j] = accn[j * 128 + 64];
        const float An = s_a[w][n];
        const float a2 = An * kLog2e;
        float a[kT];
        // ---- forward: local aggregate, scan, re-run from the true carry-in
        float H = 0.f;
#pragma unroll
        for (int j = 0; j < kT; ++j) {
          a[j] = fast_exp2(dlt[j] * a2);
          const float bu = kZOH ? (expm1f(dlt[j] * An) * fast_rcp(An)) * bv[j] * uu[j] : dlu[j] * bv[j];
          H = __builtin_fmaf(a[j], H, bu);
        }
        const float pseg = fast_exp2(a2 * ssum);
        float P = pseg;
        wave_scan_affine_fwd(P, H);
        const float run = s_h0[w][n];
        const float hend = __builtin_fmaf(P, run, H);
        const float hin = dpp_mov<kWaveShr1, 0xF>(run, hend);  // state before the lane's first step
        float hh[kT];
        {
          float h = hin;
#pragma unroll
          for (int j = 0; j < kT; ++j) {
            const float bu = kZOH ? (expm1f(dlt[j] * An) * fast_rcp(An)) * bv[j] * uu[j] : dlu[j] * bv[j];
            h = __builtin_fmaf(a[j], h, bu);
            hh[j] = h;
            accC[j] = __builtin_fmaf(g[j], h, accC[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < kT; ++j) accn[j * 128 + 64] = accC[j];
        float accB[kT];
#pragma unroll
        for (int j = 0; j < kT; ++j) accB[j] = accn[j * 128];
        // ---- reverse: local aggregate of lambda, reverse scan, re-run with true lambda
        float lam = cv[kT - 1] * g[kT - 1];
#pragma unroll
        for (int j = kT - 2; j >= 0; --j) lam = __builtin_fmaf(a[j + 1], lam, cv[j] * g[j]);
        float ra = pseg, rb = a[0] * lam;
        wave_scan_affine_rev(ra, rb, lane);
        const float mu_in = s_mu[cl][n];
        const float mu_out = readlane(__builtin_fmaf(ra, mu_in, rb), 0);
        const float ra_s = dpp_mov<kWaveShl1, 0xF>(1.f, ra);
        const float rb_s = dpp_mov<kWaveShl1, 0xF>(0.f, rb);
        lam = __builtin_fmaf(ra_s, mu_in, rb_s) + cv[kT - 1] * g[kT - 1];
        float dA_acc = 0.f;
#pragma unroll
        for (int j = kT - 1; j >= 0; --j) {
          if (j < kT - 1) lam = __builtin_fmaf(a[j + 1], lam, cv[j] * g[j]);
          const float ah = a[j] * (j > 0 ? hh[j - 1] : hin);  // a_bar_t * h_{t-1}
          const float q = lam * ah;
          float dBv;
          if constexpr (kZOH) {
            const float e = expm1f(dlt[j] * An) * fast_rcp(An);
            const float lb = lam * bv[j];
            s1[j] = __builtin_fmaf(lb, e, s1[j]);
            s2[j] = __builtin_fmaf(An, q, __builtin_fmaf(lb * uu[j], a[j], s2[j]));
            const float dedA = (dlt[j] * a[j] - e) * fast_rcp(An);
            dA_acc = __builtin_fmaf(dlt[j], q, __builtin_fmaf(lb * uu[j], dedA, dA_acc));
            dBv = lam * e * uu[j];
          } else {
            s1[j] = __builtin_fmaf(lam, bv[j], s1[j]);
            s2[j] = __builtin_fmaf(An, q, s2[j]);
            dA_acc = __builtin_fmaf(dlt[j], q, dA_acc);
            dBv = lam * dlu[j];
          }
          accB[j] += dBv;
        }
#pragma unroll
        for (int j = 0; j < kT; ++j) accn[j * 128] = accB[j];
        {  // next state's rows (after the last state: an unused in-bounds reload)
          const int nn = n + 1 == N ? 0 : n + 1;
          load_seg<kT>(Bb + nn * p.bc_sn, tl, L, fast_bc, bv);
          load_seg<kT>(Cb + nn * p.bc_sn, tl, L, fast_bc, cv);
        }
        const float dA_sum = wave_sum(dA_acc);
        if (lane == 0) {
          s_mu[cl][n] = mu_out;
          s_dA[cl][n] += dA_sum;
          if (c == 0 && p.dinit) p.dinit[chan * N + n] = mu_out;
        }
      }

      if (!active) continue;
      if constexpr (!kZOH) {
        // Euler needs u only from here on: reload it rather than hold it across the loop.
        load_seg<kT>(static_cast<const io_t*>(p.u) + row, tl, L, fast, uu);
#pragma unroll
        for (int j = 0; j < kT; ++j) uu[j] = (kFull || tl + j < len) ? uu[j] : 0.f;
      }
      // ---- per-step gradients of the row
      float dD_acc = 0.f, db_acc = 0.f;
      float duv[kT], ddv[kT];
#pragma unroll
      for (int j = 0; j < kT; ++j) {
        const bool valid = kFull || tl + j < len;
        float du_j, dd_j;
        if constexpr (kZOH) {
          du_j = __builtin_fmaf(Dv, g[j], s1[j]);
          dd_j = s2[j];
        } else {
          du_j = __builtin_fmaf(dlt[j], s1[j], Dv * g[j]);
          dd_j = __builtin_fmaf(uu[j], s1[j], s2[j]);
        }
        if (p.delta_softplus) {
          // d softplus(x)/dx = sigmoid(x) = 1 - exp(-softplus(x)); identity above 20.
          dd_j = dlt[j] > 20.f ? dd_j : dd_j * one_minus_exp_neg(dlt[j]);
        }
        du_j = valid ? du_j : 0.f;
        dd_j = valid ? dd_j : 0.f;
        dD_acc = __builtin_fmaf(g[j], uu[j], dD_acc);
        db_acc += dd_j;
        duv[j] = du_j;
        ddv[j] = dd_j;
      }
      store_seg<kT>(du_row, tl, L, fast, duv);
      store_seg<kT>(dd_row, tl, L, fast, ddv);
      const float dD_sum = wave_sum(dD_acc);
      const float db_sum = wave_sum(db_acc);
      if (lane == 0) {
        s_dD[cl] += dD_sum;
        s_db[cl] += db_sum;
      }
    }

    };
    if (full) {
      chunk_body(std::true_type{});
    } else {
      chunk_body(std::false_type{});
    }

    // ---- flush this chunk's dB/dC sums over the block's channels
    __syncthreads();
    const size_t nl = static_cast<size_t>(N) * L;
    float* part = p.part_dBC + static_cast<size_t>(blk) * p.part_stride + static_cast<size_t>(b) * 2 * nl;
    for (int row_i = 0; row_i < 2 * N; ++row_i) {  // (which, n) rows of the accumulator
      const int which = row_i >= N;
      const int n = row_i - which * N;
      float* dst = part + which * nl + static_cast<size_t>(n) * L + t0;
      // Thread -> (segment ln, quarter q): steps 4q..4q+3 of segment ln, summed over copies.
      for (int pos = tid; pos < 64 * (kT / 4); pos += kW * 64) {
        const int ln = pos & 63, q = pos >> 6;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int off = n * 2 * kChunk + (4 * q + e) * 128 + which * 64 + ln;
          float sum = 0.f;
          for (int cp = 0; cp < n_copy; ++cp) {
            sum += acc[cp * 2 * N * kChunk + off];
            acc[cp * 2 * N * kChunk + off] = 0.f;
          }
          v[e] = sum;
        }
        const int toff = ln * kT + 4 * q;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t0 + toff + e < L) dst[toff + e] = v[e];
      }
    }
    __syncthreads();
  }

  // ---- per-channel partial sums (over this row's steps)
  for (int k = 0; k < K; ++k) {
    const int cl = k * kW + w;
    const int d = blk * p.chan_per_block + cl;
    if (d >= p.dim) continue;
    const size_t chan = static_cast<size_t>(b) * p.dim + d;
    if (lane < N) p.part_dA[chan * N + lane] = s_dA[cl][lane];
    if (lane == 0) {
      p.part_dD[chan] = s_dD[cl];
      p.part_dbias[chan] = s_db[cl];
    }
  }
}

// dB/dC[b][n][t] = sum over channel blocks of the partials, fixed order. Partials are
// [block][b][B|C][n][t] (block stride `stride` floats). grid.y = partial row
// (b, which, n); threads walk the row's steps, 4 at a time (16-byte loads) when kVec
// (L a multiple of 4), keeping 4 blocks' loads in flight.
template <bool kVec, typename bc_t>
__global__ __launch_bounds__(256) void reduce_bc_kernel(const float* __restrict__ part, int n_blk,
                                                        size_t stride, int L, int N,
                                                        long long sb, long long sn,
                                                        bc_t* __restrict__ dB, bc_t* __restrict__ dC) {
  const int r = blockIdx.y;
  const int bb = r / (2 * N);
  const int rem = r - bb * 2 * N;
  const int which = rem >= N;
  const int n = rem - which * N;
  const float* src_row = part + static_cast<size_t>(r) * L;
  bc_t* dst = (which ? dC : dB) + bb * sb + n * sn;
  constexpr int kE = kVec ? 4 : 1;
  const int nvec = (L + kE - 1) / kE;
  for (int v = blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += gridDim.x * blockDim.x) {
    if constexpr (kVec) {
      const f32x4* src = reinterpret_cast<const f32x4*>(src_row) + v;
      const size_t svec = stride / 4;
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
      int k = 0;
      for (; k + 4 <= n_blk; k += 4) {
        const f32x4 a0 = src[static_cast<size_t>(k + 0) * svec];
        const f32x4 a1 = src[static_cast<size_t>(k + 1) * svec];
        const f32x4 a2 = src[static_cast<size_t>(k + 2) * svec];
        const f32x4 a3 = src[static_cast<size_t>(k + 3) * svec];
        s += a0;
        s += a1;
        s += a2;
        s += a3;
      }
      for (; k < n_blk; ++k) s += src[static_cast<size_t>(k) * svec];
      store_as(dst + 4 * v + 0, s.x);
      store_as(dst + 4 * v + 1, s.y);
      store_as(dst + 4 * v + 2, s.z);
      store_as(dst + 4 * v + 3, s.w);
    } else {
      float s = 0.f;
      for (int k = 0; k < n_blk; ++k) s += src_row[static_cast<size_t>(k) * stride + v];
      store_as(dst + v, s);
    }
  }
}

// dA[d][n] = sum_b part_dA[b][d][n]; dD[d], dbias[d] likewise (fixed order).
__global__ __launch_bounds__(256) void reduce_small_kernel(const float* __restrict__ part_dA,
                                                           const float* __restrict__ part_dD,
                                                           const float* __restrict__ part_db,
                                                           int batch, int dim, int dstate,
                                                           float* dA, float* dD, float* dbias) {
  const int dn = dim * dstate;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dn + 2 * dim;
       i += gridDim.x * blockDim.x) {
    if (i < dn) {
      float s = 0.f;
      for (int bb = 0; bb < batch; ++bb) s += part_dA[static_cast<size_t>(bb) * dn + i];
      dA[i] = s;
    } else {
      const int which = (i - dn) / dim;
      const int dd = (i - dn) - which * dim;
      const float* src = which == 0 ? part_dD : part_db;
      float* dst = which == 0 ? dD : dbias;
      if (dst == nullptr) continue;
      float s = 0.f;
      for (int bb = 0; bb < batch; ++bb) s += src[static_cast<size_t>(bb) * dim + dd];
      dst[dd] = s;
    }
  }
}

template <bool kZOH, bool kHasZ, typename io_t, typename bc_t>
static hipError_t launch_bwd_t(const BwdParams& p, hipStream_t stream) {
  dim3 grid(p.n_blocks_d, p.batch);
  hipLaunchKernelGGL((bwd_kernel<kBwdT, kBwdW, kZOH, kHasZ, io_t, bc_t>), grid, dim3(kBwdW * 64), 0,
                     stream, p);
  return hipGetLastError();
}

template <typename io_t, typename bc_t>
static hipError_t launch_bwd_io(const BwdParams& p, int zoh, hipStream_t stream) {
  const bool hz = p.z != nullptr;
  if (zoh) return hz ? launch_bwd_t<true, true, io_t, bc_t>(p, stream)
                     : launch_bwd_t<true, false, io_t, bc_t>(p, stream);
  return hz ? launch_bwd_t<false, true, io_t, bc_t>(p, stream)
            : launch_bwd_t<false, false, io_t, bc_t>(p, stream);
}

int bwd_chan_per_block(int batch, int dim, int varlen) {
  // One workgroup per CU holds the dB/dC accumulator (LDS), so the grid should fit one
  // pass over the 256 CUs: the fewest channel rounds K with batch * ceil(dim / (kW*K))
  // <= 256 (more rounds also mean fewer dB/dC partials to reduce). With variable lengths
  // rows finish at different times, so workgroups stay ~4x smaller and the hardware
  // balances them. Bounded by the LDS bookkeeping size; depends on shapes only.
  const long long per_row = (dim + kBwdW - 1) / kBwdW;  // rounds needed for a whole row
  const long long target = varlen ? 4 * kCUs : kCUs;
  long long k = (static_cast<long long>(batch) * per_row + target - 1) / target;
  if (k < 1) k = 1;
  while (k < per_row && static_cast<long long>(batch) * ((per_row + k - 1) / k) > target) ++k;
  if (k > kMaxChanPerBlock / kBwdW) k = kMaxChanPerBlock / kBwdW;
  if (k > per_row) k = per_row;
  return static_cast<int>(k) * kBwdW;
}

hipError_t launch_bwd_scan(const BwdParams& p, int zoh, int io_bf16, int bc_bf16,
                           hipStream_t stream) {
  if (io_bf16) return bc_bf16 ? launch_bwd_io<bf16_t, bf16_t>(p, zoh, stream)
                              : launch_bwd_io<bf16_t, float>(p, zoh, stream);
  return bc_bf16 ? launch_bwd_io<float, bf16_t>(p, zoh, stream)
                 : launch_bwd_io<float, float>(p, zoh, stream);
}

hipError_t launch_bwd_reduce(const BwdParams& p, int bc_bf16, void* dA, void* dB, void* dC,
                             float* dD, float* dbias, hipStream_t stream) {
  const int L = p.seqlen;
  const bool vec = (L % 4) == 0;  // partial rows are 16-byte aligned (block stride: 64 floats)
  const int nvec = vec ? L / 4 : L;
  const dim3 grid((nvec + 255) / 256, p.batch * 2 * p.dstate);
#define MSS_REDUCE_BC(VEC, T)                                                                 \
  hipLaunchKernelGGL((reduce_bc_kernel<VEC, T>), grid, dim3(256), 0, stream, p.part_dBC,       \
                     p.n_blocks_d, p.part_stride, L, p.dstate, p.bc_sb, p.bc_sn,              \
                     static_cast<T*>(dB), static_cast<T*>(dC))
  if (bc_bf16) {
    if (vec) MSS_REDUCE_BC(true, bf16_t); else MSS_REDUCE_BC(false, bf16_t);
  } else {
    if (vec) MSS_REDUCE_BC(true, float); else MSS_REDUCE_BC(false, float);
  }
#undef MSS_REDUCE_BC
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int small = p.dim * p.dstate + 2 * p.dim;
  hipLaunchKernelGGL(reduce_small_kernel, dim3((small + 255) / 256), dim3(256), 0, stream, p.part_dA,
                     p.part_dD, p.part_dbias, p.batch, p.dim, p.dstate, static_cast<float*>(dA), dD,
                     dbias);
  return hipGetLastError();
}

}  // namespace mss
