// Complex-SSM selective scan (forward and backward) for gfx950 (MI355X).
//
// Reference behaviour followed: the complex-state branch of S6 (mamba/mamba1.py:143-176):
// A = -exp(A_log.real) + i*A_imag (the caller applies that parameterisation),
// a_bar = exp(delta*A), Euler b_bar = delta*B (real) or ZOH b_bar = expm1(delta*A)/A*B
// (complex), an affine associative scan over complex states from a zero state, then
// y = sum_n C*Re(h) + D*u (``ys.real``, :175-198). The same fusions as the real scan run
// inside the kernels: softplus(delta + bias), the padding mask, the silu(z) gate, an
// optional initial state (zero reproduces the reference) and the last state. The reference
// runs this branch as an XLA associative scan and differentiates it with autodiff; the
// backward here is a hand-written adjoint that treats each complex state as a real
// 2-vector, so the transpose of multiplication by a_bar is multiplication by conj(a_bar).
//
// Mapping, as the real kernels: one wave per (batch, channel), a lane owns one 8-step
// segment, a wave pass covers a 512-step chunk, and segments are joined by a 64-lane
// inclusive scan of complex affine maps on DPP lane shifts. exp(delta*A) is
// exp2(delta*Re(A)*log2(e)) * (cos, sin)(delta*Im(A)), the angle taken in turns
// (delta*Im(A)/2pi) for the hardware sine and cosine.
#include "mss_common.h"

namespace mss {

constexpr int kCT = kSegSteps;     // steps per lane: one carry segment
constexpr int kCChunk = 64 * kCT;  // steps per wave pass
static_assert(kCChunk == kPartChunk, "the reduction's chunk is the scan's");
constexpr int kCFwdW = 4;          // waves (channels) per forward workgroup
constexpr int kCBwdW = 12;         // waves per backward workgroup (3 per SIMD, one per CU)
constexpr int kCMaxChan = 48;      // channels one backward workgroup walks, at most
// dB/dC accumulator rows of the backward: ceil(kCBwdW/N) copies of each state's row, so
// waves never share a row within one state iteration; the most over N <= 16 is 22 (N = 11).
constexpr int kCAccRows = 22;
constexpr float kInv2Pi = 0.15915494309189535f;

// Constants of exp(t * A) for one (channel, state).
struct CoefA {
  float ar2;    // Re(A) * log2(e)
  float airev;  // Im(A) / (2 pi)
  float ar, ai; // A
  float inv_a2; // 1 / |A|^2 (ZOH)
};

__device__ __forceinline__ CoefA load_coef(const float* __restrict__ A, size_t idx) {
  CoefA c;
  c.ar = A[2 * idx];
  c.ai = A[2 * idx + 1];
  c.ar2 = c.ar * kLog2e;
  c.airev = c.ai * kInv2Pi;
  c.inv_a2 = 1.f / __builtin_fmaf(c.ar, c.ar, c.ai * c.ai);
  return c;
}

// exp(t * A) = m * (cy + i sy), m = exp(t Re A).
struct CExp {
  float m, cy, sy;
};

// The angle t Im(A) in turns, reduced to [0, 1) by fract (exact), feeds the hardware
// sine and cosine (which take turns): measured on MI355X against float64 over [-8, 8]
// turns, their absolute error is at most 1.2e-7 (about one ulp of 1).
__device__ __forceinline__ CExp cexp_t(float t, const CoefA& c) {
  CExp e;
  e.m = fast_exp2(t * c.ar2);
  const float rev = __builtin_amdgcn_fractf(t * c.airev);
  e.cy = __builtin_amdgcn_cosf(rev);
  e.sy = __builtin_amdgcn_sinf(rev);
  return e;
}

// E = expm1(t A) / A (the ZOH b_bar without B) from exp(t A)'s parts. Re expm1(tA) =
// expm1(t Re A) cos y + (cos y - 1) with both terms <= 0 for t >= 0 (no cancellation
// between them), and cos y - 1 = -sin^2 y / (1 + cos y) where cos y > 0 (no cancellation
// near y = 0); Im expm1(tA) = exp(t Re A) sin y.
__device__ __forceinline__ void zoh_e(float t, const CoefA& c, const CExp& x, float& er, float& ei) {
  const float em1 = expm1f(t * c.ar);
  const float cm1 = x.cy > 0.f ? -x.sy * x.sy * fast_rcp(1.f + x.cy) : x.cy - 1.f;
  const float xr = __builtin_fmaf(em1, x.cy, cm1);
  const float xi = x.m * x.sy;
  er = __builtin_fmaf(xr, c.ar, xi * c.ai) * c.inv_a2;
  ei = __builtin_fmaf(xi, c.ar, -xr * c.ai) * c.inv_a2;
}

// One step of the 64-lane inclusive scan of complex affine maps x -> P x + H: the lane
// combines the map of the lane kCtrl selects (earlier in lane order, identity where there
// is none) with its own: (Pl, Hl) then (P, H) gives (Pl P, P Hl + H).
template <int kCtrl, int kRowMask>
__device__ __forceinline__ void caffine_step(float& pr, float& pi, float& hr, float& hi) {
  const float lpr = dpp_mov<kCtrl, kRowMask>(1.f, pr);
  const float lpi = dpp_mov<kCtrl, kRowMask>(0.f, pi);
  const float lhr = dpp_mov<kCtrl, kRowMask>(0.f, hr);
  const float lhi = dpp_mov<kCtrl, kRowMask>(0.f, hi);
  const float nhr = __builtin_fmaf(pr, lhr, __builtin_fmaf(-pi, lhi, hr));
  const float nhi = __builtin_fmaf(pr, lhi, __builtin_fmaf(pi, lhr, hi));
  const float npr = __builtin_fmaf(pr, lpr, -pi * lpi);
  const float npi = __builtin_fmaf(pr, lpi, pi * lpr);
  hr = nhr;
  hi = nhi;
  pr = npr;
  pi = npi;
}

__device__ __forceinline__ void wave_scan_caffine(float& pr, float& pi, float& hr, float& hi) {
  caffine_step<kRowShr1, 0xF>(pr, pi, hr, hi);
  caffine_step<kRowShr2, 0xF>(pr, pi, hr, hi);
  caffine_step<kRowShr4, 0xF>(pr, pi, hr, hi);
  caffine_step<kRowShr8, 0xF>(pr, pi, hr, hi);
  caffine_step<kRowBcast15, 0xA>(pr, pi, hr, hi);
  caffine_step<kRowBcast31, 0xC>(pr, pi, hr, hi);
}

// ---------------------------------------------------------------------------------
// Forward. Workgroup = kCFwdW channels of one batch row; no LDS, no block barriers. The
// running state of state n (entering the current chunk) is kept by lane n as (run_r, run_i).
template <bool kZOH, typename io_t, typename bc_t>
__global__ __launch_bounds__(kCFwdW * 64) void cfwd_kernel(FwdParams p) {
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = row_longest_first(p.seq_lens, p.batch, p.seqlen, blockIdx.y);
  const int d = blockIdx.x * kCFwdW + w;
  if (d >= p.dim) return;  // wave-uniform; the kernel has no block-level barrier
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
  const float Dv = p.D ? p.D[d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;

  float run_r = 0.f, run_i = 0.f;
  if (p.x0 && lane < N) {
    run_r = p.x0[(chan * N + lane) * 2];
    run_i = p.x0[(chan * N + lane) * 2 + 1];
  }
  const int n_chunks = (L + kCChunk - 1) / kCChunk;
  const int n_live = (len + kCChunk - 1) / kCChunk;
  for (int c = 0; c < n_chunks; ++c) {
    const int t0 = c * kCChunk;
    const int tl = t0 + lane * kCT;
    const bool fast = p.vec_io && t0 + kCChunk <= L;
    const bool fast_bc = p.vec_bc && t0 + kCChunk <= L;
    float y[kCT];
    if (c >= n_live) {
      // The whole chunk is past this row's length: the state is frozen, the output zero
      // (the backward reads no residual here, so y_pre is left unwritten).
#pragma unroll
      for (int j = 0; j < kCT; ++j) y[j] = 0.f;
      store_seg<kCT>(out_row, tl, L, fast, y);
      continue;
    }
    float dlt[kCT], uu[kCT];
    float ssum = 0.f;
    load_seg<kCT>(dl_row, tl, L, fast, dlt);
    load_seg<kCT>(u_row, tl, L, fast, uu);
#pragma unroll
    for (int j = 0; j < kCT; ++j) {
      const bool valid = tl + j < len;
      const float x = dlt[j] + bias;
      const float dv = p.delta_softplus ? softplus(x) : x;
      dlt[j] = valid ? dv : 0.f;
      uu[j] = valid ? uu[j] : 0.f;
      y[j] = Dv * uu[j];
      ssum += dlt[j];
    }
    // B and C rows of the next state are loaded one state ahead.
    float bnx[kCT], cnx[kCT];
    load_seg<kCT>(Bb, tl, L, fast_bc, bnx);
    load_seg<kCT>(Cb, tl, L, fast_bc, cnx);
    for (int n = 0; n < N; ++n) {
      const CoefA cf = load_coef(p.A, static_cast<size_t>(d) * N + n);
      float ar[kCT], ai[kCT], br[kCT], bi[kCT];
      float bv[kCT], cv[kCT];
#pragma unroll
      for (int j = 0; j < kCT; ++j) {
        bv[j] = bnx[j];
        cv[j] = cnx[j];
      }
      if (n + 1 < N) {
        load_seg<kCT>(Bb + (n + 1) * p.bc_sn, tl, L, fast_bc, bnx);
        load_seg<kCT>(Cb + (n + 1) * p.bc_sn, tl, L, fast_bc, cnx);
      }
      float hr = 0.f, hi = 0.f;
      {
#pragma unroll
        for (int j = 0; j < kCT; ++j) {
          const CExp e = cexp_t(dlt[j], cf);
          const bool valid = tl + j < len;
          ar[j] = valid ? e.m * e.cy : 1.f;
          ai[j] = valid ? e.m * e.sy : 0.f;
          if constexpr (kZOH) {
            float er, ei;
            zoh_e(dlt[j], cf, e, er, ei);
            const float s = bv[j] * uu[j];
            br[j] = er * s;
            bi[j] = ei * s;
          } else {
            br[j] = dlt[j] * uu[j] * bv[j];
            bi[j] = 0.f;
          }
          const float nr = __builtin_fmaf(ar[j], hr, __builtin_fmaf(-ai[j], hi, br[j]));
          const float ni = __builtin_fmaf(ar[j], hi, __builtin_fmaf(ai[j], hr, bi[j]));
          hr = nr;
          hi = ni;
        }
      }
      // Segment map h -> P h + H, P = exp(A * sum delta); scanned over the lanes.
      const CExp pe = cexp_t(ssum, cf);
      float pr = pe.m * pe.cy, pim = pe.m * pe.sy;
      wave_scan_caffine(pr, pim, hr, hi);
      const float rr = readlane(run_r, n), ri = readlane(run_i, n);
      // State at the lane's last step, then the previous lane's as this lane's carry-in.
      const float er = __builtin_fmaf(pr, rr, __builtin_fmaf(-pim, ri, hr));
      const float ei = __builtin_fmaf(pr, ri, __builtin_fmaf(pim, rr, hi));
      float xr = dpp_mov<kWaveShr1, 0xF>(rr, er);
      float xi = dpp_mov<kWaveShr1, 0xF>(ri, ei);
      if (lane == 0) {
        xr = rr;
        xi = ri;
      }
      if (p.carries && tl < L) {
        float2* cp = reinterpret_cast<float2*>(p.carries) + (chan * N + n) * p.n_seg + tl / kCT;
        *cp = make_float2(xr, xi);
      }
      {
#pragma unroll
        for (int j = 0; j < kCT; ++j) {
          const float nr = __builtin_fmaf(ar[j], xr, __builtin_fmaf(-ai[j], xi, br[j]));
          const float ni = __builtin_fmaf(ar[j], xi, __builtin_fmaf(ai[j], xr, bi[j]));
          xr = nr;
          xi = ni;
          y[j] = __builtin_fmaf(cv[j], xr, y[j]);
        }
      }
      const float nr = readlane(er, 63), ni = readlane(ei, 63);
      run_r = lane == n ? nr : run_r;
      run_i = lane == n ? ni : run_i;
    }
    if (p.z) {
      if (p.y_pre) {
        float yp[kCT];
#pragma unroll
        for (int j = 0; j < kCT; ++j) yp[j] = (tl + j < len) ? y[j] : 0.f;
        store_seg<kCT>(static_cast<io_t*>(p.y_pre) + row, tl, L, fast, yp);
      }
      float zv[kCT];
      load_seg<kCT>(static_cast<const io_t*>(p.z) + row, tl, L, fast, zv);
#pragma unroll
      for (int j = 0; j < kCT; ++j) y[j] *= zv[j] * sigmoid(zv[j]);
    }
#pragma unroll
    for (int j = 0; j < kCT; ++j) y[j] = (tl + j < len) ? y[j] : 0.f;
    store_seg<kCT>(out_row, tl, L, fast, y);
  }
  if (p.last && lane < N) {
    p.last[(chan * N + lane) * 2] = run_r;
    p.last[(chan * N + lane) * 2 + 1] = run_i;
  }
}

// ---------------------------------------------------------------------------------
// Backward. Workgroup = kCBwdW waves walking p.chan_per_block channels of one batch row in
// rounds of kCBwdW, chunks from last to first. Within a chunk a lane owns segment
// 63 - lane, so the adjoint (which runs backwards in time) is an inclusive scan in lane
// order. Per state: re-run the forward inside the segment from the stored segment-entry
// state (carries), aggregate the segment's adjoint map from a zero seed, scan the maps
// across the lanes, then re-run the adjoint from the true seed and form the gradients.
// dB/dC of the chunk accumulate in LDS rows: at state iteration i wave w handles state
// (i + w) mod N in copy w / N of that state's row, so no two waves share a row at once and
// the sum order is fixed; a wave adds into its row once the row's previous owner has
// counted that iteration done in LDS (no workgroup barrier per iteration). After every
// chunk the rows (copies summed in order) go to this workgroup's partial rows; a second
// kernel sums the partials over workgroups in a fixed order.
template <bool kZOH, bool kHasZ, typename io_t, typename bc_t>
__global__ __launch_bounds__(kCBwdW * 64) void cbwd_kernel(BwdParams p) {
  constexpr int W = kCBwdW;
  __shared__ __attribute__((aligned(16))) float s_acc[kCAccRows][2][kCChunk];
  __shared__ float s_mu[kCMaxChan][kMaxN][2];  // adjoint entering the chunk from the right
  __shared__ float s_dA[kCMaxChan][kMaxN][2];
  __shared__ float s_dD[kCMaxChan];
  __shared__ float s_db[kCMaxChan];
  __shared__ int s_done[W];  // state iterations of the current chunk each wave has finished

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = row_longest_first(p.seq_lens, p.batch, p.seqlen, blockIdx.y);
  const int L = p.seqlen;
  const int N = p.dstate;
  const int len = p.seq_lens ? min(max(p.seq_lens[b], 0), L) : L;
  const int cpb = p.chan_per_block;
  const int d0 = blockIdx.x * cpb;
  const int rounds = cpb / W;
  const int copies = (W + N - 1) / N;
  const int seg = 63 - lane;
  const bc_t* __restrict__ Bb = static_cast<const bc_t*>(p.B) + b * p.bc_sb;
  const bc_t* __restrict__ Cb = static_cast<const bc_t*>(p.C) + b * p.bc_sb;

  for (int i = tid; i < cpb * N; i += W * 64) {
    const int k = i / N, n = i - k * N;
    const int d = d0 + k;
    float mr = 0.f, mi = 0.f;
    if (p.dlast && d < p.dim) {
      const size_t o = ((static_cast<size_t>(b) * p.dim + d) * N + n) * 2;
      mr = p.dlast[o];
      mi = p.dlast[o + 1];
    }
    s_mu[k][n][0] = mr;
    s_mu[k][n][1] = mi;
    s_dA[k][n][0] = 0.f;
    s_dA[k][n][1] = 0.f;
  }
  for (int i = tid; i < cpb; i += W * 64) s_dD[i] = s_db[i] = 0.f;
  for (int i = tid; i < copies * N * 2 * kCChunk; i += W * 64) (&s_acc[0][0][0])[i] = 0.f;
  if (tid < W) s_done[tid] = 0;
  // The previous owner of this wave's row at chunk iteration g: the copy's next wave at
  // g - 1, or, for the copy's last wave, the copy's first wave at g - (N - w % N); every
  // wait is on an earlier iteration, so all waits resolve.
  const int wmod = w % N;
  const int copy_waves = min(N, W - (w / N) * N);
  const int pred = wmod + 1 < copy_waves ? w + 1 : w - wmod;
  const int pred_lag = wmod + 1 < copy_waves ? 1 : N - wmod;
  __syncthreads();

  const int n_chunks = (L + kCChunk - 1) / kCChunk;
  const int n_live = (len + kCChunk - 1) / kCChunk;
  for (int c = n_chunks - 1; c >= 0; --c) {
    const int t0 = c * kCChunk;
    const int ts = t0 + seg * kCT;
    const bool fast = p.vec_io && t0 + kCChunk <= L;
    const bool fast_bc = p.vec_bc && t0 + kCChunk <= L;
    const bool live = c < n_live;  // workgroup-uniform
    for (int r = 0; r < rounds; ++r) {
      const int k = r * W + w;
      const int d = d0 + k;
      const bool active = d < p.dim;
      const int dd = active ? d : p.dim - 1;
      const size_t chan = static_cast<size_t>(b) * p.dim + dd;
      const long long row = b * p.io_sb + dd * p.io_sd;
      io_t* du_row = static_cast<io_t*>(p.du) + row;
      io_t* ddl_row = static_cast<io_t*>(p.ddelta) + row;
      if (!live) {
        // Past the row's length: zero gradients; the adjoint passes through unchanged.
        if (active) {
          float zero[kCT];
#pragma unroll
          for (int j = 0; j < kCT; ++j) zero[j] = 0.f;
          store_seg<kCT>(du_row, ts, L, fast, zero);
          store_seg<kCT>(ddl_row, ts, L, fast, zero);
          if constexpr (kHasZ) store_seg<kCT>(static_cast<io_t*>(p.dz) + row, ts, L, fast, zero);
        }
        continue;
      }
      const float Dv = p.D ? p.D[dd] : 0.f;
      const float bias = p.delta_bias ? p.delta_bias[dd] : 0.f;
      float xraw[kCT], dlt[kCT], uu[kCT], g[kCT];
      load_seg<kCT>(static_cast<const io_t*>(p.delta) + row, ts, L, fast, xraw);
      load_seg<kCT>(static_cast<const io_t*>(p.u) + row, ts, L, fast, uu);
      load_seg<kCT>(static_cast<const io_t*>(p.dout) + row, ts, L, fast, g);
      float ssum = 0.f;
#pragma unroll
      for (int j = 0; j < kCT; ++j) {
        const bool valid = ts + j < len;
        xraw[j] += bias;
        const float dv = p.delta_softplus ? softplus(xraw[j]) : xraw[j];
        dlt[j] = valid ? dv : 0.f;
        uu[j] = valid ? uu[j] : 0.f;
        g[j] = valid ? g[j] : 0.f;
        ssum += dlt[j];
      }
      if constexpr (kHasZ) {
        float zv[kCT], yp[kCT], dz[kCT];
        load_seg<kCT>(static_cast<const io_t*>(p.z) + row, ts, L, fast, zv);
        load_seg<kCT>(static_cast<const io_t*>(p.y_pre) + row, ts, L, fast, yp);
#pragma unroll
        for (int j = 0; j < kCT; ++j) {
          const float sz = sigmoid(zv[j]);
          dz[j] = g[j] * yp[j] * sz * __builtin_fmaf(zv[j], 1.f - sz, 1.f);
          g[j] = g[j] * zv[j] * sz;
        }
        if (active) store_seg<kCT>(static_cast<io_t*>(p.dz) + row, ts, L, fast, dz);
      }
      float du[kCT], ddl[kCT];
#pragma unroll
      for (int j = 0; j < kCT; ++j) {
        du[j] = Dv * g[j];
        ddl[j] = 0.f;
      }

      // B, C rows and the segment-entry state of the next state are loaded one state
      // ahead, so their latency overlaps a state's arithmetic (Euler; ZOH keeps E_t per
      // step in registers and has no room for them, so it loads each state's rows in place).
      constexpr bool kAhead = !kZOH;
      const float2* __restrict__ carry_seg = reinterpret_cast<const float2*>(p.carries) +
                                             chan * N * p.n_seg + ts / kCT;
      float bnx[kCT], cnx[kCT];
      float2 hnx = make_float2(0.f, 0.f);
      if (kAhead && active) {
        const int n0 = w % N;
        load_seg<kCT>(Bb + n0 * p.bc_sn, ts, L, fast_bc, bnx);
        load_seg<kCT>(Cb + n0 * p.bc_sn, ts, L, fast_bc, cnx);
        if (ts < L) hnx = carry_seg[static_cast<size_t>(n0) * p.n_seg];
      }
      for (int it = 0; it < N; ++it) {
        const int n = (it + w) % N;
        const int arow = (w / N) * N + n;
        if (active) {
          const CoefA cf = load_coef(p.A, static_cast<size_t>(dd) * N + n);
          float bv[kCT], cv[kCT];
          float hinr, hini;
          if constexpr (kAhead) {
#pragma unroll
            for (int j = 0; j < kCT; ++j) {
              bv[j] = bnx[j];
              cv[j] = cnx[j];
            }
            hinr = hnx.x;
            hini = hnx.y;
            if (it + 1 < N) {
              const int nn = (it + 1 + w) % N;
              load_seg<kCT>(Bb + nn * p.bc_sn, ts, L, fast_bc, bnx);
              load_seg<kCT>(Cb + nn * p.bc_sn, ts, L, fast_bc, cnx);
              if (ts < L) hnx = carry_seg[static_cast<size_t>(nn) * p.n_seg];
            }
          } else {
            load_seg<kCT>(Bb + n * p.bc_sn, ts, L, fast_bc, bv);
            load_seg<kCT>(Cb + n * p.bc_sn, ts, L, fast_bc, cv);
            const float2 h0 = ts < L ? carry_seg[static_cast<size_t>(n) * p.n_seg] : make_float2(0.f, 0.f);
            hinr = h0.x;
            hini = h0.y;
          }
          // Forward re-run: a_j, the state before each step, (ZOH) E_j.
          float ar[kCT], ai[kCT], hpr[kCT], hpi[kCT], er[kCT], ei[kCT];
#pragma unroll
          for (int j = 0; j < kCT; ++j) {
            const CExp e = cexp_t(dlt[j], cf);
            const bool valid = ts + j < len;
            ar[j] = valid ? e.m * e.cy : 1.f;
            ai[j] = valid ? e.m * e.sy : 0.f;
            float brj, bij;
            if constexpr (kZOH) {
              zoh_e(dlt[j], cf, e, er[j], ei[j]);
              const float s = bv[j] * uu[j];
              brj = er[j] * s;
              bij = ei[j] * s;
            } else {
              er[j] = ei[j] = 0.f;
              brj = dlt[j] * uu[j] * bv[j];
              bij = 0.f;
            }
            hpr[j] = hinr;
            hpi[j] = hini;
            const float nr = __builtin_fmaf(ar[j], hinr, __builtin_fmaf(-ai[j], hini, brj));
            const float ni = __builtin_fmaf(ar[j], hini, __builtin_fmaf(ai[j], hinr, bij));
            hinr = nr;
            hini = ni;
          }
          // Segment adjoint map m -> Pc m + Hc (m entering at the segment end): Pc = conj of
          // the segment's product of a_bar, Hc from a zero seed.
          float hcr = 0.f, hci = 0.f;
#pragma unroll
          for (int j = kCT - 1; j >= 0; --j) {
            const float lr = __builtin_fmaf(cv[j], g[j], hcr);
            const float li = hci;
            hcr = __builtin_fmaf(ar[j], lr, ai[j] * li);
            hci = __builtin_fmaf(ar[j], li, -ai[j] * lr);
          }
          const CExp pe = cexp_t(ssum, cf);
          float pcr = pe.m * pe.cy, pci = -pe.m * pe.sy;
          wave_scan_caffine(pcr, pci, hcr, hci);
          const float mur = s_mu[k][n][0], mui = s_mu[k][n][1];
          const float oar = __builtin_fmaf(pcr, mur, __builtin_fmaf(-pci, mui, hcr));
          const float oai = __builtin_fmaf(pcr, mui, __builtin_fmaf(pci, mur, hci));
          float mr = dpp_mov<kWaveShr1, 0xF>(mur, oar);
          float mi = dpp_mov<kWaveShr1, 0xF>(mui, oai);
          if (lane == 0) {
            mr = mur;
            mi = mui;
          }
          // Lane 63 holds segment 0: its outgoing adjoint enters the previous chunk.
          if (lane == 63) {
            s_mu[k][n][0] = oar;
            s_mu[k][n][1] = oai;
          }
          float dar = 0.f, dai = 0.f;
          float accB[kCT], accC[kCT];
#pragma unroll
          for (int j = kCT - 1; j >= 0; --j) {
            const float lr = __builtin_fmaf(cv[j], g[j], mr);
            const float li = mi;
            // W = lambda * conj(a_bar h_prev): dA += delta W, ddelta += Re(W conj(A))
            const float ahr = __builtin_fmaf(ar[j], hpr[j], -ai[j] * hpi[j]);
            const float ahi = __builtin_fmaf(ar[j], hpi[j], ai[j] * hpr[j]);
            const float wr = __builtin_fmaf(lr, ahr, li * ahi);
            const float wi = __builtin_fmaf(li, ahr, -lr * ahi);
            dar = __builtin_fmaf(dlt[j], wr, dar);
            dai = __builtin_fmaf(dlt[j], wi, dai);
            ddl[j] = __builtin_fmaf(wr, cf.ar, __builtin_fmaf(wi, cf.ai, ddl[j]));
            // m = conj(a_bar) lambda: the adjoint leaving the step towards the past.
            const float nmr = __builtin_fmaf(ar[j], lr, ai[j] * li);
            const float nmi = __builtin_fmaf(ar[j], li, -ai[j] * lr);
            if constexpr (kZOH) {
              const float s = bv[j] * uu[j];
              const float ge = __builtin_fmaf(er[j], lr, ei[j] * li);  // Re(conj(E) lambda)
              du[j] = __builtin_fmaf(bv[j], ge, du[j]);
              accB[j] = uu[j] * ge;
              ddl[j] = __builtin_fmaf(s, nmr, ddl[j]);  // s Re(conj(a_bar) lambda)
              // dE/dA = (delta a_bar - E) / A
              const float xr = __builtin_fmaf(dlt[j], ar[j], -er[j]);
              const float xi = __builtin_fmaf(dlt[j], ai[j], -ei[j]);
              const float vr = __builtin_fmaf(xr, cf.ar, xi * cf.ai) * cf.inv_a2;
              const float vi = __builtin_fmaf(xi, cf.ar, -xr * cf.ai) * cf.inv_a2;
              dar = __builtin_fmaf(s, __builtin_fmaf(vr, lr, vi * li), dar);
              dai = __builtin_fmaf(s, __builtin_fmaf(vr, li, -vi * lr), dai);
              accC[j] = g[j] * __builtin_fmaf(er[j], s, ahr);
            } else {
              const float q = lr * bv[j];
              du[j] = __builtin_fmaf(dlt[j], q, du[j]);
              ddl[j] = __builtin_fmaf(uu[j], q, ddl[j]);
              const float dlu = dlt[j] * uu[j];
              accB[j] = lr * dlu;
              accC[j] = g[j] * __builtin_fmaf(dlu, bv[j], ahr);
            }
            mr = nmr;
            mi = nmi;
          }
          const float sar = wave_sum(dar), sai = wave_sum(dai);
          if (lane == 0) {
            s_dA[k][n][0] += sar;
            s_dA[k][n][1] += sai;
          }
          // This wave's rows for the iteration: accumulate the segment's dB/dC once the
          // rows' previous owner is done with them (bounded poll: it always progresses).
          {
            const int need = r * N + it - pred_lag + 1;
            if (need > 0) {
              int spins = 0;
              while (__hip_atomic_load(&s_done[pred], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < need &&
                     ++spins < (1 << 22))
                __builtin_amdgcn_s_sleep(1);
            }
            asm volatile("" ::: "memory");  // the row's reads stay below the poll
          }
          f32x4* rb = reinterpret_cast<f32x4*>(&s_acc[arow][0][seg * kCT]);
          f32x4* rc = reinterpret_cast<f32x4*>(&s_acc[arow][1][seg * kCT]);
#pragma unroll
          for (int q = 0; q < kCT / 4; ++q) {
            f32x4 vb = rb[q], vc = rc[q];
            vb.x += accB[4 * q + 0];
            vb.y += accB[4 * q + 1];
            vb.z += accB[4 * q + 2];
            vb.w += accB[4 * q + 3];
            vc.x += accC[4 * q + 0];
            vc.y += accC[4 * q + 1];
            vc.z += accC[4 * q + 2];
            vc.w += accC[4 * q + 3];
            rb[q] = vb;
            rc[q] = vc;
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the row writes have landed
        } else {
          // An inactive wave owns its rows without touching them: it passes them on after
          // their previous owner.
          const int need = r * N + it - pred_lag + 1;
          if (need > 0) {
            int spins = 0;
            while (__hip_atomic_load(&s_done[pred], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < need &&
                   ++spins < (1 << 22))
              __builtin_amdgcn_s_sleep(1);
          }
        }
        if (lane == 0) __hip_atomic_store(&s_done[w], r * N + it + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      if (active) {
        float dsum = 0.f, gsum = 0.f;
#pragma unroll
        for (int j = 0; j < kCT; ++j) {
          const bool valid = ts + j < len;
          float dx = ddl[j];
          if (p.delta_softplus) dx *= sigmoid(xraw[j]);
          dx = valid ? dx : 0.f;
          du[j] = valid ? du[j] : 0.f;
          ddl[j] = dx;
          dsum += dx;
          gsum = __builtin_fmaf(g[j], uu[j], gsum);
        }
        store_seg<kCT>(du_row, ts, L, fast, du);
        store_seg<kCT>(ddl_row, ts, L, fast, ddl);
        const float sd = wave_sum(gsum), sb = wave_sum(dsum);
        if (lane == 0) {
          s_dD[k] += sd;
          s_db[k] += sb;
        }
      }
    }
    // This chunk's dB/dC partial rows (copies summed in order), then clear the rows, after
    // every wave's last accumulation. None past the row's length: the reduction takes those
    // steps as zero (the rows stay zero).
    __syncthreads();
    if (tid < W) s_done[tid] = 0;  // (read again only after the barrier that ends the flush)
    float* part = p.part_dBC + static_cast<size_t>(blockIdx.x) * p.part_stride;
    for (int i = tid; live && i < 2 * N * kCChunk; i += W * 64) {
      const int which = i / (N * kCChunk);
      const int rem = i - which * N * kCChunk;
      const int n = rem / kCChunk;
      const int t = rem - n * kCChunk;
      float s = 0.f;
      for (int cp = 0; cp < copies; ++cp) {
        s += s_acc[cp * N + n][which][t];
        s_acc[cp * N + n][which][t] = 0.f;
      }
      if (t0 + t < L) part[(static_cast<size_t>(b) * 2 * N + which * N + n) * L + t0 + t] = s;
    }
    __syncthreads();
  }
  for (int i = tid; i < cpb * N; i += W * 64) {
    const int k = i / N, n = i - k * N;
    const int d = d0 + k;
    if (d >= p.dim) continue;
    const size_t o = ((static_cast<size_t>(b) * p.dim + d) * N + n) * 2;
    p.part_dA[o] = s_dA[k][n][0];
    p.part_dA[o + 1] = s_dA[k][n][1];
    if (p.dinit) {
      p.dinit[o] = s_mu[k][n][0];
      p.dinit[o + 1] = s_mu[k][n][1];
    }
  }
  for (int i = tid; i < cpb; i += W * 64) {
    const int d = d0 + i;
    if (d >= p.dim) continue;
    p.part_dD[static_cast<size_t>(b) * p.dim + d] = s_dD[i];
    p.part_dbias[static_cast<size_t>(b) * p.dim + d] = s_db[i];
  }
}

// ---------------------------------------------------------------------------------
// Single-token step with complex A (S6.step's complex branch, mamba/mamba1.py:200-214):
// state [B][D][N][2] float32 (interleaved complex) updated in place, out = (sum_n C Re(h) +
// D u) * silu(z). Mapping of the real step: a 16-lane DPP row per (b, d) channel, one lane
// per state, batch fastest.
template <bool kZOH, typename io_t, typename bc_t>
__global__ __launch_bounds__(256) void cssm_step_kernel(StepParams p) {
  const long long idx = (static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x) >> 4;
  const int n = threadIdx.x & 15;
  const bool ch_ok = idx < static_cast<long long>(p.batch) * p.dim;
  const int b = ch_ok ? static_cast<int>(idx % p.batch) : 0;
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
      const CoefA cf = load_coef(p.A, static_cast<size_t>(d) * N + n);
      const CExp e = cexp_t(dt, cf);
      const float s = to_f32(static_cast<const bc_t*>(p.B)[b * p.bc_sb + n * p.bc_sn]) * u;
      float br, bi;
      if constexpr (kZOH) {
        float er, ei;
        zoh_e(dt, cf, e, er, ei);
        br = er * s;
        bi = ei * s;
      } else {
        br = dt * s;
        bi = 0.f;
      }
      float2* st = reinterpret_cast<float2*>(p.state) + (static_cast<size_t>(b) * p.dim + d) * N + n;
      const float2 h = *st;
      const float ar = e.m * e.cy, ai = e.m * e.sy;
      const float nr = __builtin_fmaf(ar, h.x, __builtin_fmaf(-ai, h.y, br));
      const float ni = __builtin_fmaf(ar, h.y, __builtin_fmaf(ai, h.x, bi));
      *st = make_float2(nr, ni);
      yv = to_f32(static_cast<const bc_t*>(p.C)[b * p.bc_sb + n * p.bc_sn]) * nr;
    }
  }
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

hipError_t launch_cssm_step(const StepParams& p, bool zoh, bool io_bf16, bool bc_bf16, hipStream_t stream) {
  const long long n = static_cast<long long>(p.batch) * p.dim * 16;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256)), block(256);
#define MSS_CSTEP(Z, IO, BC) hipLaunchKernelGGL((cssm_step_kernel<Z, IO, BC>), grid, block, 0, stream, p)
  if (zoh) {
    if (io_bf16) { if (bc_bf16) MSS_CSTEP(true, bf16_t, bf16_t); else MSS_CSTEP(true, bf16_t, float); }
    else { if (bc_bf16) MSS_CSTEP(true, float, bf16_t); else MSS_CSTEP(true, float, float); }
  } else {
    if (io_bf16) { if (bc_bf16) MSS_CSTEP(false, bf16_t, bf16_t); else MSS_CSTEP(false, bf16_t, float); }
    else { if (bc_bf16) MSS_CSTEP(false, float, bf16_t); else MSS_CSTEP(false, float, float); }
  }
#undef MSS_CSTEP
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
template <bool kZOH, typename io_t, typename bc_t>
static hipError_t launch_cfwd_t(const FwdParams& p, hipStream_t stream) {
  dim3 grid((p.dim + kCFwdW - 1) / kCFwdW, p.batch);
  hipLaunchKernelGGL((cfwd_kernel<kZOH, io_t, bc_t>), grid, dim3(kCFwdW * 64), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_cfwd(const FwdParams& p, int zoh, int io_bf16, int bc_bf16, hipStream_t stream) {
  if (zoh) {
    if (io_bf16) return bc_bf16 ? launch_cfwd_t<true, bf16_t, bf16_t>(p, stream)
                                : launch_cfwd_t<true, bf16_t, float>(p, stream);
    return bc_bf16 ? launch_cfwd_t<true, float, bf16_t>(p, stream)
                   : launch_cfwd_t<true, float, float>(p, stream);
  }
  if (io_bf16) return bc_bf16 ? launch_cfwd_t<false, bf16_t, bf16_t>(p, stream)
                              : launch_cfwd_t<false, bf16_t, float>(p, stream);
  return bc_bf16 ? launch_cfwd_t<false, float, bf16_t>(p, stream)
                 : launch_cfwd_t<false, float, float>(p, stream);
}

int cbwd_chan_per_block(int batch, int dim) {
  // One workgroup per CU (registers: 3 waves per SIMD); take the fewest channel rounds K
  // with batch * ceil(dim / (kW*K)) <= 256, at most kCMaxChan channels.
  const long long per_row = (dim + kCBwdW - 1) / kCBwdW;
  long long k = 1;
  while (k < per_row && k * kCBwdW < kCMaxChan &&
         static_cast<long long>(batch) * ((per_row + k - 1) / k) > 256)
    ++k;
  return static_cast<int>(k) * kCBwdW;
}

template <bool kZOH, bool kHasZ, typename io_t, typename bc_t>
static hipError_t launch_cbwd_t(const BwdParams& p, hipStream_t stream) {
  dim3 grid(p.n_blocks_d, p.batch);
  hipLaunchKernelGGL((cbwd_kernel<kZOH, kHasZ, io_t, bc_t>), grid, dim3(kCBwdW * 64), 0, stream, p);
  return hipGetLastError();
}

template <typename io_t, typename bc_t>
static hipError_t launch_cbwd_io(const BwdParams& p, int zoh, hipStream_t stream) {
  const bool hz = p.z != nullptr;
  if (zoh) return hz ? launch_cbwd_t<true, true, io_t, bc_t>(p, stream)
                     : launch_cbwd_t<true, false, io_t, bc_t>(p, stream);
  return hz ? launch_cbwd_t<false, true, io_t, bc_t>(p, stream)
            : launch_cbwd_t<false, false, io_t, bc_t>(p, stream);
}

hipError_t launch_cbwd_scan(const BwdParams& p, int zoh, int io_bf16, int bc_bf16, hipStream_t stream) {
  if (io_bf16) return bc_bf16 ? launch_cbwd_io<bf16_t, bf16_t>(p, zoh, stream)
                              : launch_cbwd_io<bf16_t, float>(p, zoh, stream);
  return bc_bf16 ? launch_cbwd_io<float, bf16_t>(p, zoh, stream)
                 : launch_cbwd_io<float, float>(p, zoh, stream);
}

}  // namespace mss
