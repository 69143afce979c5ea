// Backward selective scan for gfx950 (MI355X).
//
// Reference behaviour followed (not its structure):
// native/upstream_mamba/selective_scan_bwd_kernel.cuh:136-299 (reverse chunk loop, forward
// states recomputed from stored residuals, reverse adjoint scan seeded by the final-state
// cotangent, du/ddelta/dA/dB/dC formulas) and its dormant fused branches :151-203,
// :442-485 (softplus, z gate, D, delta bias, initial-state gradient).
//
// Mapping: one wave per channel, lane = segment of kT = 8 steps, chunk = 64 segments = 512
// steps. Lanes hold segments in REVERSED time order (lane 0 = the chunk's last segment), so
// the adjoint, which runs backwards in time, is joined across lanes by the cheap upward
// DPP scan (row shifts + row broadcasts). A workgroup of kW waves walks K rounds of kW
// channels of one batch row and every chunk from last to first. Per chunk the B/C rows of
// all states are staged once in LDS (direct-to-LDS loads) and shared by every wave and
// round. Per (channel, state):
//   forward  from the forward pass's stored state at the segment start (no scan): a_t,
//            a_t*h_{t-1}, h_t; dC partial g_t*h_t
//   reverse  local adjoint aggregate, 64-lane scan seeded by the message from the chunk to
//            the right (dlast for the last chunk), then a re-run producing lambda_t and
//            every per-step gradient term; dB partial lambda_t*delta_t*u_t
// dB/dC are sums over channels: each wave adds its per-(n, t) terms into an LDS
// accumulator shared by the workgroup (rows owned in rotation, plain read-add-write; a wave
// takes its next row once that row's previous owner has marked the iteration done in LDS,
// no workgroup barrier per state), flushed once per chunk to a per-channel-block partial; a second
// kernel sums the partials in a fixed order. This replaces the reference's
// one-global-atomic-per-(b,d,n,t) scheme (selective_scan_bwd_kernel.cuh:295-318).
#include "mss_common.h"

namespace mss {

constexpr int kBwdT = kSegSteps;  // steps per lane: the granularity of the forward's carries
constexpr int kBwdChunk = 64 * kBwdT;
static_assert(kBwdChunk == kPartChunk, "the reduction's chunk is the scan's");
constexpr int kMaxChanPerBlock = 96;  // channels one workgroup walks, at most

// Waves per workgroup, one workgroup per CU: 12 (3 per SIMD, 168 VGPRs) for every state
// count, or 16 (4 per SIMD, 128 VGPRs) when 16 waves own exactly 16 accumulator rows
// (N divides 16), which keeps the LDS within 160 KB. 16 waves walk a round of channels
// ~1.2x slower than 12 but 16/12 as many channels per round (measured on MI355X).
constexpr bool bwd_waves_fit(int waves, int n) { return waves == 12 || (waves == 16 && 16 % n == 0); }

// Floats of LDS holding the dB/dC accumulator (ceil(kW/N) copies of 2N rows of a chunk,
// see the kernel) followed by the B/C stage (2N rows of the chunk in bc_t), maximised over
// the N the wave count serves: with 12 waves N = 11 needs two accumulator copies (22 rows)
// and is the largest.
constexpr int bwd_lds_floats(int waves, int bc_bytes) {
  int m = 0;
  for (int n = 1; n <= kMaxN; ++n) {
    if (!bwd_waves_fit(waves, n)) continue;
    const int v = ((waves + n - 1) / n) * n * 2 * kBwdChunk + n * 2 * kBwdChunk * bc_bytes / 4;
    m = v > m ? v : m;
  }
  return m;
}

// Inclusive upward scan over the 64 lanes of maps m -> P*m + H (lower lanes applied
// first: (Pl, Hl) then (Pr, Hr) gives (Pl*Pr, Pr*Hl + Hr), the operator of reference
// native/selective_scan_cuda.cu:58-63) and of plain sums S. Lane 63 ends with the
// whole wave's map and sum. Each step (lane i takes lane i - 2^k) advances the three
// chains; each DPP read comes two VALU instructions after the write of its source, the
// wait a DPP read needs, and `s_nop 1` pads the first and last step. One asm statement,
// so the compiler neither places a write between a pad and the read it guards nor pads
// between steps itself.
#define MSS_BWD_SCAN_STEP(CTRL, RM)                                \
  "v_fmac_f32_dpp %0, %0, %1 " CTRL " row_mask:" RM " bank_mask:0xf\n\t" \
  "v_add_f32_dpp %2, %2, %2 " CTRL " row_mask:" RM " bank_mask:0xf\n\t"  \
  "v_mul_f32_dpp %1, %1, %1 " CTRL " row_mask:" RM " bank_mask:0xf\n\t"
__device__ __forceinline__ void wave_scan_affine_sum(float& P, float& H, float& S) {
  asm volatile("s_nop 1\n\t"                                   //
               MSS_BWD_SCAN_STEP("row_shr:1", "0xf")            //
               MSS_BWD_SCAN_STEP("row_shr:2", "0xf")            //
               MSS_BWD_SCAN_STEP("row_shr:4", "0xf")            //
               MSS_BWD_SCAN_STEP("row_shr:8", "0xf")            //
               MSS_BWD_SCAN_STEP("row_bcast:15", "0xa")         //
               MSS_BWD_SCAN_STEP("row_bcast:31", "0xc")         //
               "s_nop 1"
               : "+v"(H), "+v"(P), "+v"(S));
}
#undef MSS_BWD_SCAN_STEP

// Sum over the 64 lanes, complete in lane 63 (other lanes hold prefix sums).
__device__ __forceinline__ float wave_sum_to_last(float v) {
  v += dpp_mov<kRowShr1, 0xF>(0.f, v);
  v += dpp_mov<kRowShr2, 0xF>(0.f, v);
  v += dpp_mov<kRowShr4, 0xF>(0.f, v);
  v += dpp_mov<kRowShr8, 0xF>(0.f, v);
  v += dpp_mov<kRowBcast15, 0xA>(0.f, v);
  v += dpp_mov<kRowBcast31, 0xC>(0.f, v);
  return v;
}

// Stage the B and C rows of all N states, steps [t0, t0 + 64*kT), into
// dst[n][B|C][slot]; segment s's q-th 16-byte slot sits at kQ*s + (q ^ slot_swz(s)) so the
// reads of 16 consecutive lanes hit distinct bank groups. dma: rows are 16-byte aligned
// and L is a multiple of the slot width; past-the-end slots re-read the last valid slot
// (finite values that only meet zero coefficients). Otherwise scalar loads, zero past L.
template <int kT, int kW, typename bc_t>
__device__ __forceinline__ void stage_chunk(const bc_t* __restrict__ Bb, const bc_t* __restrict__ Cb,
                                            int N, int t0, int L, long long sn, bool dma,
                                            uint4 (*dst)[2][64 * kT * sizeof(bc_t) / 16], int tid) {
  constexpr int kE = BcStage<bc_t>::kElemsPerSlot;
  constexpr int kQ = kT / kE;
  constexpr int kSlots = 64 * kQ;  // per row, a multiple of 64
  if (dma) {
    const int lane = tid & 63;
    const int w = tid >> 6;
    for (int f0 = w * 64; f0 < N * 2 * kSlots; f0 += kW * 64) {
      const int rowi = f0 / kSlots;  // wave-uniform
      const int n = rowi >> 1;
      const int which = rowi & 1;
      const int s0 = f0 - rowi * kSlots;
      const int s = s0 + lane;
      const int i = s / kQ;
      const int q = (s % kQ) ^ slot_swz<kQ>(i);
      int e = t0 + i * kT + q * kE;
      e = e < L ? e : L - kE;
      const bc_t* src = (which ? Cb : Bb) + n * sn + e;
      __builtin_amdgcn_global_load_lds((gbl_void_t)src, (lds_void_t)(&dst[n][which][s0]), 16, 0, 0);
    }
  } else {
    for (int f = tid; f < N * 2 * 64 * kT; f += kW * 64) {
      const int rowi = f / (64 * kT);
      const int n = rowi >> 1;
      const int which = rowi & 1;
      const int e = f - rowi * 64 * kT;
      const int i = e / kT;
      const int r = e % kT;
      const int sl = kQ * i + ((r / kE) ^ slot_swz<kQ>(i));
      const int t = t0 + e;
      bc_t v;
      if (t < L) {
        v = ((which ? Cb : Bb) + n * sn)[t];
      } else {
        store_as(&v, 0.f);
      }
      reinterpret_cast<bc_t*>(&dst[n][which][0])[sl * kE + (r % kE)] = v;
    }
  }
}

// kGroup: 0 = the whole state dimension; 1 = the first state group of a float32 scan with
// more than kMaxN states (A, the state buffers and the carries read with the strides of the
// full tensors, p.a_ld / p.state_ld / p.carry_cs; dz only where p.dz is given); 2 = a later
// group (as 1, and du/ddelta add to the values already in their buffers).
template <int kW, bool kZOH, bool kHasZ, typename io_t, typename bc_t, int kGroup = 0>
__global__ __launch_bounds__(kW * 64) void bwd_kernel(BwdParams p) {
  constexpr bool kAcc = kGroup == 2;
  constexpr int kT = kBwdT;
  constexpr int kChunk = kBwdChunk;
  constexpr int kRowSlots = kChunk * static_cast<int>(sizeof(bc_t)) / 16;
  // One LDS buffer: first the dB/dC partial sums of the workgroup's channels for one
  // chunk, acc[copy][n][j][B|C][lane] (step j of lane `lane`'s segment), conflict-free for
  // the 64 lanes of a wave. At state iteration i wave w owns row n = (i + w) mod N of copy
  // w / N, so rows are updated with plain read-add-write in a fixed order (LDS float
  // atomics are avoided: far slower than a read, an add and a write on gfx950). Then the
  // B/C rows of the current chunk, all states: stage[n][B|C][slot].
  __shared__ __attribute__((aligned(16))) float lds[bwd_lds_floats(kW, sizeof(bc_t))];
  __shared__ float s_mu[kMaxChanPerBlock][kMaxN];  // adjoint message entering the chunk
  __shared__ float s_dA[kMaxChanPerBlock][kMaxN];
  __shared__ float s_dD[kMaxChanPerBlock];
  __shared__ float s_db[kMaxChanPerBlock];
  __shared__ float s_A[kW][kMaxN];  // A row of each wave's current channel
  __shared__ int s_done[kW];         // state iterations of the current chunk each wave has finished

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int seg = 63 - lane;  // this lane's segment within a chunk (reversed time order)
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = row_longest_first(p.seq_lens, p.batch, p.seqlen, blockIdx.y);
  const int blk = blockIdx.x;
  const int L = p.seqlen;
  const int N = p.dstate;
  const int K = p.chan_per_block / kW;
  const int a_ld = kGroup ? p.a_ld : N;
  const int st_ld = kGroup ? p.state_ld : N;
  const long long carry_cs = kGroup ? p.carry_cs : static_cast<long long>(N) * p.n_seg;
  const bool has_dz = kGroup ? p.dz != nullptr : true;  // (z given: dz given, ungrouped)
  const int len = p.seq_lens ? min(max(p.seq_lens[b], 0), L) : L;
  const bool vec_io = p.vec_io != 0;
  const bool dma = p.vec_bc != 0;
  const bc_t* __restrict__ Bb = static_cast<const bc_t*>(p.B) + b * p.bc_sb;
  const bc_t* __restrict__ Cb = static_cast<const bc_t*>(p.C) + b * p.bc_sb;

  const int n_copy = (kW + N - 1) / N;
  const int acc_floats = n_copy * N * 2 * kChunk;
  float* const acc = lds;
  uint4(*const stage)[2][kRowSlots] = reinterpret_cast<uint4(*)[2][kRowSlots]>(lds + acc_floats);
  const int wmod = w % N;
  float* const acc_w = acc + (w / N) * 2 * N * kChunk;
  // Rows of a copy rotate one wave down per state iteration, so the previous owner of this
  // wave's row at chunk iteration g is the copy's next wave at g - 1 or, for the copy's last
  // wave, its first wave at g - (N - wmod): every wait is on an earlier iteration, so the
  // waits always resolve. (A workgroup barrier per iteration instead, measured on MI355X:
  // backward 906 / 357 / 3121 us at c3 / a c5 layer / c4 against 882 / 350 / 3033, c2 the
  // same.)
  const int copy_waves = min(N, kW - (w / N) * N);
  const int pred = wmod + 1 < copy_waves ? w + 1 : w - wmod;
  const int pred_lag = wmod + 1 < copy_waves ? 1 : N - wmod;
  if (tid < kW) s_done[tid] = 0;
  for (int i = tid; i < acc_floats; i += kW * 64) acc[i] = 0.f;
  for (int k = 0; k < K; ++k) {
    const int cl = k * kW + w;
    const int d = blk * p.chan_per_block + cl;
    if (lane < kMaxN) {
      float mu0 = 0.f;
      if (d < p.dim && lane < N && p.dlast) mu0 = p.dlast[(static_cast<size_t>(b) * p.dim + d) * st_ld + lane];
      s_mu[cl][lane] = mu0;
      s_dA[cl][lane] = 0.f;
    }
    if (lane == 0) {
      s_dD[cl] = 0.f;
      s_db[cl] = 0.f;
    }
  }

  const int n_chunks = (L + kChunk - 1) / kChunk;
  const int n_live = (len + kChunk - 1) / kChunk;  // chunks holding at least one valid step
  if (n_live > 0) stage_chunk<kT, kW, bc_t>(Bb, Cb, N, (n_live - 1) * kChunk, L, p.bc_sn, dma, stage, tid);
  wait_vmem_all();
  __syncthreads();

  for (int c = n_chunks - 1; c >= 0; --c) {
    const int t0 = c * kChunk;
    const int tl = t0 + seg * kT;  // first step of this lane's segment
    const bool fast = vec_io && (t0 + kChunk <= L);  // wave-uniform
    const int seg_idx = t0 / kT + seg;               // index into a carries row
    const bool seg_ok = seg_idx < p.n_seg;

    if (c >= n_live) {
      // Whole chunk past this row's length: zero gradients; the adjoint message passes
      // through the identity steps unchanged.
      for (int k = 0; k < K; ++k) {
        const int cl = k * kW + w;
        const int d = blk * p.chan_per_block + cl;
        if (d >= p.dim) continue;
        const long long row = b * p.io_sb + d * p.io_sd;
        float zero[kT];
#pragma unroll
        for (int j = 0; j < kT; ++j) zero[j] = 0.f;
        if constexpr (!kAcc) {  // (accumulating: adding zero changes nothing)
          store_seg<kT>(static_cast<io_t*>(p.du) + row, tl, L, fast, zero);
          store_seg<kT>(static_cast<io_t*>(p.ddelta) + row, tl, L, fast, zero);
        }
        if constexpr (kHasZ)
          if (has_dz) store_seg<kT>(static_cast<io_t*>(p.dz) + row, tl, L, fast, zero);
        if (c == 0 && p.dinit && lane < N)
          p.dinit[(static_cast<size_t>(b) * p.dim + d) * st_ld + lane] = s_mu[cl][lane];
      }
      // No dB/dC partials: the reduction takes this chunk's steps as zero.
      continue;
    }

    for (int k = 0; k < K; ++k) {
      const int cl = k * kW + w;
      const int d_raw = blk * p.chan_per_block + cl;
      const bool active = d_raw < p.dim;
      const int d = active ? d_raw : p.dim - 1;
      const size_t chan = static_cast<size_t>(b) * p.dim + d;
      const long long row = b * p.io_sb + d * p.io_sd;
      // Carries of this channel and chunk: a uniform base per state plus the lane's segment,
      // so the loads take a scalar base and a fixed per-lane offset (no per-load address
      // registers for later instructions to wait on).
      const float* __restrict__ carry_chunk = p.carries + chan * carry_cs + t0 / kT;

      // ---- per-step inputs of the row
      // A row through LDS: a global load feeding the state loop would put a wait on all
      // outstanding loads (the carry prefetch included) inside the loop.
      if (lane < N) s_A[w][lane] = p.A[static_cast<size_t>(d) * a_ld + lane];
      const float Dv = p.D ? p.D[d] : 0.f;
      const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
      float dlt[kT], dlu[kT], uu[kT], g[kT], s1[kT], s2[kT];
      float ssum = 0.f;
      float hin_next = 0.f;
      if (active && seg_ok) hin_next = (carry_chunk + static_cast<size_t>(wmod) * p.n_seg)[seg];
      {
        // Unconditional, so no per-step value needs a copy for the inactive path: a wave past
        // the last channel reads the clamped channel's row and never stores or accumulates.
        load_seg<kT>(static_cast<const io_t*>(p.delta) + row, tl, L, fast, dlt);
        load_seg<kT>(static_cast<const io_t*>(p.u) + row, tl, L, fast, uu);
        load_seg<kT>(static_cast<const io_t*>(p.dout) + row, tl, L, fast, g);
        if constexpr (kHasZ) {
          // g = dout * silu(z); dz = dout * y * sigmoid(z) * (1 + z * (1 - sigmoid(z))). With the
          // forward's out = y z sigmoid(z): dz = dout * out * (1 / z + 1 - sigmoid(z)), and where
          // |z| < kZTiny (out / z imprecise) y itself, which the forward kept there.
          float zr[kT], yp[kT];
          load_seg<kT>(static_cast<const io_t*>(p.z) + row, tl, L, fast, zr);
          load_seg<kT>(static_cast<const io_t*>(p.out) + row, tl, L, fast, yp);
          const io_t* __restrict__ ykept = static_cast<const io_t*>(p.y_pre) + row;
#pragma unroll
          for (int j = 0; j < kT; ++j) {
            const bool valid = tl + j < len;
            const float go = valid ? g[j] : 0.f;
            const float sz = sigmoid(zr[j]);
            float d = go * yp[j] * (fast_rcp(zr[j]) + (1.f - sz));
            if (valid && __builtin_fabsf(zr[j]) < kZTiny)
              d = go * to_f32(ykept[tl + j]) * sz * __builtin_fmaf(zr[j], 1.f - sz, 1.f);
            yp[j] = valid ? d : 0.f;
            g[j] = go * zr[j] * sz;
          }
          if (active && has_dz) store_seg<kT>(static_cast<io_t*>(p.dz) + row, tl, L, fast, yp);
        }
#pragma unroll
        for (int j = 0; j < kT; ++j) {
          const bool valid = tl + j < len;
          const float x = dlt[j] + bias;
          float dv = p.delta_softplus ? softplus(x) : x;
          dv = valid ? dv : 0.f;
          uu[j] = valid ? uu[j] : 0.f;
          dlt[j] = dv;
          dlu[j] = kZOH ? uu[j] : dv * uu[j];
          if constexpr (!kHasZ) g[j] = valid ? g[j] : 0.f;
          s1[j] = 0.f;
          s2[j] = 0.f;
          ssum += dv;
        }
      }

      // ---- states, in the wave's rotated order (see the accumulator). dA of state n rides
      // on the next state's scan; the last one is reduced after the loop.
      float dA_pend = 0.f;
      int n_pend = -1;
      for (int i = 0; i < N; ++i) {
        int n = i + wmod;
        n = n >= N ? n - N : n;
        const float hin = hin_next;
        if (active && seg_ok && i + 1 < N) {
          const int nn = n + 1 == N ? 0 : n + 1;
          hin_next = (carry_chunk + static_cast<size_t>(nn) * p.n_seg)[seg];
        }
        // The stage does not change within a chunk: its reads go out before the barrier, so
        // their latency overlaps the wait.
        float bv[kT], cg[kT];
        read_staged<kT, bc_t>(stage[n][0], seg, bv);
        read_staged<kT, bc_t>(stage[n][1], seg, cg);
        const int gi = k * N + i;  // state iteration within the chunk
        {
          // Row n is free once its previous owner has finished its iteration. The poll is
          // bounded only so that it ends in every case; the owner always progresses.
          const int need = gi - pred_lag + 1;
          if (need > 0) {
            int spins = 0;
            while (__hip_atomic_load(&s_done[pred], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < need &&
                   ++spins < (1 << 22))
              __builtin_amdgcn_s_sleep(1);
          }
          asm volatile("" ::: "memory");  // the row's reads stay below the poll
        }
        if (!active) {  // owns the row without touching it: passes it on
          if (lane == 0) __hip_atomic_store(&s_done[w], gi + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          continue;
        }
        // The wave holding an accumulator row issues ahead of the waves still polling, so the
        // row is handed on sooner (measured on MI355X, interleaved: backward 868 -> 845 us at
        // c3, 343 -> 334 us at a c5 layer, 3109 -> 3036 us at c4; c2's 12-wave plan within 1 %).
        __builtin_amdgcn_s_setprio(1);
        const float An = s_A[w][n];
        const float a2 = An * kLog2e;
        const float mu = s_mu[cl][n];
        const float dA_old = n_pend >= 0 ? s_dA[cl][n_pend] : 0.f;
        // This wave owns accumulator row n until the next barrier.
        float* accn = acc_w + n * 2 * kChunk + lane;
        float a[kT], ah[kT], accB[kT];
#pragma unroll
        for (int j = 0; j < kT; ++j) accB[j] = accn[j * 128];  // used by the re-run; fetched early
        {
          float accC[kT];
#pragma unroll
          for (int j = 0; j < kT; ++j) accC[j] = accn[j * 128 + 64];
          float h = hin;
#pragma unroll
          for (int j = 0; j < kT; ++j) {
            a[j] = fast_exp2(dlt[j] * a2);
            const float bu = kZOH ? (expm1f(dlt[j] * An) * fast_rcp(An)) * bv[j] * uu[j] : dlu[j] * bv[j];
            ah[j] = a[j] * h;  // a_bar_t * h_{t-1}
            h = ah[j] + bu;
            accC[j] = __builtin_fmaf(g[j], h, accC[j]);
          }
#pragma unroll
          for (int j = 0; j < kT; ++j) accn[j * 128 + 64] = accC[j];
        }
        // ---- reverse: local adjoint aggregate, scan, re-run with the true message
#pragma unroll
        for (int j = 0; j < kT; ++j) cg[j] *= g[j];
        float lam = cg[kT - 1];
#pragma unroll
        for (int j = kT - 2; j >= 0; --j) lam = __builtin_fmaf(a[j + 1], lam, cg[j]);
        float P = fast_exp2(a2 * ssum);  // product of the segment's a_bar
        float Q = a[0] * lam;            // message the segment sends left, zero input
        float S = dA_pend;
        wave_scan_affine_sum(P, Q, S);
        const float mo = __builtin_fmaf(P, mu, Q);       // message leaving this lane's segment
        const float m_in = dpp_mov<kWaveShr1, 0xF>(mu, mo);  // message entering it
        if (lane == 63) {
          s_mu[cl][n] = mo;  // after chunk 0: d h_{-1} = a_bar_0 * lambda_0 (written below)
          if (n_pend >= 0) s_dA[cl][n_pend] = dA_old + S;
        }
        lam = m_in + cg[kT - 1];
        float dA_l = 0.f;
#pragma unroll
        for (int j = kT - 1; j >= 0; --j) {
          if (j < kT - 1) lam = __builtin_fmaf(a[j + 1], lam, cg[j]);
          const float q = lam * ah[j];
          if constexpr (kZOH) {
            const float e = expm1f(dlt[j] * An) * fast_rcp(An);
            const float lb = lam * bv[j];
            s1[j] = __builtin_fmaf(lb, e, s1[j]);
            s2[j] = __builtin_fmaf(An, q, __builtin_fmaf(lb * uu[j], a[j], s2[j]));
            const float dedA = (dlt[j] * a[j] - e) * fast_rcp(An);
            dA_l = __builtin_fmaf(dlt[j], q, __builtin_fmaf(lb * uu[j], dedA, dA_l));
            accB[j] = __builtin_fmaf(lam * e, uu[j], accB[j]);
          } else {
            s1[j] = __builtin_fmaf(lam, bv[j], s1[j]);
            s2[j] = __builtin_fmaf(An, q, s2[j]);
            dA_l = __builtin_fmaf(dlt[j], q, dA_l);
            accB[j] = __builtin_fmaf(lam, dlu[j], accB[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < kT; ++j) accn[j * 128] = accB[j];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's row writes have landed
        if (lane == 0) __hip_atomic_store(&s_done[w], gi + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __builtin_amdgcn_s_setprio(0);
        dA_pend = dA_l;
        n_pend = n;
      }
      if (!active) continue;
      {
        const float S = wave_sum_to_last(dA_pend);
        if (lane == 63) s_dA[cl][n_pend] += S;
      }
      if (c == 0 && p.dinit && lane < N) p.dinit[chan * st_ld + lane] = s_mu[cl][lane];

      // ---- per-step gradients of the row
      if constexpr (!kZOH) {
        // Euler needs u only from here on: reload it rather than hold it across the loop.
        load_seg<kT>(static_cast<const io_t*>(p.u) + row, tl, L, fast, uu);
      }
      float dD_acc = 0.f, db_acc = 0.f;
      float duv[kT], ddv[kT];
#pragma unroll
      for (int j = 0; j < kT; ++j) {
        const bool valid = tl + j < len;
        const float uv = valid ? uu[j] : 0.f;
        float du_j, dd_j;
        if constexpr (kZOH) {
          du_j = __builtin_fmaf(Dv, g[j], s1[j]);
          dd_j = s2[j];
        } else {
          du_j = __builtin_fmaf(dlt[j], s1[j], Dv * g[j]);
          dd_j = __builtin_fmaf(uv, s1[j], s2[j]);
        }
        if (p.delta_softplus) {
          // d softplus(x)/dx = sigmoid(x) = 1 - exp(-softplus(x)); identity above 20.
          dd_j = dlt[j] > 20.f ? dd_j : dd_j * one_minus_exp_neg(dlt[j]);
        }
        du_j = valid ? du_j : 0.f;
        dd_j = valid ? dd_j : 0.f;
        dD_acc = __builtin_fmaf(g[j], uv, dD_acc);
        db_acc += dd_j;
        duv[j] = du_j;
        ddv[j] = dd_j;
      }
      if constexpr (kAcc) {
        float prev[kT];
        load_seg<kT>(static_cast<const io_t*>(p.du) + row, tl, L, fast, prev);
#pragma unroll
        for (int j = 0; j < kT; ++j) duv[j] += prev[j];
        load_seg<kT>(static_cast<const io_t*>(p.ddelta) + row, tl, L, fast, prev);
#pragma unroll
        for (int j = 0; j < kT; ++j) ddv[j] += prev[j];
      }
      store_seg<kT>(static_cast<io_t*>(p.du) + row, tl, L, fast, duv);
      store_seg<kT>(static_cast<io_t*>(p.ddelta) + row, tl, L, fast, ddv);
      const float dD_sum = wave_sum_to_last(dD_acc);
      const float db_sum = wave_sum_to_last(db_acc);
      if (lane == 63) {
        s_dD[cl] += dD_sum;
        s_db[cl] += db_sum;
      }
    }

    // ---- all waves are done with this chunk's stage and accumulator: start staging the
    // next chunk (to the left), then flush this chunk's dB/dC sums over the block's channels.
    __syncthreads();
    if (tid < kW) s_done[tid] = 0;  // (read again only after the barrier that ends the flush)
    if (c > 0) stage_chunk<kT, kW, bc_t>(Bb, Cb, N, t0 - kChunk, L, p.bc_sn, dma, stage, tid);
    const size_t nl = static_cast<size_t>(N) * L;
    float* part = p.part_dBC + static_cast<size_t>(blk) * p.part_stride + static_cast<size_t>(b) * 2 * nl;
    const bool vec_part = (L % 4) == 0;
    for (int task = tid; task < 2 * N * 128; task += kW * 64) {
      // Row (which, n); acc lane ln (segment 63 - ln); steps 4qq..4qq+3 of the segment.
      const int rowi = task >> 7;
      const int which = rowi >= N;
      const int n = rowi - which * N;
      const int ln = task & 63;
      const int qq = (task >> 6) & 1;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int off = n * 2 * kChunk + (4 * qq + e) * 128 + which * 64 + ln;
        float sum = 0.f;
        for (int cp = 0; cp < n_copy; ++cp) {
          sum += acc[cp * 2 * N * kChunk + off];
          acc[cp * 2 * N * kChunk + off] = 0.f;
        }
        v[e] = sum;
      }
      const int t = t0 + (63 - ln) * kT + 4 * qq;
      float* dst = part + which * nl + static_cast<size_t>(n) * L + t;
      if (vec_part && t + 4 <= L) {
        const f32x4 x = {v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4*>(dst) = x;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t + e < L) dst[e] = v[e];
      }
    }
    wait_vmem_all();
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

// One launch finishes every cross-block sum, in a fixed order:
//   blocks [0, n_bc_blocks): dB/dC[b][n][t] = sum over channel blocks of the partials
//     ([block][b][B|C][n][t], block stride `stride` floats). The block's row is
//     blockIdx / x_blocks = (b, which, n); threads walk the row's steps, 4 at a time (16-byte
//     loads) when kVec (L a multiple of 4), keeping kDepth blocks' loads in flight (8 when
//     there are 64 or more channel blocks: c2's 64 blocks reduce in 14.7 us instead of 17.6
//     on MI355X; with 32 blocks depth 8 was slower). The sum runs over blocks in order
//     either way, so both depths give the same bits. With
//     seq_lens, steps from live_part_end(len, L) on are zero (the scans write no partials
//     there);
//   the remaining blocks: dA[d][n] = sum_b part_dA[b][d][n] (dA rows a_ld apart); dD[d],
//     dbias[d] likewise (dbias added to its current value when acc_bias: a state group of a
//     wider scan).
template <bool kVec, typename bc_t, int kDepth>
__global__ __launch_bounds__(256) void reduce_kernel(const float* __restrict__ part, int n_blk,
                                                     size_t stride, int L, int N, int x_blocks,
                                                     int n_bc_blocks, long long sb, long long sn,
                                                     bc_t* __restrict__ dB, bc_t* __restrict__ dC,
                                                     const float* __restrict__ part_dA,
                                                     const float* __restrict__ part_dD,
                                                     const float* __restrict__ part_db, int batch,
                                                     int dim, int na, int a_ld, int acc_bias,
                                                     float* dA, float* dD, float* dbias,
                                                     const int* __restrict__ seq_lens) {
  if (static_cast<int>(blockIdx.x) >= n_bc_blocks) {
    const int dn = dim * na;  // dA row width: dstate (real A) or 2 * dstate (complex A)
    const int i = (blockIdx.x - n_bc_blocks) * blockDim.x + threadIdx.x;
    if (i < dn) {
      float s = 0.f;
      for (int bb = 0; bb < batch; ++bb) s += part_dA[static_cast<size_t>(bb) * dn + i];
      dA[static_cast<size_t>(i / na) * a_ld + i % na] = s;
    } else if (i < dn + 2 * dim) {
      const int which = (i - dn) / dim;
      const int dd = (i - dn) - which * dim;
      const float* src = which == 0 ? part_dD : part_db;
      float* dst = which == 0 ? dD : dbias;
      if (dst != nullptr) {
        float s = 0.f;
        for (int bb = 0; bb < batch; ++bb) s += src[static_cast<size_t>(bb) * dim + dd];
        dst[dd] = (acc_bias && which == 1) ? dst[dd] + s : s;
      }
    }
    return;
  }
  const int r = blockIdx.x / x_blocks;
  const int xb = blockIdx.x - r * x_blocks;
  const int bb = r / (2 * N);
  const int rem = r - bb * 2 * N;
  const int which = rem >= N;
  const int n = rem - which * N;
  const float* src_row = part + static_cast<size_t>(r) * L;
  bc_t* dst = (which ? dC : dB) + bb * sb + n * sn;
  constexpr int kE = kVec ? 4 : 1;
  const int nvec = (L + kE - 1) / kE;
  // Elements (of kE steps) holding partials; live_part_end is a multiple of 4 or L.
  const int nlive = seq_lens ? (live_part_end(min(max(seq_lens[bb], 0), L), L) + kE - 1) / kE : nvec;
  for (int v = xb * blockDim.x + threadIdx.x; v < nvec; v += x_blocks * blockDim.x) {
    if (v >= nlive) {
#pragma unroll
      for (int e = 0; e < kE; ++e) store_as(dst + kE * v + e, 0.f);
      continue;
    }
    if constexpr (kVec) {
      const f32x4* src = reinterpret_cast<const f32x4*>(src_row) + v;
      const size_t svec = stride / 4;
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
      int k = 0;
      for (; k + kDepth <= n_blk; k += kDepth) {
        f32x4 a[kDepth];
#pragma unroll
        for (int q = 0; q < kDepth; ++q) a[q] = src[static_cast<size_t>(k + q) * svec];
#pragma unroll
        for (int q = 0; q < kDepth; ++q) s += a[q];
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

template <bool kZOH, bool kHasZ, typename io_t, typename bc_t, int kGroup>
static hipError_t launch_bwd_a(const BwdParams& p, hipStream_t stream) {
  dim3 grid(p.n_blocks_d, p.batch);
  if (p.waves == 16) {
    if (!bwd_waves_fit(16, p.dstate) || p.chan_per_block % 16 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL((bwd_kernel<16, kZOH, kHasZ, io_t, bc_t, kGroup>), grid, dim3(16 * 64), 0, stream, p);
  } else {
    if (p.waves != 12 || p.chan_per_block % 12 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL((bwd_kernel<12, kZOH, kHasZ, io_t, bc_t, kGroup>), grid, dim3(12 * 64), 0, stream, p);
  }
  return hipGetLastError();
}

template <bool kZOH, bool kHasZ, typename io_t, typename bc_t>
static hipError_t launch_bwd_t(const BwdParams& p, hipStream_t stream) {
  if (p.dstate == p.a_ld) return launch_bwd_a<kZOH, kHasZ, io_t, bc_t, 0>(p, stream);
  // state groups of a wider scan exist only for float32 scans
  if constexpr (sizeof(io_t) == 4 && sizeof(bc_t) == 4) {
    if (p.acc_out) return launch_bwd_a<kZOH, kHasZ, io_t, bc_t, 2>(p, stream);
    return launch_bwd_a<kZOH, kHasZ, io_t, bc_t, 1>(p, stream);
  }
  return hipErrorInvalidValue;
}

template <typename io_t, typename bc_t>
static hipError_t launch_bwd_io(const BwdParams& p, int zoh, hipStream_t stream) {
  const bool hz = p.z != nullptr;
  if (zoh) return hz ? launch_bwd_t<true, true, io_t, bc_t>(p, stream)
                     : launch_bwd_t<true, false, io_t, bc_t>(p, stream);
  return hz ? launch_bwd_t<false, true, io_t, bc_t>(p, stream)
            : launch_bwd_t<false, false, io_t, bc_t>(p, stream);
}

// Channels one workgroup of `waves` waves walks: the fewest channel rounds K with
// batch * ceil(dim / (waves*K)) <= target workgroups (more rounds also mean fewer dB/dC
// partials to reduce), bounded by the LDS bookkeeping size.
static int chan_per_block_for(int waves, int batch, int dim, long long target) {
  const long long per_row = (dim + waves - 1) / waves;  // rounds needed for a whole row
  long long k = (static_cast<long long>(batch) * per_row + target - 1) / target;
  if (k < 1) k = 1;
  while (k < per_row && static_cast<long long>(batch) * ((per_row + k - 1) / k) > target) ++k;
  if (k > kMaxChanPerBlock / waves) k = kMaxChanPerBlock / waves;
  if (k > per_row) k = per_row;
  return static_cast<int>(k) * waves;
}

BwdPlan bwd_plan(int batch, int dim, int dstate, int varlen) {
  // One workgroup per CU holds the B/C stage and the dB/dC accumulator (LDS), so the grid
  // should fit one pass over the 256 CUs. With variable lengths rows finish at different
  // times, so workgroups stay ~2x smaller and the hardware balances them (rows are handed
  // out longest first; measured on MI355X at B=16 D=2560 L=8192: 2x 4.68 ms per step, 4x
  // 4.83 with twice the dB/dC partials, 1x 4.99 with a longer tail). Of 12 and 16
  // waves the plan takes the one with the smaller modelled time: workgroup passes x rounds
  // x time of a round (16 waves: 1.2x that of 12). Depends on shapes only.
  const long long target = varlen ? 2 * kCUs : kCUs;
  auto cost = [&](int waves, int cpb) {
    const long long grid = static_cast<long long>(batch) * ((dim + cpb - 1) / cpb);
    const double rounds = static_cast<double>(cpb / waves) * (waves == 16 ? 1.2 : 1.0);
    const double passes = varlen ? static_cast<double>(grid) / kCUs
                                 : static_cast<double>((grid + kCUs - 1) / kCUs);
    return passes * rounds;
  };
  BwdPlan plan{12, chan_per_block_for(12, batch, dim, target)};
  if (bwd_waves_fit(16, dstate)) {
    const int cpb16 = chan_per_block_for(16, batch, dim, target);
    if (cost(16, cpb16) < cost(12, plan.chan_per_block)) plan = BwdPlan{16, cpb16};
  }
  return plan;
}

hipError_t launch_bwd_scan(const BwdParams& p, int zoh, int io_bf16, int bc_bf16,
                           hipStream_t stream) {
  if (io_bf16) return bc_bf16 ? launch_bwd_io<bf16_t, bf16_t>(p, zoh, stream)
                              : launch_bwd_io<bf16_t, float>(p, zoh, stream);
  return bc_bf16 ? launch_bwd_io<float, bf16_t>(p, zoh, stream)
                 : launch_bwd_io<float, float>(p, zoh, stream);
}

hipError_t launch_bwd_reduce(const BwdParams& p, int bc_bf16, int a_width, int a_ld, int acc_bias,
                             void* dA, void* dB, void* dC, float* dD, float* dbias, hipStream_t stream) {
  const int L = p.seqlen;
  const bool vec = (L % 4) == 0;  // partial rows are 16-byte aligned (block stride: 64 floats)
  const int nvec = vec ? L / 4 : L;
  const int x_blocks = (nvec + 255) / 256;
  const int n_bc_blocks = x_blocks * p.batch * 2 * p.dstate;
  const int small = p.dim * a_width + 2 * p.dim;
  const dim3 grid(n_bc_blocks + (small + 255) / 256);
  const bool deep = p.n_blocks_d >= 64;
#define MSS_REDUCE(VEC, T)                                                                       \
  hipLaunchKernelGGL((deep ? reduce_kernel<VEC, T, 8> : reduce_kernel<VEC, T, 4>), grid, dim3(256), \
                     0, stream, p.part_dBC, p.n_blocks_d,                                          \
                     p.part_stride, L, p.dstate, x_blocks, n_bc_blocks, p.bc_sb, p.bc_sn,          \
                     static_cast<T*>(dB), static_cast<T*>(dC), p.part_dA, p.part_dD, p.part_dbias,  \
                     p.batch, p.dim, a_width, a_ld, acc_bias, static_cast<float*>(dA), dD, dbias, \
                     p.seq_lens)
  if (bc_bf16) {
    if (vec) MSS_REDUCE(true, bf16_t); else MSS_REDUCE(false, bf16_t);
  } else {
    if (vec) MSS_REDUCE(true, float); else MSS_REDUCE(false, float);
  }
#undef MSS_REDUCE
  return hipGetLastError();
}

}  // namespace mss
