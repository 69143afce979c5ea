// C ABI of the selective-scan engine: argument validation, parameter packing, dispatch.
//
// Every check runs on the host before the first HIP call, so each error path is
// reachable (and tested) without a GPU. Error contract mirrors the reference handlers:
// invalid shapes/attributes -> MSS_ERR_INVALID_ARGUMENT (reference returns
// ffi::Error::InvalidArgument, native/selective_scan_cuda.cu:400-440 and
// native/selective_scan_bwd.cu:45-79); runtime failures -> MSS_ERR_HIP with the HIP
// error text kept per thread (reference: ffi::Error::Internal with cudaGetErrorString,
// native/selective_scan_cuda.cu:334-337).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <cmath>
#include <cstddef>
#include <algorithm>
#include <mutex>
#include <string>

#include "../../include/mamba_selective_scan.h"
#include "mss_common.h"

namespace mss {
hipError_t launch_fwd(const FwdParams& p, int zoh, int io_bf16, int bc_bf16, hipStream_t stream);
hipError_t launch_carry_rebuild(const FwdParams& p, hipStream_t stream);
hipError_t launch_bwd_scan(const BwdParams& p, int zoh, int io_bf16, int bc_bf16,
                           hipStream_t stream);
hipError_t launch_bwd_reduce(const BwdParams& p, int bc_bf16, int a_width, int a_ld, int acc_bias,
                             void* dA, void* dB, void* dC, float* dD, float* dbias, hipStream_t stream);
BwdPlan bwd_plan(int batch, int dim, int dstate, int varlen);
hipError_t launch_cfwd(const FwdParams& p, int zoh, int io_bf16, int bc_bf16, hipStream_t stream);
hipError_t launch_cbwd_scan(const BwdParams& p, int zoh, int io_bf16, int bc_bf16, hipStream_t stream);
int cbwd_chan_per_block(int batch, int dim);
hipError_t launch_cssm_step(const StepParams& p, bool zoh, bool io_bf16, bool bc_bf16, hipStream_t stream);
hipError_t launch_conv(const ConvParams& p, bool bwd, bool vec, bool silu, bool io_bf16,
                       hipStream_t stream);
hipError_t launch_conv_reduce(const ConvParams& p, int n_tiles, float* dw, float* dbias,
                              hipStream_t stream);
int conv_tile_steps(int vec, int io_bf16);
hipError_t launch_norm_fwd(const NormParams& p, bool io_bf16, hipStream_t stream);
hipError_t launch_norm_bwd(const NormParams& p, bool io_bf16, float* dw, hipStream_t stream);
int norm_blocks(int tokens);
hipError_t launch_xent(const XentParams& p, bool bwd, bool vec, hipStream_t stream);
hipError_t launch_xent_fused(const XentParams& p, hipStream_t stream);
hipError_t launch_xent_rescale(bf16_t* dz, long long n, const float* factor, hipStream_t stream);
hipError_t launch_ssm_step(const StepParams& p, bool zoh, bool io_bf16, bool bc_bf16, hipStream_t stream);
hipError_t launch_conv_step(const ConvStepParams& p, bool io_bf16, hipStream_t stream);
hipError_t launch_gemv(const GemvParams& p, hipStream_t stream);
hipError_t launch_proj(const ProjParams& p, hipStream_t stream);
hipError_t launch_wgrad(const WgradParams& p, hipStream_t stream);
hipError_t launch_shadow_refresh(const ShadowParams& p, hipStream_t stream);
hipError_t launch_adamw(const AdamWParams& p, hipStream_t stream);
hipError_t launch_embed_cm(const EmbedParams& p, hipStream_t stream);
hipError_t launch_embed_cm_backward(const EmbedParams& p, hipStream_t stream);
}  // namespace mss

namespace {

thread_local std::string g_last_hip_error;

int hip_fail(hipError_t e, const char* what) {
  g_last_hip_error = std::string(what) + ": " + hipGetErrorString(e);
  return MSS_ERR_HIP;
}

size_t dtype_size(int dt) { return dt == MSS_BF16 ? 2 : 4; }

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// max_dstate: MSS_MAX_DSTATE, or MSS_MAX_DSTATE_WIDE for the float32 real-A scans (the
// backward then runs over groups of at most MSS_MAX_DSTATE states).
int check_dims(int32_t batch, int32_t dim, int32_t seqlen, int32_t dstate,
               int32_t max_dstate = MSS_MAX_DSTATE) {
  if (batch <= 0 || dim <= 0 || seqlen <= 0) return MSS_ERR_INVALID_ARGUMENT;
  if (dstate <= 0 || dstate > MSS_MAX_DSTATE_WIDE) return MSS_ERR_INVALID_ARGUMENT;
  if (dstate > max_dstate) return MSS_ERR_UNSUPPORTED;
  // Grid limits: batch rows (and the dB/dC reduction's batch*2*dstate rows, per state
  // group) on grid.y.
  if (static_cast<long long>(batch) * 2 * (dstate < MSS_MAX_DSTATE ? dstate : MSS_MAX_DSTATE) > 65535)
    return MSS_ERR_UNSUPPORTED;
  // Index arithmetic inside the kernels uses 64-bit offsets; per-row steps are int.
  return MSS_OK;
}

// Largest dstate of a scan with these dtypes: wide for float32 real-A scans.
int32_t max_dstate_for(int32_t io_dtype, int32_t bc_dtype, bool cplx) {
  return (!cplx && io_dtype == MSS_F32 && bc_dtype == MSS_F32) ? MSS_MAX_DSTATE_WIDE : MSS_MAX_DSTATE;
}

// State groups of a backward wider than MSS_MAX_DSTATE: G balanced groups, group g holding
// states [group_begin(g), group_begin(g + 1)).
int state_groups(int32_t dstate) { return (dstate + MSS_MAX_DSTATE - 1) / MSS_MAX_DSTATE; }
int group_begin(int32_t dstate, int g) {
  return static_cast<int>(static_cast<long long>(g) * dstate / state_groups(dstate));
}

int check_common(int32_t discretization, int32_t softplus, int32_t io_dtype, int32_t bc_dtype) {
  if (discretization != MSS_EULER && discretization != MSS_ZOH) return MSS_ERR_INVALID_ARGUMENT;
  if (softplus != 0 && softplus != 1) return MSS_ERR_INVALID_ARGUMENT;
  if ((io_dtype != MSS_F32 && io_dtype != MSS_BF16) || (bc_dtype != MSS_F32 && bc_dtype != MSS_BF16))
    return MSS_ERR_INVALID_ARGUMENT;
  return MSS_OK;
}

// Row strides with the contiguous defaults filled in.
struct Strides {
  long long io_sb = 0, io_sd = 0, bc_sb = 0, bc_sn = 0;
};

// Rows (i, j) start at i*s_i + j*s_j and are `len` long (i < n_i, j < n_j): true when no
// two of them overlap.
bool rows_disjoint(long long n_i, long long s_i, long long n_j, long long s_j, long long len) {
  if (n_i == 1 && n_j == 1) return true;
  if (n_i == 1) return s_j >= len;
  if (n_j == 1) return s_i >= len;
  const bool i_inner = s_i <= s_j;
  const long long lo = i_inner ? s_i : s_j, hi = i_inner ? s_j : s_i;
  const long long n_lo = i_inner ? n_i : n_j;
  return lo >= len && hi >= (n_lo - 1) * lo + len;
}

int resolve_strides(const mss_strides& in, int32_t batch, int32_t dim, int32_t seqlen,
                    int32_t dstate, Strides* out) {
  constexpr long long kMaxStride = 1LL << 40;
  const long long L = seqlen;
  out->io_sb = in.io_batch ? in.io_batch : static_cast<long long>(dim) * L;
  out->io_sd = in.io_dim ? in.io_dim : L;
  out->bc_sb = in.bc_batch ? in.bc_batch : static_cast<long long>(dstate) * L;
  out->bc_sn = in.bc_state ? in.bc_state : L;
  for (long long v : {out->io_sb, out->io_sd, out->bc_sb, out->bc_sn})
    if (v < 0 || v > kMaxStride) return MSS_ERR_INVALID_ARGUMENT;
  if (!rows_disjoint(batch, out->io_sb, dim, out->io_sd, L)) return MSS_ERR_INVALID_ARGUMENT;
  if (!rows_disjoint(batch, out->bc_sb, dstate, out->bc_sn, L)) return MSS_ERR_INVALID_ARGUMENT;
  return MSS_OK;
}

// 16-byte vector access of every row: aligned bases and strides.
bool strides_aligned(long long s0, long long s1, size_t esz) {
  return (static_cast<size_t>(s0) * esz) % 16 == 0 && (static_cast<size_t>(s1) * esz) % 16 == 0;
}

int n_seg_of(int32_t seqlen) { return (seqlen + MSS_SEG_STEPS - 1) / MSS_SEG_STEPS; }

struct BwdLayout {
  int waves = 12, chan_per_block = 0, n_blocks_d = 0;
  size_t part_stride = 0;  // floats per channel block of dB/dC partials (multiple of 64)
  size_t off_dA = 0, off_dD = 0, off_db = 0, total = 0;
};

// cplx: the complex-A backward (its own channel blocking; dA partials are complex).
BwdLayout bwd_layout(int32_t batch, int32_t dim, int32_t seqlen, int32_t dstate, bool varlen,
                     bool cplx = false) {
  BwdLayout l;
  if (cplx) {
    l.chan_per_block = mss::cbwd_chan_per_block(batch, dim);
  } else {
    const mss::BwdPlan plan = mss::bwd_plan(batch, dim, dstate, varlen ? 1 : 0);
    l.waves = plan.waves;
    l.chan_per_block = plan.chan_per_block;
  }
  l.n_blocks_d = (dim + l.chan_per_block - 1) / l.chan_per_block;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  l.part_stride = (static_cast<size_t>(batch) * 2 * dstate * seqlen + 63) / 64 * 64;
  const size_t bc = static_cast<size_t>(l.n_blocks_d) * l.part_stride * sizeof(float);
  l.off_dA = up(bc);
  l.off_dD = l.off_dA + up(static_cast<size_t>(batch) * dim * dstate * (cplx ? 2 : 1) * sizeof(float));
  l.off_db = l.off_dD + up(static_cast<size_t>(batch) * dim * sizeof(float));
  l.total = l.off_db + up(static_cast<size_t>(batch) * dim * sizeof(float));
  return l;
}

// Workspace layout of a backward call: for more than MSS_MAX_DSTATE states the groups run
// one after another in one workspace, sized for the larger of the two group sizes (its
// plan is the one reported for the call).
BwdLayout bwd_layout_call(int32_t batch, int32_t dim, int32_t seqlen, int32_t dstate, bool varlen,
                          bool cplx = false) {
  if (cplx || dstate <= MSS_MAX_DSTATE) return bwd_layout(batch, dim, seqlen, dstate, varlen, cplx);
  const int G = state_groups(dstate);
  const BwdLayout hi = bwd_layout(batch, dim, seqlen, (dstate + G - 1) / G, varlen);
  const BwdLayout lo = bwd_layout(batch, dim, seqlen, dstate / G, varlen);
  return hi.total >= lo.total ? hi : lo;
}

int validate_fwd(const mss_fwd_args* a, bool cplx = false) {
  if (a == nullptr) return MSS_ERR_INVALID_ARGUMENT;
  int s = check_common(a->discretization, a->delta_softplus, a->io_dtype, a->bc_dtype);
  if (s != MSS_OK) return s;
  s = check_dims(a->batch, a->dim, a->seqlen, a->dstate, max_dstate_for(a->io_dtype, a->bc_dtype, cplx));
  if (s != MSS_OK) return s;
  if (!a->u || !a->delta || !a->A || !a->B || !a->C || !a->out) return MSS_ERR_INVALID_ARGUMENT;
  Strides st;
  return resolve_strides(a->strides, a->batch, a->dim, a->seqlen, a->dstate, &st);
}

int validate_bwd(const mss_bwd_args* a, bool cplx = false) {
  if (a == nullptr) return MSS_ERR_INVALID_ARGUMENT;
  int s = check_common(a->discretization, a->delta_softplus, a->io_dtype, a->bc_dtype);
  if (s != MSS_OK) return s;
  s = check_dims(a->batch, a->dim, a->seqlen, a->dstate, max_dstate_for(a->io_dtype, a->bc_dtype, cplx));
  if (s != MSS_OK) return s;
  if (!a->u || !a->delta || !a->A || !a->B || !a->C || !a->carries || !a->dout) return MSS_ERR_INVALID_ARGUMENT;
  if (!a->du || !a->ddelta || !a->dA || !a->dB || !a->dC) return MSS_ERR_INVALID_ARGUMENT;
  if (a->D && !a->dD) return MSS_ERR_INVALID_ARGUMENT;
  if (a->z && (!a->dz || !a->y_pre || (!cplx && !a->out))) return MSS_ERR_INVALID_ARGUMENT;
  if (a->delta_bias && !a->ddelta_bias) return MSS_ERR_INVALID_ARGUMENT;
  Strides st;
  return resolve_strides(a->strides, a->batch, a->dim, a->seqlen, a->dstate, &st);
}

int run_fwd(const mss_fwd_args* a, float* ref_states, hipStream_t stream, bool cplx = false) {
  mss::FwdParams p{};
  p.batch = a->batch;
  p.dim = a->dim;
  p.seqlen = a->seqlen;
  p.dstate = a->dstate;
  p.delta_softplus = a->delta_softplus;
  Strides st;
  resolve_strides(a->strides, a->batch, a->dim, a->seqlen, a->dstate, &st);  // validated
  p.io_sb = st.io_sb;
  p.io_sd = st.io_sd;
  p.bc_sb = st.bc_sb;
  p.bc_sn = st.bc_sn;
  const size_t io_e = dtype_size(a->io_dtype), bc_e = dtype_size(a->bc_dtype);
  const size_t bc_row = static_cast<size_t>(a->seqlen) * bc_e;
  p.vec_io = strides_aligned(st.io_sb, st.io_sd, io_e) && aligned16(a->u) && aligned16(a->delta) &&
             aligned16(a->z) && aligned16(a->out) && aligned16(a->y_pre);
  // B/C staging also needs L to be a multiple of the 16-byte slot width.
  p.vec_bc = (bc_row % 16 == 0) && strides_aligned(st.bc_sb, st.bc_sn, bc_e) && aligned16(a->B) &&
             aligned16(a->C);
  p.n_seg = n_seg_of(a->seqlen);
  p.n_ref = (a->seqlen + MSS_REF_CHUNK - 1) / MSS_REF_CHUNK;
  p.u = a->u;
  p.delta = a->delta;
  p.A = a->A;
  p.B = a->B;
  p.C = a->C;
  p.D = a->D;
  p.z = a->z;
  p.delta_bias = a->delta_bias;
  p.x0 = a->initial_state;
  p.seq_lens = a->seq_lens;
  p.out = a->out;
  p.last = a->last_state;
  p.carries = a->carries;
  p.ref_states = ref_states;
  p.y_pre = a->z ? a->y_pre : nullptr;
  const int zoh = a->discretization == MSS_ZOH;
  const int io_bf16 = a->io_dtype == MSS_BF16, bc_bf16 = a->bc_dtype == MSS_BF16;
  const hipError_t e = cplx ? mss::launch_cfwd(p, zoh, io_bf16, bc_bf16, stream)
                            : mss::launch_fwd(p, zoh, io_bf16, bc_bf16, stream);
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching selective scan forward");
}

enum BwdPhase { kPhaseScan = 1, kPhaseReduce = 2, kPhaseBoth = 3 };

mss::BwdParams pack_bwd(const mss_bwd_args* a, const BwdLayout& l, char* ws) {
  mss::BwdParams p{};
  p.batch = a->batch;
  p.dim = a->dim;
  p.seqlen = a->seqlen;
  p.dstate = a->dstate;
  p.delta_softplus = a->delta_softplus;
  Strides st;
  resolve_strides(a->strides, a->batch, a->dim, a->seqlen, a->dstate, &st);  // validated
  p.io_sb = st.io_sb;
  p.io_sd = st.io_sd;
  p.bc_sb = st.bc_sb;
  p.bc_sn = st.bc_sn;
  const size_t io_e = dtype_size(a->io_dtype), bc_e = dtype_size(a->bc_dtype);
  const size_t bc_row = static_cast<size_t>(a->seqlen) * bc_e;
  p.vec_io = strides_aligned(st.io_sb, st.io_sd, io_e) && aligned16(a->u) && aligned16(a->delta) &&
             aligned16(a->z) && aligned16(a->dout) && aligned16(a->du) && aligned16(a->ddelta) &&
             aligned16(a->dz) && aligned16(a->y_pre) && aligned16(a->out);
  p.vec_bc = (bc_row % 16 == 0) && strides_aligned(st.bc_sb, st.bc_sn, bc_e) && aligned16(a->B) &&
             aligned16(a->C);
  p.n_seg = n_seg_of(a->seqlen);
  p.waves = l.waves;
  p.chan_per_block = l.chan_per_block;
  p.n_blocks_d = l.n_blocks_d;
  p.u = a->u;
  p.delta = a->delta;
  p.A = a->A;
  p.B = a->B;
  p.C = a->C;
  p.D = a->D;
  p.z = a->z;
  p.delta_bias = a->delta_bias;
  p.x0 = a->initial_state;
  p.seq_lens = a->seq_lens;
  p.carries = a->carries;
  p.y_pre = a->y_pre;
  p.out = a->z ? a->out : nullptr;
  p.dout = a->dout;
  p.dlast = a->dlast_state;
  p.du = a->du;
  p.ddelta = a->ddelta;
  p.dz = a->dz;
  p.dinit = a->dinitial_state;
  p.a_ld = a->dstate;
  p.state_ld = a->dstate;
  p.carry_cs = static_cast<long long>(a->dstate) * p.n_seg;
  p.acc_out = 0;
  p.part_dBC = reinterpret_cast<float*>(ws);
  p.part_stride = l.part_stride;
  p.part_dA = reinterpret_cast<float*>(ws + l.off_dA);
  p.part_dD = reinterpret_cast<float*>(ws + l.off_dD);
  p.part_dbias = reinterpret_cast<float*>(ws + l.off_db);
  return p;
}

int run_bwd(const mss_bwd_args* a, int phases, hipStream_t stream, bool cplx = false) {
  const bool varlen = a->seq_lens != nullptr;
  const bool grouped = !cplx && a->dstate > MSS_MAX_DSTATE;
  // State groups hand the du/ddelta/ddelta_bias sums from one group to the next, so the two
  // phases cannot be split across calls.
  if (grouped && phases != kPhaseBoth) return MSS_ERR_UNSUPPORTED;
  const BwdLayout l = bwd_layout_call(a->batch, a->dim, a->seqlen, a->dstate, varlen, cplx);
  char* ws = static_cast<char*>(a->workspace);
  bool owned = false;
  if (ws == nullptr) {
    // Split phases hand partial sums from one call to the next through the workspace.
    if (phases != kPhaseBoth) return MSS_ERR_WORKSPACE;
    const hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&ws), l.total, stream);
    if (e != hipSuccess) return hip_fail(e, "allocating backward workspace");
    owned = true;
  } else if (a->workspace_bytes < l.total || !aligned16(ws)) {
    return MSS_ERR_WORKSPACE;
  }
  const int zoh = a->discretization == MSS_ZOH;
  const int io_bf16 = a->io_dtype == MSS_BF16;
  const int bc_bf16 = a->bc_dtype == MSS_BF16;
  hipError_t e = hipSuccess;
  if (!grouped) {
    const mss::BwdParams p = pack_bwd(a, l, ws);
    if (phases & kPhaseScan)
      e = cplx ? mss::launch_cbwd_scan(p, zoh, io_bf16, bc_bf16, stream)
               : mss::launch_bwd_scan(p, zoh, io_bf16, bc_bf16, stream);
    if (e == hipSuccess && (phases & kPhaseReduce)) {
      const int na = a->dstate * (cplx ? 2 : 1);
      e = mss::launch_bwd_reduce(p, bc_bf16, na, na, 0, a->dA, a->dB, a->dC, a->dD, a->ddelta_bias, stream);
    }
  } else {
    // One backward per state group (float32 only), in order on the stream, each in the same
    // workspace: group 0 writes du/ddelta (with the D term), dz, dD and ddelta_bias; later
    // groups add their state sums to du/ddelta/ddelta_bias. A, the state buffers and the
    // carries are read with the full dstate as row stride; dB/dC/dA rows of a group are its
    // own.
    const int N = a->dstate;
    for (int g = 0; g < state_groups(N) && e == hipSuccess; ++g) {
      const int n0 = group_begin(N, g), ng = group_begin(N, g + 1) - n0;
      mss::BwdParams p = pack_bwd(a, bwd_layout(a->batch, a->dim, a->seqlen, ng, varlen), ws);
      const size_t bc_off = static_cast<size_t>(n0) * p.bc_sn * sizeof(float);
      p.dstate = ng;
      p.A = a->A + n0;
      p.B = static_cast<const char*>(a->B) + bc_off;
      p.C = static_cast<const char*>(a->C) + bc_off;
      p.x0 = a->initial_state ? a->initial_state + n0 : nullptr;
      p.dlast = a->dlast_state ? a->dlast_state + n0 : nullptr;
      p.dinit = a->dinitial_state ? a->dinitial_state + n0 : nullptr;
      p.carries = a->carries + static_cast<size_t>(n0) * p.n_seg;
      if (g > 0) {
        p.D = nullptr;
        p.dz = nullptr;
        p.acc_out = 1;
      }
      e = mss::launch_bwd_scan(p, zoh, io_bf16, bc_bf16, stream);
      if (e == hipSuccess)
        e = mss::launch_bwd_reduce(p, bc_bf16, ng, N, g > 0, a->dA + n0, static_cast<char*>(a->dB) + bc_off,
                                   static_cast<char*>(a->dC) + bc_off, g == 0 ? a->dD : nullptr,
                                   a->ddelta_bias, stream);
    }
  }
  if (owned) {
    const hipError_t f = hipFreeAsync(ws, stream);
    if (e == hipSuccess) e = f;
  }
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching selective scan backward");
}

// ---- Fixed device scratch of mss_bwd_noalloc: the backward's workspace (dB/dC and
// dA/dD/dbias partial sums) for callers that cannot allocate. One array per device, held
// until the process ends. In host code `scratch` names a host-side stand-in: kernels get
// the device address that hipGetSymbolAddress returns for the current device.
constexpr size_t kScratchBytes = static_cast<size_t>(MSS_NOALLOC_SCRATCH_BYTES);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device.
int scratch_of_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "querying the current device");
  if (dev < 0 || dev >= kMaxDevices) return MSS_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "looking up the backward scratch");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MSS_OK;
}

}  // namespace

// ---- causal conv1d
int validate_conv(const mss_conv_args* a, bool bwd) {
  if (a == nullptr) return MSS_ERR_INVALID_ARGUMENT;
  if (a->batch <= 0 || a->dim <= 0 || a->seqlen <= 0) return MSS_ERR_INVALID_ARGUMENT;
  if (a->width < 1 || a->width > 4) return MSS_ERR_INVALID_ARGUMENT;
  if (a->batch > 65535 || a->dim > 65535) return MSS_ERR_UNSUPPORTED;
  if (a->io_dtype != MSS_F32 && a->io_dtype != MSS_BF16) return MSS_ERR_INVALID_ARGUMENT;
  if (a->activation != 0 && a->activation != 1) return MSS_ERR_INVALID_ARGUMENT;
  if (!a->x || !a->weight) return MSS_ERR_INVALID_ARGUMENT;
  if (!bwd && !a->y) return MSS_ERR_INVALID_ARGUMENT;
  if (bwd && (!a->dy || !a->dx || !a->dweight)) return MSS_ERR_INVALID_ARGUMENT;
  if (bwd && a->bias && !a->dbias) return MSS_ERR_INVALID_ARGUMENT;
  Strides st;
  return resolve_strides(a->strides, a->batch, a->dim, a->seqlen, 1, &st);
}

struct ConvSetup {
  mss::ConvParams p{};
  bool vec = false;
  int n_tiles = 0;
  size_t ws_bytes = 0;
};

ConvSetup conv_setup(const mss_conv_args* a) {
  ConvSetup c;
  Strides st;
  resolve_strides(a->strides, a->batch, a->dim, a->seqlen, 1, &st);  // validated
  c.p.batch = a->batch;
  c.p.dim = a->dim;
  c.p.seqlen = a->seqlen;
  c.p.width = a->width;
  c.p.sb = st.io_sb;
  c.p.sd = st.io_sd;
  c.p.x = a->x;
  c.p.w = a->weight;
  c.p.bias = a->bias;
  c.p.seq_lens = a->seq_lens;
  c.p.y = a->y;
  c.p.dy = a->dy;
  c.p.dx = a->dx;
  const size_t esz = dtype_size(a->io_dtype);
  c.vec = strides_aligned(st.io_sb, st.io_sd, esz) && aligned16(a->x) && aligned16(a->y) &&
          aligned16(a->dy) && aligned16(a->dx);
  const int tile = mss::conv_tile_steps(c.vec, a->io_dtype == MSS_BF16);
  c.n_tiles = (a->seqlen + tile - 1) / tile;
  c.ws_bytes = static_cast<size_t>(a->dim) * a->batch * c.n_tiles * (a->width + 1) * sizeof(float);
  return c;
}

extern "C" {

int mss_abi_version(void) { return MSS_ABI_VERSION; }

const char* mss_strerror(int status) {
  switch (status) {
    case MSS_OK: return "ok";
    case MSS_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MSS_ERR_UNSUPPORTED:
      return "unsupported configuration (a size beyond this build's limits, e.g. dstate > 16 or "
             "batch * 2 * dstate > 65535; each entry point's limits are in mamba_selective_scan.h)";
    case MSS_ERR_HIP: return "HIP runtime error";
    case MSS_ERR_WORKSPACE: return "workspace too small";
    case MSS_ERR_SCRATCH_LIMIT:
      return "request needs more backward scratch than mss_bwd_noalloc holds "
             "(MSS_NOALLOC_SCRATCH_BYTES; use mss_bwd with a workspace)";
    default: return "unknown status";
  }
}

const char* mss_last_hip_error(void) { return g_last_hip_error.c_str(); }

size_t mss_bwd_workspace_bytes(const mss_bwd_args* a) {
  if (a == nullptr ||
      check_dims(a->batch, a->dim, a->seqlen, a->dstate, max_dstate_for(a->io_dtype, a->bc_dtype, false)) != MSS_OK)
    return 0;
  return bwd_layout_call(a->batch, a->dim, a->seqlen, a->dstate, a->seq_lens != nullptr).total;
}

int mss_bwd_plan(const mss_bwd_args* args, int32_t* waves, int32_t* chan_per_block) {
  if (waves == nullptr || chan_per_block == nullptr) return MSS_ERR_INVALID_ARGUMENT;
  const int s = validate_bwd(args);
  if (s != MSS_OK) return s;
  const BwdLayout l = bwd_layout_call(args->batch, args->dim, args->seqlen, args->dstate, args->seq_lens != nullptr);
  *waves = l.waves;
  *chan_per_block = l.chan_per_block;
  return MSS_OK;
}

int mss_fwd(const mss_fwd_args* args, void* stream) {
  const int s = validate_fwd(args);
  if (s != MSS_OK) return s;
  return run_fwd(args, nullptr, static_cast<hipStream_t>(stream));
}

int mss_bwd(const mss_bwd_args* args, void* stream) {
  const int s = validate_bwd(args);
  if (s != MSS_OK) return s;
  return run_bwd(args, kPhaseBoth, static_cast<hipStream_t>(stream));
}

int mss_bwd_noalloc(const mss_bwd_args* args, void* stream) {
  const int s = validate_bwd(args);
  if (s != MSS_OK) return s;
  const BwdLayout l = bwd_layout_call(args->batch, args->dim, args->seqlen, args->dstate, args->seq_lens != nullptr);
  if (l.total > kScratchBytes) return MSS_ERR_SCRATCH_LIMIT;
  void* ws = nullptr;
  const int t = scratch_of_current_device(&ws);
  if (t != MSS_OK) return t;
  mss_bwd_args a = *args;
  a.workspace = ws;
  a.workspace_bytes = kScratchBytes;
  return run_bwd(&a, kPhaseBoth, static_cast<hipStream_t>(stream));
}

int mss_bwd_scan(const mss_bwd_args* args, void* stream) {
  const int s = validate_bwd(args);
  if (s != MSS_OK) return s;
  return run_bwd(args, kPhaseScan, static_cast<hipStream_t>(stream));
}

int mss_bwd_reduce(const mss_bwd_args* args, void* stream) {
  const int s = validate_bwd(args);
  if (s != MSS_OK) return s;
  return run_bwd(args, kPhaseReduce, static_cast<hipStream_t>(stream));
}

// Complex A: the same argument blocks with A, dA and every state buffer read as interleaved
// (real, imaginary) float32 pairs; the carry segments hold complex states, 8-byte aligned.
size_t mss_cbwd_workspace_bytes(const mss_bwd_args* a) {
  if (a == nullptr || check_dims(a->batch, a->dim, a->seqlen, a->dstate) != MSS_OK) return 0;
  return bwd_layout(a->batch, a->dim, a->seqlen, a->dstate, a->seq_lens != nullptr, true).total;
}

int mss_cfwd(const mss_fwd_args* args, void* stream) {
  const int s = validate_fwd(args, true);
  if (s != MSS_OK) return s;
  if (!aligned8(args->A) || !aligned8(args->initial_state) || !aligned8(args->last_state) ||
      !aligned8(args->carries))
    return MSS_ERR_INVALID_ARGUMENT;
  return run_fwd(args, nullptr, static_cast<hipStream_t>(stream), true);
}

int mss_cbwd(const mss_bwd_args* args, void* stream) {
  const int s = validate_bwd(args, true);
  if (s != MSS_OK) return s;
  if (!aligned8(args->A) || !aligned8(args->carries)) return MSS_ERR_INVALID_ARGUMENT;
  return run_bwd(args, kPhaseBoth, static_cast<hipStream_t>(stream), true);
}

size_t mss_conv_bwd_workspace_bytes(const mss_conv_args* a) {
  // Shapes only: sized for the scalar path, which has the most step tiles.
  if (a == nullptr || a->batch <= 0 || a->dim <= 0 || a->seqlen <= 0 || a->width < 1 || a->width > 4)
    return 0;
  const int tile = mss::conv_tile_steps(0, 0);
  const size_t tiles = (static_cast<size_t>(a->seqlen) + tile - 1) / tile;
  return static_cast<size_t>(a->dim) * a->batch * tiles * (a->width + 1) * sizeof(float);
}

int mss_conv_fwd(const mss_conv_args* args, void* stream) {
  const int s = validate_conv(args, false);
  if (s != MSS_OK) return s;
  ConvSetup c = conv_setup(args);
  const hipError_t e = mss::launch_conv(c.p, false, c.vec, args->activation == 1,
                                        args->io_dtype == MSS_BF16, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching conv1d forward");
}

int mss_conv_bwd(const mss_conv_args* args, void* stream) {
  const int s = validate_conv(args, true);
  if (s != MSS_OK) return s;
  ConvSetup c = conv_setup(args);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(args->workspace);
  bool owned = false;
  if (ws == nullptr) {
    const hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&ws), c.ws_bytes, st);
    if (e != hipSuccess) return hip_fail(e, "allocating conv1d workspace");
    owned = true;
  } else if (args->workspace_bytes < c.ws_bytes || !aligned16(ws)) {
    return MSS_ERR_WORKSPACE;
  }
  c.p.part = reinterpret_cast<float*>(ws);
  hipError_t e = mss::launch_conv(c.p, true, c.vec, args->activation == 1, args->io_dtype == MSS_BF16, st);
  if (e == hipSuccess) e = mss::launch_conv_reduce(c.p, c.n_tiles, args->dweight, args->dbias, st);
  if (owned) {
    const hipError_t f = hipFreeAsync(ws, st);
    if (e == hipSuccess) e = f;
  }
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching conv1d backward");
}

static int validate_norm(const mss_norm_args* a, bool bwd) {
  if (a == nullptr || a->features <= 0 || a->tokens <= 0) return MSS_ERR_INVALID_ARGUMENT;
  if (!(a->eps >= 0.f)) return MSS_ERR_INVALID_ARGUMENT;
  if (a->io_dtype != MSS_F32 && a->io_dtype != MSS_BF16) return MSS_ERR_INVALID_ARGUMENT;
  if (!a->h || !a->weight || !a->rstd) return MSS_ERR_INVALID_ARGUMENT;
  if (a->delta && !a->hn) return MSS_ERR_INVALID_ARGUMENT;
  if (!bwd && !a->x) return MSS_ERR_INVALID_ARGUMENT;
  if (bwd && (!a->dx || !a->dhn || !a->dweight)) return MSS_ERR_INVALID_ARGUMENT;
  return MSS_OK;
}

static mss::NormParams pack_norm(const mss_norm_args* a) {
  mss::NormParams p{};
  p.features = a->features;
  p.tokens = a->tokens;
  p.eps = a->eps;
  p.h = a->h;
  p.delta = a->delta;
  p.w = a->weight;
  p.hn = a->hn;
  p.x = a->x;
  p.rstd = a->rstd;
  p.dx = a->dx;
  p.dhn_in = a->dhn_in;
  p.dhn = a->dhn;
  p.ddelta = a->ddelta;
  return p;
}

size_t mss_norm_bwd_workspace_bytes(const mss_norm_args* a) {
  if (a == nullptr || a->features <= 0 || a->tokens <= 0) return 0;
  return static_cast<size_t>(mss::norm_blocks(a->tokens)) * a->features * sizeof(float);
}

int mss_norm_fwd(const mss_norm_args* args, void* stream) {
  const int s = validate_norm(args, false);
  if (s != MSS_OK) return s;
  const hipError_t e = mss::launch_norm_fwd(pack_norm(args), args->io_dtype == MSS_BF16,
                                            static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching rmsnorm forward");
}

int mss_norm_bwd(const mss_norm_args* args, void* stream) {
  const int s = validate_norm(args, true);
  if (s != MSS_OK) return s;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t need = mss_norm_bwd_workspace_bytes(args);
  char* ws = static_cast<char*>(args->workspace);
  bool owned = false;
  if (ws == nullptr) {
    const hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&ws), need, st);
    if (e != hipSuccess) return hip_fail(e, "allocating rmsnorm workspace");
    owned = true;
  } else if (args->workspace_bytes < need) {
    return MSS_ERR_WORKSPACE;
  }
  mss::NormParams p = pack_norm(args);
  p.dw_part = reinterpret_cast<float*>(ws);
  hipError_t e = mss::launch_norm_bwd(p, args->io_dtype == MSS_BF16, args->dweight, st);
  if (owned) {
    const hipError_t f = hipFreeAsync(ws, st);
    if (e == hipSuccess) e = f;
  }
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching rmsnorm backward");
}

namespace {
bool spans_overlap(const void* a, long long rows_a, long long ld_a, long long cols_a, const void* b,
                   long long rows_b, long long ld_b, long long cols_b);
}  // namespace

static int validate_xent(const mss_xent_args* a, bool bwd) {
  if (a == nullptr || a->rows <= 0 || a->vocab <= 0) return MSS_ERR_INVALID_ARGUMENT;
  if (!a->logits || !a->targets || !a->lse) return MSS_ERR_INVALID_ARGUMENT;
  if (!bwd && !a->loss) return MSS_ERR_INVALID_ARGUMENT;
  if (bwd && (!a->grad_scale || !a->dlogits)) return MSS_ERR_INVALID_ARGUMENT;
  return MSS_OK;
}

static int run_xent(const mss_xent_args* a, bool bwd, hipStream_t st) {
  mss::XentParams p{};
  p.rows = a->rows;
  p.vocab = a->vocab;
  p.z = static_cast<const mss::bf16_t*>(a->logits);
  p.target = reinterpret_cast<const long long*>(a->targets);
  p.loss = a->loss;
  p.lse = a->lse;
  p.grad_scale = a->grad_scale;
  p.dz = static_cast<mss::bf16_t*>(a->dlogits);
  const bool vec = (a->vocab % 8 == 0) && aligned16(a->logits) && aligned16(a->dlogits);
  const hipError_t e = mss::launch_xent(p, bwd, vec, st);
  return e == hipSuccess ? MSS_OK : hip_fail(e, bwd ? "launching cross-entropy backward" : "launching cross-entropy forward");
}

int mss_xent_fwd(const mss_xent_args* args, void* stream) {
  const int s = validate_xent(args, false);
  return s != MSS_OK ? s : run_xent(args, false, static_cast<hipStream_t>(stream));
}

int mss_xent_bwd(const mss_xent_args* args, void* stream) {
  const int s = validate_xent(args, true);
  return s != MSS_OK ? s : run_xent(args, true, static_cast<hipStream_t>(stream));
}

int mss_xent_fwd_grad(const mss_xent_args* a, void* stream) {
  if (a == nullptr || a->rows <= 0 || a->vocab <= 0 || !a->logits || !a->targets || !a->lse || !a->loss ||
      !a->grad_scale || !a->dlogits)
    return MSS_ERR_INVALID_ARGUMENT;
  static_assert(mss::kXentFusedMaxVocab == MSS_XENT_FUSED_MAX_VOCAB, "header and kernel disagree");
  if (a->vocab % 8 != 0 || a->vocab > MSS_XENT_FUSED_MAX_VOCAB || !aligned16(a->logits) || !aligned16(a->dlogits))
    return MSS_ERR_UNSUPPORTED;
  const long long n = static_cast<long long>(a->rows) * a->vocab;
  if (spans_overlap(a->logits, 1, 0, n, a->dlogits, 1, 0, n)) return MSS_ERR_INVALID_ARGUMENT;
  mss::XentParams p{};
  p.rows = a->rows;
  p.vocab = a->vocab;
  p.z = static_cast<const mss::bf16_t*>(a->logits);
  p.target = reinterpret_cast<const long long*>(a->targets);
  p.loss = a->loss;
  p.lse = a->lse;
  p.grad_scale = a->grad_scale;
  p.dz = static_cast<mss::bf16_t*>(a->dlogits);
  const hipError_t e = mss::launch_xent_fused(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching cross-entropy forward + gradient");
}

int mss_xent_rescale(void* dlogits, int64_t n, const float* factor, void* stream) {
  if (!dlogits || !factor || n < 0) return MSS_ERR_INVALID_ARGUMENT;
  if (n == 0) return MSS_OK;
  const hipError_t e = mss::launch_xent_rescale(static_cast<mss::bf16_t*>(dlogits), n, factor,
                                                static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching gradient rescale");
}

namespace {
bool spans_overlap(const void* a, long long rows_a, long long ld_a, long long cols_a, const void* b,
                   long long rows_b, long long ld_b, long long cols_b) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  const uintptr_t xe = x + static_cast<uintptr_t>(((rows_a - 1) * ld_a + cols_a) * 2);
  const uintptr_t ye = y + static_cast<uintptr_t>(((rows_b - 1) * ld_b + cols_b) * 2);
  return x < ye && y < xe;
}

}  // namespace

int mss_proj(const mss_proj_args* a, void* stream) {
  if (a == nullptr || a->M <= 0 || a->K <= 0 || a->T <= 0 || !a->W || !a->X || !a->C)
    return MSS_ERR_INVALID_ARGUMENT;
  if (a->ldw < (a->w_trans ? a->M : a->K) || a->ldx < a->T || a->ldc < a->T) return MSS_ERR_INVALID_ARGUMENT;
  if (a->ldw % 8 != 0 || a->ldx % 8 != 0 || a->ldc % 8 != 0 || !aligned16(a->W) || !aligned16(a->X) ||
      !aligned16(a->C))
    return MSS_ERR_INVALID_ARGUMENT;
  const bool expand = a->K <= mss::kProjExpandMaxK && a->K % 16 == 0;
  const bool reduce = a->K % 64 == 0 && a->M <= mss::kProjReduceMaxM;
  if (a->M % 16 != 0 || a->T % 64 != 0 || (!expand && !reduce)) return MSS_ERR_UNSUPPORTED;
  if (static_cast<long long>(a->M) * a->ldc >= (1LL << 40) || static_cast<long long>(a->K) * a->ldx >= (1LL << 40))
    return MSS_ERR_UNSUPPORTED;
  if ((a->w_trans ? spans_overlap(a->C, a->M, a->ldc, a->T, a->W, a->K, a->ldw, a->M)
                  : spans_overlap(a->C, a->M, a->ldc, a->T, a->W, a->M, a->ldw, a->K)) ||
      spans_overlap(a->C, a->M, a->ldc, a->T, a->X, a->K, a->ldx, a->T))
    return MSS_ERR_INVALID_ARGUMENT;
  mss::ProjParams p{};
  p.M = a->M;
  p.K = a->K;
  p.T = a->T;
  p.accumulate = a->accumulate != 0;
  p.w_trans = a->w_trans != 0;
  p.ldw = a->ldw;
  p.ldx = a->ldx;
  p.ldc = a->ldc;
  p.W = a->W;
  p.X = a->X;
  p.C = a->C;
  const hipError_t e = mss::launch_proj(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching projection GEMM");
}



namespace {
// The split count of a supported weight-gradient shape, 0 for shapes the kernel does not take.
int wgrad_shape_splits(int32_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || N % 4 != 0 || K % 64 != 0) return 0;
  return mss::wgrad_splits(M, N, K);
}
}  // namespace

int64_t mss_wgrad_workspace_bytes(int32_t M, int32_t N, int32_t K) {
  const int s = wgrad_shape_splits(M, N, K);
  return s > 1 ? static_cast<int64_t>(s) * M * N * 4 : 0;
}

int mss_wgrad(const mss_wgrad_args* a, void* stream) {
  if (a == nullptr || a->M <= 0 || a->N <= 0 || a->K <= 0 || !a->A || !a->B || !a->C) return MSS_ERR_INVALID_ARGUMENT;
  if (a->lda < a->K || a->ldb < a->K || a->ldc < a->N) return MSS_ERR_INVALID_ARGUMENT;
  if (a->lda % 8 != 0 || a->ldb % 8 != 0 || a->ldc % 4 != 0 || !aligned16(a->A) || !aligned16(a->B) ||
      !aligned16(a->C))
    return MSS_ERR_INVALID_ARGUMENT;
  const int splits = wgrad_shape_splits(a->M, a->N, a->K);
  if (splits == 0) return MSS_ERR_UNSUPPORTED;
  if (static_cast<long long>(a->M) * a->lda >= (1LL << 40) || static_cast<long long>(a->N) * a->ldb >= (1LL << 40) ||
      static_cast<long long>(a->M) * a->ldc >= (1LL << 40))
    return MSS_ERR_UNSUPPORTED;
  const long long ws_bytes = mss_wgrad_workspace_bytes(a->M, a->N, a->K);
  if (ws_bytes > 0 && (!a->workspace || a->workspace_bytes < ws_bytes || !aligned16(a->workspace)))
    return MSS_ERR_INVALID_ARGUMENT;
  // C (float32, 2 bf16 elements per column) against the operands and the workspace.
  if (spans_overlap(a->C, a->M, 2 * a->ldc, 2 * a->N, a->A, a->M, a->lda, a->K) ||
      spans_overlap(a->C, a->M, 2 * a->ldc, 2 * a->N, a->B, a->N, a->ldb, a->K) ||
      (ws_bytes > 0 && spans_overlap(a->C, a->M, 2 * a->ldc, 2 * a->N, a->workspace, 1, 0, ws_bytes / 2)))
    return MSS_ERR_INVALID_ARGUMENT;
  mss::WgradParams p{};
  p.M = a->M;
  p.N = a->N;
  p.K = a->K;
  p.splits = splits;
  p.accumulate = a->accumulate != 0;
  p.lda = a->lda;
  p.ldb = a->ldb;
  p.ldc = a->ldc;
  p.A = a->A;
  p.B = a->B;
  p.C = a->C;
  p.workspace = static_cast<float*>(a->workspace);
  const hipError_t e = mss::launch_wgrad(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching weight-gradient GEMM");
}


static_assert(sizeof(mss_shadow_entry) == sizeof(mss::ShadowEntry) &&
                  offsetof(mss_shadow_entry, ld_t) == offsetof(mss::ShadowEntry, ld_t) &&
                  offsetof(mss_shadow_entry, tile0) == offsetof(mss::ShadowEntry, tile0),
              "public and kernel shadow entries share one layout");

int mss_shadow_refresh(const mss_shadow_entry* entries, int32_t n_entries, int64_t n_tiles, void* stream) {
  if (!entries || n_entries <= 0 || n_tiles <= 0) return MSS_ERR_INVALID_ARGUMENT;
  mss::ShadowParams p{};
  p.entries = reinterpret_cast<const mss::ShadowEntry*>(entries);
  p.n_entries = n_entries;
  p.n_tiles = n_tiles;
  const hipError_t e = mss::launch_shadow_refresh(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching shadow refresh");
}

static_assert(sizeof(mss_adamw_entry) == sizeof(mss::AdamWEntry) &&
                  offsetof(mss_adamw_entry, step) == offsetof(mss::AdamWEntry, step) &&
                  offsetof(mss_adamw_entry, shadow_t) == offsetof(mss::AdamWEntry, shadow_t) &&
                  offsetof(mss_adamw_entry, rows) == offsetof(mss::AdamWEntry, rows) &&
                  offsetof(mss_adamw_entry, numel) == offsetof(mss::AdamWEntry, numel),
              "public and kernel AdamW entries share one layout");

namespace {
// Work units of a valid entry (flat 4096-element runs, or 64 x 64 tiles with a transposed
// shadow), 0 for an invalid one.
long long adamw_units(const mss_adamw_entry& e) {
  if (!e.param || !e.grad || !e.exp_avg || !e.exp_avg_sq || !e.step || e.numel <= 0 || e.numel >= (1LL << 40))
    return 0;
  if (!aligned16(e.param) || !aligned16(e.grad) || !aligned16(e.exp_avg) || !aligned16(e.exp_avg_sq) ||
      (e.shadow && !aligned8(e.shadow)))
    return 0;
  if (!e.shadow_t) return (e.numel + mss::kAdamWUnit - 1) / mss::kAdamWUnit;
  if (e.rows <= 0 || e.cols <= 0 || e.cols % 4 != 0 || static_cast<long long>(e.rows) * e.cols != e.numel ||
      e.ld_t < e.rows || e.ld_t % 8 != 0 || !aligned16(e.shadow_t))
    return 0;
  return static_cast<long long>((e.rows + 63) / 64) * ((e.cols + 63) / 64);
}
}  // namespace

int mss_adamw(const mss_adamw_args* a, void* stream) {
  if (!a || !a->entries || a->n_entries <= 0) return MSS_ERR_INVALID_ARGUMENT;
  const bool finite = std::isfinite(a->lr) && std::isfinite(a->beta1) && std::isfinite(a->beta2) &&
                      std::isfinite(a->eps) && std::isfinite(a->weight_decay);
  if (!finite || a->lr < 0.f || a->beta1 < 0.f || a->beta1 >= 1.f || a->beta2 < 0.f || a->beta2 >= 1.f ||
      a->eps <= 0.f || a->weight_decay < 0.f)
    return MSS_ERR_INVALID_ARGUMENT;
  for (int32_t i = 0; i < a->n_entries; ++i)
    if (adamw_units(a->entries[i]) == 0) return MSS_ERR_INVALID_ARGUMENT;
  // Launches of up to kAdamWMaxEntries entries each, in order.
  for (int32_t i0 = 0; i0 < a->n_entries; i0 += mss::kAdamWMaxEntries) {
    mss::AdamWParams p{};
    p.n = std::min(mss::kAdamWMaxEntries, a->n_entries - i0);
    p.lr = a->lr;
    p.beta1 = a->beta1;
    p.beta2 = a->beta2;
    p.eps = a->eps;
    p.weight_decay = a->weight_decay;
    long long u = 0;
    for (int k = 0; k < p.n; ++k) {
      std::memcpy(&p.e[k], &a->entries[i0 + k], sizeof(mss::AdamWEntry));
      p.unit0[k] = u;
      u += adamw_units(a->entries[i0 + k]);
    }
    p.unit0[p.n] = u;
    if (u >= (1LL << 31)) return MSS_ERR_UNSUPPORTED;
    const hipError_t e = mss::launch_adamw(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "launching AdamW");
  }
  return MSS_OK;
}


int mss_embed_cm(const int64_t* tokens, int64_t T, const float* E, int32_t V, int32_t D, float* h, int64_t ldh,
                 void* stream) {
  if (!tokens || !E || !h || T <= 0 || T >= (1LL << 31) || V <= 0 || D <= 0 || ldh < T) return MSS_ERR_INVALID_ARGUMENT;
  // (the grid: 64 x 64 tiles of 256 threads, fewer than 2^32 threads)
  if (static_cast<long long>(D) * ldh >= (1LL << 40) || static_cast<long long>(V) * D >= (1LL << 40) ||
      ((T + 63) / 64) * ((D + 63) / 64) >= (1LL << 24))
    return MSS_ERR_UNSUPPORTED;
  if (spans_overlap(h, D, 2 * ldh, 2 * T, E, V, 2LL * D, 2LL * D) || spans_overlap(h, D, 2 * ldh, 2 * T, tokens, 1, 0, 4 * T))
    return MSS_ERR_INVALID_ARGUMENT;
  mss::EmbedParams p{};
  p.T = T;
  p.V = V;
  p.D = D;
  p.ldh = ldh;
  p.tokens = reinterpret_cast<const long long*>(tokens);
  p.E = E;
  p.h = h;
  const hipError_t e = mss::launch_embed_cm(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching embedding gather");
}

int mss_embed_cm_backward(const float* dh, int64_t ldh, const int64_t* sorted_tokens, const int64_t* order, int64_t T,
                          int32_t V, int32_t D, float* dE, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!dh || !sorted_tokens || !order || !dE || !workspace || T <= 0 || T >= (1LL << 31) || V <= 0 || D <= 0 ||
      ldh < T)
    return MSS_ERR_INVALID_ARGUMENT;
  if (D % 4 != 0 || D > mss::kEmbedMaxD) return MSS_ERR_UNSUPPORTED;
  if (static_cast<long long>(D) * ldh >= (1LL << 40) || static_cast<long long>(V) * D >= (1LL << 40) ||
      ((T + 63) / 64) * ((D + 63) / 64) >= (1LL << 24))
    return MSS_ERR_UNSUPPORTED;
  if (!aligned16(dE) || !aligned16(workspace) || workspace_bytes < 4 * T * D) return MSS_ERR_INVALID_ARGUMENT;
  // dE (float32, 2 bf16-sized units per element) against dh and the workspace.
  if (spans_overlap(dE, V, 2LL * D, 2LL * D, dh, D, 2 * ldh, 2 * T) ||
      spans_overlap(dE, V, 2LL * D, 2LL * D, workspace, 1, 0, 2 * T * D) ||
      spans_overlap(workspace, 1, 0, 2 * T * D, dh, D, 2 * ldh, 2 * T))
    return MSS_ERR_INVALID_ARGUMENT;
  mss::EmbedParams p{};
  p.T = T;
  p.V = V;
  p.D = D;
  p.ldh = ldh;
  p.dh = dh;
  p.sorted_tokens = reinterpret_cast<const long long*>(sorted_tokens);
  p.order = reinterpret_cast<const long long*>(order);
  p.work = static_cast<float*>(workspace);
  p.dE = dE;
  const hipError_t e = mss::launch_embed_cm_backward(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching embedding gradient");
}


namespace {
// Validated StepParams of a scan-step call; need_delta false when delta comes from elsewhere.
int step_params(const mss_step_args* a, bool cplx, bool need_delta, mss::StepParams* p) {
  if (a == nullptr) return MSS_ERR_INVALID_ARGUMENT;
  int s = check_dims(a->batch, a->dim, 1, a->dstate);
  if (s != MSS_OK) return s;
  s = check_common(a->discretization, a->delta_softplus, a->io_dtype, a->bc_dtype);
  if (s != MSS_OK) return s;
  if (!a->state || !a->u || (need_delta && !a->delta) || !a->A || !a->B || !a->C || !a->out)
    return MSS_ERR_INVALID_ARGUMENT;
  if (cplx && (!aligned8(a->state) || !aligned8(a->A))) return MSS_ERR_INVALID_ARGUMENT;
  Strides st;
  // Rows of one step: the per-row "length" is 1.
  s = resolve_strides(a->strides, a->batch, a->dim, 1, a->dstate, &st);
  if (s != MSS_OK) return s;
  p->batch = a->batch;
  p->dim = a->dim;
  p->dstate = a->dstate;
  p->delta_softplus = a->delta_softplus;
  p->io_sb = st.io_sb;
  p->io_sd = st.io_sd;
  p->bc_sb = st.bc_sb;
  p->bc_sn = st.bc_sn;
  p->state = a->state;
  p->u = a->u;
  p->delta = a->delta;
  p->z = a->z;
  p->B = a->B;
  p->C = a->C;
  p->A = a->A;
  p->D = a->D;
  p->delta_bias = a->delta_bias;
  p->out = a->out;
  return MSS_OK;
}

int run_scan_step(const mss_step_args* a, void* stream, bool cplx) {
  mss::StepParams p{};
  const int s = step_params(a, cplx, true, &p);
  if (s != MSS_OK) return s;
  const bool zoh = a->discretization == MSS_ZOH;
  const bool io_bf16 = a->io_dtype == MSS_BF16, bc_bf16 = a->bc_dtype == MSS_BF16;
  const hipStream_t st_ = static_cast<hipStream_t>(stream);
  const hipError_t e = cplx ? mss::launch_cssm_step(p, zoh, io_bf16, bc_bf16, st_)
                            : mss::launch_ssm_step(p, zoh, io_bf16, bc_bf16, st_);
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching scan step");
}

// Validated ConvStepParams; need_x false when x comes from elsewhere.
int conv_step_params(const mss_conv_step_args* a, bool need_x, mss::ConvStepParams* p) {
  if (a == nullptr || a->batch <= 0 || a->dim <= 0) return MSS_ERR_INVALID_ARGUMENT;
  if (a->width < 1 || a->width > 4) return MSS_ERR_INVALID_ARGUMENT;
  if (a->io_dtype != MSS_F32 && a->io_dtype != MSS_BF16) return MSS_ERR_INVALID_ARGUMENT;
  if (a->activation != 0 && a->activation != 1) return MSS_ERR_INVALID_ARGUMENT;
  if ((need_x && !a->x) || !a->weight || !a->y || (a->width > 1 && !a->conv_state))
    return MSS_ERR_INVALID_ARGUMENT;
  Strides st;
  const int s = resolve_strides(a->strides, a->batch, a->dim, 1, 1, &st);
  if (s != MSS_OK) return s;
  p->batch = a->batch;
  p->dim = a->dim;
  p->width = a->width;
  p->act = a->activation;
  p->sb = st.io_sb;
  p->sd = st.io_sd;
  p->state = a->conv_state;
  p->x = a->x;
  p->w = a->weight;
  p->bias = a->bias;
  p->y = a->y;
  return MSS_OK;
}

// Validated GemvParams; need_y false when an epilogue replaces every store to Y, need_x
// false when a prologue computes X.
int gemv_params(const mss_gemv_args* a, bool need_y, mss::GemvParams* p, bool need_x = true) {
  if (a == nullptr || a->M <= 0 || a->K <= 0 || a->K % 8 != 0) return MSS_ERR_INVALID_ARGUMENT;
  if (a->N != 1 && a->N != 2 && a->N != 4 && a->N != 8) return MSS_ERR_UNSUPPORTED;
  if (a->ldw < a->K || a->ldw % 8 != 0 || !a->W || (need_x && !a->X) || (need_y && !a->Y))
    return MSS_ERR_INVALID_ARGUMENT;
  if (!aligned16(a->W) || (need_x && !aligned16(a->X)) || reinterpret_cast<uintptr_t>(a->Y) % 2 != 0)
    return MSS_ERR_INVALID_ARGUMENT;
  if (static_cast<long long>(a->K) * a->N * 2 > 65536) return MSS_ERR_UNSUPPORTED;  // X staged in LDS
  p->M = a->M;
  p->K = a->K;
  p->N = a->N;
  p->ldw = a->ldw;
  p->W = a->W;
  p->X = a->X;
  p->Y = a->Y;
  return MSS_OK;
}

int run_gemv(const mss::GemvParams& p, void* stream) {
  const hipError_t e = mss::launch_gemv(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching gemv");
}
}  // namespace

int mss_scan_step(const mss_step_args* a, void* stream) { return run_scan_step(a, stream, false); }

int mss_cscan_step(const mss_step_args* a, void* stream) { return run_scan_step(a, stream, true); }

int mss_conv_step(const mss_conv_step_args* a, void* stream) {
  mss::ConvStepParams p{};
  const int s = conv_step_params(a, true, &p);
  if (s != MSS_OK) return s;
  const hipError_t e = mss::launch_conv_step(p, a->io_dtype == MSS_BF16, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSS_OK : hip_fail(e, "launching conv step");
}

int mss_gemv(const mss_gemv_args* a, void* stream) {
  mss::GemvParams p{};
  const int s = gemv_params(a, true, &p);
  return s != MSS_OK ? s : run_gemv(p, stream);
}

namespace {
// GemvParams of a GEMM with the conv-window step fused on its first conv->dim rows.
int gemv_conv_params(const mss_gemv_args* g, const mss_conv_step_args* c, bool need_x, mss::GemvParams* p) {
  if (g == nullptr || c == nullptr) return MSS_ERR_INVALID_ARGUMENT;
  int s = gemv_params(g, c->dim < g->M, p, need_x);
  if (s == MSS_OK) s = conv_step_params(c, false, &p->cs);
  if (s != MSS_OK) return s;
  if (c->io_dtype != MSS_BF16 || c->batch != g->N || c->dim > g->M) return MSS_ERR_INVALID_ARGUMENT;
  // the fused kernel indexes the step's operands with int offsets
  const long long span = (c->batch - 1LL) * p->cs.sb + (c->dim - 1LL) * p->cs.sd;
  if (span >= (1LL << 31) || static_cast<long long>(c->batch) * c->dim * c->width >= (1LL << 31))
    return MSS_ERR_UNSUPPORTED;
  p->epi = 1;
  return MSS_OK;
}

bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return a != nullptr && b != nullptr && x < y + nb && y < x + na;
}
}  // namespace

int mss_gemv_conv_step(const mss_gemv_args* g, const mss_conv_step_args* c, void* stream) {
  mss::GemvParams p{};
  const int s = gemv_conv_params(g, c, true, &p);
  return s != MSS_OK ? s : run_gemv(p, stream);
}

int mss_norm_gemv_conv_step(const mss_norm_args* n, const mss_gemv_args* g, const mss_conv_step_args* c,
                            void* stream) {
  if (n == nullptr) return MSS_ERR_INVALID_ARGUMENT;
  mss::GemvParams p{};
  const int s = gemv_conv_params(g, c, false, &p);
  if (s != MSS_OK) return s;
  if (n->features != g->K || n->tokens != g->N || n->io_dtype != MSS_BF16 || !(n->eps >= 0.f) || !n->h ||
      !n->weight || (n->delta && !n->hn))
    return MSS_ERR_INVALID_ARGUMENT;
  if (!aligned16(n->h) || !aligned16(n->delta) || !aligned16(n->hn)) return MSS_ERR_INVALID_ARGUMENT;
  // workgroup 0 writes hn while the others still read h and delta
  const size_t stream_bytes = static_cast<size_t>(n->features) * n->tokens * sizeof(float);
  if (n->delta && (overlaps(n->hn, stream_bytes, n->h, stream_bytes) ||
                   overlaps(n->hn, stream_bytes, n->delta, stream_bytes / 2)))
    return MSS_ERR_INVALID_ARGUMENT;
  static_assert(mss::kNormGemvMaxFeatures == MSS_NORM_GEMV_MAX_FEATURES, "header and kernel disagree");
  if (n->features > MSS_NORM_GEMV_MAX_FEATURES) return MSS_ERR_UNSUPPORTED;
  p.norm = 1;
  p.nm.features = n->features;
  p.nm.tokens = n->tokens;
  p.nm.eps = n->eps;
  p.nm.h = n->h;
  p.nm.delta = n->delta;
  p.nm.w = n->weight;
  p.nm.hn = n->hn;
  p.nm.rstd = n->rstd;
  return run_gemv(p, stream);
}

int mss_gemv_scan_step(const mss_gemv_args* g, const mss_step_args* a, void* stream) {
  if (g == nullptr || a == nullptr) return MSS_ERR_INVALID_ARGUMENT;
  mss::GemvParams p{};
  int s = gemv_params(g, false, &p);
  if (s == MSS_OK) s = step_params(a, false, false, &p.ss);
  if (s != MSS_OK) return s;
  if (a->io_dtype != MSS_BF16 || a->bc_dtype != MSS_BF16 || a->batch != g->N || a->dim != g->M)
    return MSS_ERR_INVALID_ARGUMENT;
  // the fused kernel indexes the step's operands with int offsets
  const mss::StepParams& q = p.ss;
  const long long io_span = (q.batch - 1LL) * q.io_sb + (q.dim - 1LL) * q.io_sd;
  const long long bc_span = (q.batch - 1LL) * q.bc_sb + (q.dstate - 1LL) * q.bc_sn;
  if (io_span >= (1LL << 31) || bc_span >= (1LL << 31) ||
      static_cast<long long>(q.batch) * q.dim * q.dstate >= (1LL << 31))
    return MSS_ERR_UNSUPPORTED;
  p.epi = 2;
  p.zoh = a->discretization == MSS_ZOH;
  return run_gemv(p, stream);
}

int mss_scan_fwd_repeat(void* stream, int32_t discretization, int32_t repeats, int32_t batch,
                        int32_t length, int32_t dim, int32_t dstate, const float* A,
                        const float* deltas, const float* B, const float* C, const float* u,
                        const float* initial_x, float* y, float* final_x, float* chunk_states) {
  if (repeats <= 0) return MSS_ERR_INVALID_ARGUMENT;
  int s = check_dims(batch, dim, length, dstate, MSS_MAX_DSTATE_WIDE);
  if (s != MSS_OK) return s;
  if (discretization != MSS_EULER && discretization != MSS_ZOH) return MSS_ERR_INVALID_ARGUMENT;
  if (!A || !deltas || !B || !C || !u || !initial_x || !y || !final_x || !chunk_states)
    return MSS_ERR_INVALID_ARGUMENT;
  mss_fwd_args a{};
  a.batch = batch;
  a.dim = dim;
  a.seqlen = length;
  a.dstate = dstate;
  a.discretization = discretization;
  a.io_dtype = MSS_F32;
  a.bc_dtype = MSS_F32;
  a.u = u;
  a.delta = deltas;
  a.A = A;
  a.B = B;
  a.C = C;
  a.initial_state = initial_x;
  a.out = y;
  a.last_state = final_x;
  for (int r = 0; r < repeats; ++r) {
    s = run_fwd(&a, chunk_states, static_cast<hipStream_t>(stream));
    if (s != MSS_OK) return s;
  }
  return MSS_OK;
}

int mss_scan_fwd(void* stream, int32_t discretization, int32_t batch, int32_t length, int32_t dim,
                 int32_t dstate, const float* A, const float* deltas, const float* B,
                 const float* C, const float* u, const float* initial_x, float* y, float* final_x,
                 float* chunk_states) {
  return mss_scan_fwd_repeat(stream, discretization, 1, batch, length, dim, dstate, A, deltas, B, C,
                             u, initial_x, y, final_x, chunk_states);
}

// Workspace of mss_scan_bwd_ws: the 8-step state carries, then mss_bwd's workspace.
static size_t scan_bwd_carry_bytes(int32_t batch, int32_t length, int32_t dim, int32_t dstate) {
  const size_t b = static_cast<size_t>(batch) * dim * dstate * n_seg_of(length) * sizeof(float);
  return (b + 255) / 256 * 256;
}

size_t mss_scan_bwd_workspace_bytes(int32_t batch, int32_t length, int32_t dim, int32_t dstate) {
  if (check_dims(batch, dim, length, dstate, MSS_MAX_DSTATE_WIDE) != MSS_OK) return 0;
  return scan_bwd_carry_bytes(batch, length, dim, dstate) + bwd_layout_call(batch, dim, length, dstate, false).total;
}

int mss_scan_bwd_ws(void* stream, int32_t batch, int32_t length, int32_t dim, int32_t dstate,
                    const float* A, const float* deltas, const float* B, const float* C,
                    const float* u, const float* initial_x, const float* chunk_states,
                    const float* dout, const float* dfinal_x, float* dA, float* ddeltas, float* dB,
                    float* dC, float* du, float* dinitial_x, void* workspace, size_t workspace_bytes) {
  int s = check_dims(batch, dim, length, dstate, MSS_MAX_DSTATE_WIDE);
  if (s != MSS_OK) return s;
  if (!A || !deltas || !B || !C || !u || !initial_x || !chunk_states || !dout || !dfinal_x || !dA ||
      !ddeltas || !dB || !dC || !du || !dinitial_x)
    return MSS_ERR_INVALID_ARGUMENT;
  // The carry rebuild runs one grid slice per 2048-step block (grid.z).
  if ((length + MSS_REF_CHUNK - 1) / MSS_REF_CHUNK > 65535) return MSS_ERR_UNSUPPORTED;
  if (workspace == nullptr || !aligned16(workspace) ||
      workspace_bytes < mss_scan_bwd_workspace_bytes(batch, length, dim, dstate))
    return MSS_ERR_WORKSPACE;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* carries = reinterpret_cast<float*>(ws);
  const size_t carry_bytes = scan_bwd_carry_bytes(batch, length, dim, dstate);
  // The backward re-runs each 8-step segment from the state entering it; the reference
  // residual holds the state at 2048-step block ends only, so each block's recurrence is
  // re-run from it first (one state pass, blocks in parallel).
  mss::FwdParams p{};
  p.batch = batch;
  p.dim = dim;
  p.seqlen = length;
  p.dstate = dstate;
  const size_t row = static_cast<size_t>(length) * sizeof(float);
  p.vec_io = (row % 16 == 0) && aligned16(u) && aligned16(deltas);
  p.vec_bc = (row % 16 == 0) && aligned16(B);
  p.n_seg = n_seg_of(length);
  p.n_ref = (length + MSS_REF_CHUNK - 1) / MSS_REF_CHUNK;
  p.u = u;
  p.delta = deltas;
  p.A = A;
  p.B = B;
  p.x0 = initial_x;
  p.ref_states = const_cast<float*>(chunk_states);
  p.carries = carries;
  hipError_t e = mss::launch_carry_rebuild(p, st);
  if (e != hipSuccess) return hip_fail(e, "launching carry rebuild");
  mss_bwd_args a{};
  a.batch = batch;
  a.dim = dim;
  a.seqlen = length;
  a.dstate = dstate;
  a.io_dtype = MSS_F32;
  a.bc_dtype = MSS_F32;
  a.u = u;
  a.delta = deltas;
  a.A = A;
  a.B = B;
  a.C = C;
  a.initial_state = initial_x;
  a.carries = carries;
  a.dout = dout;
  a.dlast_state = dfinal_x;
  a.du = du;
  a.ddelta = ddeltas;
  a.dA = dA;
  a.dB = dB;
  a.dC = dC;
  a.dinitial_state = dinitial_x;
  a.workspace = ws + carry_bytes;
  a.workspace_bytes = workspace_bytes - carry_bytes;
  return run_bwd(&a, kPhaseBoth, st);
}

int mss_scan_bwd(void* stream, int32_t batch, int32_t length, int32_t dim, int32_t dstate,
                 const float* A, const float* deltas, const float* B, const float* C,
                 const float* u, const float* initial_x, const float* chunk_states,
                 const float* dout, const float* dfinal_x, float* dA, float* ddeltas, float* dB,
                 float* dC, float* du, float* dinitial_x) {
  int s = check_dims(batch, dim, length, dstate, MSS_MAX_DSTATE_WIDE);
  if (s != MSS_OK) return s;
  if (!A || !deltas || !B || !C || !u || !initial_x || !chunk_states || !dout || !dfinal_x || !dA ||
      !ddeltas || !dB || !dC || !du || !dinitial_x)
    return MSS_ERR_INVALID_ARGUMENT;
  if ((length + MSS_REF_CHUNK - 1) / MSS_REF_CHUNK > 65535) return MSS_ERR_UNSUPPORTED;
  // The reference signature has no workspace operand: one stream-ordered allocation per call
  // (mss_scan_bwd_ws takes a caller's workspace and allocates nothing).
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t bytes = mss_scan_bwd_workspace_bytes(batch, length, dim, dstate);
  void* ws = nullptr;
  hipError_t e = hipMallocAsync(&ws, bytes, st);
  if (e != hipSuccess) return hip_fail(e, "allocating backward workspace");
  s = mss_scan_bwd_ws(stream, batch, length, dim, dstate, A, deltas, B, C, u, initial_x, chunk_states, dout,
                      dfinal_x, dA, ddeltas, dB, dC, du, dinitial_x, ws, bytes);
  e = hipFreeAsync(ws, st);
  if (s != MSS_OK) return s;
  return e == hipSuccess ? MSS_OK : hip_fail(e, "freeing backward workspace");
}

}  // extern "C"
