/*
 * mamba_selective_scan.h — C ABI of the MI355X (gfx950) Mamba-1 selective-scan engine.
 *
 * Library: libmamba_selective_scan_hip.so (built from jax-mambas_amd/csrc/).
 *
 * Everything here is plain C: pointers, sizes and int32 flags. Tensors are device
 * pointers in the physical layout the reference's kernel boundary uses (reference
 * mamba/selective_scan_cuda.py:135-147 declares XLA layouts (0,2,1), i.e. channel-major
 * [B][D][L] for u/delta/z/out and [B][N][L] for B/C). The fused entry points also take
 * row strides (mss_strides): steps are always contiguous, but rows may be laid out as
 * e.g. [D][B][L] — the layout of a (D, B*L) activation matrix, which lets a model keep
 * every projection a plain 2-D GEMM with no transposes around the scan:
 *
 *   u, delta, z, out, du, ddelta, dz, dout : [batch][dim][seqlen]
 *   B, C, dB, dC                          : [batch][dstate][seqlen]
 *   A, dA                                 : [dim][dstate]            (float32)
 *   D, dD, delta_bias, ddelta_bias        : [dim]                    (float32)
 *   initial_state, last_state, dlast_state, dinitial_state : [batch][dim][dstate] (float32)
 *   seq_lens                              : [batch] int32 (optional variable lengths)
 *   carries                               : [batch][dim][dstate][ceil(seqlen/8)] float32
 *                                           state h entering every 8-step segment
 *                                           (segment 0: initial_state)
 *   y_pre                                 : [batch][dim][seqlen] y before the z gate (real A:
 *                                           only where |z| < 1e-20; other elements unwritten)
 *   (carries and y_pre are residuals for the backward: with seq_lens, their values in
 *   512-step chunks past a row's length are unspecified; the backward does not read them)
 *
 * All entry points are asynchronous on the given stream (a hipStream_t passed as
 * void*; NULL = the default stream), re-entrant, and validate every argument before
 * any HIP call, returning an mss_status code (never throwing across the ABI).
 *
 * Semantics (per batch b, channel d, state n, step t):
 *   delta_t = delta_raw_t + bias_d;  if delta_softplus: delta_t = softplus(delta_t)
 *             (identity above 20);  delta_t = 0 for t >= seq_lens[b]
 *   a_bar   = exp(delta_t * A_dn)
 *   Euler:  bu = delta_t * B_nt * u_t      ZOH: bu = expm1(delta_t*A_dn)/A_dn * B_nt * u_t
 *   h_t     = a_bar * h_{t-1} + bu,  h_{-1} = initial_state (0 if NULL)
 *   y_t     = sum_n C_nt h_t + D_d u_t;   out_t = y_t * silu(z_t) (if z);  out_t = 0 for t >= len
 *   last_state = h at the final step.
 */
#ifndef MAMBA_SELECTIVE_SCAN_H_
#define MAMBA_SELECTIVE_SCAN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSS_ABI_VERSION 16
/* dstate limits (MSS_ERR_UNSUPPORTED beyond, MSS_ERR_INVALID_ARGUMENT beyond 256):
 * MSS_MAX_DSTATE_WIDE for the float32 real-A scans — mss_fwd / mss_bwd / mss_bwd_noalloc with
 * io and bc dtype MSS_F32, and the reference-signature mss_scan_* entry points (whose C
 * handlers accept N <= 256, reference native/selective_scan_cuda.cu:34, 410-411); their
 * backward runs over groups of at most MSS_MAX_DSTATE states, so mss_bwd_scan /
 * mss_bwd_reduce (split phases) stay at MSS_MAX_DSTATE. MSS_MAX_DSTATE for bf16 scans, the
 * complex-A scan, the decode steps and the split phases. */
#define MSS_MAX_DSTATE 16
#define MSS_MAX_DSTATE_WIDE 256
#define MSS_SEG_STEPS 8     /* step granularity of the `carries` residual */
#define MSS_REF_CHUNK 2048   /* step granularity of the reference's chunk_states */
#define MSS_NOALLOC_SCRATCH_BYTES (128u << 20) /* fixed per-device scratch of mss_bwd_noalloc */
#define MSS_NORM_GEMV_MAX_FEATURES 1024 /* largest norm->features of mss_norm_gemv_conv_step */
#define MSS_XENT_FUSED_MAX_VOCAB 65536 /* largest vocab of mss_xent_fwd_grad */

typedef enum mss_status {
  MSS_OK = 0,
  MSS_ERR_INVALID_ARGUMENT = 1, /* bad shape, null required pointer, bad flag */
  MSS_ERR_UNSUPPORTED = 2,      /* valid request this build does not implement */
  MSS_ERR_HIP = 3,              /* a HIP runtime call failed; see mss_last_hip_error */
  MSS_ERR_WORKSPACE = 4,        /* caller workspace too small */
  MSS_ERR_SCRATCH_LIMIT = 5     /* mss_bwd_noalloc: shapes need more than its fixed scratch */
} mss_status;

typedef enum mss_dtype { MSS_F32 = 0, MSS_BF16 = 1 } mss_dtype;
typedef enum mss_discretization { MSS_EULER = 0, MSS_ZOH = 1 } mss_discretization;

/* Row strides, in elements, of the fused entry points' tensors. The step axis is always
 * contiguous. 0 selects the contiguous default. Rows must not overlap. */
typedef struct mss_strides {
  int64_t io_batch; /* u, delta, z, out, y_pre, dout, du, ddelta, dz: (b,d)->(b+1,d); default dim*seqlen */
  int64_t io_dim;   /* (b,d) -> (b,d+1); default seqlen */
  int64_t bc_batch; /* B, C, dB, dC: (b,n) -> (b+1,n); default dstate*seqlen */
  int64_t bc_state; /* (b,n) -> (b,n+1); default seqlen */
} mss_strides;

/* Forward of the fused scan (no counterpart symbol in the reference: it generalises
 * MambaSelectiveScan, native/selective_scan_cuda.cu:554-573, with the fusions the
 * reference model applies around the scan, mamba/mamba1.py:160-198, 300-337). */
typedef struct mss_fwd_args {
  int32_t batch, dim, seqlen, dstate;
  int32_t discretization; /* mss_discretization */
  int32_t delta_softplus; /* 0 / 1 */
  int32_t io_dtype;       /* dtype of u, delta, z, out */
  int32_t bc_dtype;       /* dtype of B, C */
  const void* u;
  const void* delta;
  const float* A;
  const void* B;
  const void* C;
  const float* D;             /* optional */
  const void* z;              /* optional */
  const float* delta_bias;    /* optional */
  const float* initial_state; /* optional */
  const int32_t* seq_lens;    /* optional */
  void* out;
  float* last_state; /* optional */
  float* carries;    /* optional; required by mss_bwd */
  void* y_pre;       /* optional [B][D][L] (io dtype, io strides): y before the silu(z)
                        gate, the residual mss_bwd needs when z is given. Real A: written
                        only where |z| < 1e-20 (mss_bwd takes y sigma(z) from out / z
                        elsewhere); complex A (mss_cfwd): written everywhere */
  mss_strides strides;
} mss_fwd_args;

/* Backward of the fused scan. Outputs are fully overwritten (no accumulation).
 * dA/dD/dB/dC/ddelta_bias are deterministic sums over batch and channels up to the
 * order of fp32 adds inside one workgroup. */
typedef struct mss_bwd_args {
  int32_t batch, dim, seqlen, dstate;
  int32_t discretization;
  int32_t delta_softplus;
  int32_t io_dtype; /* dtype of u, delta, z, dout, du, ddelta, dz */
  int32_t bc_dtype; /* dtype of B, C, dB, dC */
  const void* u;
  const void* delta;
  const float* A;
  const void* B;
  const void* C;
  const float* D;
  const void* z;
  const float* delta_bias;
  const float* initial_state;
  const int32_t* seq_lens;
  const float* carries;     /* from mss_fwd with the same inputs; required */
  const void* y_pre;        /* from mss_fwd; required iff z given */
  const void* out;          /* mss_fwd's out; required iff z given (real A; unused by mss_cbwd) */
  const void* dout;
  const float* dlast_state; /* optional cotangent of last_state */
  void* du;
  void* ddelta;
  float* dA;
  void* dB;
  void* dC;
  float* dD;             /* required iff D given */
  void* dz;              /* required iff z given */
  float* ddelta_bias;    /* required iff delta_bias given */
  float* dinitial_state; /* optional */
  void* workspace;       /* device scratch; NULL = library allocates stream-ordered */
  size_t workspace_bytes;
  mss_strides strides;   /* the forward's strides; also those of dout/du/ddelta/dz, dB/dC */
} mss_bwd_args;

/* Size of the scratch mss_bwd needs for these shapes and for whether seq_lens is given
 * (0 on invalid arguments). */
size_t mss_bwd_workspace_bytes(const mss_bwd_args* args);

/* Launch plan mss_bwd would use for these arguments: waves per workgroup of the backward
 * scan kernel and channels one workgroup walks (it depends on the shapes and on whether
 * seq_lens is given). Validates like mss_bwd; launches nothing. No counterpart in the
 * reference, whose backward launch shape is fixed by its traits
 * (native/upstream_mamba/selective_scan_bwd_kernel.cuh:499-535). */
int mss_bwd_plan(const mss_bwd_args* args, int32_t* waves, int32_t* chan_per_block);

int mss_fwd(const mss_fwd_args* args, void* stream);
int mss_bwd(const mss_bwd_args* args, void* stream);

/* mss_bwd without any allocation, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. args->workspace is ignored: the workspace is a fixed
 * per-device array of MSS_NOALLOC_SCRATCH_BYTES inside the library, held by every device
 * the library runs this entry point on until the process ends. Shapes whose workspace
 * (mss_bwd_workspace_bytes) exceeds it return MSS_ERR_SCRATCH_LIMIT before any launch.
 * Results equal mss_bwd's bit for bit (same kernels, same plan). All calls on one device
 * share the one array: calls whose executions overlap on a device (concurrent streams, or
 * threads) race and must be serialised by the caller. The array's device address is looked
 * up once per device and kept for the life of the process: after hipDeviceReset on a device
 * (which unloads the library's code objects) this entry point must not be called there. */
int mss_bwd_noalloc(const mss_bwd_args* args, void* stream);

/* mss_bwd in two stream-ordered phases sharing a caller-provided workspace (NULL ->
 * MSS_ERR_WORKSPACE): mss_bwd_scan writes du/ddelta/dz/dinitial_state and per-block
 * partial sums of dA/dB/dC/dD/ddelta_bias into the workspace; mss_bwd_reduce sums the
 * partials in a fixed order into dA/dB/dC/dD/ddelta_bias. mss_bwd == scan then reduce.
 * Both phases take the same arguments (the reduction reads seq_lens: no partials are written
 * for 512-step chunks past a row's length, whose dB/dC steps it sets to zero).
 * (The reference backward, native/selective_scan_bwd.cu:166-190, is one call; the split
 * lets a caller time or defer the cross-channel reduction.) */
int mss_bwd_scan(const mss_bwd_args* args, void* stream);
int mss_bwd_reduce(const mss_bwd_args* args, void* stream);

/* --- Complex-A scan (complex SSM). -------------------------------------------------
 * Replaces the complex_ssm branch of S6.__call__ (reference mamba/mamba1.py:143-176,
 * 195-198; no FFI symbol there: it runs as jax.lax.associative_scan over complex64 states
 * and is differentiated by JAX autodiff). Same argument blocks as mss_fwd / mss_bwd, with
 * complex tensors stored as interleaved (real, imaginary) float32 pairs (complex64 memory):
 *   A, dA                                 : [dim][dstate][2]
 *   initial_state, last_state, dlast_state, dinitial_state : [batch][dim][dstate][2]
 *   carries                               : [batch][dim][dstate][ceil(seqlen/8)][2]
 * (A, the state buffers and carries 8-byte aligned). Semantics as at the top of this file
 * with complex a_bar = exp(delta A), ZOH b_bar = expm1(delta A)/A * B, complex h, and
 * y_t = sum_n C_nt Re(h_t) + D_d u_t. The reference's A = -exp(A_log.real) + i*A_imag
 * parameterisation (mamba/mamba1.py:162) is the caller's. Gradients of complex inputs are
 * (dL/dRe, dL/dIm) of the real loss; dlast_state is read in the same convention.
 * mss_cbwd allocates its workspace (stream-ordered) when args->workspace is NULL; size
 * from mss_cbwd_workspace_bytes. dB/dC sums inside one workgroup use a fixed order. */
size_t mss_cbwd_workspace_bytes(const mss_bwd_args* args);
int mss_cfwd(const mss_fwd_args* args, void* stream);
int mss_cbwd(const mss_bwd_args* args, void* stream);

/* --- Causal depthwise conv1d + activation (the Mamba-1 block's short convolution). ---
 * No counterpart symbol in the reference: it runs there as an XLA convolution
 * (mamba/mamba1.py:250-255, 313-329: nnx.Conv(feature_group_count=channels,
 * padding="CAUSAL"), then silu, with the padding mask applied before and after).
 * Rows of x/y/dy/dx use the io strides of `strides` (bc strides unused):
 *   pre[t] = bias[d] + sum_{k<width} weight[d][k] * x[t - (width-1) + k]   (x[t<0] = 0)
 *   y[t]   = silu(pre[t]) (activation 1) or pre[t] (activation 0);  y[t] = 0 for t >= seq_lens[b]
 * The backward recomputes pre from x and overwrites dx, dweight and dbias. */
typedef struct mss_conv_args {
  int32_t batch, dim, seqlen;
  int32_t width;      /* taps, 1..4 */
  int32_t io_dtype;   /* x, y, dy, dx */
  int32_t activation; /* 0 none, 1 silu */
  const void* x;
  const float* weight;     /* [dim][width] */
  const float* bias;       /* [dim], optional */
  const int32_t* seq_lens; /* optional */
  void* y;                 /* forward output */
  const void* dy;          /* backward inputs / outputs */
  void* dx;
  float* dweight;          /* [dim][width] */
  float* dbias;            /* optional (required iff bias given) */
  void* workspace;         /* backward scratch; NULL = library allocates stream-ordered */
  size_t workspace_bytes;
  mss_strides strides;
} mss_conv_args;

size_t mss_conv_bwd_workspace_bytes(const mss_conv_args* args);
int mss_conv_fwd(const mss_conv_args* args, void* stream);
int mss_conv_bwd(const mss_conv_args* args, void* stream);

/* --- Single-token recurrent step (decode). ----------------------------------------
 * Replaces S6.step / Mamba.step (mamba/mamba1.py:200-214, 339-363; no FFI symbol in the
 * reference). For each (b, d), with the scan's fused extras:
 *   delta = softplus(delta_raw + bias) (if delta_softplus),  a_bar = exp(delta A[d][n]),
 *   state[b][d][n] = a_bar*state + b_bar*u  (Euler b_bar = delta*B, ZOH expm1(delta A)/A*B),
 *   y = sum_n C state + D u,  out = y * silu(z) (if z)
 * state is [batch][dim][dstate] float32, updated in place (the scan's last_state layout).
 * u/delta/z/out are [batch][dim] and B/C [batch][dstate] with the row strides of
 * `strides` (0 = contiguous; e.g. io_batch=1, io_dim=batch for a (dim, batch) matrix). */
typedef struct mss_step_args {
  int32_t batch, dim, dstate;
  int32_t discretization, delta_softplus;
  int32_t io_dtype, bc_dtype;
  float* state;
  const void* u;
  const void* delta;
  const float* A;
  const void* B;
  const void* C;
  const float* D;          /* optional */
  const void* z;           /* optional */
  const float* delta_bias; /* optional */
  void* out;
  mss_strides strides;
} mss_step_args;

int mss_scan_step(const mss_step_args* args, void* stream);

/* mss_scan_step with complex A (the complex branch of S6.step, mamba/mamba1.py:200-214):
 * A [dim][dstate][2] and state [batch][dim][dstate][2] as interleaved (real, imaginary)
 * float32 pairs, 8-byte aligned (the complex scan's last_state layout); the state is
 * updated in place and out = (sum_n C Re(state) + D u) * silu(z). */
int mss_cscan_step(const mss_step_args* args, void* stream);

/* Causal-conv window update for one token: window = [conv_state[b][d][0..width-2], x];
 * y = act(bias + sum_k weight[d][k] window[k]); conv_state shifts left and takes x.
 * conv_state is [batch][dim][width-1] in the activation dtype, updated in place; x/y use
 * the io strides of `strides`. */
typedef struct mss_conv_step_args {
  int32_t batch, dim, width, io_dtype, activation;
  void* conv_state;
  const void* x;
  const float* weight; /* [dim][width] */
  const float* bias;   /* optional */
  void* y;
  mss_strides strides;
} mss_conv_step_args;

int mss_conv_step(const mss_conv_step_args* args, void* stream);

/* --- Decode-shaped GEMM: Y = W X. -------------------------------------------------------
 * No counterpart symbol in the reference (its decode step, mamba/mamba1.py:200-214,
 * 339-363, runs the block's projections as XLA dot products). W [M][K] bf16 with row
 * stride ldw (16-byte aligned, ldw >= K, ldw % 8 == 0); X [K][N] bf16 (16-byte aligned)
 * and Y [M][N] bf16 with rows of N contiguous values; K % 8 == 0; N in {1, 2, 4, 8} and
 * 2*K*N <= 65536 bytes (X is staged in LDS; MSS_ERR_UNSUPPORTED otherwise). Float32
 * accumulation, Y rounded to bf16 once. */
typedef struct mss_gemv_args {
  int32_t M, K, N;
  int64_t ldw;
  const void* W;
  const void* X;
  void* Y;
} mss_gemv_args;

int mss_gemv(const mss_gemv_args* args, void* stream);

/* mss_gemv with the next decode step fused behind it (no counterpart symbol in the
 * reference: Mamba.step, mamba/mamba1.py:339-363, applies the conv window and S6.step,
 * :200-214, to the projections' outputs). Each entry computes the products with float32
 * sums rounded to bf16 once, then, instead of storing some rows of Y, applies the step to
 * those bf16 rows exactly as the separate step call would (bit for bit, given the same rows).
 * The rows themselves equal mss_gemv's bit for bit except where the fused entry sums on the
 * matrix cores and mss_gemv does not: mss_gemv_conv_step (and mss_norm_gemv_conv_step) with
 * K % 64 == 0 and M below 4096 rows, where the two summation orders can leave a row one
 * bf16 rounding apart.
 *
 * mss_gemv_conv_step: rows [0, conv->dim) of W X are conv->x (ignored, may be null) of
 * mss_conv_step: conv_state and conv->y are updated as that call would, and those rows of
 * Y are not written (Y may be null when conv->dim == M). conv->batch == N, conv->dim <= M,
 * io_dtype MSS_BF16.
 *
 * mss_gemv_scan_step: W X is step->delta (ignored, may be null) of mss_scan_step (real A):
 * state and step->out are updated as that call would; Y is not written (may be null).
 * step->batch == N, step->dim == M, io_dtype and bc_dtype MSS_BF16. */
int mss_gemv_conv_step(const mss_gemv_args* gemv, const mss_conv_step_args* conv, void* stream);
int mss_gemv_scan_step(const mss_gemv_args* gemv, const mss_step_args* step, void* stream);

/* --- Residual add + RMSNorm over the features of a channel-major stream. ----------
 * No counterpart symbol in the reference (mamba/mamba1.py:300-337 applies
 * nnx.RMSNorm(epsilon) to the residual stream and adds each block's output back).
 * Matrices are [features][tokens], row-major (tokens contiguous):
 *   forward   hn = h + delta (delta optional; hn written only then),
 *             rstd[t] = 1/sqrt(mean_f hn^2 + eps),  x = hn * rstd * w
 *   backward  xhat = hn*rstd,  c = mean_f w dx xhat,
 *             dhn = dhn_in + rstd*(w dx - xhat c)  (dhn_in optional), ddelta = dhn in the
 *             activation dtype (optional), dw = sum_t dx xhat. */
typedef struct mss_norm_args {
  int32_t features, tokens;
  float eps;
  int32_t io_dtype;    /* dtype of delta, x, dx, ddelta (the stream h/hn/dhn is float32) */
  const float* h;      /* forward input; backward: the forward's normalised input (hn) */
  const void* delta;   /* optional */
  const float* weight; /* [features] */
  float* hn;           /* written when delta is given */
  void* x;
  float* rstd;         /* [tokens] */
  const void* dx;      /* backward */
  const float* dhn_in; /* optional */
  float* dhn;
  void* ddelta;        /* optional */
  float* dweight;
  void* workspace;     /* NULL = library allocates stream-ordered */
  size_t workspace_bytes;
} mss_norm_args;

size_t mss_norm_bwd_workspace_bytes(const mss_norm_args* args);
int mss_norm_fwd(const mss_norm_args* args, void* stream);
int mss_norm_bwd(const mss_norm_args* args, void* stream);

/* mss_norm_fwd followed by mss_gemv_conv_step on its output, as one launch (no counterpart
 * symbol in the reference: Mamba.step, mamba/mamba1.py:339-363, normalises the residual
 * stream and feeds it to the in-projection, whose first rows go through the conv window).
 * A decode step's block entry: the results (norm->hn, norm->rstd when not NULL,
 * conv_state, conv->y and the rows of gemv->Y past conv->dim) equal those two calls bit
 * for bit; norm->x and gemv->X are ignored (may be NULL): every workgroup recomputes the
 * normalised tokens. norm->features == gemv->K <= MSS_NORM_GEMV_MAX_FEATURES
 * (MSS_ERR_UNSUPPORTED above),
 * norm->tokens == gemv->N, io_dtype MSS_BF16, h/delta/hn 16-byte aligned, hn not
 * overlapping h or delta; the conv and GEMM conditions of mss_gemv_conv_step. */
int mss_norm_gemv_conv_step(const mss_norm_args* norm, const mss_gemv_args* gemv,
                            const mss_conv_step_args* conv, void* stream);

/* --- Cross-entropy over bf16 logits [rows][vocab] with fp32 math. -------------------
 * No counterpart symbol in the reference (its training loss is optax softmax
 * cross-entropy, experiments/mamba_inductionheads.py:129-136):
 *   forward   lse[r] = log sum_v exp(z[r][v]),  loss[r] = lse[r] - z[r][target[r]]
 *             (NaN for a target outside [0, vocab))
 *   backward  dz[r][v] = (*grad_scale) * (softmax(z[r])[v] - [v == target[r]])  (bf16) */
typedef struct mss_xent_args {
  int32_t rows, vocab;
  const void* logits;        /* bf16 */
  const int64_t* targets;    /* [rows] */
  float* loss;               /* [rows] */
  float* lse;                /* [rows] */
  const float* grad_scale;   /* backward: device scalar */
  void* dlogits;             /* backward: bf16 */
} mss_xent_args;

int mss_xent_fwd(const mss_xent_args* args, void* stream);
int mss_xent_bwd(const mss_xent_args* args, void* stream);

/* Forward and backward in one pass over the logits (each row read once), for a loss that
 * will be differentiated: loss and lse as mss_xent_fwd (the row's float32 partial sums
 * merged in another fixed order, so within a few units of the last place of its lse), and
 * dlogits = (*grad_scale) * (softmax - onehot) as mss_xent_bwd computes it from that lse. vocab % 8 == 0 and vocab <= MSS_XENT_FUSED_MAX_VOCAB, logits and dlogits 16-byte aligned and not
 * overlapping; MSS_ERR_UNSUPPORTED for other shapes.
 * mss_xent_rescale multiplies n bf16 values by *factor (a device scalar, e.g. the upstream
 * gradient of the loss), rounding once, and does nothing when *factor == 1. */
int mss_xent_fwd_grad(const mss_xent_args* args, void* stream);
int mss_xent_rescale(void* dlogits, int64_t n, const float* factor, void* stream);

/* --- Skinny projection GEMMs of the training step (bf16, float32 sums). ------------
 * No counterpart symbol in the reference: its S6 input projections (s_B, s_C, Linear_R:
 * d_inner -> R + 2N; Linear_Delta: R -> d_inner, mamba/mamba1.py:52-67, 107-124) run as
 * XLA dot products. Matrices are row-major; activations channel-major [features][tokens].
 *
 * mss_proj: C[M][T] = W[M][K] X[K][T] (+ C when accumulate != 0, the old C read as bf16 and
 * the sum rounded once), C rounded to bf16. With w_trans != 0 the weight is passed as its
 * transpose, W^T [K][M] with row stride ldw >= M (e.g. the input-gradient products W^T dY
 * from the stored W). M % 16 == 0, T % 64 == 0, and either K <= 128 with K % 16 == 0, or
 * K % 64 == 0 with M <= 128; W, X, C 16-byte aligned with ldw, ldx, ldc multiples of 8
 * (elements); C overlapping neither W nor X. MSS_ERR_UNSUPPORTED for other shapes. */
typedef struct mss_proj_args {
  int32_t M, K, T, accumulate, w_trans;
  int64_t ldw, ldx, ldc;
  const void* W;
  const void* X;
  void* C;
} mss_proj_args;

int mss_proj(const mss_proj_args* args, void* stream);

/* --- Weight-gradient GEMM of the training step (bf16 operands, float32 output). -------
 * No counterpart symbol in the reference: the gradients of its block projections
 * (mamba/mamba1.py:52-67, 107-124, 272-276, 330-337) are XLA dot products.
 *
 * mss_wgrad: C[M][N] = A[M][K] B[N][K]^T (+ C when accumulate != 0), float32, i.e.
 * dW = dY X^T over channel-major activations (rows contiguous along K, the tokens).
 * N a multiple of 4, K a multiple of 64 (192 x 192 output tiles, partial at the edges);
 * A, B 16-byte aligned with lda, ldb >= K,
 * multiples of 8 (elements); C 16-byte aligned with ldc >= N, a multiple of 4; C overlapping
 * neither operand nor the workspace. The tokens are split over workgroups and the partial
 * tiles added in a fixed order (results do not depend on timing): `workspace` holds
 * mss_wgrad_workspace_bytes(M, N, K) bytes, 16-byte aligned (may be NULL when that is 0).
 * MSS_ERR_UNSUPPORTED for other shapes (mss_wgrad_workspace_bytes returns 0 for them). */
typedef struct mss_wgrad_args {
  int32_t M, N, K, accumulate;
  int64_t lda, ldb, ldc;
  const void* A;
  const void* B;
  float* C;
  void* workspace;
  int64_t workspace_bytes;
} mss_wgrad_args;

int64_t mss_wgrad_workspace_bytes(int32_t M, int32_t N, int32_t K);
int mss_wgrad(const mss_wgrad_args* args, void* stream);

/* --- bf16 shadows of float32 master weights, refreshed once per training step. --------
 * No counterpart symbol in the reference (its parameters are used in their own dtype).
 * For each entry: dst = bf16(src) (round to nearest even) when dst is not NULL, and
 * dst_t[c * ld_t + r] = bf16(src[r][c]) when dst_t is not NULL (the transposed copy the
 * input-gradient GEMMs W^T dY read as a contiguous operand). src is [rows][cols] float32
 * with rows contiguous, dst [rows][cols] bf16. The table lives in DEVICE memory (built once,
 * read by every refresh, e.g. each replay of a captured step); entries are 64 x 64 tiles
 * numbered consecutively: entry i covers tiles [tile0_i, tile0_i + ceil(rows/64) *
 * ceil(cols/64)), tile0 increasing from 0, n_tiles the total. The table is not checked
 * here (it is device memory); one launch refreshes every entry. */
typedef struct mss_shadow_entry {
  const float* src;
  void* dst;
  void* dst_t;
  int32_t rows, cols;
  int64_t ld_t;
  int64_t tile0;
} mss_shadow_entry;

int mss_shadow_refresh(const mss_shadow_entry* entries, int32_t n_entries, int64_t n_tiles, void* stream);

/* --- AdamW over float32 master weights, writing their bf16 shadows. --------------------
 * No counterpart symbol in the reference (its training step leaves the optimizer to the
 * caller: optax, experiments/mamba_inductionheads.py:126-139). Updates every entry in float32,
 * with decoupled weight decay (Loshchilov & Hutter) and bias-corrected moments:
 *   p <- p (1 - lr wd);  m <- m + (1 - beta1)(g - m);  v <- beta2 v + (1 - beta2) g^2;
 *   p <- p - lr / (1 - beta1^t) * m / (sqrt(v) / sqrt(1 - beta2^t) + eps),
 * t the float32 at the entry's `step` (device memory; the caller advances it before the call,
 * so a captured step replays with the right count). Then shadow = bf16(p) where shadow is not
 * NULL, and shadow_t[c * ld_t + r] = bf16(p[r][c]) where shadow_t is not NULL (as
 * mss_shadow_refresh). The entry array is HOST memory, read during the call: entries travel
 * to the GPU as kernel arguments, up to 40 per launch, so nothing is allocated or copied
 * and a captured call replays as it was made. Per entry: param, grad, exp_avg, exp_avg_sq
 * (numel float32 each) 16-byte aligned, shadow (bf16) 8-byte aligned; with shadow_t, the
 * parameter is [rows][cols] (rows * cols == numel, cols a multiple of 4) and shadow_t
 * 16-byte aligned with ld_t >= rows a multiple of 8. MSS_ERR_INVALID_ARGUMENT otherwise,
 * before any launch. Entries must not overlap one another. */
typedef struct mss_adamw_entry {
  float* param;
  const float* grad;
  float* exp_avg;
  float* exp_avg_sq;
  const float* step;
  void* shadow;
  void* shadow_t;
  int32_t rows, cols;
  int64_t ld_t;
  int64_t numel;
} mss_adamw_entry;

typedef struct mss_adamw_args {
  const mss_adamw_entry* entries;
  int32_t n_entries;
  float lr, beta1, beta2, eps, weight_decay;
} mss_adamw_args;

int mss_adamw(const mss_adamw_args* args, void* stream);

/* --- Token embedding into a channel-major stream, and its gradient. -------------------
 * Replace the XLA gather of the reference LM's input embedding (nnx.Embed,
 * mamba/mamba1.py:378-380) and its scatter-add gradient, for a stream kept as [D][T].
 * mss_embed_cm: h[f * ldh + t] = E[tokens[t] * D + f] for t < T, f < D (float32; E [V][D]
 * rows contiguous, ldh >= T); a token outside [0, V) gives a column of NaN (nothing is read
 * for it). h must not overlap E or tokens.
 * mss_embed_cm_backward: dE[v * D + f] += sum of dh[f * ldh + t] over t with tokens[t] == v,
 * given the tokens sorted stably (sorted_tokens ascending, order[i] the position of
 * sorted_tokens[i]; e.g. a stable sort's values and indices). Each row of dE is updated by
 * one workgroup, the run's terms added in a fixed association: the result does not depend on
 * timing. Tokens outside [0, V) are skipped. D a multiple of 4 and at most 1024, and at most
 * 2^24 tiles of 64 x 64 in both calls (MSS_ERR_UNSUPPORTED otherwise); dE and workspace 16-byte aligned, workspace >= 4 * T * D
 * bytes (dh transposed token-major); dE overlapping neither dh nor the workspace. */
int mss_embed_cm(const int64_t* tokens, int64_t T, const float* E, int32_t V, int32_t D, float* h, int64_t ldh,
                 void* stream);
int mss_embed_cm_backward(const float* dh, int64_t ldh, const int64_t* sorted_tokens, const int64_t* order, int64_t T,
                          int32_t V, int32_t D, float* dE, void* workspace, int64_t workspace_bytes, void* stream);


/* --- Reference-compatible entry points (float32, no fusions). ---------------------
 * Same argument order, attribute meaning and buffer shapes as the reference's XLA-FFI
 * handlers; physical layouts as listed at the top of this file. */

/* Replaces MambaSelectiveScan (reference native/selective_scan_cuda.cu:554-573).
 * discretization: 0 Euler, 1 ZOH. chunk_states: [B][D][ceil(L/2048)][N][2] holding
 * (prod a_bar over [0, chunk end], h at chunk end), as selective_scan_cuda.cu:306-320. */
int mss_scan_fwd(void* stream, int32_t discretization, int32_t batch, int32_t length,
                 int32_t dim, int32_t dstate, const float* A, const float* deltas,
                 const float* B, const float* C, const float* u, const float* initial_x,
                 float* y, float* final_x, float* chunk_states);

/* Replaces MambaSelectiveScanBenchmark (reference native/selective_scan_cuda.cu:578-598):
 * the forward launched `repeats` times back to back. */
int mss_scan_fwd_repeat(void* stream, int32_t discretization, int32_t repeats, int32_t batch,
                        int32_t length, int32_t dim, int32_t dstate, const float* A,
                        const float* deltas, const float* B, const float* C, const float* u,
                        const float* initial_x, float* y, float* final_x, float* chunk_states);

/* Replaces MambaSelectiveScanBackward (reference native/selective_scan_bwd.cu:166-190),
 * Euler discretization, from the forward's chunk_states as the reference does
 * (native/upstream_mamba/selective_scan_bwd_kernel.cuh:254-264): each 2048-step block's
 * state recurrence is re-run from the state chunk_states holds at the previous block's end
 * (initial_x for the first), all blocks in parallel, giving the state entering every
 * 8-step segment; then the backward kernels run from those. The reference signature has no
 * workspace operand, so this call makes one stream-ordered allocation of
 * mss_scan_bwd_workspace_bytes; mss_scan_bwd_ws takes a caller workspace instead (e.g. an
 * XLA FFI handler's scratch allocation) and allocates nothing. Outputs are overwritten. */
int mss_scan_bwd(void* stream, int32_t batch, int32_t length, int32_t dim, int32_t dstate,
                 const float* A, const float* deltas, const float* B, const float* C,
                 const float* u, const float* initial_x, const float* chunk_states,
                 const float* dout, const float* dfinal_x, float* dA, float* ddeltas, float* dB,
                 float* dC, float* du, float* dinitial_x);
size_t mss_scan_bwd_workspace_bytes(int32_t batch, int32_t length, int32_t dim, int32_t dstate);
int mss_scan_bwd_ws(void* stream, int32_t batch, int32_t length, int32_t dim, int32_t dstate,
                    const float* A, const float* deltas, const float* B, const float* C,
                    const float* u, const float* initial_x, const float* chunk_states,
                    const float* dout, const float* dfinal_x, float* dA, float* ddeltas, float* dB,
                    float* dC, float* du, float* dinitial_x, void* workspace, size_t workspace_bytes);

/* Human-readable text for a status code. */
const char* mss_strerror(int status);
/* Text of the last HIP error seen by this thread (for MSS_ERR_HIP). */
const char* mss_last_hip_error(void);
int mss_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA_SELECTIVE_SCAN_H_ */
