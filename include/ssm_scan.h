/* ssm_scan.h -- C ABI of the MI355X (gfx950) selective-scan engine.
 *
 * One shared library, libssmscan.so, built from mamba-ssm-benchmark_amd/csrc/.  Every
 * entry point takes plain pointers, element strides and sizes; no C++ or framework types
 * cross the boundary.  The library never allocates device memory and never synchronizes:
 * callers pass outputs and workspaces (sizes from the *_bytes queries) and a HIP stream
 * (hipStream_t passed as void*; NULL = the null stream).  Kernels are enqueued on that
 * stream only.  Calls are re-entrant; the last error message is thread-local.
 *
 * Logical layouts follow the reference (models/scan.py:279): x, delta, z, out (B,L,D);
 * A (D,N); Bm, Cm (B,L,N); h0, last (B,D,N); D skip (D,).  Strides are in elements and
 * may be anything (including 0 for broadcast, e.g. the scalar-decay A of
 * models/mamba.py:82-83); the fast path is any tensor whose L or D axis has stride 1.
 *
 * Error model (mirrors the reference's Python exceptions):
 *   SSM_EINVAL  bad argument           -> ValueError  (models/scan.py:55; kernels/triton_scan.py:324-328)
 *   SSM_EKEY    unknown scan name       -> KeyError    (models/scan.py:261)
 *   SSM_ESPACE  workspace too small     -> ValueError
 *   SSM_EHIP    HIP launch/runtime error -> RuntimeError
 */
#ifndef SSM_SCAN_H
#define SSM_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SSM_ABI_VERSION 8

enum { SSM_OK = 0, SSM_EINVAL = 1, SSM_EKEY = 2, SSM_ESPACE = 3, SSM_EHIP = 4 };

/* Discretizations; the values are the reference's METHODS (kernels/triton_scan.py:23-24). */
enum { SSM_ZOH = 0, SSM_EULER = 1, SSM_BILINEAR = 2 };

/* Element types.  The state/compute type is float64 when dtype is SSM_F64 and float32
 * otherwise (the reference computes in promote(dtype, float32), models/scan.py:289). */
enum { SSM_F32 = 0, SSM_BF16 = 1, SSM_F16 = 2, SSM_F64 = 3 };

/* Scan algorithm ids: the reference's `scan=` names (models/scan.py:281-283, 168-173). */
enum {
  SSM_SCAN_REFERENCE = 0,
  SSM_SCAN_SEQUENTIAL = 1,
  SSM_SCAN_HILLIS_STEELE = 2,
  SSM_SCAN_BLELLOCH = 3,
  SSM_SCAN_CHUNKED = 4,
  SSM_SCAN_FUSED = 5, /* the reference's 'triton' fused kernels; here the fused HIP engine */
  SSM_SCAN_AUTO = 6
};

/* A strided tensor view.  data == NULL means "absent" for optional tensors. */
typedef struct ssm_tensor {
  void *data;
  int64_t stride[3];
} ssm_tensor;

/* ------------------------------------------------------------------ fused forward
 * Replaces TritonSelectiveScanFn.forward / _launch_fwd / _fwd_kernel
 * (kernels/triton_scan.py:27-74, 253-286) and the forward of SelectiveScanFn
 * (models/scan.py:202-217), with the D skip and SiLU gate of models/mamba.py:124 fused:
 *   delta' = softplus(delta + delta_bias) (each part optional), h_t = a_t h_{t-1} + b_t,
 *   y_t = sum_n C_t[n] h_t[n],   out = (y + Dskip * x) * silu(z)   (each part optional). */
typedef struct ssm_fwd_args {
  int64_t batch, seqlen, dim, dstate;
  int32_t method;          /* SSM_ZOH / SSM_EULER / SSM_BILINEAR */
  int32_t dtype;           /* type of x, delta, Bm, Cm, z, out */
  ssm_tensor x, delta;     /* (B,L,D) */
  ssm_tensor A;            /* (D,N), state type */
  ssm_tensor Bm, Cm;       /* (B,L,N) */
  ssm_tensor Dskip;        /* (D,) state type, optional */
  ssm_tensor z;            /* (B,L,D), optional gate */
  ssm_tensor delta_bias;   /* (D,) state type, optional */
  int32_t delta_softplus;  /* nonzero: delta' = softplus(delta + bias) */
  int32_t segments;        /* time segments scanned in parallel: 0 = chosen by the library
                              (more than 1 only when B x D alone cannot fill the GPU, e.g.
                              one long sequence); the segment-end states are combined
                              exactly like scan_chunked's chunk summaries
                              (models/scan.py:158-164) and need ssm_fwd_workspace_bytes() */
  ssm_tensor h0;           /* (B,D,N) state type, optional initial state */
  ssm_tensor out;          /* (B,L,D) dtype, required */
  ssm_tensor last;         /* (B,D,N) state type, optional final state */
  void *saved;             /* optional: ssm_fwd_saved_bytes() of device memory; when given,
                              the forward stores what ssm_bwd needs (chunk-boundary
                              states and, with a gate, the pre-gate output) */
  void *workspace;         /* scratch of ssm_fwd_workspace_bytes() (long-sequence path) */
  int64_t workspace_bytes;
  /* Optional low-rank delta: the dt_proj GEMM of models/mamba.py:76 done while the delta
   * tiles are staged.  With delta_rank R in 1..16, `delta` is the (B,L,R) input dt (dtype)
   * and the delta the scan uses is delta @ delta_proj^T, delta_proj (D,R) in the state type,
   * before delta_bias / softplus; no (B,L,D) delta is read.  delta_rank = 0: off.  Needs
   * dstate <= 16 and a 16- or 32-bit dtype. */
  ssm_tensor delta_proj;
  int64_t delta_rank;
  /* A_is_log = 1: `A` holds log(-A), the A_log parameter of models/mamba.py:61,81 (A =
   * -exp(A_log), :81), and the kernels form A themselves; 0: `A` is A. */
  int32_t A_is_log;
  int32_t reserved1;
} ssm_fwd_args;

/* ------------------------------------------------------------------ fused backward
 * Replaces TritonSelectiveScanFn.backward / _bwd_kernel (kernels/triton_scan.py:143-226,
 * 288-319) and SelectiveScanFn.backward (models/scan.py:219-255).  Recomputes states
 * inside each chunk from the saved chunk-boundary states; every reduction (dA, dB, dC,
 * dD, ddelta_bias) is done in a fixed order, so results are bitwise reproducible. */
typedef struct ssm_bwd_args {
  int64_t batch, seqlen, dim, dstate;
  int32_t method, dtype;
  ssm_tensor x, delta, A, Bm, Cm, Dskip, z, delta_bias; /* as in ssm_fwd_args */
  int32_t delta_softplus;
  int32_t segments;        /* time segments walked back in parallel: 0 = chosen by the library
                              (more than 1 only when B x D alone cannot fill the GPU); each
                              segment starts from the adjoint carried in from the later ones,
                              combined as the forward combines its segments, in reverse.
                              Float64 inputs always use one segment. */
  ssm_tensor h0;
  const void *saved;       /* the `saved` buffer of the matching ssm_fwd call, or NULL
                              (then the states are recomputed into the workspace) */
  ssm_tensor dout;         /* (B,L,D) dtype: gradient of out */
  ssm_tensor dlast;        /* (B,D,N) state type, optional: gradient of last */
  ssm_tensor dx, ddelta;   /* (B,L,D) dtype; ddelta is w.r.t. the raw delta input */
  ssm_tensor dA;           /* (D,N) state type */
  ssm_tensor dBm, dCm;     /* (B,L,N) dtype */
  ssm_tensor dD;           /* (D,) state type, required iff Dskip */
  ssm_tensor dz;           /* (B,L,D) dtype, required iff z; any strides (e.g. the gate half
                              of an in_proj-output gradient, as z may be) */
  ssm_tensor ddelta_bias;  /* (D,) state type, required iff delta_bias */
  ssm_tensor dh0;          /* (B,D,N) state type, optional (gradient of h0) */
  void *workspace;         /* ssm_bwd_workspace_bytes() */
  int64_t workspace_bytes;
  /* Low-rank delta as in ssm_fwd_args; ddelta is then the (B,L,D) gradient of the projected
   * delta (before bias / softplus), from which the caller's GEMMs form the gradients of the
   * (B,L,R) input and of delta_proj. */
  ssm_tensor delta_proj;
  int64_t delta_rank;
  int32_t A_is_log;        /* as in ssm_fwd_args; dA is then the gradient of A_log */
  int32_t reserved1;
} ssm_bwd_args;

/* ------------------------------------------------------------------ decode step
 * Replaces the inline recurrent step of Mamba.forward (models/mamba.py:113-118,122-124):
 *   h <- a h + b (in place),  out = (sum_n C[n] h[n] + Dskip x) * silu(z). */
typedef struct ssm_step_args {
  int64_t batch, dim, dstate;
  int32_t method, dtype;
  ssm_tensor x, delta;     /* (B,D) */
  ssm_tensor A;            /* (D,N) state type */
  ssm_tensor Bm, Cm;       /* (B,N) */
  ssm_tensor Dskip;        /* (D,) optional */
  ssm_tensor z;            /* (B,D) optional */
  ssm_tensor delta_bias;   /* (D,) optional */
  int32_t delta_softplus;
  int32_t reserved0;
  ssm_tensor h;            /* (B,D,N) state type, read and updated in place */
  ssm_tensor out;          /* (B,D) dtype */
} ssm_step_args;

/* ------------------------------------------------------------------ fused decode layer
 * The scan-path part of one Mamba layer's recurrent decode step (models/mamba.py:93-124 at
 * L = 1 with a state, preceded by the block's RMSNorm, models/lm.py Block / models/common.py:8-16),
 * in one launch per layer.  The caller runs the two large projections as GEMMs:
 *   xz = u @ (W_in diag(norm_w))^T        (in_proj with the RMSNorm weight folded in)
 * and, after this call, u += y @ W_out^T (out_proj + residual).  Per batch row this step
 *   s = rsqrt(mean(u^2) + eps);  x = s xz[:, :D], z = s xz[:, D:]      (the RMSNorm scale)
 *   x = silu(conv(conv_state, x) + conv_bias);  conv_state <- shifted  (models/mamba.py:104-107)
 *   dt, B, C = x_proj(x);  delta = softplus(dt_proj(dt) + dt_bias)     (:75-76)
 *   h <- a h + b (ssm_state, in place);  y = (C h + Dskip x) silu(z)   (:113-118, :124)
 * All tensors float32 (the conv state float32 or bf16) and row-major; dstate <= 64; one
 * workgroup per batch row. */
typedef struct ssm_decode_args {
  int64_t batch, dim, dstate, width, dt_rank, d_model;
  int32_t method;          /* SSM_ZOH / SSM_EULER / SSM_BILINEAR */
  int32_t conv_state_dtype; /* SSM_F32 or SSM_BF16 (the state of a bf16-autocast model) */
  float eps;               /* RMSNorm epsilon */
  float reserved1;
  const float *u;          /* (B, d_model) block input (the residual stream) */
  const float *xz;         /* (B, 2*dim) = u @ (W_in diag(norm_w))^T */
  const float *conv_w;     /* (dim, width) */
  const float *conv_b;     /* (dim,) */
  void *conv_state;        /* (B, dim, width-1) of conv_state_dtype, updated in place (a bf16
                              state stores the new inputs rounded to bf16; NULL when width is 1) */
  const float *x_proj_wt;  /* (dim, dt_rank + 2*dstate): x_proj's weight transposed */
  const float *dt_proj_w;  /* (dim, dt_rank) */
  const float *dt_bias;    /* (dim,) */
  const float *A_log;      /* (dim, dstate): A = -exp(A_log) */
  const float *Dskip;      /* (dim,) */
  float *ssm_state;        /* (B, dim, dstate), updated in place */
  float *y;                /* (B, dim) output, the input of out_proj */
} ssm_decode_args;

/* ------------------------------------------------------------------ decode step of a block stack
 * The recurrent decode step of a stack of Mamba blocks: the loop over blocks of
 * models/lm.py:124-128 with states, each block x = x + mixer(norm1(x), state)
 * (models/lm.py:82-83; RMSNorm models/common.py:14-16; the mixer models/mamba.py:93-124 at
 * L = 1), in two launches per block plus one at the end.  Unlike ssm_decode_step, the in_proj
 * and out_proj GEMMs are part of the step, tiled with the rest of the block over the whole GPU.
 * u (B, d_model) holds the residual stream entering the first block and is replaced by the one
 * leaving the last (the input of the final norm and head).  Optionally the call also covers the
 * token step's ends (models/lm.py:125,128): with `tokens`, the residual stream entering the
 * first block is the tokens' embedding rows (u is then output only; an id outside
 * [0, vocab) reads a zero row, where the reference's embedding raises); with `head_w4`, the
 * logits of the final RMSNorm and the head are written.  The GEMM weights come in a layout of
 * four consecutive k per column (w_in4, w_out4, head_w4), so a lane reads 16 bytes at a time.
 * Every block has the same dimensions; tensors are float32 and row-major (conv states float32
 * or bf16), states are updated in place, and every sum runs in a fixed order (the step is
 * deterministic).
 * Supported: d_model <= 512, dim <= 1024, both multiples of 4, dstate 8 or 16, dt_rank 8, 16
 * or 32, width <= 4; u, embed and every weight read four floats at a time (w_in4, w_out4,
 * head_w4, A_log, dt_proj_w) and ssm_state 16-byte aligned;
 * ssm_decode_stack_check names the limit a shape breaks. */
typedef struct ssm_decode_block {
  const float *w_in4;      /* (d_model/4, 2*dim, 4): element [g][c][j] = W[c][4g + j] for
                              W = W_in diag(norm_w), in_proj with the RMSNorm weight folded in */
  const float *conv_w;     /* (dim, width) */
  const float *conv_b;     /* (dim,) */
  const float *x_proj_wt;  /* (dim, dt_rank + 2*dstate): x_proj's weight transposed */
  const float *dt_proj_w;  /* (dim, dt_rank) */
  const float *dt_bias;    /* (dim,) */
  const float *A_log;      /* (dim, dstate): A = -exp(A_log) */
  const float *Dskip;      /* (dim,) */
  const float *w_out4;     /* (dim/4, d_model, 4): element [g][c][j] = W_out[c][4g + j] */
  void *conv_state;        /* (B, dim, width-1) of conv_state_dtype, updated in place (may be
                              NULL when width is 1) */
  float *ssm_state;        /* (B, dim, dstate), updated in place */
  float eps;               /* the block's RMSNorm epsilon */
  int32_t reserved0;
} ssm_decode_block;

typedef struct ssm_decode_stack_args {
  int64_t batch, dim, dstate, width, dt_rank, d_model;
  int32_t method;          /* SSM_ZOH / SSM_EULER / SSM_BILINEAR */
  int32_t conv_state_dtype; /* SSM_F32 or SSM_BF16 */
  int32_t n_blocks;
  int32_t reserved0;
  const ssm_decode_block *blocks;  /* host array of n_blocks, read during the call only */
  float *u;                /* (B, d_model) residual stream, replaced in place */
  void *workspace;         /* device memory of ssm_decode_stack_workspace_bytes() */
  int64_t workspace_bytes;
  const int64_t *tokens;   /* (B,) token ids on the device, or NULL; an id outside [0, vocab)
                              reads a zero embedding row and sets the status word (below) */
  const float *embed;      /* (vocab, d_model) embedding table, read when tokens is set */
  const float *head_w4;    /* (d_model/4, vocab, 4): element [g][v][j] = W[v][4g + j] for
                              W = W_head diag(norm_f_w), or NULL (no head) */
  float *logits;           /* (B, vocab), written when head_w4 is set */
  int64_t vocab;
  float head_eps;          /* the final RMSNorm's epsilon */
  int32_t reserved1;
} ssm_decode_stack_args;

/* ------------------------------------------------------------------ linear scans
 * Replaces the scan algorithms of models/scan.py:70-165 (scan_sequential,
 * scan_hillis_steele, scan_blelloch, scan_chunked) on (a, b) of shape (B, L, M):
 *   h_t = a_t h_{t-1} + b_t,  h_{-1} = h0 (or 0).   With reverse != 0 the recurrence
 * runs from t = L-1 down to 0 (used by the composed backward, models/scan.py:240). */
typedef struct ssm_lscan_args {
  int64_t batch, seqlen, width;
  int32_t algo;            /* SSM_SCAN_SEQUENTIAL .. SSM_SCAN_CHUNKED */
  int32_t dtype;           /* SSM_F32 or SSM_F64 (a, b, h0, h all this type) */
  int32_t reverse;
  int32_t reserved0;
  int64_t chunk;           /* SSM_SCAN_CHUNKED: chunk size; 0 = ssm_default_chunk(L) */
  ssm_tensor a, b;         /* (B,L,M) */
  ssm_tensor h0;           /* (B,M) optional */
  ssm_tensor h;            /* (B,L,M) output */
  void *workspace;         /* ssm_lscan_workspace_bytes() */
  int64_t workspace_bytes;
} ssm_lscan_args;

/* Adjoint of ssm_lscan: given dh = dL/dh (B,L,M), returns da, db (B,L,M) and dh0 (B,M).
 * It is the reverse scan lambda_t = dh_t + a_{t+1} lambda_{t+1} run with the same algorithm
 * (models/scan.py:239-240 scans a_next with the forward's scan_fn), then da_t = lambda_t h_{t-1},
 * db_t = lambda_t, dh0 = a_0 lambda_0 (models/scan.py:242-248).  `reverse` is the direction of
 * the forward scan being differentiated. */
typedef struct ssm_lscan_bwd_args {
  int64_t batch, seqlen, width;
  int32_t algo, dtype, reverse, reserved0;
  int64_t chunk;
  ssm_tensor a;            /* forward input (B,L,M) */
  ssm_tensor h0;           /* forward input (B,M), optional */
  ssm_tensor h;            /* forward output (B,L,M) */
  ssm_tensor dh;           /* upstream gradient (B,L,M) */
  ssm_tensor da, db;       /* outputs (B,L,M) */
  ssm_tensor dh0;          /* output (B,M), optional */
  void *workspace;         /* ssm_lscan_bwd_workspace_bytes() */
  int64_t workspace_bytes;
} ssm_lscan_bwd_args;

/* ------------------------------------------------------------------ discretization
 * models/scan.py:39-55, materialized: a, b (B,L,D,N), contiguous.  The backward maps
 * (da, db) to (ddelta, dA, dBm, dx) exactly as autograd does through discretize
 * (models/scan.py:249). */
typedef struct ssm_disc_args {
  int64_t batch, seqlen, dim, dstate;
  int32_t method, dtype;   /* dtype: SSM_F32 or SSM_F64 for every tensor */
  ssm_tensor delta, x;     /* (B,L,D) */
  ssm_tensor A;            /* (D,N) */
  ssm_tensor Bm;           /* (B,L,N) */
  void *a, *b;             /* forward outputs (B,L,D,N) contiguous */
  const void *da, *db;     /* backward inputs (B,L,D,N) contiguous */
  ssm_tensor ddelta, dx;   /* backward outputs (B,L,D) */
  ssm_tensor dA;           /* backward output (D,N) */
  ssm_tensor dBm;          /* backward output (B,L,N) */
  void *workspace;         /* ssm_disc_workspace_bytes() */
  int64_t workspace_bytes;
} ssm_disc_args;

/* ------------------------------------------------------------------ causal depthwise conv
 * models/mamba.py:101-107: y = silu(conv1d(pad_left(x), w, bias, groups=D)), with the
 * chronological shift state of :104-106 (the previous width-1 inputs). */
typedef struct ssm_conv_args {
  int64_t batch, seqlen, dim, width;
  int32_t dtype;           /* x, out, dx, dout; weight/bias in float32 (float64 for F64) */
  int32_t silu;
  ssm_tensor x;            /* (B,L,D) */
  ssm_tensor weight;       /* (D,W) */
  ssm_tensor bias;         /* (D,) optional */
  ssm_tensor state_in;     /* (B,D,W-1) optional previous inputs (zeros when absent) */
  ssm_tensor out;          /* (B,L,D) forward output */
  ssm_tensor state_out;    /* (B,D,W-1) optional: the last W-1 inputs after this call */
  ssm_tensor dout;         /* backward: (B,L,D) */
  ssm_tensor dx;           /* backward: (B,L,D) */
  ssm_tensor dweight;      /* backward: (D,W) float32/64 */
  ssm_tensor dbias;        /* backward: (D,) optional */
  void *workspace;         /* ssm_conv_workspace_bytes() */
  int64_t workspace_bytes;
} ssm_conv_args;

/* ------------------------------------------------------------------ RMSNorm
 * models/common.py:8-16 (the LM's pre-norms, models/lm.py:63,95):
 *   y = (x * r) * weight,  r = 1 / sqrt(mean(x^2, last dim) + eps)  per row.
 * Rows of `dim` <= 1024 elements with unit column stride; float32 or float64 throughout. */
typedef struct ssm_norm_args {
  int64_t rows, dim;
  int32_t dtype;           /* SSM_F32 or SSM_F64: x, weight, out, rstd, dout, dx, dweight */
  int32_t reserved0;
  double eps;
  ssm_tensor x;            /* (rows, dim): stride[0] = row stride, stride[1] = 1 */
  ssm_tensor weight;       /* (dim,) contiguous */
  ssm_tensor out;          /* forward: (rows, dim) */
  void *rstd;              /* (rows,) r per row: written by the forward, read by the backward */
  ssm_tensor dout;         /* backward: (rows, dim) */
  ssm_tensor dx;           /* backward: (rows, dim) */
  void *dweight;           /* backward: (dim,) */
  void *workspace;         /* backward: ssm_norm_workspace_bytes() */
  int64_t workspace_bytes;
} ssm_norm_args;

/* ------------------------------------------------------------------ entry points */
int ssm_abi_version(void);
const char *ssm_last_error(void);

/* Host-only argument validation (no device needed).  Returns SSM_OK or an error code. */
int ssm_fwd_check(const ssm_fwd_args *args);
int ssm_bwd_check(const ssm_bwd_args *args);
int ssm_step_check(const ssm_step_args *args);
int ssm_decode_check(const ssm_decode_args *args);
int ssm_decode_stack_check(const ssm_decode_stack_args *args);
int ssm_lscan_check(const ssm_lscan_args *args);
int ssm_lscan_bwd_check(const ssm_lscan_bwd_args *args);
int ssm_disc_check(const ssm_disc_args *args);
int ssm_conv_check(const ssm_conv_args *args);
int ssm_norm_check(const ssm_norm_args *args);

/* Buffer sizes in bytes (host-only). */
int64_t ssm_fwd_saved_bytes(const ssm_fwd_args *args);
int64_t ssm_fwd_workspace_bytes(const ssm_fwd_args *args);
int64_t ssm_bwd_workspace_bytes(const ssm_bwd_args *args);
int64_t ssm_lscan_workspace_bytes(const ssm_lscan_args *args);
int64_t ssm_lscan_bwd_workspace_bytes(const ssm_lscan_bwd_args *args);
int64_t ssm_disc_workspace_bytes(const ssm_disc_args *args);
int64_t ssm_conv_workspace_bytes(const ssm_conv_args *args);
int64_t ssm_norm_workspace_bytes(const ssm_norm_args *args);
int64_t ssm_decode_stack_workspace_bytes(const ssm_decode_stack_args *args);
/* Byte offset inside the decode-stack workspace of an int32 status word: ssm_decode_stack sets
 * it to 1 when a token id lies outside [0, vocab) (the reference's nn.Embedding,
 * models/lm.py:125, raises on such ids; the step itself reads a zero row and goes on).  The
 * library never clears it: the caller zeroes it (e.g. when it allocates the workspace) and
 * reads it when it wants to check, so the step stays free of host synchronization and can be
 * captured in a graph.  No counterpart in the reference.  -1 for invalid dimensions. */
int64_t ssm_decode_stack_status_offset(const ssm_decode_stack_args *args);

/* Launches (asynchronous on `stream`). */
int ssm_fwd(const ssm_fwd_args *args, void *stream);
int ssm_bwd(const ssm_bwd_args *args, void *stream);
int ssm_step(const ssm_step_args *args, void *stream);
int ssm_decode_step(const ssm_decode_args *args, void *stream);
int ssm_decode_stack(const ssm_decode_stack_args *args, void *stream);
int ssm_lscan(const ssm_lscan_args *args, void *stream);
int ssm_lscan_bwd(const ssm_lscan_bwd_args *args, void *stream);
int ssm_disc_fwd(const ssm_disc_args *args, void *stream);
int ssm_disc_bwd(const ssm_disc_args *args, void *stream);
int ssm_conv_fwd(const ssm_conv_args *args, void *stream);
int ssm_conv_bwd(const ssm_conv_args *args, void *stream);
int ssm_norm_fwd(const ssm_norm_args *args, void *stream);   /* models/common.py:14-16 */
int ssm_norm_bwd(const ssm_norm_args *args, void *stream);   /* autograd of :14-16 */

/* ssm_fwd without allocation.  No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as ssm_fwd, except that args->workspace and
 * args->workspace_bytes are ignored: the long-sequence (segmented) path uses a fixed device
 * array of SSM_FWD_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.  With
 * args->segments = 0 a plan whose ssm_fwd_workspace_bytes() exceeds the array runs the most
 * segments that fit it; a forced count that exceeds it fails with SSM_ESPACE.  The stream must belong
 * to the current device.  Calls on one GPU share the array: calls that overlap on one GPU
 * race (serialize them, e.g. on one stream). */
#define SSM_FWD_NOALLOC_SCRATCH_BYTES (8 * 1024 * 1024)
int ssm_fwd_noalloc(const ssm_fwd_args *args, void *stream);

/* ------------------------------------------------------------------ plans (host-only, exact integers)
 * The reference's integer planning functions, returned bit-exactly. */
int64_t ssm_default_chunk(int64_t seqlen);                        /* models/scan.py:138-139 */
int64_t ssm_scan_blocks(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                        int64_t d_block, int64_t *bounds, int64_t capacity);
                                                                  /* models/scan.py:185-190; writes
                                                                     (start, end) pairs, returns count */
int64_t ssm_block_d(int64_t batch, int64_t dim);                  /* kernels/triton_scan.py:245-250 */
int64_t ssm_bwd_tile(int64_t batch, int64_t seqlen, int64_t dstate, int64_t block_d);
                                                                  /* kernels/triton_scan.py:305 */
int32_t ssm_resolve_scan(int32_t scan_id, int32_t on_gpu, int32_t method, int64_t dstate,
                         int32_t engine_available);               /* models/scan.py:286-287, 305-314;
                                                                     -1 for an unknown id */

#ifdef __cplusplus
}
#endif
#endif /* SSM_SCAN_H */
