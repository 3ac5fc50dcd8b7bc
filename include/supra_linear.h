/*
 * supra_linear.h - C ABI of the MI355X (gfx950) linear layer: the projections either side of the
 * attention operator in the DiT block (qkv, proj, q, kv, cproj, fc1, fc2; app/models/dit.js:165-192).
 *
 * Replaces `linear(gpu, x, W, {rows, aOff, out, resid, gate, gOff, act, bias})`
 * (app/gpu/ops.js:33-43) and the GEMM it dispatches, `matmulShader` with A mode "rows" and B format
 * "f32" (app/gpu/gemm.js:116-223, epilogue at gemm.js:127-137, activations at gemm.js:21-36).
 * Same library as supra_attn.h (libsupra_attn.so), same conventions: device pointers, offsets and
 * strides in floats, stream-ordered asynchronous calls, SA_OK or a negative SA_ERR_* status with
 * sa_last_error(), nothing allocated inside the call.
 */
#ifndef SUPRA_LINEAR_H
#define SUPRA_LINEAR_H

#include "supra_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- activation applied after the bias (app/gpu/gemm.js:21-36, 128-130) ---- */
#define SA_ACT_NONE 0
#define SA_ACT_GELU 1      /* 0.5 x (1 + erf(x / sqrt(2))) */
#define SA_ACT_GELU_TANH 2 /* 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), PyTorch approximate="tanh" */
#define SA_ACT_SILU 3      /* x / (1 + exp(-x)) */

/* ---- how the result reaches y (app/gpu/gemm.js:131) ---- */
#define SA_EPI_STORE 0      /* y[m][n] = r */
#define SA_EPI_RESID 1      /* y[m][n] += r (residual, in place) */
#define SA_EPI_RESID_GATE 2 /* y[m][n] += gate[gate_off + n] * r (AdaLN-Zero gated residual) */

/*
 * One linear layer: for m < M, n < N,
 *
 *   r = act(alpha * sum_k X[m][k] W[n][k] + bias[n])
 *
 * with X[m][k] = x[x_off + m*ldx + k], W[n][k] = w[n*ldw + k] (the PyTorch [out, in] weight layout
 * the reference uploads, app/weights.js:89-96), bias optional, then stored or added into
 * Y[m][n] = y[y_off + m*ldy + n] as `epilogue` says. Strides of 0 default to K (ldx, ldw) and N
 * (ldy); offsets and strides must be below 2^40. y must not overlap x, w, bias or gate. Set struct_size = sizeof(sa_linear_args) and
 * alpha (1 for a plain layer; the reference's default).
 */
typedef struct sa_linear_args {
  uint32_t struct_size;
  int32_t M; /* rows (app/gpu/ops.js:36: rows, default x.size / K) */
  int32_t N; /* output features */
  int32_t K; /* input features */
  const float* x;
  int64_t x_off; /* app/gpu/ops.js:40 aOff */
  int64_t ldx;
  const float* w;
  int64_t ldw;
  const float* bias; /* [N] or NULL */
  float alpha;
  int32_t act;      /* SA_ACT_* */
  int32_t epilogue; /* SA_EPI_* */
  const float* gate; /* SA_EPI_RESID_GATE only */
  int64_t gate_off;  /* app/gpu/ops.js:41 gOff */
  float* y;
  int64_t y_off;
  int64_t ldy;
} sa_linear_args;

/* Launch one linear layer on `stream` (a hipStream_t, NULL = null stream). Replaces
 * app/gpu/ops.js:35-43 + app/gpu/gemm.js:116-223. */
int sa_linear_f32(const sa_linear_args* args, void* stream);

/* Name of the kernel sa_linear_f32 would launch for `args` ("linear_mfma_128x192", ...,
 * "linear_generic"), or NULL if the arguments are invalid. Host only; no counterpart in the
 * reference (its app/gpu/ops.js:17-24 tile choice is internal). */
const char* sa_linear_kernel_name(const sa_linear_args* args);

#ifdef __cplusplus
}
#endif

#endif /* SUPRA_LINEAR_H */
