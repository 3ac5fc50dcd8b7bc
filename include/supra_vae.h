/*
 * supra_vae.h - C ABI of the SD-VAE mid-block attention on MI355X (gfx950): the whole block of
 * app/models/vae.js:77-94 in one call,
 *
 *   n   = GroupNorm(x; groups, eps, gamma, beta)                       (vae.js:81)
 *   q|k|v = n Wqkv^T + bqkv                                            (vae.js:82-84)
 *   a   = softmax(q k^T / sqrt(C)) v, one head of dim C                (vae.js:86)
 *   out = x + a Wo^T + bo                                              (vae.js:88-90)
 *
 * over an NHWC image x [HW, C]. Same library and conventions as supra_attn.h (device pointers,
 * stream-ordered asynchronous calls, SA_OK or a negative SA_ERR_* status with sa_last_error()).
 * The intermediates (normalized image, q|k|v, attention output, the attention's merge scratch)
 * live in a caller-provided workspace of sa_vae_attention_workspace_bytes() bytes: nothing is
 * allocated inside the call.
 */
#ifndef SUPRA_VAE_H
#define SUPRA_VAE_H

#include "supra_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sa_vae_attn_args {
  uint32_t struct_size;
  int32_t HW;     /* pixels (h * w; 1024 for the 32x32 latent) */
  int32_t C;      /* channels = the single head's dim (512) */
  int32_t groups; /* GroupNorm groups (32); C % groups == 0 */
  float eps;      /* GroupNorm epsilon (1e-6) */
  const float* x; /* [HW, C] input image, rows contiguous */
  const float* gamma; /* [C] GroupNorm weight */
  const float* beta;  /* [C] GroupNorm bias */
  const float* wqkv;  /* [3C, C]: the q, k and v projection weights stacked (PyTorch [out, in] layout) */
  const float* bqkv;  /* [3C] or NULL */
  const float* wo;    /* [C, C] output projection */
  const float* bo;    /* [C] or NULL */
  float* out;         /* [HW, C]; may be x itself (in place), must not overlap anything else */
  void* workspace;    /* device scratch, 16-byte aligned, >= sa_vae_attention_workspace_bytes() */
  int64_t workspace_bytes;
} sa_vae_attn_args;

/* Run the block (replaces VAEDecoder.attention, app/models/vae.js:77-94: GroupNorm, three linears,
 * the attention operator, the output linear and the residual add). */
int sa_vae_attention_f32(const sa_vae_attn_args* args, void* stream);

/* Bytes of device workspace sa_vae_attention_f32 needs for `args`, or a negative SA_ERR_* status
 * (only the sizes are read). Host only; no counterpart in the reference, whose intermediates are
 * pooled tensors (app/gpu/device.js:57-88). */
int64_t sa_vae_attention_workspace_bytes(const sa_vae_attn_args* args);

#ifdef __cplusplus
}
#endif

#endif /* SUPRA_VAE_H */
