/*
 * supra_attn.h - C ABI of the MI355X (gfx950) fused attention operator.
 *
 * This library replaces the attention hot path of Supra2-Img Web: the JS operator
 * `attention(gpu, {q, k, v, Lq, Lk, H, D, ldq, ldk, ldv, qOff, kOff, vOff, oOff, scale, bias, out})`
 * (app/gpu/ops.js:103-149), its fused WGSL kernel (app/gpu/kernels.js:164-316), and the unfused
 * QK^T GEMM -> softmax(+bias) -> PV GEMM chain it falls back to (app/gpu/ops.js:119-147,
 * app/gpu/kernels.js:27-63, app/gpu/gemm.js:116-223). The device-buffer helpers replace the parts
 * of the WebGPU runtime that the operator's callers touch (app/gpu/device.js:41-55, 144-191,
 * 255-269).
 *
 * Conventions
 *  - Every pointer argument named q/k/v/o/bias/key_len/key_mask is a DEVICE pointer.
 *  - Offsets and strides are in ELEMENTS (floats for q/k/v/o/bias), as in app/gpu/ops.js.
 *  - All calls are stream-ordered and asynchronous unless documented otherwise; `stream` is a
 *    hipStream_t passed as void* (NULL = the null stream). Nothing in the attention call
 *    allocates device memory: the kernels that merge partial results across workgroups use a
 *    caller-provided workspace (sa_attention_workspace_bytes).
 *  - Status codes: SA_OK (0) or a negative SA_ERR_* value. A failed call launches nothing.
 *    sa_last_error() returns a thread-local message describing the last failure.
 *  - q, k and v may alias one another (the DiT passes one packed qkv buffer as all three,
 *    app/models/dit.js:172). o must not overlap any of them.
 */
#ifndef SUPRA_ATTN_H
#define SUPRA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SA_ABI_VERSION 5

/* ---- status codes ---- */
#define SA_OK 0
#define SA_ERR_INVALID (-1)     /* invalid argument (null pointer, non-positive size, bad stride) */
#define SA_ERR_UNSUPPORTED (-2) /* a valid request outside what this build implements */
#define SA_ERR_HIP (-3)         /* the HIP runtime reported an error */
#define SA_ERR_ALIAS (-4)       /* the output overlaps an input */
#define SA_ERR_NOT_FOUND (-5)   /* a named tensor is not in the weight file (supra_weights.h) */
#define SA_ERR_IO (-6)          /* a weight file could not be opened, sized or mapped */
#define SA_ERR_FORMAT (-7)      /* a weight file is not well-formed safetensors */

/* ---- additive score bias ---- */
#define SA_BIAS_NONE 0
/* Dense bias, element (b, h, i, j) at bias[b*sbias + (h*Lq + i)*Lk + j]: the [H, Lq, Lk] layout
 * that app/models/t5.js:55-65 builds and app/gpu/kernels.js:34 adds (sbias = 0 shares one bias
 * across the batch). */
#define SA_BIAS_DENSE 1
/* Relative-position bias gathered in-kernel (HF T5 compute_bias, mirrored by
 * app/models/t5.js:55-65): element (b, h, i, j) = bias[bucket_lut[j - i + Lq - 1] * H + h], with
 * bias the [num_buckets, H] table of app/models/t5.js:44 and bucket_lut an int32 device array of
 * Lq + Lk - 1 buckets (fill it with sa_t5_bucket_lut). A bucket id outside [0, num_buckets) is
 * clamped into it (every kernel, and sa_t5_position_bias, apply the same rule). */
#define SA_BIAS_RELPOS 2

/* ---- key masking (on top of the Lk bound) ---- */
#define SA_MASK_NONE 0
/* Per-sequence key length: keys j >= key_len[b] are masked (0 <= key_len[b] <= Lk). This is the
 * padded form of app/models/dit.js:182-185, which runs each sample at its own Lk. */
#define SA_MASK_KEY_LEN 1
/* Boolean key-padding mask, key_mask[b*smask + j] != 0 means "attend": the
 * F.scaled_dot_product_attention boolean convention of tools/reference.py:78. */
#define SA_MASK_KEY_MASK 2

/*
 * Arguments of one attention call: for every sequence b < B, head h < H and query i < Lq,
 *
 *   s_ij   = scale * sum_d Q[b,i,h,d] K[b,j,h,d] + bias(b,h,i,j)
 *   O[b,i,h,:] = sum_{j attended} softmax_j(s_ij) V[b,j,h,:]
 *
 * with Q[b,i,h,d] = q[q_off + b*sq + i*ldq + h*D + d] (likewise k, v, o). A query row whose keys
 * are all masked produces zeros (the F.scaled_dot_product_attention convention).
 *
 * Set struct_size = sizeof(sa_attn_args) (checked, so that later ABI revisions can grow the
 * struct; the revision-2 size, which ends at workspace_bytes, is still accepted). Zero-initialise
 * unused fields.
 */
typedef struct sa_attn_args {
  uint32_t struct_size;
  int32_t B;  /* sequences in the batch (app/models/dit.js loops these on the host) */
  int32_t H;  /* heads */
  int32_t D;  /* head dim */
  int32_t Lq; /* queries per sequence */
  int32_t Lk; /* keys per sequence (the padded length when a mask is used) */
  const float* q;
  const float* k;
  const float* v;
  float* o;
  int64_t q_off, k_off, v_off, o_off; /* element offsets (qOff/kOff/vOff/oOff in ops.js) */
  int64_t ldq, ldk, ldv, ldo;         /* row strides; ldo <= 0 means H*D (ops.js:114) */
  int64_t sq, sk, sv, so;             /* batch strides; ignored when B == 1. Offsets and strides < 2^40 */
  float scale;                        /* softmax scale; the JS default 1/sqrt(D) is set by callers */
  int32_t bias_mode;                  /* SA_BIAS_* */
  const float* bias;                  /* DENSE: [B?][H, Lq, Lk]; RELPOS: table [num_buckets, H] */
  int64_t sbias;                      /* DENSE batch stride in elements (0 = shared) */
  const int32_t* bucket_lut;          /* RELPOS: Lq + Lk - 1 bucket ids, index j - i + Lq - 1 */
  int32_t num_buckets;                /* RELPOS: rows of the table */
  int32_t mask_mode;                  /* SA_MASK_* */
  const int32_t* key_len;             /* KEY_LEN: [B] */
  const uint8_t* key_mask;            /* KEY_MASK: [B, smask] */
  int64_t smask;                      /* KEY_MASK batch stride (bytes = elements); <= 0 means Lk */
  void* workspace;                    /* device scratch, 16-byte aligned, when the call needs it */
  int64_t workspace_bytes;            /* its size (>= sa_attention_workspace_bytes(args)) */
  /* Revision 3. KEY_LEN: an optional HOST copy of key_len[0..B), read during the call and used
   * only to shape the launch: the flash kernel schedules the sequences (balanced by key blocks over
   * the device's L2 domains and CUs) when 8 <= B <= 256, bit for bit neutral; the 16-query
   * small-launch kernel packs sequences of at most 64 keys into fewer workgroups when B <= 16 and
   * the launch would exceed one workgroup per CU (the order of the fp32 sums changes, within the
   * usual rounding). The results come from the device key_len either way, so a stale copy costs
   * speed, never correctness. The DiT caller knows its prompt lengths on the host
   * (app/models/dit.js:137-144). */
  const int32_t* key_len_host;
} sa_attn_args;

/* Fused attention, fp32 in and out, fp32 MFMA arithmetic. Replaces ops.attention
 * (app/gpu/ops.js:103-149) for every caller in app/models/{dit,t5,vae}.js; B folds the
 * per-sample host loops of app/models/dit.js:170-185 into one launch. Asynchronous on `stream`. */
int sa_attention_f32(const sa_attn_args* args, void* stream);

/* Scratch the allocation-free entry point has per GPU: 32 MiB of device memory, held from the
 * library's first use on that GPU (below) until the process ends. */
#define SA_NOALLOC_SCRATCH_BYTES (32 << 20)

/* sa_attention_f32 for callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc. No counterpart in the reference.
 * args->workspace and workspace_bytes are ignored: the kernels that merge partial results across
 * workgroups use the library's own per-GPU scratch (a static device array of
 * SA_NOALLOC_SCRATCH_BYTES). The library plans those merges to fit it, so every call
 * sa_attention_f32 takes runs here too; a call that would need more (sa_attention_workspace_bytes)
 * would fail with SA_ERR_UNSUPPORTED before any launch. Nothing in the call allocates. The library looks up a
 * GPU's scratch address (hipGetSymbolAddress, which loads the library's device code on that GPU if
 * nothing has yet) once, at its first use on that GPU: sa_set_device, sa_malloc, sa_stream_create or
 * any operator call there. A caller that captures these calls into a HIP graph makes one of those
 * calls on the GPU before it begins the capture; otherwise the first call in the capture does the
 * lookup. Every call on one GPU shares its scratch: calls ordered on one stream are fine, calls
 * that overlap on one GPU (other streams, other threads) race. The scratch holds nothing that must
 * start at zero. */
int sa_attention_f32_noalloc(const sa_attn_args* args, void* stream);

/* Device scratch bytes sa_attention_f32 needs for these arguments on the current device (0 for
 * most calls; the wide-head kernel splits long key ranges across workgroups and merges their
 * partial results through it), or a negative SA_ERR_* status if the arguments are rejected.
 * The workspace holds no state between calls, but calls that run concurrently must not share one.
 * Host only: no device work. There is no counterpart in the reference, whose unfused path keeps
 * its score matrix in buffers the caller's pool provides (app/gpu/ops.js:125-128). */
int64_t sa_attention_workspace_bytes(const sa_attn_args* args);

/* Which kernel sa_attention_f32 would launch for these arguments (a static name such as
 * "flash_mfma_d64"), or NULL with sa_last_error() set if the arguments are rejected (the status
 * is then sa_last_status()). Host only. */
const char* sa_attention_kernel_name(const sa_attn_args* args);

/* ---- kernel plan: the compiled kernel a call launches, and every compiled variant ----
 * The reference picks a matmul tile (app/gpu/ops.js:15-31) and decides fused vs unfused
 * (ops.js:111-112) inside the operator; these host-only queries make the equivalent choice of
 * this library inspectable, so tests can show that every compiled variant runs. */
#define SA_KERNEL_FLASH 1   /* flash_mfma_kernel<head_dim, key_split, bias_mode, mask_variant> */
#define SA_KERNEL_WIDE 2    /* wide_mfma_kernel<head_dim, bias_mode, mask_variant> (no bias or a dense one), + a
                                merge kernel when key_chunks > 1 */
#define SA_KERNEL_GENERIC 3 /* generic_kernel (any head dim <= 1024, any alignment) */
#define SA_KERNEL_FLASH_SMALL 4 /* flash_small_kernel<key_split waves, bias_mode, mask_variant>: head dim 64,
                                   one workgroup per 32 queries, for launches of at most 256 such groups */
#define SA_KERNEL_FLASH_SMALL16 5 /* flash_small16_kernel<bias_mode, mask_variant>: head dim 64, one workgroup
                                     (key_split 4 waves) per 16 queries, for launches of at most 256 such groups */
/* mask_variant beyond the SA_MASK_* values: per-sequence key lengths plus a launch shaped by their
 * host copy (SA_MASK_KEY_LEN with key_len_host). FLASH: the host sequence schedule (8 <= B <= 256,
 * order not the identity). FLASH_SMALL16: sequences of at most 64 keys packed at 2 (or, if that is
 * not enough, 1) waves per 16-query group, shortest first, until a launch of more than 256 groups
 * fits 256 workgroups (B <= 16); workgroups then counts the packed grid. */
#define SA_MASK_VARIANT_KEY_LEN_SCHEDULED 3

typedef struct sa_attn_plan {
  uint32_t struct_size;    /* set to sizeof(sa_attn_plan) before the call */
  int32_t kernel;          /* SA_KERNEL_* */
  int32_t head_dim;        /* head dim the kernel is compiled for (the call's D for GENERIC) */
  int32_t key_split;       /* FLASH, FLASH_SMALL: waves of a workgroup that split one query group's key blocks */
  int32_t key_chunks;      /* WIDE: workgroups that split one query group's keys (merged after) */
  int32_t bias_mode;       /* SA_BIAS_* compiled into the kernel */
  int32_t mask_variant;    /* SA_MASK_* compiled into the kernel, or SA_MASK_VARIANT_KEY_LEN_SCHEDULED */
  int32_t keys_per_step;   /* FLASH: keys a workgroup stages per loop step (32 per splitting wave); WIDE: keys per chunk */
  int64_t workgroups;      /* grid of the attention kernel */
  int64_t workspace_bytes; /* sa_attention_workspace_bytes(args) */
  const char* name;        /* sa_attention_kernel_name(args) (static storage) */
  /* FLASH launches of more units (query tiles) than fit the GPU at once whose last round holds
   * few units: those last units run at one workgroup per CU, in a second launch of the
   * small-launch kernel (tail_kernel SA_KERNEL_FLASH_SMALL, tail_key_split 4 waves per 32 queries)
   * or of the flash kernel split by keys over 2 waves per 32 queries (SA_KERNEL_FLASH, 2), or, when
   * tail_folded is 1, as 64-query units of the latter run inside the first launch (see tail_folded);
   * tail_kernel is 0 when there are no such units, tail_workgroups the number of workgroups (or, folded,
   * of 64-query units) they take. WIDE calls whose query groups fill whole rounds of workgroups
   * (one per CU at head dim 512, two at 256) and a few more: the whole rounds run unsplit (key_chunks
   * 1, workgroups = their groups) and the groups past them follow in a second launch of the wide
   * kernel (tail_kernel SA_KERNEL_WIDE), each split into tail_key_split key chunks merged after;
   * tail_workgroups is that launch's grid. */
  int32_t tail_kernel;
  int32_t tail_key_split;
  int64_t tail_workgroups;
  /* Revision 2 (appended: a revision-1 struct, which ends at tail_workgroups, is still accepted and
   * these fields are then not written). The host sequence schedule of a FLASH call whose
   * mask_variant is SA_MASK_VARIANT_KEY_LEN_SCHEDULED: sequence_order[r] is the sequence launched at
   * rank r (r < B; L2 domain x takes the ranks from x*B/8 on, rounded as the grid's tiles split, to
   * the next domain's first) and order_n is B; otherwise order_n is 0 and sequence_order all zero. */
  int32_t order_n;
  uint8_t sequence_order[256];
  /* Revision 3 (appended: revision-1 and revision-2 structs are still accepted, without it). 1 when
   * the units past the first round run inside the first launch: a launch of one round plus at most
   * half a round, whose first tail_workgroups workgroups (the first one on each CU) each run one
   * 64-query unit of them, split by keys over 2 waves per 32 queries, after their own unit; 0 otherwise. */
  int32_t tail_folded;
} sa_attn_plan;

/* Fills *plan for these arguments: SA_OK, or the status sa_attention_f32 would return for a
 * rejected call (nothing is launched either way). plan->struct_size: sizeof(sa_attn_plan), or the
 * revision-2 size (offsetof(sa_attn_plan, tail_folded)) or the revision-1 size
 * (offsetof(sa_attn_plan, order_n)). Host only. */
int sa_attention_plan(const sa_attn_args* args, sa_attn_plan* plan);

/* Number of compiled kernel variants; sa_attention_variant(i, plan) describes variant i
 * (kernel, head_dim, key_split, bias_mode, mask_variant, name; the other fields 0). FLASH
 * variants come first, one per <head_dim, key_split, bias_mode, mask_variant>. Host only. */
int32_t sa_attention_variant_count(void);
int sa_attention_variant(int32_t index, sa_attn_plan* plan);

/* T5 bidirectional/unidirectional relative-position bucket of each relative position
 * rel = j - i for j in [0, Lk), i in [0, Lq): out[rel + Lq - 1] for the Lq + Lk - 1 values of rel.
 * Follows HF T5Attention._relative_position_bucket in float32, as app/models/t5.js:14-23 does.
 * Host memory, synchronous. */
int sa_t5_bucket_lut(int32_t Lq, int32_t Lk, int32_t num_buckets, int32_t max_distance,
                     int32_t bidirectional, int32_t* out);

/* Dense [H, Lq, Lk] bias from a [num_buckets, H] table and a bucket LUT, written to device memory
 * `out` (app/models/t5.js:55-65, for callers that pass a dense bias). Asynchronous on `stream`. */
int sa_t5_position_bias(const float* table, const int32_t* bucket_lut, int32_t num_buckets, int32_t H,
                        int32_t Lq, int32_t Lk, float* out, void* stream);

/* ---- device runtime helpers (app/gpu/device.js: GPU.empty/fromArray/upload/read/sync) ---- */
int sa_device_count(int32_t* count);
int sa_set_device(int32_t device);
int sa_malloc(void** ptr, size_t bytes);   /* device memory; synchronous */
int sa_free(void* ptr);                    /* synchronous (waits for the device) */
int sa_malloc_host(void** ptr, size_t bytes); /* pinned host memory (hipHostMalloc), e.g. sa_st_upload staging */
int sa_free_host(void* ptr);               /* synchronous (waits for the device) */
int sa_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream); /* returns when copied */
int sa_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream); /* waits for stream */
int sa_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream); /* stream-ordered */
int sa_memset(void* dst, int value, size_t bytes, void* stream);
int sa_stream_create(void** stream);       /* a non-blocking stream at the default priority */
int sa_stream_destroy(void* stream);
int sa_stream_sync(void* stream);          /* the JS shim's gpu.sync() */
int sa_device_sync(void);

/* ---- timing (the timestamp profiler of app/gpu/device.js:272-325) ---- */
int sa_event_create(void** event);
int sa_event_destroy(void* event);
int sa_event_record(void* event, void* stream);
int sa_event_elapsed_ms(float* ms, void* start, void* stop); /* waits for stop */

/* ---- diagnostics ---- */
int sa_version(void);             /* SA_ABI_VERSION */
const char* sa_last_error(void);  /* thread-local; "" when the last call succeeded */
/* Thread-local status of the last library call that returned one (SA_OK after a success), also
 * for the calls whose failure is a NULL name (sa_attention_kernel_name, sa_linear_kernel_name);
 * the reference's async errors surface the same way at sync (app/gpu/device.js:262-268). */
int sa_last_status(void);

#ifdef __cplusplus
}
#endif

#endif /* SUPRA_ATTN_H */
