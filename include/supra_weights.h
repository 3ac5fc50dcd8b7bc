/*
 * supra_weights.h - safetensors weights into MI355X (gfx950) device memory.
 *
 * Replaces the weight loader of Supra2-Img Web (app/weights.js): SafeTensors.open / has / info /
 * f32 / rows, toF32 with its BF16 and F16 decoders, and uploadVector / uploadLinear / uploadConv3
 * (app/weights.js:6-118), which the model loaders call for every tensor (app/models/dit.js:67-104,
 * app/models/t5.js:25-46, 72, app/models/vae.js:14-55).
 *
 * The reference decodes each tensor on the CPU into a Float32Array and uploads it. Here the host
 * side only parses the header and moves the file's raw data section to device memory in one bulk
 * copy (sa_st_upload); every decode, gather and re-layout then runs on the device from that
 * resident copy (sa_to_f32, sa_rows_f32, sa_conv3_pack_f32), at HBM speed.
 *
 * Same library and conventions as supra_attn.h: SA_OK or a negative SA_ERR_* status with
 * sa_last_error(); device calls are stream-ordered and asynchronous; nothing allocates device
 * memory. Element counts and offsets are in elements of the named dtype unless they say bytes.
 */
#ifndef SUPRA_WEIGHTS_H
#define SUPRA_WEIGHTS_H

#include "supra_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- safetensors dtypes (the header's "dtype" strings) ---- */
#define SA_DT_OTHER 0 /* a dtype name this build does not know: listed by sa_st_info, never decoded */
#define SA_DT_F32 1
#define SA_DT_F16 2
#define SA_DT_BF16 3
#define SA_DT_F64 4
#define SA_DT_I64 5
#define SA_DT_I32 6
#define SA_DT_I16 7
#define SA_DT_I8 8
#define SA_DT_U8 9
#define SA_DT_BOOL 10
/* known sizes, not decoded to f32 (app/weights.js:35 throws "unsupported dtype" for them) */
#define SA_DT_U16 11
#define SA_DT_U32 12
#define SA_DT_U64 13
#define SA_DT_F8_E4M3 14
#define SA_DT_F8_E5M2 15

#define SA_ST_MAX_DIMS 8

typedef struct sa_st_file sa_st_file; /* an opened safetensors file or buffer (host side) */

typedef struct sa_st_tensor {
  uint32_t struct_size;          /* sizeof(sa_st_tensor) */
  int32_t dtype;                 /* SA_DT_* */
  int32_t elem_bytes;            /* bytes per element (0 for SA_DT_OTHER) */
  int32_t ndim;                  /* entries of shape[] in use (0 for a scalar) */
  int64_t shape[SA_ST_MAX_DIMS];
  int64_t numel;                 /* product of shape (1 for a scalar) */
  int64_t begin, end;            /* "data_offsets": bytes [begin, end) of the data section */
  char dtype_name[16];           /* the header's dtype string, NUL-terminated */
} sa_st_tensor;

/* SafeTensors.open (app/weights.js:40-47): maps the file and parses its header. A header that is
 * not a JSON object of {dtype, shape, data_offsets} entries (plus an optional "__metadata__"
 * object), or an entry whose bytes do not fit the data section or do not match shape x dtype size,
 * is SA_ERR_FORMAT. Host only: no device call. */
int sa_st_open(const char* path, sa_st_file** out);
/* The same over a caller-owned buffer of the whole file, which must outlive the handle. */
int sa_st_open_memory(const void* bytes, int64_t size, sa_st_file** out);
int sa_st_close(sa_st_file* file);

int64_t sa_st_count(const sa_st_file* file);                /* tensors, in header order */
const char* sa_st_name(const sa_st_file* file, int64_t i);  /* NULL when i is out of range */
/* has() / info() (app/weights.js:56-64): SA_OK, or SA_ERR_NOT_FOUND ("missing tensor <name>"). */
int sa_st_info(const sa_st_file* file, const char* name, sa_st_tensor* out);

/* "__metadata__" (app/weights.js:44): string values as stored, any other JSON value as its text. */
int64_t sa_st_metadata_count(const sa_st_file* file);
const char* sa_st_metadata_key(const sa_st_file* file, int64_t i);
const char* sa_st_metadata_value(const sa_st_file* file, const char* key); /* NULL when absent */

int64_t sa_st_data_bytes(const sa_st_file* file);  /* size of the data section */
const void* sa_st_data(const sa_st_file* file);    /* host address of the data section */

/* Copies bytes [begin, end) of the data section to device memory at dst, and returns when the copy
 * has completed. With `staging` (pinned host memory from hipHostMalloc, at least 2 MiB) the copy
 * runs in chunks through the two halves of it, so that filling one half from the file (several host
 * threads) overlaps the DMA of the other; with staging == NULL the runtime copies from the mapping
 * itself. */
int sa_st_upload(const sa_st_file* file, int64_t begin, int64_t end, void* dst, void* staging,
                 int64_t staging_bytes, void* stream);

/* ---- device-side decoding from a resident copy of the data section ---- */

/* toF32 (app/weights.js:28-37): dst[i] = element i of src as float32, for n elements of `dtype`:
 * F32 bit copy; BF16 bits << 16 (bf16ToF32, :6-12); F16 exactly (f16ToF32, :14-25; every NaN
 * becomes the quiet NaN 0x7fc00000, as JS's NaN does); F64 rounded to nearest even; I64 via the
 * nearest double (Number(), then rounded to float32); I32/I16/I8/U8/BOOL exactly. src needs only
 * the alignment of its dtype (any byte offset for 1-byte types); dst is 4-byte aligned. The other
 * SA_DT_* values are SA_ERR_UNSUPPORTED, as the reference throws for them. */
int sa_to_f32(const void* src, int32_t dtype, int64_t n, float* dst, void* stream);

/* rows (app/weights.js:73-83): dst[i, :] = toF32(table[ids[i], :]) for a [rows, dim] table, n_ids
 * device int32 ids. An id outside [0, rows) gives a zero row (the reference reads the bytes that
 * follow the table in the file instead). */
int sa_rows_f32(const void* table, int32_t dtype, int64_t rows, int64_t dim, const int32_t* ids,
                int64_t n_ids, float* dst, void* stream);

/* uploadConv3 (app/weights.js:105-118): a 3x3 conv weight [cout, cin, 3, 3] of `dtype` into the
 * implicit-GEMM layout [cout, 3, 3, cin_pad] float32, dst[(o*9 + t)*cin_pad + i] = w[(o*cin + i)*9
 * + t], zero for cin <= i < cin_pad (cin_pad 0 means cin; otherwise cin_pad >= cin). */
int sa_conv3_pack_f32(const void* w, int32_t dtype, int32_t cout, int32_t cin, int32_t cin_pad,
                      float* dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SUPRA_WEIGHTS_H */
