/*
 * Node.js N-API addon over the attention library's C ABI (include/supra_attn.h).
 *
 * It gives the JS shim (js/device.js, js/ops.js) what app/gpu/device.js gave app/gpu/ops.js:
 * device buffers (GPU.empty / fromArray / read, device.js:144-191), one in-order queue
 * (device.js:1-5: work is stream-ordered, so a buffer released right after a call is safe to
 * reuse) and sync (device.js:255-259). The attention call itself maps ops.attention's options
 * object (app/gpu/ops.js:109) onto sa_attn_args.
 *
 * Device pointers cross into JS as External values. Every C ABI status other than SA_OK becomes a
 * thrown JS Error whose code is the status ("SA_ERR_INVALID", ...) and whose message is
 * sa_last_error(). The stream is created on first use, so loading the addon on a host without a
 * GPU succeeds (only calls that need the device fail).
 */
#include <node_api.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "supra_attn.h"
#include "supra_linear.h"
#include "supra_vae.h"
#include "supra_weights.h"

static void* g_stream = NULL;
static int g_stream_ready = 0;

#define NAPI_CALL(env, call)                                         \
  do {                                                               \
    napi_status st_ = (call);                                        \
    if (st_ != napi_ok) {                                            \
      const napi_extended_error_info* info_ = NULL;                  \
      napi_get_last_error_info((env), &info_);                       \
      napi_throw_error((env), "SA_NAPI",                             \
                       info_ && info_->error_message                 \
                           ? info_->error_message                    \
                           : "N-API call failed");                   \
      return NULL;                                                   \
    }                                                                \
  } while (0)

static const char* status_code(int rc) {
  switch (rc) {
    case SA_ERR_INVALID: return "SA_ERR_INVALID";
    case SA_ERR_UNSUPPORTED: return "SA_ERR_UNSUPPORTED";
    case SA_ERR_HIP: return "SA_ERR_HIP";
    case SA_ERR_ALIAS: return "SA_ERR_ALIAS";
    case SA_ERR_NOT_FOUND: return "SA_ERR_NOT_FOUND";
    case SA_ERR_IO: return "SA_ERR_IO";
    case SA_ERR_FORMAT: return "SA_ERR_FORMAT";
    default: return "SA_ERR";
  }
}

/* Throws for a failed C ABI status; returns 1 if it threw. */
static int throw_if(napi_env env, int rc) {
  if (rc == SA_OK) return 0;
  const char* msg = sa_last_error();
  napi_throw_error(env, status_code(rc), msg && msg[0] ? msg : "supra_attn call failed");
  return 1;
}

static int ensure_stream(napi_env env) {
  if (g_stream_ready) return 0;
  if (throw_if(env, sa_stream_create(&g_stream))) return 1;
  g_stream_ready = 1;
  return 0;
}

static napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok) {
    napi_throw_error(env, "SA_NAPI", "cannot read arguments");
    return 1;
  }
  for (size_t i = argc; i < want; ++i) napi_get_undefined(env, &argv[i]);
  return 0;
}

static int is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok) return 1;
  return t == napi_undefined || t == napi_null;
}

/* External -> pointer; undefined/null -> NULL. Anything else throws. */
static int get_ptr(napi_env env, napi_value v, void** out, const char* what) {
  *out = NULL;
  if (is_nullish(env, v)) return 0;
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_external) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s must be a device buffer handle", what);
    napi_throw_type_error(env, "SA_ERR_INVALID", msg);
    return 1;
  }
  return napi_get_value_external(env, v, out) == napi_ok ? 0 : 1;
}

static int get_i64(napi_env env, napi_value v, int64_t dflt, int64_t* out, const char* what) {
  if (is_nullish(env, v)) {
    *out = dflt;
    return 0;
  }
  double d;
  if (napi_get_value_double(env, v, &d) != napi_ok || d != d || d != (double)(int64_t)d) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s must be an integer", what);
    napi_throw_type_error(env, "SA_ERR_INVALID", msg);
    return 1;
  }
  *out = (int64_t)d;
  return 0;
}

static int get_f64(napi_env env, napi_value v, double dflt, double* out, const char* what) {
  if (is_nullish(env, v)) {
    *out = dflt;
    return 0;
  }
  if (napi_get_value_double(env, v, out) != napi_ok) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s must be a number", what);
    napi_throw_type_error(env, "SA_ERR_INVALID", msg);
    return 1;
  }
  return 0;
}

static int prop(napi_env env, napi_value obj, const char* name, napi_value* out) {
  bool has = false;
  if (napi_has_named_property(env, obj, name, &has) != napi_ok) return 1;
  if (!has) {
    napi_get_undefined(env, out);
    return 0;
  }
  return napi_get_named_property(env, obj, name, out) == napi_ok ? 0 : 1;
}

static int prop_i64(napi_env env, napi_value obj, const char* name, int64_t dflt, int64_t* out) {
  napi_value v;
  if (prop(env, obj, name, &v)) return 1;
  return get_i64(env, v, dflt, out, name);
}

static int prop_ptr(napi_env env, napi_value obj, const char* name, void** out) {
  napi_value v;
  if (prop(env, obj, name, &v)) return 1;
  return get_ptr(env, v, out, name);
}

/* opts -> sa_attn_args. Field names are those of app/gpu/ops.js:109 (q, k, v, Lq, Lk, H, D, ldq,
 * ldk, ldv, qOff, kOff, vOff, oOff, scale) plus out -> o, and the extension fields B, ldo, sq, sk,
 * sv, so, biasMode, bias, sbias, bucketLut, numBuckets, maskMode, keyLen, keyMask, smask,
 * workspace, workspaceBytes. */
static int fill_args(napi_env env, napi_value o, sa_attn_args* a) {
  memset(a, 0, sizeof *a);
  a->struct_size = sizeof *a;
  int64_t B, H, D, Lq, Lk, bm, mm, nb;
  void *q, *k, *v, *out, *bias, *lut, *kl, *km, *ws;
  double scale;
  napi_value sv;
  if (prop_i64(env, o, "B", 1, &B) || prop_i64(env, o, "H", -1, &H) || prop_i64(env, o, "D", -1, &D) ||
      prop_i64(env, o, "Lq", -1, &Lq) || prop_i64(env, o, "Lk", -1, &Lk))
    return 1;
  if (prop_ptr(env, o, "q", &q) || prop_ptr(env, o, "k", &k) || prop_ptr(env, o, "v", &v) ||
      prop_ptr(env, o, "out", &out) || prop_ptr(env, o, "bias", &bias) || prop_ptr(env, o, "bucketLut", &lut) ||
      prop_ptr(env, o, "keyLen", &kl) || prop_ptr(env, o, "keyMask", &km) || prop_ptr(env, o, "workspace", &ws))
    return 1;
  if (prop_i64(env, o, "qOff", 0, &a->q_off) || prop_i64(env, o, "kOff", 0, &a->k_off) ||
      prop_i64(env, o, "vOff", 0, &a->v_off) || prop_i64(env, o, "oOff", 0, &a->o_off) ||
      prop_i64(env, o, "ldq", -1, &a->ldq) || prop_i64(env, o, "ldk", -1, &a->ldk) ||
      prop_i64(env, o, "ldv", -1, &a->ldv) || prop_i64(env, o, "ldo", 0, &a->ldo) ||
      prop_i64(env, o, "sq", 0, &a->sq) || prop_i64(env, o, "sk", 0, &a->sk) || prop_i64(env, o, "sv", 0, &a->sv) ||
      prop_i64(env, o, "so", 0, &a->so) || prop_i64(env, o, "sbias", 0, &a->sbias) ||
      prop_i64(env, o, "smask", 0, &a->smask) || prop_i64(env, o, "biasMode", SA_BIAS_NONE, &bm) ||
      prop_i64(env, o, "maskMode", SA_MASK_NONE, &mm) || prop_i64(env, o, "numBuckets", 0, &nb) ||
      prop_i64(env, o, "workspaceBytes", 0, &a->workspace_bytes))
    return 1;
  if (prop(env, o, "scale", &sv) || get_f64(env, sv, 1.0, &scale, "scale")) return 1;
  if (B < -0x7fffffffLL || B > 0x7fffffffLL || H > 0x7fffffffLL || D > 0x7fffffffLL || Lq > 0x7fffffffLL ||
      Lk > 0x7fffffffLL) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "sizes must fit in int32");
    return 1;
  }
  a->B = (int32_t)B;
  a->H = (int32_t)H;
  a->D = (int32_t)D;
  a->Lq = (int32_t)Lq;
  a->Lk = (int32_t)Lk;
  a->q = (const float*)q;
  a->k = (const float*)k;
  a->v = (const float*)v;
  a->o = (float*)out;
  a->scale = (float)scale;
  a->bias_mode = (int32_t)bm;
  a->bias = (const float*)bias;
  a->bucket_lut = (const int32_t*)lut;
  a->num_buckets = (int32_t)nb;
  a->mask_mode = (int32_t)mm;
  a->key_len = (const int32_t*)kl;
  a->key_mask = (const uint8_t*)km;
  a->workspace = ws;
  return 0;
}

/* opts -> sa_linear_args: M, N, K, x, xOff, ldx, w, ldw, bias, alpha (default 1), act, epilogue,
 * gate, gateOff, y, yOff, ldy (the JS shim maps app/gpu/ops.js:35-43's linear() onto these). */
static int fill_linear(napi_env env, napi_value o, sa_linear_args* a) {
  memset(a, 0, sizeof *a);
  a->struct_size = sizeof *a;
  int64_t M, N, K, act, epi;
  void *x, *w, *bias, *gate, *y;
  double alpha;
  napi_value av;
  if (prop_i64(env, o, "M", -1, &M) || prop_i64(env, o, "N", -1, &N) || prop_i64(env, o, "K", -1, &K) ||
      prop_i64(env, o, "act", SA_ACT_NONE, &act) || prop_i64(env, o, "epilogue", SA_EPI_STORE, &epi) ||
      prop_i64(env, o, "xOff", 0, &a->x_off) || prop_i64(env, o, "ldx", 0, &a->ldx) ||
      prop_i64(env, o, "ldw", 0, &a->ldw) || prop_i64(env, o, "gateOff", 0, &a->gate_off) ||
      prop_i64(env, o, "yOff", 0, &a->y_off) || prop_i64(env, o, "ldy", 0, &a->ldy))
    return 1;
  if (prop_ptr(env, o, "x", &x) || prop_ptr(env, o, "w", &w) || prop_ptr(env, o, "bias", &bias) ||
      prop_ptr(env, o, "gate", &gate) || prop_ptr(env, o, "y", &y))
    return 1;
  if (prop(env, o, "alpha", &av) || get_f64(env, av, 1.0, &alpha, "alpha")) return 1;
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL || M < -1 || N < -1 || K < -1) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "sizes must fit in int32");
    return 1;
  }
  a->M = (int32_t)M;
  a->N = (int32_t)N;
  a->K = (int32_t)K;
  a->x = (const float*)x;
  a->w = (const float*)w;
  a->bias = (const float*)bias;
  a->alpha = (float)alpha;
  a->act = (int32_t)act;
  a->epilogue = (int32_t)epi;
  a->gate = (const float*)gate;
  a->y = (float*)y;
  return 0;
}

static napi_value js_linear(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_linear_args a;
  if (fill_linear(env, argv[0], &a)) return NULL;
  /* validate before touching the device, so a bad call reports its own error on any host */
  if (sa_linear_kernel_name(&a) == NULL) {
    throw_if(env, SA_ERR_INVALID);
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_linear_f32(&a, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_linear_kernel_name(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_linear_args a;
  if (fill_linear(env, argv[0], &a)) return NULL;
  const char* name = sa_linear_kernel_name(&a);
  if (!name) {
    throw_if(env, SA_ERR_INVALID);
    return NULL;
  }
  napi_value r;
  NAPI_CALL(env, napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &r));
  return r;
}

/* opts -> sa_vae_attn_args: HW, C, groups (32), eps (1e-6), x, gamma, beta, wqkv, bqkv, wo, bo,
 * out, workspace, workspaceBytes. */
static int fill_vae(napi_env env, napi_value o, sa_vae_attn_args* a) {
  memset(a, 0, sizeof *a);
  a->struct_size = sizeof *a;
  int64_t HW, C, G;
  double eps;
  napi_value ev;
  void *x, *gamma, *beta, *wqkv, *bqkv, *wo, *bo, *out, *ws;
  if (prop_i64(env, o, "HW", -1, &HW) || prop_i64(env, o, "C", -1, &C) || prop_i64(env, o, "groups", 32, &G) ||
      prop_i64(env, o, "workspaceBytes", 0, &a->workspace_bytes))
    return 1;
  if (prop(env, o, "eps", &ev) || get_f64(env, ev, 1e-6, &eps, "eps")) return 1;
  if (prop_ptr(env, o, "x", &x) || prop_ptr(env, o, "gamma", &gamma) || prop_ptr(env, o, "beta", &beta) ||
      prop_ptr(env, o, "wqkv", &wqkv) || prop_ptr(env, o, "bqkv", &bqkv) || prop_ptr(env, o, "wo", &wo) ||
      prop_ptr(env, o, "bo", &bo) || prop_ptr(env, o, "out", &out) || prop_ptr(env, o, "workspace", &ws))
    return 1;
  if (HW > 0x7fffffffLL || C > 0x7fffffffLL || G > 0x7fffffffLL || HW < -1 || C < -1 || G < -1) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "sizes must fit in int32");
    return 1;
  }
  a->HW = (int32_t)HW;
  a->C = (int32_t)C;
  a->groups = (int32_t)G;
  a->eps = (float)eps;
  a->x = (const float*)x;
  a->gamma = (const float*)gamma;
  a->beta = (const float*)beta;
  a->wqkv = (const float*)wqkv;
  a->bqkv = (const float*)bqkv;
  a->wo = (const float*)wo;
  a->bo = (const float*)bo;
  a->out = (float*)out;
  a->workspace = ws;
  return 0;
}

static napi_value js_vae_attention(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_vae_attn_args a;
  if (fill_vae(env, argv[0], &a)) return NULL;
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_vae_attention_f32(&a, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_vae_workspace_bytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_vae_attn_args a;
  if (fill_vae(env, argv[0], &a)) return NULL;
  const int64_t n = sa_vae_attention_workspace_bytes(&a);
  if (n < 0) {
    throw_if(env, (int)n);
    return NULL;
  }
  napi_value r;
  NAPI_CALL(env, napi_create_double(env, (double)n, &r));
  return r;
}

static napi_value js_attention(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_attn_args a;
  if (fill_args(env, argv[0], &a)) return NULL;
  /* validate before touching the device, so a bad call reports its own error on any host */
  if (sa_attention_kernel_name(&a) == NULL) {
    throw_if(env, SA_ERR_INVALID);
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_attention_f32(&a, g_stream))) return NULL;
  return undefined(env);
}

/* Bytes of device workspace the call needs (sa_attention_workspace_bytes); throws if rejected. */
static napi_value js_workspace_bytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_attn_args a;
  if (fill_args(env, argv[0], &a)) return NULL;
  const int64_t n = sa_attention_workspace_bytes(&a);
  if (n < 0) {
    throw_if(env, (int)n);
    return NULL;
  }
  napi_value r;
  NAPI_CALL(env, napi_create_double(env, (double)n, &r));
  return r;
}

static napi_value js_kernel_name(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_attn_args a;
  if (fill_args(env, argv[0], &a)) return NULL;
  const char* name = sa_attention_kernel_name(&a);
  if (!name) {
    throw_if(env, SA_ERR_INVALID);
    return NULL;
  }
  napi_value r;
  NAPI_CALL(env, napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &r));
  return r;
}

static napi_value js_version(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value r;
  NAPI_CALL(env, napi_create_int32(env, sa_version(), &r));
  return r;
}

static napi_value js_device_count(napi_env env, napi_callback_info info) {
  (void)info;
  int32_t n = 0;
  sa_device_count(&n); /* 0 when no device is visible */
  napi_value r;
  NAPI_CALL(env, napi_create_int32(env, n, &r));
  return r;
}

static napi_value js_malloc(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  int64_t bytes;
  if (get_i64(env, argv[0], -1, &bytes, "bytes")) return NULL;
  if (bytes < 0) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "bytes must be >= 0");
    return NULL;
  }
  void* p = NULL;
  if (throw_if(env, sa_malloc(&p, (size_t)bytes))) return NULL;
  napi_value r;
  NAPI_CALL(env, napi_create_external(env, p, NULL, NULL, &r));
  return r;
}

static napi_value js_free(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  void* p;
  if (get_ptr(env, argv[0], &p, "buffer")) return NULL;
  if (g_stream_ready && throw_if(env, sa_stream_sync(g_stream))) return NULL;
  if (throw_if(env, sa_free(p))) return NULL;
  return undefined(env);
}

/* (buffer, typedArray, byteOffset) -> the typed array's bytes at buffer + byteOffset */
static int typed_bytes(napi_env env, napi_value ta, void** data, size_t* bytes) {
  bool is_ta = false;
  napi_is_typedarray(env, ta, &is_ta);
  if (!is_ta) {
    napi_throw_type_error(env, "SA_ERR_INVALID", "expected a TypedArray");
    return 1;
  }
  napi_typedarray_type type;
  size_t length, offset;
  napi_value ab;
  if (napi_get_typedarray_info(env, ta, &type, &length, data, &ab, &offset) != napi_ok) {
    napi_throw_error(env, "SA_NAPI", "cannot read TypedArray");
    return 1;
  }
  size_t elem = 1;
  switch (type) {
    case napi_int16_array: case napi_uint16_array: elem = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
    default: elem = 1; break;
  }
  *bytes = length * elem;
  return 0;
}

static napi_value js_upload(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (get_args(env, info, 3, argv)) return NULL;
  void* dst;
  void* src;
  size_t bytes;
  int64_t off;
  if (get_ptr(env, argv[0], &dst, "buffer") || typed_bytes(env, argv[1], &src, &bytes) ||
      get_i64(env, argv[2], 0, &off, "byteOffset"))
    return NULL;
  if (!dst || off < 0) {
    napi_throw_error(env, "SA_ERR_INVALID", "upload needs a buffer and byteOffset >= 0");
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_memcpy_h2d((char*)dst + off, src, bytes, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_download(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (get_args(env, info, 3, argv)) return NULL;
  void* src;
  void* dst;
  size_t bytes;
  int64_t off;
  if (get_ptr(env, argv[0], &src, "buffer") || typed_bytes(env, argv[1], &dst, &bytes) ||
      get_i64(env, argv[2], 0, &off, "byteOffset"))
    return NULL;
  if (!src || off < 0) {
    napi_throw_error(env, "SA_ERR_INVALID", "download needs a buffer and byteOffset >= 0");
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_memcpy_d2h(dst, (const char*)src + off, bytes, g_stream))) return NULL;
  return argv[1];
}

static napi_value js_memset(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (get_args(env, info, 3, argv)) return NULL;
  void* dst;
  int64_t value, bytes;
  if (get_ptr(env, argv[0], &dst, "buffer") || get_i64(env, argv[1], 0, &value, "value") ||
      get_i64(env, argv[2], -1, &bytes, "bytes"))
    return NULL;
  if (bytes < 0) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "bytes must be >= 0");
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_memset(dst, (int)value, (size_t)bytes, g_stream))) return NULL;
  return undefined(env);
}

/* (dst, dstByteOffset, src, srcByteOffset, bytes): device-to-device copy, stream-ordered */
static napi_value js_copy(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (get_args(env, info, 5, argv)) return NULL;
  void* dst;
  void* src;
  int64_t doff, soff, bytes;
  if (get_ptr(env, argv[0], &dst, "dst") || get_i64(env, argv[1], 0, &doff, "dstByteOffset") ||
      get_ptr(env, argv[2], &src, "src") || get_i64(env, argv[3], 0, &soff, "srcByteOffset") ||
      get_i64(env, argv[4], -1, &bytes, "bytes"))
    return NULL;
  if (!dst || !src || doff < 0 || soff < 0 || bytes < 0) {
    napi_throw_error(env, "SA_ERR_INVALID", "copy needs two buffers and offsets, bytes >= 0");
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_memcpy_d2d((char*)dst + doff, (const char*)src + soff, (size_t)bytes, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_sync(napi_env env, napi_callback_info info) {
  (void)info;
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_stream_sync(g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_bucket_lut(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (get_args(env, info, 5, argv)) return NULL;
  int64_t Lq, Lk, nb, md, bidir;
  if (get_i64(env, argv[0], -1, &Lq, "Lq") || get_i64(env, argv[1], -1, &Lk, "Lk") ||
      get_i64(env, argv[2], 32, &nb, "numBuckets") || get_i64(env, argv[3], 128, &md, "maxDistance"))
    return NULL;
  bool b = true;
  if (!is_nullish(env, argv[4]) && napi_get_value_bool(env, argv[4], &b) != napi_ok) {
    napi_throw_type_error(env, "SA_ERR_INVALID", "bidirectional must be a boolean");
    return NULL;
  }
  bidir = b ? 1 : 0;
  if (Lq < 1 || Lk < 1 || Lq > 0x3fffffff || Lk > 0x3fffffff) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "Lq and Lk must be in [1, 2^30)");
    return NULL;
  }
  const size_t n = (size_t)(Lq + Lk - 1);
  napi_value ab, arr;
  void* data = NULL;
  NAPI_CALL(env, napi_create_arraybuffer(env, n * sizeof(int32_t), &data, &ab));
  if (throw_if(env, sa_t5_bucket_lut((int32_t)Lq, (int32_t)Lk, (int32_t)nb, (int32_t)md, (int32_t)bidir,
                                     (int32_t*)data)))
    return NULL;
  NAPI_CALL(env, napi_create_typedarray(env, napi_int32_array, n, ab, 0, &arr));
  return arr;
}

static napi_value js_position_bias(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (get_args(env, info, 7, argv)) return NULL;
  void *table, *lut, *out;
  int64_t nb, H, Lq, Lk;
  if (get_ptr(env, argv[0], &table, "table") || get_ptr(env, argv[1], &lut, "bucketLut") ||
      get_i64(env, argv[2], -1, &nb, "numBuckets") || get_i64(env, argv[3], -1, &H, "H") ||
      get_i64(env, argv[4], -1, &Lq, "Lq") || get_i64(env, argv[5], -1, &Lk, "Lk") ||
      get_ptr(env, argv[6], &out, "out"))
    return NULL;
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_t5_position_bias((const float*)table, (const int32_t*)lut, (int32_t)nb, (int32_t)H,
                                        (int32_t)Lq, (int32_t)Lk, (float*)out, g_stream)))
    return NULL;
  return undefined(env);
}

static napi_value js_event_create(napi_env env, napi_callback_info info) {
  (void)info;
  void* ev = NULL;
  if (throw_if(env, sa_event_create(&ev))) return NULL;
  napi_value r;
  NAPI_CALL(env, napi_create_external(env, ev, NULL, NULL, &r));
  return r;
}

static napi_value js_event_record(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  void* ev;
  if (get_ptr(env, argv[0], &ev, "event")) return NULL;
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_event_record(ev, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_event_elapsed(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (get_args(env, info, 2, argv)) return NULL;
  void *a, *b;
  if (get_ptr(env, argv[0], &a, "start") || get_ptr(env, argv[1], &b, "stop")) return NULL;
  float ms = 0.f;
  if (throw_if(env, sa_event_elapsed_ms(&ms, a, b))) return NULL;
  napi_value r;
  NAPI_CALL(env, napi_create_double(env, ms, &r));
  return r;
}

static napi_value js_event_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  void* ev;
  if (get_ptr(env, argv[0], &ev, "event")) return NULL;
  if (throw_if(env, sa_event_destroy(ev))) return NULL;
  return undefined(env);
}

/* ---- safetensors (include/supra_weights.h) ---- */

/* The JS handle of an opened file: closed by stClose or, failing that, when collected. Bytes
 * opened from a JS array are copied, so that the handle does not depend on the array's storage. */
typedef struct StHandle {
  sa_st_file* f;
  void* copy;
} StHandle;

static void st_finalize(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  StHandle* h = (StHandle*)data;
  if (h->f) sa_st_close(h->f);
  free(h->copy);
  free(h);
}

static napi_value st_wrap(napi_env env, sa_st_file* f, void* copy) {
  StHandle* h = (StHandle*)calloc(1, sizeof *h);
  if (!h) {
    sa_st_close(f);
    free(copy);
    napi_throw_error(env, "SA_NAPI", "out of host memory");
    return NULL;
  }
  h->f = f;
  h->copy = copy;
  napi_value r;
  if (napi_create_external(env, h, st_finalize, NULL, &r) != napi_ok) {
    st_finalize(env, h, NULL);
    napi_throw_error(env, "SA_NAPI", "cannot create the file handle");
    return NULL;
  }
  return r;
}

static int st_get(napi_env env, napi_value v, sa_st_file** out) {
  void* p = NULL;
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_external || napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, "SA_ERR_INVALID", "expected a safetensors handle");
    return 1;
  }
  *out = ((StHandle*)p)->f;
  if (!*out) {
    napi_throw_error(env, "SA_ERR_INVALID", "the safetensors handle is closed");
    return 1;
  }
  return 0;
}

static int get_string(napi_env env, napi_value v, char* buf, size_t cap, const char* what) {
  size_t len = 0;
  if (napi_get_value_string_utf8(env, v, buf, cap, &len) != napi_ok || len + 1 >= cap) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s must be a string shorter than %zu bytes", what, cap - 1);
    napi_throw_type_error(env, "SA_ERR_INVALID", msg);
    return 1;
  }
  return 0;
}

static napi_value js_st_open(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  char path[4096];
  if (get_string(env, argv[0], path, sizeof path, "path")) return NULL;
  sa_st_file* f = NULL;
  if (throw_if(env, sa_st_open(path, &f))) return NULL;
  return st_wrap(env, f, NULL);
}

static napi_value js_st_open_bytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  void* data;
  size_t bytes;
  if (typed_bytes(env, argv[0], &data, &bytes)) return NULL;
  void* copy = malloc(bytes ? bytes : 1);
  if (!copy) {
    napi_throw_error(env, "SA_NAPI", "out of host memory");
    return NULL;
  }
  memcpy(copy, data, bytes);
  sa_st_file* f = NULL;
  if (throw_if(env, sa_st_open_memory(copy, (int64_t)bytes, &f))) {
    free(copy);
    return NULL;
  }
  return st_wrap(env, f, copy);
}

static napi_value js_st_close(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  void* p = NULL;
  napi_valuetype t;
  if (napi_typeof(env, argv[0], &t) == napi_ok && t == napi_external && napi_get_value_external(env, argv[0], &p) == napi_ok &&
      p) {
    StHandle* h = (StHandle*)p;
    if (h->f) sa_st_close(h->f);
    h->f = NULL;
    free(h->copy);
    h->copy = NULL;
  }
  return undefined(env);
}

static napi_value js_st_names(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_st_file* f;
  if (st_get(env, argv[0], &f)) return NULL;
  const int64_t n = sa_st_count(f);
  napi_value arr, s;
  NAPI_CALL(env, napi_create_array_with_length(env, (size_t)n, &arr));
  for (int64_t i = 0; i < n; ++i) {
    NAPI_CALL(env, napi_create_string_utf8(env, sa_st_name(f, i), NAPI_AUTO_LENGTH, &s));
    NAPI_CALL(env, napi_set_element(env, arr, (uint32_t)i, s));
  }
  return arr;
}

/* (handle, name) -> {dtype, shape, data_offsets, code} (the header entry, app/weights.js:60-64) */
static napi_value js_st_info(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (get_args(env, info, 2, argv)) return NULL;
  sa_st_file* f;
  char name[4096];
  if (st_get(env, argv[0], &f) || get_string(env, argv[1], name, sizeof name, "name")) return NULL;
  sa_st_tensor t;
  memset(&t, 0, sizeof t);
  t.struct_size = sizeof t;
  if (throw_if(env, sa_st_info(f, name, &t))) return NULL;
  napi_value o, v, shape, offs;
  NAPI_CALL(env, napi_create_object(env, &o));
  NAPI_CALL(env, napi_create_string_utf8(env, t.dtype_name, NAPI_AUTO_LENGTH, &v));
  NAPI_CALL(env, napi_set_named_property(env, o, "dtype", v));
  NAPI_CALL(env, napi_create_array_with_length(env, (size_t)t.ndim, &shape));
  for (int i = 0; i < t.ndim; ++i) {
    NAPI_CALL(env, napi_create_double(env, (double)t.shape[i], &v));
    NAPI_CALL(env, napi_set_element(env, shape, (uint32_t)i, v));
  }
  NAPI_CALL(env, napi_set_named_property(env, o, "shape", shape));
  NAPI_CALL(env, napi_create_array_with_length(env, 2, &offs));
  NAPI_CALL(env, napi_create_double(env, (double)t.begin, &v));
  NAPI_CALL(env, napi_set_element(env, offs, 0, v));
  NAPI_CALL(env, napi_create_double(env, (double)t.end, &v));
  NAPI_CALL(env, napi_set_element(env, offs, 1, v));
  NAPI_CALL(env, napi_set_named_property(env, o, "data_offsets", offs));
  NAPI_CALL(env, napi_create_int32(env, t.dtype, &v));
  NAPI_CALL(env, napi_set_named_property(env, o, "code", v));
  NAPI_CALL(env, napi_create_double(env, (double)t.numel, &v));
  NAPI_CALL(env, napi_set_named_property(env, o, "numel", v));
  return o;
}

static napi_value js_st_has(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (get_args(env, info, 2, argv)) return NULL;
  sa_st_file* f;
  char name[4096];
  if (st_get(env, argv[0], &f) || get_string(env, argv[1], name, sizeof name, "name")) return NULL;
  sa_st_tensor t;
  memset(&t, 0, sizeof t);
  t.struct_size = sizeof t;
  napi_value r;
  NAPI_CALL(env, napi_get_boolean(env, sa_st_info(f, name, &t) == SA_OK, &r));
  return r;
}

static napi_value js_st_metadata(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_st_file* f;
  if (st_get(env, argv[0], &f)) return NULL;
  napi_value o, v;
  NAPI_CALL(env, napi_create_object(env, &o));
  const int64_t n = sa_st_metadata_count(f);
  for (int64_t i = 0; i < n; ++i) {
    const char* k = sa_st_metadata_key(f, i);
    NAPI_CALL(env, napi_create_string_utf8(env, sa_st_metadata_value(f, k), NAPI_AUTO_LENGTH, &v));
    NAPI_CALL(env, napi_set_named_property(env, o, k, v));
  }
  return o;
}

static napi_value js_st_data_bytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_st_file* f;
  if (st_get(env, argv[0], &f)) return NULL;
  napi_value r;
  NAPI_CALL(env, napi_create_double(env, (double)sa_st_data_bytes(f), &r));
  return r;
}

/* (handle, begin, end, dst, dstByteOffset, staging|null, stagingBytes): returns when copied */
static napi_value js_st_upload(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (get_args(env, info, 7, argv)) return NULL;
  sa_st_file* f;
  int64_t begin, end, doff, sbytes;
  void *dst, *staging;
  if (st_get(env, argv[0], &f) || get_i64(env, argv[1], 0, &begin, "begin") || get_i64(env, argv[2], -1, &end, "end") ||
      get_ptr(env, argv[3], &dst, "dst") || get_i64(env, argv[4], 0, &doff, "dstByteOffset") ||
      get_ptr(env, argv[5], &staging, "staging") || get_i64(env, argv[6], 0, &sbytes, "stagingBytes"))
    return NULL;
  if (doff < 0) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "dstByteOffset must be >= 0");
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_st_upload(f, begin, end, dst ? (char*)dst + doff : NULL, staging, sbytes, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_malloc_host(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  int64_t bytes;
  if (get_i64(env, argv[0], -1, &bytes, "bytes")) return NULL;
  if (bytes < 0) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "bytes must be >= 0");
    return NULL;
  }
  void* p = NULL;
  if (throw_if(env, sa_malloc_host(&p, (size_t)bytes))) return NULL;
  napi_value r;
  NAPI_CALL(env, napi_create_external(env, p, NULL, NULL, &r));
  return r;
}

static napi_value js_free_host(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  void* p;
  if (get_ptr(env, argv[0], &p, "buffer")) return NULL;
  if (throw_if(env, sa_free_host(p))) return NULL;
  return undefined(env);
}

/* (src, srcByteOffset, dtype, n, dst, dstByteOffset) */
static napi_value js_to_f32(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  if (get_args(env, info, 6, argv)) return NULL;
  void *src, *dst;
  int64_t soff, dtype, n, doff;
  if (get_ptr(env, argv[0], &src, "src") || get_i64(env, argv[1], 0, &soff, "srcByteOffset") ||
      get_i64(env, argv[2], -1, &dtype, "dtype") || get_i64(env, argv[3], -1, &n, "n") ||
      get_ptr(env, argv[4], &dst, "dst") || get_i64(env, argv[5], 0, &doff, "dstByteOffset"))
    return NULL;
  if (!src || !dst || soff < 0 || doff < 0) {
    napi_throw_error(env, "SA_ERR_INVALID", "toF32 needs two buffers and offsets >= 0");
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_to_f32((char*)src + soff, (int32_t)dtype, n, (float*)((char*)dst + doff), g_stream))) return NULL;
  return undefined(env);
}

/* (table, tableByteOffset, dtype, rows, dim, ids, nIds, dst) */
static napi_value js_rows_f32(napi_env env, napi_callback_info info) {
  napi_value argv[8];
  if (get_args(env, info, 8, argv)) return NULL;
  void *table, *ids, *dst;
  int64_t toff, dtype, rows, dim, n_ids;
  if (get_ptr(env, argv[0], &table, "table") || get_i64(env, argv[1], 0, &toff, "tableByteOffset") ||
      get_i64(env, argv[2], -1, &dtype, "dtype") || get_i64(env, argv[3], -1, &rows, "rows") ||
      get_i64(env, argv[4], -1, &dim, "dim") || get_ptr(env, argv[5], &ids, "ids") ||
      get_i64(env, argv[6], -1, &n_ids, "nIds") || get_ptr(env, argv[7], &dst, "dst"))
    return NULL;
  if (!table || toff < 0) {
    napi_throw_error(env, "SA_ERR_INVALID", "rowsF32 needs a table and tableByteOffset >= 0");
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_rows_f32((char*)table + toff, (int32_t)dtype, rows, dim, (const int32_t*)ids, n_ids, (float*)dst,
                                g_stream)))
    return NULL;
  return undefined(env);
}

/* (w, wByteOffset, dtype, cout, cin, cinPad, dst) */
static napi_value js_conv3_pack(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (get_args(env, info, 7, argv)) return NULL;
  void *w, *dst;
  int64_t woff, dtype, cout, cin, cp;
  if (get_ptr(env, argv[0], &w, "w") || get_i64(env, argv[1], 0, &woff, "wByteOffset") ||
      get_i64(env, argv[2], -1, &dtype, "dtype") || get_i64(env, argv[3], -1, &cout, "cout") ||
      get_i64(env, argv[4], -1, &cin, "cin") || get_i64(env, argv[5], 0, &cp, "cinPad") || get_ptr(env, argv[6], &dst, "dst"))
    return NULL;
  if (!w || woff < 0 || cout > INT32_MAX || cin > INT32_MAX || cp > INT32_MAX) {
    napi_throw_error(env, "SA_ERR_INVALID", "conv3Pack needs a weight buffer, wByteOffset >= 0 and 32-bit sizes");
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_conv3_pack_f32((char*)w + woff, (int32_t)dtype, (int32_t)cout, (int32_t)cin, (int32_t)cp,
                                      (float*)dst, g_stream)))
    return NULL;
  return undefined(env);
}

static napi_value init(napi_env env, napi_value exports) {
  const napi_property_descriptor props[] = {
      {"attention", NULL, js_attention, NULL, NULL, NULL, napi_enumerable, NULL},
      {"kernelName", NULL, js_kernel_name, NULL, NULL, NULL, napi_enumerable, NULL},
      {"workspaceBytes", NULL, js_workspace_bytes, NULL, NULL, NULL, napi_enumerable, NULL},
      {"linear", NULL, js_linear, NULL, NULL, NULL, napi_enumerable, NULL},
      {"vaeAttention", NULL, js_vae_attention, NULL, NULL, NULL, napi_enumerable, NULL},
      {"vaeWorkspaceBytes", NULL, js_vae_workspace_bytes, NULL, NULL, NULL, napi_enumerable, NULL},
      {"linearKernelName", NULL, js_linear_kernel_name, NULL, NULL, NULL, napi_enumerable, NULL},
      {"version", NULL, js_version, NULL, NULL, NULL, napi_enumerable, NULL},
      {"deviceCount", NULL, js_device_count, NULL, NULL, NULL, napi_enumerable, NULL},
      {"malloc", NULL, js_malloc, NULL, NULL, NULL, napi_enumerable, NULL},
      {"free", NULL, js_free, NULL, NULL, NULL, napi_enumerable, NULL},
      {"upload", NULL, js_upload, NULL, NULL, NULL, napi_enumerable, NULL},
      {"download", NULL, js_download, NULL, NULL, NULL, napi_enumerable, NULL},
      {"memset", NULL, js_memset, NULL, NULL, NULL, napi_enumerable, NULL},
      {"copy", NULL, js_copy, NULL, NULL, NULL, napi_enumerable, NULL},
      {"sync", NULL, js_sync, NULL, NULL, NULL, napi_enumerable, NULL},
      {"bucketLut", NULL, js_bucket_lut, NULL, NULL, NULL, napi_enumerable, NULL},
      {"positionBias", NULL, js_position_bias, NULL, NULL, NULL, napi_enumerable, NULL},
      {"eventCreate", NULL, js_event_create, NULL, NULL, NULL, napi_enumerable, NULL},
      {"eventRecord", NULL, js_event_record, NULL, NULL, NULL, napi_enumerable, NULL},
      {"eventElapsed", NULL, js_event_elapsed, NULL, NULL, NULL, napi_enumerable, NULL},
      {"eventDestroy", NULL, js_event_destroy, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stOpen", NULL, js_st_open, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stOpenBytes", NULL, js_st_open_bytes, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stClose", NULL, js_st_close, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stNames", NULL, js_st_names, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stInfo", NULL, js_st_info, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stHas", NULL, js_st_has, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stMetadata", NULL, js_st_metadata, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stDataBytes", NULL, js_st_data_bytes, NULL, NULL, NULL, napi_enumerable, NULL},
      {"stUpload", NULL, js_st_upload, NULL, NULL, NULL, napi_enumerable, NULL},
      {"mallocHost", NULL, js_malloc_host, NULL, NULL, NULL, napi_enumerable, NULL},
      {"freeHost", NULL, js_free_host, NULL, NULL, NULL, napi_enumerable, NULL},
      {"toF32", NULL, js_to_f32, NULL, NULL, NULL, napi_enumerable, NULL},
      {"rowsF32", NULL, js_rows_f32, NULL, NULL, NULL, napi_enumerable, NULL},
      {"conv3Pack", NULL, js_conv3_pack, NULL, NULL, NULL, napi_enumerable, NULL},
  };
  NAPI_CALL(env, napi_define_properties(env, exports, sizeof props / sizeof props[0], props));
  napi_value c;
#define CONST(name, val)                                      \
  NAPI_CALL(env, napi_create_int32(env, (val), &c));          \
  NAPI_CALL(env, napi_set_named_property(env, exports, name, c));
  CONST("SA_BIAS_NONE", SA_BIAS_NONE)
  CONST("SA_BIAS_DENSE", SA_BIAS_DENSE)
  CONST("SA_BIAS_RELPOS", SA_BIAS_RELPOS)
  CONST("SA_MASK_NONE", SA_MASK_NONE)
  CONST("SA_MASK_KEY_LEN", SA_MASK_KEY_LEN)
  CONST("SA_MASK_KEY_MASK", SA_MASK_KEY_MASK)
  CONST("SA_DT_F32", SA_DT_F32)
  CONST("SA_DT_F16", SA_DT_F16)
  CONST("SA_DT_BF16", SA_DT_BF16)
  CONST("SA_DT_F64", SA_DT_F64)
  CONST("SA_DT_I64", SA_DT_I64)
  CONST("SA_DT_I32", SA_DT_I32)
  CONST("SA_DT_I16", SA_DT_I16)
  CONST("SA_DT_I8", SA_DT_I8)
  CONST("SA_DT_U8", SA_DT_U8)
  CONST("SA_DT_BOOL", SA_DT_BOOL)
#undef CONST
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
