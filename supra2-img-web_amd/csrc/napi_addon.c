/*
 * Node.js N-API addon over the attention library's C ABI (include/supra_attn.h).
 *
 * It gives the JS shim (js/device.js, js/ops.js) what app/gpu/device.js gave app/gpu/ops.js:
 * device buffers (GPU.empty / fromArray / read, device.js:144-191), one in-order queue
 * (device.js:1-5: work is stream-ordered, so a buffer released right after a call is safe to
 * reuse) and sync (device.js:255-259). The attention call itself maps ops.attention's options
 * object (app/gpu/ops.js:109) onto sa_attn_args.
 *
 * Device buffers, pinned host buffers, events and opened safetensors files cross into JS as
 * handles: plain objects tagged as this addon's and wrapping a record of the pointer and, for
 * buffers, the allocation size. Every call checks each handle's tag and kind, that it has not been
 * released, and that every byte range it touches lies inside the buffer (for the attention, linear
 * and VAE calls, the whole strided extent of each operand) - the validation WebGPU applies to
 * buffer bindings and writeBuffer, so no call from JS reaches memory outside an allocation, and a
 * use after free() throws instead of faulting. Every C ABI status other than SA_OK becomes a thrown
 * JS Error whose code is the status ("SA_ERR_INVALID", ...) and whose message is sa_last_error().
 * The stream is created on first use, so loading the addon on a host without a GPU succeeds (only
 * calls that need the device fail).
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

/* Throws the status of the library call that just returned NULL: its own status, or
 * SA_ERR_INVALID should it ever have left none, so the JS call always throws. */
static void throw_last(napi_env env) {
  const int rc = sa_last_status();
  throw_if(env, rc != SA_OK ? rc : SA_ERR_INVALID);
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

/* ---- handles ----
 * The memory behind a handle is released only by free / freeHost / eventDestroy / stClose (buffers
 * are destroyed explicitly, as app/gpu/device.js does); a handle collected first frees its record
 * and, for a file, closes the file. */
enum { H_DEVICE = 1, H_HOST = 2, H_EVENT = 3, H_FILE = 4 };

typedef struct Handle {
  int kind;
  void* ptr;     /* the memory, the hipEvent_t or the sa_st_file; NULL once released */
  int64_t bytes; /* buffers: the allocation size */
  void* copy;    /* H_FILE opened from bytes: the host copy the file reads from */
} Handle;

static const napi_type_tag kHandleTag = {0x9d3c6a4f18e2b705ULL, 0x4b71e0c2d95a3f86ULL};

static const char* kind_name(int kind) {
  switch (kind) {
    case H_DEVICE: return "a device buffer handle";
    case H_HOST: return "a pinned host buffer handle";
    case H_EVENT: return "an event handle";
    default: return "a safetensors handle";
  }
}

static void handle_finalize(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  Handle* h = (Handle*)data;
  if (h->kind == H_FILE && h->ptr) sa_st_close((sa_st_file*)h->ptr);
  free(h->copy);
  free(h);
}

/* A new handle object for `ptr`. It owns an H_FILE's file and copy from here on (closed if this
 * fails); device or host memory and events stay the caller's to release when it returns NULL. */
static napi_value new_handle(napi_env env, int kind, void* ptr, int64_t bytes, void* copy) {
  Handle* h = (Handle*)calloc(1, sizeof *h);
  if (!h) {
    if (kind == H_FILE) sa_st_close((sa_st_file*)ptr);
    free(copy);
    napi_throw_error(env, "SA_NAPI", "out of host memory");
    return NULL;
  }
  h->kind = kind;
  h->ptr = ptr;
  h->bytes = bytes;
  h->copy = copy;
  napi_value obj;
  if (napi_create_object(env, &obj) != napi_ok || napi_wrap(env, obj, h, handle_finalize, NULL, NULL) != napi_ok) {
    if (kind != H_FILE) h->ptr = NULL;
    handle_finalize(env, h, NULL);
    napi_throw_error(env, "SA_NAPI", "cannot create a handle");
    return NULL;
  }
  if (napi_type_tag_object(env, obj, &kHandleTag) != napi_ok) {
    if (kind != H_FILE) h->ptr = NULL; /* the wrapper's finalizer frees the record */
    napi_throw_error(env, "SA_NAPI", "cannot tag a handle");
    return NULL;
  }
  return obj;
}

/* The live handle of `kind` in v; undefined/null gives NULL when `optional`. Anything else throws. */
static int get_handle(napi_env env, napi_value v, int kind, int optional, const char* what, Handle** out) {
  char msg[160];
  *out = NULL;
  if (is_nullish(env, v)) {
    if (optional) return 0;
    snprintf(msg, sizeof msg, "%s must be %s (got null or undefined)", what, kind_name(kind));
    napi_throw_type_error(env, "SA_ERR_INVALID", msg);
    return 1;
  }
  napi_valuetype t;
  bool tagged = false;
  void* p = NULL;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_object ||
      napi_check_object_type_tag(env, v, &kHandleTag, &tagged) != napi_ok || !tagged ||
      napi_unwrap(env, v, &p) != napi_ok || !p || ((Handle*)p)->kind != kind) {
    snprintf(msg, sizeof msg, "%s must be %s", what, kind_name(kind));
    napi_throw_type_error(env, "SA_ERR_INVALID", msg);
    return 1;
  }
  if (!((Handle*)p)->ptr) {
    snprintf(msg, sizeof msg, "%s: %s that has been released", what, kind_name(kind));
    napi_throw_error(env, "SA_ERR_INVALID", msg);
    return 1;
  }
  *out = (Handle*)p;
  return 0;
}

static void* ptr_of(const Handle* h) { return h ? h->ptr : NULL; }

/* Checks that bytes [off, off + len) lie inside buffer h (a NULL h passes: the C ABI decides
 * whether the operand may be absent); len < 0 stands for an extent that overflowed. */
static int in_bounds(napi_env env, const Handle* h, int64_t off, int64_t len, const char* what) {
  if (!h) return 0;
  if (off < 0 || len < 0 || off > h->bytes || len > h->bytes - off) {
    char msg[200];
    if (len < 0)
      snprintf(msg, sizeof msg, "%s: the extent overflows 64-bit sizes", what);
    else
      snprintf(msg, sizeof msg, "%s: %lld bytes at byte offset %lld lie outside the %lld-byte buffer", what,
               (long long)len, (long long)off, (long long)h->bytes);
    napi_throw_range_error(env, "SA_ERR_INVALID", msg);
    return 1;
  }
  return 0;
}

/* elem * (off + (nb - 1)*sb + (nr - 1)*ld + row): the bytes a strided operand spans from its
 * buffer's start, or -1 if that overflows. */
static int64_t extent_bytes(int64_t elem, int64_t off, int64_t nb, int64_t sb, int64_t nr, int64_t ld, int64_t row) {
  int64_t acc = off, t = 0;
  if (nb > 1 && (__builtin_mul_overflow(nb - 1, sb, &t) || __builtin_add_overflow(acc, t, &acc))) return -1;
  if (nr > 1 && (__builtin_mul_overflow(nr - 1, ld, &t) || __builtin_add_overflow(acc, t, &acc))) return -1;
  if (__builtin_add_overflow(acc, row, &acc) || __builtin_mul_overflow(acc, elem, &acc) || acc < 0) return -1;
  return acc;
}

/* a * b * c, or -1 if that overflows or a factor is negative */
static int64_t mul3(int64_t a, int64_t b, int64_t c) {
  int64_t r;
  if (a < 0 || b < 0 || c < 0 || __builtin_mul_overflow(a, b, &r) || __builtin_mul_overflow(r, c, &r)) return -1;
  return r;
}

/* Event handles (no size) */
static int get_event(napi_env env, napi_value v, const char* what, void** out) {
  Handle* h;
  if (get_handle(env, v, H_EVENT, 0, what, &h)) return 1;
  *out = h->ptr;
  return 0;
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

static int prop_buf(napi_env env, napi_value obj, const char* name, Handle** out) {
  napi_value v;
  if (prop(env, obj, name, &v)) return 1;
  return get_handle(env, v, H_DEVICE, 1, name, out);
}

/* opts -> sa_attn_args. Field names are those of app/gpu/ops.js:109 (q, k, v, Lq, Lk, H, D, ldq,
 * ldk, ldv, qOff, kOff, vOff, oOff, scale) plus out -> o, and the extension fields B, ldo, sq, sk,
 * sv, so, biasMode, bias, sbias, bucketLut, numBuckets, maskMode, keyLen, keyLenHost, keyMask,
 * smask, workspace, workspaceBytes. */
typedef struct AttnHandles {
  Handle *q, *k, *v, *out, *bias, *lut, *kl, *km, *ws;
} AttnHandles;

static int fill_args(napi_env env, napi_value o, sa_attn_args* a, AttnHandles* hs) {
  memset(a, 0, sizeof *a);
  memset(hs, 0, sizeof *hs);
  a->struct_size = sizeof *a;
  int64_t B, H, D, Lq, Lk, bm, mm, nb;
  double scale;
  napi_value sv;
  if (prop_i64(env, o, "B", 1, &B) || prop_i64(env, o, "H", -1, &H) || prop_i64(env, o, "D", -1, &D) ||
      prop_i64(env, o, "Lq", -1, &Lq) || prop_i64(env, o, "Lk", -1, &Lk))
    return 1;
  if (prop_buf(env, o, "q", &hs->q) || prop_buf(env, o, "k", &hs->k) || prop_buf(env, o, "v", &hs->v) ||
      prop_buf(env, o, "out", &hs->out) || prop_buf(env, o, "bias", &hs->bias) ||
      prop_buf(env, o, "bucketLut", &hs->lut) || prop_buf(env, o, "keyLen", &hs->kl) ||
      prop_buf(env, o, "keyMask", &hs->km) || prop_buf(env, o, "workspace", &hs->ws))
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
  /* keyLenHost: optional Int32Array host copy of keyLen (>= B entries), read during the call */
  napi_value klh;
  if (prop(env, o, "keyLenHost", &klh)) return 1;
  if (!is_nullish(env, klh)) {
    bool is_ta = false;
    napi_typedarray_type type;
    size_t length = 0, offset = 0;
    void* data = NULL;
    napi_value ab;
    if (napi_is_typedarray(env, klh, &is_ta) != napi_ok || !is_ta ||
        napi_get_typedarray_info(env, klh, &type, &length, &data, &ab, &offset) != napi_ok || type != napi_int32_array ||
        B < 1 || (int64_t)length < B) {
      napi_throw_type_error(env, "SA_ERR_INVALID", "keyLenHost must be an Int32Array of at least B lengths");
      return 1;
    }
    a->key_len_host = (const int32_t*)data;
  }
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
  if (bm < INT32_MIN || bm > INT32_MAX || mm < INT32_MIN || mm > INT32_MAX || nb < INT32_MIN || nb > INT32_MAX) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "biasMode, maskMode and numBuckets must fit in int32");
    return 1;
  }
  a->q = (const float*)ptr_of(hs->q);
  a->k = (const float*)ptr_of(hs->k);
  a->v = (const float*)ptr_of(hs->v);
  a->o = (float*)ptr_of(hs->out);
  a->scale = (float)scale;
  a->bias_mode = (int32_t)bm;
  a->bias = (const float*)ptr_of(hs->bias);
  a->bucket_lut = (const int32_t*)ptr_of(hs->lut);
  a->num_buckets = (int32_t)nb;
  a->mask_mode = (int32_t)mm;
  a->key_len = (const int32_t*)ptr_of(hs->kl);
  a->key_mask = (const uint8_t*)ptr_of(hs->km);
  a->workspace = ptr_of(hs->ws);
  return 0;
}

/* Every operand's strided extent inside its buffer (`a` already accepted by the C ABI). */
static int check_attn(napi_env env, const sa_attn_args* a, const AttnHandles* hs) {
  const int64_t HD = (int64_t)a->H * a->D, ldo = a->ldo > 0 ? a->ldo : HD, B = a->B;
  if (in_bounds(env, hs->q, 0, extent_bytes(4, a->q_off, B, a->sq, a->Lq, a->ldq, HD), "q") ||
      in_bounds(env, hs->k, 0, extent_bytes(4, a->k_off, B, a->sk, a->Lk, a->ldk, HD), "k") ||
      in_bounds(env, hs->v, 0, extent_bytes(4, a->v_off, B, a->sv, a->Lk, a->ldv, HD), "v") ||
      in_bounds(env, hs->out, 0, extent_bytes(4, a->o_off, B, a->so, a->Lq, ldo, HD), "out"))
    return 1;
  if (a->bias_mode == SA_BIAS_DENSE &&
      in_bounds(env, hs->bias, 0, extent_bytes(4, 0, B, a->sbias, 1, 0, mul3(a->H, a->Lq, a->Lk)), "bias"))
    return 1;
  if (a->bias_mode == SA_BIAS_RELPOS &&
      (in_bounds(env, hs->bias, 0, mul3(4, a->num_buckets, a->H), "bias") ||
       in_bounds(env, hs->lut, 0, mul3(4, (int64_t)a->Lq + a->Lk - 1, 1), "bucketLut")))
    return 1;
  if (a->mask_mode == SA_MASK_KEY_LEN && in_bounds(env, hs->kl, 0, mul3(4, B, 1), "keyLen")) return 1;
  if (a->mask_mode == SA_MASK_KEY_MASK &&
      in_bounds(env, hs->km, 0, extent_bytes(1, 0, B, a->smask > 0 ? a->smask : a->Lk, 1, 0, a->Lk), "keyMask"))
    return 1;
  return in_bounds(env, hs->ws, 0, a->workspace_bytes, "workspace");
}

/* opts -> sa_linear_args: M, N, K, x, xOff, ldx, w, ldw, bias, alpha (default 1), act, epilogue,
 * gate, gateOff, y, yOff, ldy (the JS shim maps app/gpu/ops.js:35-43's linear() onto these). */
typedef struct LinearHandles {
  Handle *x, *w, *bias, *gate, *y;
} LinearHandles;

static int fill_linear(napi_env env, napi_value o, sa_linear_args* a, LinearHandles* hs) {
  memset(a, 0, sizeof *a);
  memset(hs, 0, sizeof *hs);
  a->struct_size = sizeof *a;
  int64_t M, N, K, act, epi;
  double alpha;
  napi_value av;
  if (prop_i64(env, o, "M", -1, &M) || prop_i64(env, o, "N", -1, &N) || prop_i64(env, o, "K", -1, &K) ||
      prop_i64(env, o, "act", SA_ACT_NONE, &act) || prop_i64(env, o, "epilogue", SA_EPI_STORE, &epi) ||
      prop_i64(env, o, "xOff", 0, &a->x_off) || prop_i64(env, o, "ldx", 0, &a->ldx) ||
      prop_i64(env, o, "ldw", 0, &a->ldw) || prop_i64(env, o, "gateOff", 0, &a->gate_off) ||
      prop_i64(env, o, "yOff", 0, &a->y_off) || prop_i64(env, o, "ldy", 0, &a->ldy))
    return 1;
  if (prop_buf(env, o, "x", &hs->x) || prop_buf(env, o, "w", &hs->w) || prop_buf(env, o, "bias", &hs->bias) ||
      prop_buf(env, o, "gate", &hs->gate) || prop_buf(env, o, "y", &hs->y))
    return 1;
  if (prop(env, o, "alpha", &av) || get_f64(env, av, 1.0, &alpha, "alpha")) return 1;
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL || M < -1 || N < -1 || K < -1 || act < INT32_MIN ||
      act > INT32_MAX || epi < INT32_MIN || epi > INT32_MAX) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "sizes, act and epilogue must fit in int32");
    return 1;
  }
  a->M = (int32_t)M;
  a->N = (int32_t)N;
  a->K = (int32_t)K;
  a->x = (const float*)ptr_of(hs->x);
  a->w = (const float*)ptr_of(hs->w);
  a->bias = (const float*)ptr_of(hs->bias);
  a->alpha = (float)alpha;
  a->act = (int32_t)act;
  a->epilogue = (int32_t)epi;
  a->gate = (const float*)ptr_of(hs->gate);
  a->y = (float*)ptr_of(hs->y);
  return 0;
}

/* Every operand's extent inside its buffer (`a` already accepted by the C ABI). */
static int check_linear(napi_env env, const sa_linear_args* a, const LinearHandles* hs) {
  const int64_t ldx = a->ldx ? a->ldx : a->K, ldw = a->ldw ? a->ldw : a->K, ldy = a->ldy ? a->ldy : a->N;
  return in_bounds(env, hs->x, 0, extent_bytes(4, a->x_off, 1, 0, a->M, ldx, a->K), "x") ||
         in_bounds(env, hs->w, 0, extent_bytes(4, 0, 1, 0, a->N, ldw, a->K), "w") ||
         in_bounds(env, hs->bias, 0, mul3(4, a->N, 1), "bias") ||
         (a->epilogue == SA_EPI_RESID_GATE &&
          in_bounds(env, hs->gate, 0, extent_bytes(4, a->gate_off, 1, 0, 1, 0, a->N), "gate")) ||
         in_bounds(env, hs->y, 0, extent_bytes(4, a->y_off, 1, 0, a->M, ldy, a->N), "y");
}

static napi_value js_linear(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_linear_args a;
  LinearHandles hs;
  if (fill_linear(env, argv[0], &a, &hs)) return NULL;
  /* validate before touching the device, so a bad call reports its own error on any host */
  if (sa_linear_kernel_name(&a) == NULL) {
    throw_last(env);
    return NULL;
  }
  if (check_linear(env, &a, &hs) || ensure_stream(env)) return NULL;
  if (throw_if(env, sa_linear_f32(&a, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_linear_kernel_name(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_linear_args a;
  LinearHandles hs;
  if (fill_linear(env, argv[0], &a, &hs)) return NULL;
  const char* name = sa_linear_kernel_name(&a);
  if (!name) {
    throw_last(env);
    return NULL;
  }
  napi_value r;
  NAPI_CALL(env, napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &r));
  return r;
}

/* opts -> sa_vae_attn_args: HW, C, groups (32), eps (1e-6), x, gamma, beta, wqkv, bqkv, wo, bo,
 * out, workspace, workspaceBytes. */
typedef struct VaeHandles {
  Handle *x, *gamma, *beta, *wqkv, *bqkv, *wo, *bo, *out, *ws;
} VaeHandles;

static int fill_vae(napi_env env, napi_value o, sa_vae_attn_args* a, VaeHandles* hs) {
  memset(a, 0, sizeof *a);
  memset(hs, 0, sizeof *hs);
  a->struct_size = sizeof *a;
  int64_t HW, C, G;
  double eps;
  napi_value ev;
  if (prop_i64(env, o, "HW", -1, &HW) || prop_i64(env, o, "C", -1, &C) || prop_i64(env, o, "groups", 32, &G) ||
      prop_i64(env, o, "workspaceBytes", 0, &a->workspace_bytes))
    return 1;
  if (prop(env, o, "eps", &ev) || get_f64(env, ev, 1e-6, &eps, "eps")) return 1;
  if (prop_buf(env, o, "x", &hs->x) || prop_buf(env, o, "gamma", &hs->gamma) || prop_buf(env, o, "beta", &hs->beta) ||
      prop_buf(env, o, "wqkv", &hs->wqkv) || prop_buf(env, o, "bqkv", &hs->bqkv) || prop_buf(env, o, "wo", &hs->wo) ||
      prop_buf(env, o, "bo", &hs->bo) || prop_buf(env, o, "out", &hs->out) || prop_buf(env, o, "workspace", &hs->ws))
    return 1;
  if (HW > 0x7fffffffLL || C > 0x7fffffffLL || G > 0x7fffffffLL || HW < -1 || C < -1 || G < -1) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "sizes must fit in int32");
    return 1;
  }
  a->HW = (int32_t)HW;
  a->C = (int32_t)C;
  a->groups = (int32_t)G;
  a->eps = (float)eps;
  a->x = (const float*)ptr_of(hs->x);
  a->gamma = (const float*)ptr_of(hs->gamma);
  a->beta = (const float*)ptr_of(hs->beta);
  a->wqkv = (const float*)ptr_of(hs->wqkv);
  a->bqkv = (const float*)ptr_of(hs->bqkv);
  a->wo = (const float*)ptr_of(hs->wo);
  a->bo = (const float*)ptr_of(hs->bo);
  a->out = (float*)ptr_of(hs->out);
  a->workspace = ptr_of(hs->ws);
  return 0;
}

/* Every operand inside its buffer (sizes already accepted by the C ABI). */
static int check_vae(napi_env env, const sa_vae_attn_args* a, const VaeHandles* hs) {
  const int64_t img = mul3(4, a->HW, a->C), vec = mul3(4, a->C, 1);
  return in_bounds(env, hs->x, 0, img, "x") || in_bounds(env, hs->gamma, 0, vec, "gamma") ||
         in_bounds(env, hs->beta, 0, vec, "beta") || in_bounds(env, hs->wqkv, 0, mul3(12, a->C, a->C), "wqkv") ||
         in_bounds(env, hs->bqkv, 0, mul3(12, a->C, 1), "bqkv") || in_bounds(env, hs->wo, 0, mul3(4, a->C, a->C), "wo") ||
         in_bounds(env, hs->bo, 0, vec, "bo") || in_bounds(env, hs->out, 0, img, "out") ||
         in_bounds(env, hs->ws, 0, a->workspace_bytes, "workspace");
}

static napi_value js_vae_attention(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_vae_attn_args a;
  VaeHandles hs;
  if (fill_vae(env, argv[0], &a, &hs)) return NULL;
  const int64_t need = sa_vae_attention_workspace_bytes(&a); /* validates the sizes, host only */
  if (need < 0) {
    throw_if(env, (int)need);
    return NULL;
  }
  if (check_vae(env, &a, &hs) || ensure_stream(env)) return NULL;
  if (throw_if(env, sa_vae_attention_f32(&a, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_vae_workspace_bytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_vae_attn_args a;
  VaeHandles hs;
  if (fill_vae(env, argv[0], &a, &hs)) return NULL;
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
  AttnHandles hs;
  if (fill_args(env, argv[0], &a, &hs)) return NULL;
  /* validate before touching the device, so a bad call reports its own error on any host */
  if (sa_attention_kernel_name(&a) == NULL) {
    throw_last(env);
    return NULL;
  }
  if (check_attn(env, &a, &hs) || ensure_stream(env)) return NULL;
  if (throw_if(env, sa_attention_f32(&a, g_stream))) return NULL;
  return undefined(env);
}

/* Bytes of device workspace the call needs (sa_attention_workspace_bytes); throws if rejected. */
static napi_value js_workspace_bytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  sa_attn_args a;
  AttnHandles hs;
  if (fill_args(env, argv[0], &a, &hs)) return NULL;
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
  AttnHandles hs;
  if (fill_args(env, argv[0], &a, &hs)) return NULL;
  const char* name = sa_attention_kernel_name(&a);
  if (!name) {
    throw_last(env);
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
  napi_value r = new_handle(env, H_DEVICE, p, bytes, NULL);
  if (!r) sa_free(p);
  return r;
}

static napi_value js_free(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  Handle* h;
  if (get_handle(env, argv[0], H_DEVICE, 0, "buffer", &h)) return NULL;
  if (g_stream_ready && throw_if(env, sa_stream_sync(g_stream))) return NULL;
  if (throw_if(env, sa_free(h->ptr))) return NULL;
  h->ptr = NULL;
  h->bytes = 0;
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
  Handle* h;
  void* src;
  size_t bytes;
  int64_t off;
  if (get_handle(env, argv[0], H_DEVICE, 0, "buffer", &h) || typed_bytes(env, argv[1], &src, &bytes) ||
      get_i64(env, argv[2], 0, &off, "byteOffset") || in_bounds(env, h, off, (int64_t)bytes, "upload"))
    return NULL;
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_memcpy_h2d((char*)h->ptr + off, src, bytes, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_download(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (get_args(env, info, 3, argv)) return NULL;
  Handle* h;
  void* dst;
  size_t bytes;
  int64_t off;
  if (get_handle(env, argv[0], H_DEVICE, 0, "buffer", &h) || typed_bytes(env, argv[1], &dst, &bytes) ||
      get_i64(env, argv[2], 0, &off, "byteOffset") || in_bounds(env, h, off, (int64_t)bytes, "download"))
    return NULL;
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_memcpy_d2h(dst, (const char*)h->ptr + off, bytes, g_stream))) return NULL;
  return argv[1];
}

static napi_value js_memset(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (get_args(env, info, 3, argv)) return NULL;
  Handle* h;
  int64_t value, bytes;
  if (get_handle(env, argv[0], H_DEVICE, 0, "buffer", &h) || get_i64(env, argv[1], 0, &value, "value") ||
      get_i64(env, argv[2], -1, &bytes, "bytes") || in_bounds(env, h, 0, bytes, "memset"))
    return NULL;
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_memset(h->ptr, (int)value, (size_t)bytes, g_stream))) return NULL;
  return undefined(env);
}

/* (dst, dstByteOffset, src, srcByteOffset, bytes): device-to-device copy, stream-ordered */
static napi_value js_copy(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (get_args(env, info, 5, argv)) return NULL;
  Handle *dst, *src;
  int64_t doff, soff, bytes;
  if (get_handle(env, argv[0], H_DEVICE, 0, "dst", &dst) || get_i64(env, argv[1], 0, &doff, "dstByteOffset") ||
      get_handle(env, argv[2], H_DEVICE, 0, "src", &src) || get_i64(env, argv[3], 0, &soff, "srcByteOffset") ||
      get_i64(env, argv[4], -1, &bytes, "bytes") || in_bounds(env, dst, doff, bytes, "copy dst") ||
      in_bounds(env, src, soff, bytes, "copy src"))
    return NULL;
  if (dst == src && bytes > 0 && doff < soff + bytes && soff < doff + bytes) {
    napi_throw_error(env, "SA_ERR_ALIAS", "copy: the source and destination ranges overlap");
    return NULL;
  }
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_memcpy_d2d((char*)dst->ptr + doff, (const char*)src->ptr + soff, (size_t)bytes, g_stream)))
    return NULL;
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
  Handle *table, *lut, *out;
  int64_t nb, H, Lq, Lk;
  if (get_handle(env, argv[0], H_DEVICE, 0, "table", &table) || get_handle(env, argv[1], H_DEVICE, 0, "bucketLut", &lut) ||
      get_i64(env, argv[2], -1, &nb, "numBuckets") || get_i64(env, argv[3], -1, &H, "H") ||
      get_i64(env, argv[4], -1, &Lq, "Lq") || get_i64(env, argv[5], -1, &Lk, "Lk") ||
      get_handle(env, argv[6], H_DEVICE, 0, "out", &out))
    return NULL;
  if (nb < 1 || H < 1 || Lq < 1 || Lk < 1 || nb > INT32_MAX || H > INT32_MAX || Lq > 0x3fffffff || Lk > 0x3fffffff) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "numBuckets, H >= 1 (int32) and Lq, Lk in [1, 2^30)");
    return NULL;
  }
  if (in_bounds(env, table, 0, mul3(4, nb, H), "table") || in_bounds(env, lut, 0, mul3(4, Lq + Lk - 1, 1), "bucketLut") ||
      in_bounds(env, out, 0, mul3(4 * H, Lq, Lk), "out") || ensure_stream(env))
    return NULL;
  if (throw_if(env, sa_t5_position_bias((const float*)table->ptr, (const int32_t*)lut->ptr, (int32_t)nb, (int32_t)H,
                                        (int32_t)Lq, (int32_t)Lk, (float*)out->ptr, g_stream)))
    return NULL;
  return undefined(env);
}

static napi_value js_event_create(napi_env env, napi_callback_info info) {
  (void)info;
  void* ev = NULL;
  if (throw_if(env, sa_event_create(&ev))) return NULL;
  napi_value r = new_handle(env, H_EVENT, ev, 0, NULL);
  if (!r) sa_event_destroy(ev);
  return r;
}

static napi_value js_event_record(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  void* ev;
  if (get_event(env, argv[0], "event", &ev)) return NULL;
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_event_record(ev, g_stream))) return NULL;
  return undefined(env);
}

static napi_value js_event_elapsed(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (get_args(env, info, 2, argv)) return NULL;
  void *a, *b;
  if (get_event(env, argv[0], "start", &a) || get_event(env, argv[1], "stop", &b)) return NULL;
  float ms = 0.f;
  if (throw_if(env, sa_event_elapsed_ms(&ms, a, b))) return NULL;
  napi_value r;
  NAPI_CALL(env, napi_create_double(env, ms, &r));
  return r;
}

static napi_value js_event_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  Handle* h;
  if (get_handle(env, argv[0], H_EVENT, 0, "event", &h)) return NULL;
  if (throw_if(env, sa_event_destroy(h->ptr))) return NULL;
  h->ptr = NULL;
  return undefined(env);
}

/* ---- safetensors (include/supra_weights.h) ---- */

/* An opened file is an H_FILE handle: closed by stClose or, failing that, when collected. Bytes
 * opened from a JS array are copied, so that the handle does not depend on the array's storage. */
static int st_get(napi_env env, napi_value v, sa_st_file** out) {
  Handle* h;
  if (get_handle(env, v, H_FILE, 0, "file", &h)) return 1;
  *out = (sa_st_file*)h->ptr;
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
  return new_handle(env, H_FILE, f, 0, NULL);
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
  return new_handle(env, H_FILE, f, 0, copy);
}

static napi_value js_st_close(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  /* closing twice is allowed (app/weights.js never closes; a loader may close in a finally) */
  napi_valuetype t;
  bool tagged = false;
  void* p = NULL;
  if (napi_typeof(env, argv[0], &t) != napi_ok || t != napi_object ||
      napi_check_object_type_tag(env, argv[0], &kHandleTag, &tagged) != napi_ok || !tagged ||
      napi_unwrap(env, argv[0], &p) != napi_ok || !p || ((Handle*)p)->kind != H_FILE) {
    napi_throw_type_error(env, "SA_ERR_INVALID", "file must be a safetensors handle");
    return NULL;
  }
  Handle* h = (Handle*)p;
  if (h->ptr) sa_st_close((sa_st_file*)h->ptr);
  h->ptr = NULL;
  free(h->copy);
  h->copy = NULL;
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
  Handle *dst, *staging;
  if (st_get(env, argv[0], &f) || get_i64(env, argv[1], 0, &begin, "begin") || get_i64(env, argv[2], -1, &end, "end") ||
      get_handle(env, argv[3], H_DEVICE, 0, "dst", &dst) || get_i64(env, argv[4], 0, &doff, "dstByteOffset") ||
      get_handle(env, argv[5], H_HOST, 1, "staging", &staging) || get_i64(env, argv[6], 0, &sbytes, "stagingBytes"))
    return NULL;
  if (begin < 0 || end < begin) {
    napi_throw_range_error(env, "SA_ERR_INVALID", "need 0 <= begin <= end");
    return NULL;
  }
  if (in_bounds(env, dst, doff, end - begin, "stUpload dst") || (staging && in_bounds(env, staging, 0, sbytes, "staging")) ||
      ensure_stream(env))
    return NULL;
  if (throw_if(env, sa_st_upload(f, begin, end, (char*)dst->ptr + doff, ptr_of(staging), staging ? sbytes : 0, g_stream)))
    return NULL;
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
  napi_value r = new_handle(env, H_HOST, p, bytes, NULL);
  if (!r) sa_free_host(p);
  return r;
}

static napi_value js_free_host(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (get_args(env, info, 1, argv)) return NULL;
  Handle* h;
  if (get_handle(env, argv[0], H_HOST, 0, "buffer", &h)) return NULL;
  if (throw_if(env, sa_free_host(h->ptr))) return NULL;
  h->ptr = NULL;
  h->bytes = 0;
  return undefined(env);
}

/* Bytes per element of a decodable SA_DT_* code, 0 for the others (the C ABI rejects those). */
static int64_t dt_bytes(int64_t dtype) {
  switch (dtype) {
    case SA_DT_F64: case SA_DT_I64: return 8;
    case SA_DT_F32: case SA_DT_I32: return 4;
    case SA_DT_F16: case SA_DT_BF16: case SA_DT_I16: return 2;
    case SA_DT_I8: case SA_DT_U8: case SA_DT_BOOL: return 1;
    default: return 0;
  }
}

/* Throws unless dtype is decodable and every size is >= 0 and (for the 32-bit ones) fits in int32. */
static int check_decode(napi_env env, int64_t dtype, const int64_t* sizes, int n, int int32_sizes) {
  for (int i = 0; i < n; ++i)
    if (sizes[i] < 0 || (int32_sizes && sizes[i] > INT32_MAX)) {
      napi_throw_range_error(env, "SA_ERR_INVALID", int32_sizes ? "sizes must be in [0, 2^31)" : "sizes must be >= 0");
      return 1;
    }
  if (dt_bytes(dtype) == 0) {
    napi_throw_error(env, "SA_ERR_UNSUPPORTED", "dtype is not one of the decodable SA_DT_* codes");
    return 1;
  }
  return 0;
}

/* (src, srcByteOffset, dtype, n, dst, dstByteOffset) */
static napi_value js_to_f32(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  if (get_args(env, info, 6, argv)) return NULL;
  Handle *src, *dst;
  int64_t soff, dtype, n, doff;
  if (get_handle(env, argv[0], H_DEVICE, 0, "src", &src) || get_i64(env, argv[1], 0, &soff, "srcByteOffset") ||
      get_i64(env, argv[2], -1, &dtype, "dtype") || get_i64(env, argv[3], -1, &n, "n") ||
      get_handle(env, argv[4], H_DEVICE, 0, "dst", &dst) || get_i64(env, argv[5], 0, &doff, "dstByteOffset") ||
      check_decode(env, dtype, &n, 1, 0) || in_bounds(env, src, soff, mul3(dt_bytes(dtype), n, 1), "toF32 src") ||
      in_bounds(env, dst, doff, mul3(4, n, 1), "toF32 dst"))
    return NULL;
  if (ensure_stream(env)) return NULL;
  if (throw_if(env, sa_to_f32((char*)src->ptr + soff, (int32_t)dtype, n, (float*)((char*)dst->ptr + doff), g_stream)))
    return NULL;
  return undefined(env);
}

/* (table, tableByteOffset, dtype, rows, dim, ids, nIds, dst) */
static napi_value js_rows_f32(napi_env env, napi_callback_info info) {
  napi_value argv[8];
  if (get_args(env, info, 8, argv)) return NULL;
  Handle *table, *ids, *dst;
  int64_t toff, dtype, rows, dim, n_ids;
  if (get_handle(env, argv[0], H_DEVICE, 0, "table", &table) || get_i64(env, argv[1], 0, &toff, "tableByteOffset") ||
      get_i64(env, argv[2], -1, &dtype, "dtype") || get_i64(env, argv[3], -1, &rows, "rows") ||
      get_i64(env, argv[4], -1, &dim, "dim") || get_handle(env, argv[5], H_DEVICE, 0, "ids", &ids) ||
      get_i64(env, argv[6], -1, &n_ids, "nIds") || get_handle(env, argv[7], H_DEVICE, 0, "dst", &dst))
    return NULL;
  const int64_t sizes[3] = {rows, dim, n_ids};
  if (check_decode(env, dtype, sizes, 3, 0) || in_bounds(env, table, toff, mul3(dt_bytes(dtype), rows, dim), "rowsF32 table") ||
      in_bounds(env, ids, 0, mul3(4, n_ids, 1), "rowsF32 ids") || in_bounds(env, dst, 0, mul3(4, n_ids, dim), "rowsF32 dst") ||
      ensure_stream(env))
    return NULL;
  if (throw_if(env, sa_rows_f32((char*)table->ptr + toff, (int32_t)dtype, rows, dim, (const int32_t*)ids->ptr, n_ids,
                                (float*)dst->ptr, g_stream)))
    return NULL;
  return undefined(env);
}

/* (w, wByteOffset, dtype, cout, cin, cinPad, dst) */
static napi_value js_conv3_pack(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (get_args(env, info, 7, argv)) return NULL;
  Handle *w, *dst;
  int64_t woff, dtype, cout, cin, cp;
  if (get_handle(env, argv[0], H_DEVICE, 0, "w", &w) || get_i64(env, argv[1], 0, &woff, "wByteOffset") ||
      get_i64(env, argv[2], -1, &dtype, "dtype") || get_i64(env, argv[3], -1, &cout, "cout") ||
      get_i64(env, argv[4], -1, &cin, "cin") || get_i64(env, argv[5], 0, &cp, "cinPad") ||
      get_handle(env, argv[6], H_DEVICE, 0, "dst", &dst))
    return NULL;
  const int64_t sizes[3] = {cout, cin, cp};
  if (check_decode(env, dtype, sizes, 3, 1) || in_bounds(env, w, woff, mul3(9 * dt_bytes(dtype), cout, cin), "conv3Pack w") ||
      in_bounds(env, dst, 0, mul3(36, cout, cp > 0 ? cp : cin), "conv3Pack dst") || ensure_stream(env))
    return NULL;
  if (throw_if(env, sa_conv3_pack_f32((char*)w->ptr + woff, (int32_t)dtype, (int32_t)cout, (int32_t)cin, (int32_t)cp,
                                      (float*)dst->ptr, g_stream)))
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
