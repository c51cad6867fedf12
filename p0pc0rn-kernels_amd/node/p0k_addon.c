/* p0k_addon.c — Node N-API addon over the C ABI of libp0k (include/p0k.h). It is the thin native layer under the
 * JavaScript shim (index.mjs), which keeps the reference's API: createGpu / Gpu.buffer / upload / read / free / done
 * (src/core/gpu.js) and gemm(gpu, args) (src/ops/gemm.js). Device buffers cross into JavaScript as BigInt addresses;
 * every argument check happens in libp0k, whose message becomes the thrown Error's message.
 *
 * Exports: ctxCreate, ctxDestroy, deviceInfo, alloc, free, upload, download, copy, sync, poolStats, drainPool,
 *          gemm, gemmCheck, selectTile, rowstats, attention, pixstats, gn, gnPartBytes, packQ4, packQ8, packF16, tensorBytes,
 *          lastError, abiVersion
 * (N-API version 6 or later: BigInt support; Node 12.17+).
 */
#define NAPI_VERSION 6
#include <node_api.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "p0k.h"

#define CHECK_NAPI(env, call)                                  \
  do {                                                         \
    if ((call) != napi_ok) {                                   \
      napi_throw_error((env), NULL, "p0k addon: N-API call failed: " #call); \
      return NULL;                                             \
    }                                                          \
  } while (0)

static napi_value throw_p0k(napi_env env, int code) {
  char c[16];
  snprintf(c, sizeof c, "P0K_E%d", code);
  napi_throw_error(env, c, p0k_last_error());
  return NULL;
}

static napi_value undef(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value *argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok) return 0;
  for (size_t i = argc; i < want; i++) napi_get_undefined(env, &argv[i]);
  return 1;
}

static int to_u64(napi_env env, napi_value v, uint64_t *out) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_bigint) {
    bool lossless;
    return napi_get_value_bigint_uint64(env, v, out, &lossless) == napi_ok;
  }
  if (t == napi_number) {
    double d;
    if (napi_get_value_double(env, v, &d) != napi_ok || d < 0) return 0;
    *out = (uint64_t)d;
    return 1;
  }
  if (t == napi_undefined || t == napi_null) { *out = 0; return 1; }
  return 0;
}

static p0k_ctx *get_ctx(napi_env env, napi_value v) {
  void *p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok) return NULL;
  return (p0k_ctx *)p;
}

static napi_value mk_u64(napi_env env, uint64_t v) {
  napi_value r;
  napi_create_bigint_uint64(env, v, &r);
  return r;
}

static napi_value mk_num(napi_env env, double v) {
  napi_value r;
  napi_create_double(env, v, &r);
  return r;
}

/* bytes of a TypedArray / ArrayBuffer / Buffer argument */
static int get_bytes(napi_env env, napi_value v, void **data, size_t *len) {
  bool is;
  if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
    napi_typedarray_type t;
    size_t n, off;
    napi_value ab;
    void *base;
    if (napi_get_typedarray_info(env, v, &t, &n, &base, &ab, &off) != napi_ok) return 0;
    size_t es = (t == napi_int8_array || t == napi_uint8_array || t == napi_uint8_clamped_array) ? 1
              : (t == napi_int16_array || t == napi_uint16_array) ? 2
              : (t == napi_float64_array || t == napi_bigint64_array || t == napi_biguint64_array) ? 8 : 4;
    *data = base;
    *len = n * es;
    return 1;
  }
  if (napi_is_arraybuffer(env, v, &is) == napi_ok && is) return napi_get_arraybuffer_info(env, v, data, len) == napi_ok;
  if (napi_is_dataview(env, v, &is) == napi_ok && is) {
    napi_value ab;
    size_t off;
    return napi_get_dataview_info(env, v, len, data, &ab, &off) == napi_ok;
  }
  return 0;
}

/* ------------------------------------------------------------------ context */
static void ctx_finalize(napi_env env, void *data, void *hint) {
  (void)env; (void)hint; (void)data;   /* destroyed explicitly by ctxDestroy; a context outliving JS is reclaimed at exit */
}

static napi_value ctxCreate(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  int32_t dev = 0;
  napi_valuetype t;
  napi_typeof(env, argv[0], &t);
  if (t == napi_number) napi_get_value_int32(env, argv[0], &dev);
  p0k_ctx *ctx = NULL;
  int r = p0k_ctx_create(dev, &ctx);
  if (r) return throw_p0k(env, r);
  napi_value ext;
  CHECK_NAPI(env, napi_create_external(env, ctx, ctx_finalize, NULL, &ext));
  return ext;
}

static napi_value ctxDestroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  p0k_ctx *ctx = get_ctx(env, argv[0]);
  if (ctx) p0k_ctx_destroy(ctx);
  return undef(env);
}

static napi_value deviceInfo(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  p0k_device_info d;
  int r = p0k_device_info_get(get_ctx(env, argv[0]), &d);
  if (r) return throw_p0k(env, r);
  napi_value o, s;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, d.name, NAPI_AUTO_LENGTH, &s); napi_set_named_property(env, o, "name", s);
  napi_create_string_utf8(env, d.arch, NAPI_AUTO_LENGTH, &s); napi_set_named_property(env, o, "arch", s);
  napi_set_named_property(env, o, "cus", mk_num(env, d.cus));
  napi_set_named_property(env, o, "hbmBytes", mk_num(env, (double)d.hbm_bytes));
  napi_set_named_property(env, o, "clockKhz", mk_num(env, d.clock_khz));
  return o;
}

/* ------------------------------------------------------------------ buffers */
static napi_value alloc(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  uint64_t n;
  if (!to_u64(env, argv[1], &n)) { napi_throw_type_error(env, NULL, "alloc: size must be a number"); return NULL; }
  void *p = NULL;
  int r = p0k_alloc(get_ctx(env, argv[0]), n, &p);
  if (r) return throw_p0k(env, r);
  return mk_u64(env, (uint64_t)(uintptr_t)p);
}

static napi_value free_(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  uint64_t p;
  if (!to_u64(env, argv[1], &p)) { napi_throw_type_error(env, NULL, "free: bad buffer"); return NULL; }
  int r = p0k_free(get_ctx(env, argv[0]), (void *)(uintptr_t)p);
  if (r) return throw_p0k(env, r);
  return undef(env);
}

static napi_value upload(napi_env env, napi_callback_info info) {   /* (ctx, ptr, off, data) */
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return NULL;
  uint64_t p, off;
  void *data;
  size_t len;
  if (!to_u64(env, argv[1], &p) || !to_u64(env, argv[2], &off) || !get_bytes(env, argv[3], &data, &len)) {
    napi_throw_type_error(env, NULL, "upload: (ctx, buffer, offset, TypedArray | ArrayBuffer)");
    return NULL;
  }
  int r = p0k_upload(get_ctx(env, argv[0]), (void *)(uintptr_t)p, off, data, len);
  if (r) return throw_p0k(env, r);
  return undef(env);
}

static napi_value download(napi_env env, napi_callback_info info) {   /* (ctx, ptr, off, size) -> ArrayBuffer */
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return NULL;
  uint64_t p, off, n;
  if (!to_u64(env, argv[1], &p) || !to_u64(env, argv[2], &off) || !to_u64(env, argv[3], &n)) {
    napi_throw_type_error(env, NULL, "download: (ctx, buffer, offset, size)");
    return NULL;
  }
  void *dst;
  napi_value ab;
  CHECK_NAPI(env, napi_create_arraybuffer(env, n, &dst, &ab));
  int r = p0k_download(get_ctx(env, argv[0]), (void *)(uintptr_t)p, off, dst, n);
  if (r) return throw_p0k(env, r);
  return ab;
}

static napi_value copy(napi_env env, napi_callback_info info) {   /* (ctx, dst, dstOff, src, srcOff, n) */
  napi_value argv[6];
  if (!get_args(env, info, 6, argv)) return NULL;
  uint64_t d, doff, s, soff, n;
  if (!to_u64(env, argv[1], &d) || !to_u64(env, argv[2], &doff) || !to_u64(env, argv[3], &s) ||
      !to_u64(env, argv[4], &soff) || !to_u64(env, argv[5], &n)) {
    napi_throw_type_error(env, NULL, "copy: (ctx, dst, dstOff, src, srcOff, size)");
    return NULL;
  }
  int r = p0k_copy(get_ctx(env, argv[0]), (void *)(uintptr_t)d, doff, (const void *)(uintptr_t)s, soff, n);
  if (r) return throw_p0k(env, r);
  return undef(env);
}

static napi_value sync_(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  int r = p0k_sync(get_ctx(env, argv[0]));
  if (r) return throw_p0k(env, r);
  return undef(env);
}

static napi_value poolStats(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  p0k_pool_stats s;
  int r = p0k_pool_stats_get(get_ctx(env, argv[0]), &s);
  if (r) return throw_p0k(env, r);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "alive", mk_num(env, (double)s.alive));
  napi_set_named_property(env, o, "peak", mk_num(env, (double)s.peak));
  napi_set_named_property(env, o, "pooled", mk_num(env, (double)s.pooled));
  napi_set_named_property(env, o, "highWater", mk_num(env, (double)s.high_water));
  napi_set_named_property(env, o, "maxBuf", mk_num(env, (double)s.max_buf));
  napi_set_named_property(env, o, "creates", mk_num(env, (double)s.creates));
  napi_set_named_property(env, o, "reuses", mk_num(env, (double)s.reuses));
  napi_set_named_property(env, o, "evictions", mk_num(env, (double)s.evictions));
  napi_set_named_property(env, o, "buffers", mk_num(env, (double)s.live_buffers));
  napi_set_named_property(env, o, "pooledN", mk_num(env, (double)s.pooled_buffers));
  return o;
}

static napi_value drainPool(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  int r = p0k_drain_pool(get_ctx(env, argv[0]));
  if (r) return throw_p0k(env, r);
  return undef(env);
}

/* ------------------------------------------------------------------ the op: a flat descriptor object -> p0k_gemm_args */
static int field_u64(napi_env env, napi_value o, const char *name, uint64_t *out) {
  bool has = false;
  napi_has_named_property(env, o, name, &has);
  if (!has) { *out = 0; return 1; }
  napi_value v;
  if (napi_get_named_property(env, o, name, &v) != napi_ok) return 0;
  return to_u64(env, v, out);
}

static int field_f32(napi_env env, napi_value o, const char *name, float *out) {
  bool has = false;
  napi_has_named_property(env, o, name, &has);
  *out = 0.0f;
  if (!has) return 1;
  napi_value v;
  double d = 0;
  if (napi_get_named_property(env, o, name, &v) != napi_ok) return 0;
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_undefined || t == napi_null) return 1;
  if (napi_get_value_double(env, v, &d) != napi_ok) return 0;
  *out = (float)d;
  return 1;
}

#define U64(name, dst)                                                             \
  do {                                                                             \
    uint64_t t_;                                                                   \
    if (!field_u64(env, o, name, &t_)) { napi_throw_type_error(env, NULL, "gemm descriptor field " name); return 0; } \
    dst = t_;                                                                      \
  } while (0)
#define PTR(name, dst, type)                                                       \
  do {                                                                             \
    uint64_t t_;                                                                   \
    if (!field_u64(env, o, name, &t_)) { napi_throw_type_error(env, NULL, "gemm descriptor field " name); return 0; } \
    dst = (type)(uintptr_t)t_;                                                     \
  } while (0)

static int parse_gemm(napi_env env, napi_value o, p0k_gemm_args *a) {
  memset(a, 0, sizeof *a);
  a->struct_size = sizeof *a;
  U64("w_enc", a->w_enc); PTR("w_buf", a->w_buf, const void *); U64("w_off", a->w_off); U64("w_bytes", a->w_bytes);
  U64("w_rows", a->w_rows); U64("w_cols", a->w_cols); U64("w_ld", a->w_ld);
  PTR("x_buf", a->x_buf, const void *); U64("x_off", a->x_off); U64("x_size", a->x_size);
  U64("x_ld", a->x_ld); U64("x_k0", a->x_k0); U64("x_mode", a->x_mode);
  PTR("y_buf", a->y_buf, void *); U64("y_off", a->y_off); U64("y_size", a->y_size); U64("y_ld", a->y_ld); U64("y_n0", a->y_n0);
  U64("M", a->M); U64("N", a->N); U64("K", a->K); U64("epi", a->epi); U64("acc", a->acc);
  U64("tile_bm", a->tile_bm); U64("tile_bn", a->tile_bn); U64("wr0", a->wr0); U64("wr1", a->wr1); U64("wk0", a->wk0);
  PTR("ev_buf", a->ev_buf, const float *); U64("ev_off", a->ev_off); U64("ev_size", a->ev_size);
  PTR("st_buf", a->st_buf, const float *); U64("st_off", a->st_off); U64("st_size", a->st_size);
  PTR("pv_buf", a->pv_buf, const float *); U64("pv_off", a->pv_off); U64("pv_stride", a->pv_stride); U64("pv_size", a->pv_size);
  PTR("bv_buf", a->bv_buf, const float *); U64("bv_off", a->bv_off); U64("bv_up", a->bv_up); U64("bv_size", a->bv_size);
  PTR("gt_buf", a->gt_buf, const void *); U64("gt_size", a->gt_size);
  PTR("rope_buf", a->rope_buf, const float *); U64("rope_size", a->rope_size);
  U64("res", a->res); U64("store", a->store); U64("act", a->act);
  U64("h_Ltot", a->h_Ltot); U64("h_Hq", a->h_Hq); U64("h_Hkv", a->h_Hkv); U64("h_rowOff", a->h_rowOff);
  if (!field_f32(env, o, "h_eps", &a->h_eps)) { napi_throw_type_error(env, NULL, "gemm descriptor field h_eps"); return 0; }
  U64("h_rope_mode", a->h_rope_mode);
  U64("c_Hi", a->c_Hi); U64("c_Wi", a->c_Wi); U64("c_Ci", a->c_Ci); U64("c_Ho", a->c_Ho); U64("c_Wo", a->c_Wo);
  U64("c_stride", a->c_stride); U64("c_padT", a->c_padT); U64("c_padL", a->c_padL); U64("c_ks", a->c_ks);
  U64("c_up2", a->c_up2); U64("c_gn", a->c_gn); U64("c_pn", a->c_pn);
  return 1;
}

static napi_value gemm(napi_env env, napi_callback_info info) {   /* (ctx, desc) */
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  p0k_gemm_args a;
  if (!parse_gemm(env, argv[1], &a)) return NULL;
  int r = p0k_gemm(get_ctx(env, argv[0]), &a);
  if (r) return throw_p0k(env, r);
  return mk_num(env, p0k_gemm_flops(&a));
}

static napi_value gemmCheck(napi_env env, napi_callback_info info) {   /* (desc): host-only validation */
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  p0k_gemm_args a;
  if (!parse_gemm(env, argv[0], &a)) return NULL;
  int r = p0k_gemm_check(&a);
  if (r) return throw_p0k(env, r);
  return undef(env);
}

static napi_value selectTile(napi_env env, napi_callback_info info) {   /* (desc[, ctx]): with a context, its plan */
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  p0k_gemm_args a;
  if (!parse_gemm(env, argv[0], &a)) return NULL;
  p0k_tile t;
  p0k_ctx *ctx = get_ctx(env, argv[1]);
  int r = ctx ? p0k_gemm_plan(ctx, &a, &t) : p0k_select_tile(&a, &t);
  if (r) return throw_p0k(env, r);
  napi_value o, s;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "BM", mk_num(env, t.bm));
  napi_set_named_property(env, o, "BN", mk_num(env, t.bn));
  napi_create_string_utf8(env, t.kernel == 1 ? "gemv" : t.kernel == 2 ? "gemv_mfma" : t.kernel == 3 ? "mfma_dma" : t.kernel == 4 ? "gemv_short" : "mfma", NAPI_AUTO_LENGTH, &s);
  napi_set_named_property(env, o, "kernel", s);
  return o;
}

static napi_value rowstats(napi_env env, napi_callback_info info) {   /* (ctx, {x_buf, x_off, x_size, ld, c0, rows, cols, mode, eps, st_buf, st_off, st_size}) */
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  napi_value o = argv[1];
  p0k_rowstats_args a;
  memset(&a, 0, sizeof a);
  a.struct_size = sizeof a;
  uint64_t t;
#define RS(name, dst) do { if (!field_u64(env, o, name, &t)) { napi_throw_type_error(env, NULL, "rowstats field " name); return NULL; } dst = t; } while (0)
  RS("x_buf", t); a.x_buf = (const void *)(uintptr_t)t;
  RS("x_off", a.x_off); RS("x_size", a.x_size); RS("ld", a.ld); RS("c0", a.c0); RS("rows", a.rows); RS("cols", a.cols);
  RS("mode", a.mode);
  RS("st_buf", t); a.st_buf = (float *)(uintptr_t)t;
  RS("st_off", a.st_off); RS("st_size", a.st_size);
#undef RS
  if (!field_f32(env, o, "eps", &a.eps)) { napi_throw_type_error(env, NULL, "rowstats field eps"); return NULL; }
  int r = p0k_rowstats(get_ctx(env, argv[0]), &a);
  if (r) return throw_p0k(env, r);
  return undef(env);
}

/* ------------------------------------------------------------------ pixstats / GroupNorm statistics */
#define FIELD(obj, name, dst, ...)                                                        \
  do {                                                                                    \
    uint64_t t_;                                                                          \
    if (!field_u64(env, obj, name, &t_)) { napi_throw_type_error(env, NULL, "field " name); return NULL; } \
    dst = __VA_ARGS__ t_;                                                                 \
  } while (0)

static napi_value pixstats(napi_env env, napi_callback_info info) {   /* (ctx, {x_buf, x_off, x_size, V, C, eps, r_buf, ro, r_size}) */
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  napi_value o = argv[1];
  p0k_pixstats_args a;
  memset(&a, 0, sizeof a);
  a.struct_size = sizeof a;
  FIELD(o, "x_buf", a.x_buf, (const void *)(uintptr_t));
  FIELD(o, "x_off", a.x_off, ); FIELD(o, "x_size", a.x_size, ); FIELD(o, "V", a.V, ); FIELD(o, "C", a.C, );
  FIELD(o, "r_buf", a.r_buf, (float *)(uintptr_t));
  FIELD(o, "ro", a.ro, ); FIELD(o, "r_size", a.r_size, );
  if (!field_f32(env, o, "eps", &a.eps)) { napi_throw_type_error(env, NULL, "field eps"); return NULL; }
  int r = p0k_pixstats(get_ctx(env, argv[0]), &a);
  if (r) return throw_p0k(env, r);
  return undef(env);
}

static napi_value gn(napi_env env, napi_callback_info info) {   /* (ctx, desc, what 1 | 2 | 3) -> partial rows written */
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  napi_value o = argv[1];
  int32_t what = 3;
  napi_get_value_int32(env, argv[2], &what);
  p0k_gn_args a;
  memset(&a, 0, sizeof a);
  a.struct_size = sizeof a;
  FIELD(o, "x_buf", a.x_buf, (const void *)(uintptr_t));
  FIELD(o, "x_off", a.x_off, ); FIELD(o, "x_size", a.x_size, ); FIELD(o, "pix", a.pix, ); FIELD(o, "C", a.C, );
  FIELD(o, "part_buf", a.part_buf, (float *)(uintptr_t));
  FIELD(o, "wg_off", a.wg_off, ); FIELD(o, "nwg", a.nwg, ); FIELD(o, "part_size", a.part_size, );
  FIELD(o, "gb_buf", a.gb_buf, (const float *)(uintptr_t));
  FIELD(o, "g_off", a.g_off, ); FIELD(o, "b_off", a.b_off, ); FIELD(o, "gb_size", a.gb_size, );
  FIELD(o, "ab_buf", a.ab_buf, (float *)(uintptr_t));
  FIELD(o, "ab_off", a.ab_off, ); FIELD(o, "ab_size", a.ab_size, );
  if (!field_f32(env, o, "eps", &a.eps)) { napi_throw_type_error(env, NULL, "field eps"); return NULL; }
  p0k_ctx *ctx = get_ctx(env, argv[0]);
  uint32_t nwg = 0;
  int r = what == 1 ? p0k_gn_partial(ctx, &a, &nwg) : what == 2 ? p0k_gn_finalize(ctx, &a) : p0k_groupnorm_stats(ctx, &a);
  if (r) return throw_p0k(env, r);
  return mk_num(env, nwg);
}

static napi_value attention(napi_env env, napi_callback_info info) {   /* (ctx, desc) -> flops */
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  napi_value o = argv[1];
  p0k_attn_args a;
  memset(&a, 0, sizeof a);
  a.struct_size = sizeof a;
  FIELD(o, "q_buf", a.q_buf, (const void *)(uintptr_t)); FIELD(o, "q_off", a.q_off, ); FIELD(o, "q_size", a.q_size, );
  FIELD(o, "k_buf", a.k_buf, (const void *)(uintptr_t)); FIELD(o, "k_off", a.k_off, ); FIELD(o, "k_size", a.k_size, );
  FIELD(o, "v_buf", a.v_buf, (const void *)(uintptr_t)); FIELD(o, "v_off", a.v_off, ); FIELD(o, "v_size", a.v_size, );
  FIELD(o, "o_buf", a.o_buf, (void *)(uintptr_t)); FIELD(o, "o_off", a.o_off, ); FIELD(o, "o_size", a.o_size, );
  FIELD(o, "ldo", a.ldo, ); FIELD(o, "Lq", a.Lq, ); FIELD(o, "Lk", a.Lk, ); FIELD(o, "Hq", a.Hq, ); FIELD(o, "Hkv", a.Hkv, );
  FIELD(o, "mode", a.mode, ); FIELD(o, "nvalid", a.nvalid, );
  if (!field_f32(env, o, "scale", &a.scale) || !field_f32(env, o, "cap", &a.cap)) {
    napi_throw_type_error(env, NULL, "field scale / cap");
    return NULL;
  }
  int r = p0k_attention(get_ctx(env, argv[0]), &a);
  if (r) return throw_p0k(env, r);
  return mk_num(env, p0k_attention_flops(&a));
}

static napi_value gnPartBytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  uint64_t pix;
  if (!to_u64(env, argv[0], &pix)) return NULL;
  return mk_num(env, (double)p0k_gn_part_bytes((uint32_t)pix));
}

/* ------------------------------------------------------------------ encoders (host) */
static napi_value pack_q(napi_env env, napi_callback_info info, int enc) {   /* (Float32Array W, rows, K, deq?) -> Uint8Array */
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return NULL;
  void *w;
  size_t wl;
  uint64_t rows, K;
  if (!get_bytes(env, argv[0], &w, &wl) || !to_u64(env, argv[1], &rows) || !to_u64(env, argv[2], &K)) {
    napi_throw_type_error(env, NULL, "pack: (Float32Array, rows, K[, deq Float32Array])");
    return NULL;
  }
  if (wl < rows * K * 4) { napi_throw_range_error(env, NULL, "pack: W holds fewer than rows * K floats"); return NULL; }
  float *deq = NULL;
  napi_valuetype t;
  napi_typeof(env, argv[3], &t);
  if (t != napi_undefined && t != napi_null) {
    void *d;
    size_t dl;
    if (!get_bytes(env, argv[3], &d, &dl) || dl < rows * K * 4) { napi_throw_type_error(env, NULL, "pack: deq must hold rows * K floats"); return NULL; }
    deq = (float *)d;
  }
  uint64_t nb = p0k_tensor_bytes(enc, (uint32_t)rows, (uint32_t)K);
  void *out;
  napi_value ab, arr;
  CHECK_NAPI(env, napi_create_arraybuffer(env, nb, &out, &ab));
  int r = enc == P0K_ENC_Q4G32A_T64 ? p0k_pack_q4((const float *)w, (uint32_t)rows, (uint32_t)K, (uint8_t *)out, deq)
                                    : p0k_pack_q8((const float *)w, (uint32_t)rows, (uint32_t)K, (uint8_t *)out, deq);
  if (r) {
    napi_throw_error(env, "P0K_E1", enc == P0K_ENC_Q4G32A_T64 ? "q4g32a.t64 needs rows % 64 == 0 and K % 32 == 0"
                                                               : "q8g64s.t64 needs rows % 64 == 0 and K % 64 == 0");
    return NULL;
  }
  CHECK_NAPI(env, napi_create_typedarray(env, napi_uint8_array, nb, ab, 0, &arr));
  return arr;
}
static napi_value packQ4(napi_env env, napi_callback_info info) { return pack_q(env, info, P0K_ENC_Q4G32A_T64); }
static napi_value packQ8(napi_env env, napi_callback_info info) { return pack_q(env, info, P0K_ENC_Q8G64S_T64); }

static napi_value packF16(napi_env env, napi_callback_info info) {   /* (Float32Array) -> Uint16Array */
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  void *w;
  size_t wl;
  if (!get_bytes(env, argv[0], &w, &wl)) { napi_throw_type_error(env, NULL, "packF16: Float32Array"); return NULL; }
  size_t n = wl / 4;
  void *out;
  napi_value ab, arr;
  CHECK_NAPI(env, napi_create_arraybuffer(env, n * 2, &out, &ab));
  p0k_pack_f16((const float *)w, n, (uint16_t *)out);
  CHECK_NAPI(env, napi_create_typedarray(env, napi_uint16_array, n, ab, 0, &arr));
  return arr;
}

static napi_value tensorBytes(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  uint64_t e, r, c;
  if (!to_u64(env, argv[0], &e) || !to_u64(env, argv[1], &r) || !to_u64(env, argv[2], &c)) return NULL;
  return mk_num(env, (double)p0k_tensor_bytes((int)e, (uint32_t)r, (uint32_t)c));
}

static napi_value lastError(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value s;
  napi_create_string_utf8(env, p0k_last_error(), NAPI_AUTO_LENGTH, &s);
  return s;
}

static napi_value abiVersion(napi_env env, napi_callback_info info) {
  (void)info;
  return mk_num(env, p0k_abi_version());
}

static napi_value init(napi_env env, napi_value exports) {
  const struct { const char *n; napi_callback f; } fns[] = {
      {"ctxCreate", ctxCreate}, {"ctxDestroy", ctxDestroy}, {"deviceInfo", deviceInfo}, {"alloc", alloc},
      {"free", free_}, {"upload", upload}, {"download", download}, {"copy", copy}, {"sync", sync_},
      {"poolStats", poolStats}, {"drainPool", drainPool}, {"gemm", gemm}, {"gemmCheck", gemmCheck},
      {"selectTile", selectTile}, {"rowstats", rowstats}, {"packQ4", packQ4}, {"packQ8", packQ8},
      {"packF16", packF16}, {"tensorBytes", tensorBytes}, {"lastError", lastError}, {"abiVersion", abiVersion},
      {"pixstats", pixstats}, {"gn", gn}, {"gnPartBytes", gnPartBytes}, {"attention", attention},
  };
  for (size_t i = 0; i < sizeof fns / sizeof fns[0]; i++) {
    napi_value f;
    if (napi_create_function(env, fns[i].n, NAPI_AUTO_LENGTH, fns[i].f, NULL, &f) != napi_ok) return NULL;
    if (napi_set_named_property(env, exports, fns[i].n, f) != napi_ok) return NULL;
  }
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
