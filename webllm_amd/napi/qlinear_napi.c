/*
 * Node-API binding of libqlinear.so (include/qlinear.h) for the reference's TypeScript host.
 *
 * Thin and synchronous: each function forwards to one C-ABI entry point; GPU work stays
 * asynchronous inside the library's stream. Handles are JS externals; offsets and sizes are JS
 * numbers (exact up to 2^53). A failing status throws an Error carrying ql_last_error() and a
 * `code` property (QL_E_*), the way the reference throws `new Error(msg)` (quant.ts:46-79).
 */
#define NAPI_VERSION 6
#include <node_api.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/qlinear.h"

#define CHECK_NAPI(env, call)                                             \
    do {                                                                  \
        if ((call) != napi_ok) {                                          \
            napi_throw_error((env), "QL_E_NAPI", "Node-API call failed: " #call); \
            return NULL;                                                  \
        }                                                                 \
    } while (0)

static const char* code_name(int rc)
{
    switch (rc) {
    case QL_E_BITS: return "QL_E_BITS";
    case QL_E_GROUP: return "QL_E_GROUP";
    case QL_E_DIMS: return "QL_E_DIMS";
    case QL_E_QWEIGHT_SHORT: return "QL_E_QWEIGHT_SHORT";
    case QL_E_SCALES_SHORT: return "QL_E_SCALES_SHORT";
    case QL_E_QZEROS_SHORT: return "QL_E_QZEROS_SHORT";
    case QL_E_GROUP_PACK: return "QL_E_GROUP_PACK";
    case QL_E_INVALID: return "QL_E_INVALID";
    case QL_E_RANGE: return "QL_E_RANGE";
    case QL_E_ALIGN: return "QL_E_ALIGN";
    case QL_E_HIP: return "QL_E_HIP";
    case QL_E_STATE: return "QL_E_STATE";
    default: return "QL_E_UNKNOWN";
    }
}

/* returns 1 (and throws) when rc is an error */
static int throw_rc(napi_env env, int rc)
{
    if (rc == QL_OK) return 0;
    char msg[600];
    snprintf(msg, sizeof msg, "%s: %s", code_name(rc), ql_last_error());
    napi_throw_error(env, code_name(rc), msg);
    return 1;
}

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv)
{
    size_t argc = want;
    if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok || argc < want) {
        napi_throw_type_error(env, "QL_E_INVALID", "too few arguments");
        return 1;
    }
    return 0;
}

static int get_ptr(napi_env env, napi_value v, void** out)
{
    napi_valuetype t;
    if (napi_typeof(env, v, &t) != napi_ok || t != napi_external ||
        napi_get_value_external(env, v, out) != napi_ok) {
        napi_throw_type_error(env, "QL_E_INVALID", "expected a qlinear handle");
        return 1;
    }
    return 0;
}

static int get_i32(napi_env env, napi_value v, int32_t* out)
{
    if (napi_get_value_int32(env, v, out) != napi_ok) {
        napi_throw_type_error(env, "QL_E_INVALID", "expected an integer");
        return 1;
    }
    return 0;
}

/* non-negative integer offset/size as a JS number; null/undefined -> QL_NONE when allow_none */
static int get_u64(napi_env env, napi_value v, uint64_t* out, int allow_none)
{
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (allow_none && (t == napi_null || t == napi_undefined)) {
        *out = QL_NONE;
        return 0;
    }
    double d;
    if (t != napi_number || napi_get_value_double(env, v, &d) != napi_ok || d < 0 ||
        d > 9007199254740992.0 || d != (double)(uint64_t)d) {
        napi_throw_type_error(env, "QL_E_INVALID", "expected a non-negative integer");
        return 1;
    }
    *out = (uint64_t)d;
    return 0;
}

static napi_value make_u64(napi_env env, uint64_t v)
{
    napi_value r;
    napi_create_double(env, (double)v, &r);
    return r;
}

static napi_value make_i32(napi_env env, int32_t v)
{
    napi_value r;
    napi_create_int32(env, v, &r);
    return r;
}

static int prop(napi_env env, napi_value obj, const char* name, napi_value* out)
{
    if (napi_get_named_property(env, obj, name, out) != napi_ok) {
        napi_throw_type_error(env, "QL_E_INVALID", name);
        return 1;
    }
    return 0;
}

/* {qweightOff, qzerosOff|null, scalesOff, biasOff|null, K, N, group, bits} -> ql_gptq_desc */
static int get_desc(napi_env env, napi_value obj, ql_gptq_desc* d)
{
    napi_value v;
    memset(d, 0, sizeof *d);
    if (prop(env, obj, "qweightOff", &v) || get_u64(env, v, &d->qweight_off, 0)) return 1;
    if (prop(env, obj, "qzerosOff", &v) || get_u64(env, v, &d->qzeros_off, 1)) return 1;
    if (prop(env, obj, "scalesOff", &v) || get_u64(env, v, &d->scales_off, 0)) return 1;
    if (prop(env, obj, "biasOff", &v) || get_u64(env, v, &d->bias_off, 1)) return 1;
    if (prop(env, obj, "K", &v) || get_i32(env, v, &d->K)) return 1;
    if (prop(env, obj, "N", &v) || get_i32(env, v, &d->N)) return 1;
    if (prop(env, obj, "group", &v) || get_i32(env, v, &d->group)) return 1;
    if (prop(env, obj, "bits", &v) || get_i32(env, v, &d->bits)) return 1;
    return 0;
}

/* bytes of a TypedArray / Buffer / ArrayBuffer / DataView */
static int get_bytes(napi_env env, napi_value v, void** data, size_t* len)
{
    bool is;
    if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
        napi_typedarray_type type;
        size_t n, off;
        napi_value ab;
        void* base;
        if (napi_get_typedarray_info(env, v, &type, &n, &base, &ab, &off) != napi_ok) goto bad;
        size_t es = 1;
        switch (type) {
        case napi_int16_array: case napi_uint16_array: es = 2; break;
        case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
        case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
        default: es = 1;
        }
        *data = base;
        *len = n * es;
        return 0;
    }
    if (napi_is_dataview(env, v, &is) == napi_ok && is) {
        napi_value ab;
        size_t off;
        if (napi_get_dataview_info(env, v, len, data, &ab, &off) != napi_ok) goto bad;
        return 0;
    }
    if (napi_is_arraybuffer(env, v, &is) == napi_ok && is) {
        if (napi_get_arraybuffer_info(env, v, data, len) != napi_ok) goto bad;
        return 0;
    }
bad:
    napi_throw_type_error(env, "QL_E_INVALID", "expected a TypedArray, DataView or ArrayBuffer");
    return 1;
}

/* ---------------------------------------------------------------------------------- context */

static napi_value js_create(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    int32_t dev = 0;
    size_t argc = 1;
    CHECK_NAPI(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
    if (argc >= 1 && get_i32(env, argv[0], &dev)) return NULL;
    ql_ctx* ctx = NULL;
    if (throw_rc(env, ql_create(dev, &ctx))) return NULL;
    napi_value r;
    CHECK_NAPI(env, napi_create_external(env, ctx, NULL, NULL, &r));
    return r;
}

static napi_value js_destroy(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* ctx;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &ctx)) return NULL;
    throw_rc(env, ql_destroy((ql_ctx*)ctx));
    return NULL;
}

static napi_value js_device_info(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* ctx;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &ctx)) return NULL;
    char name[256];
    int cus = 0;
    uint64_t hbm = 0;
    if (throw_rc(env, ql_device_info((ql_ctx*)ctx, name, sizeof name, &cus, &hbm))) return NULL;
    napi_value o, s;
    CHECK_NAPI(env, napi_create_object(env, &o));
    CHECK_NAPI(env, napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &s));
    napi_set_named_property(env, o, "name", s);
    napi_set_named_property(env, o, "cuCount", make_i32(env, cus));
    napi_set_named_property(env, o, "hbmBytes", make_u64(env, hbm));
    return o;
}

static napi_value js_last_error(napi_env env, napi_callback_info info)
{
    (void)info;
    napi_value s;
    CHECK_NAPI(env, napi_create_string_utf8(env, ql_last_error(), NAPI_AUTO_LENGTH, &s));
    return s;
}

/* ----------------------------------------------------------------------------------- arenas */

static napi_value js_arena_reserve(napi_env env, napi_callback_info info)
{
    napi_value argv[2];
    void* ctx;
    uint64_t bytes;
    if (get_args(env, info, 2, argv) || get_ptr(env, argv[0], &ctx) || get_u64(env, argv[1], &bytes, 0))
        return NULL;
    ql_arena* a = NULL;
    if (throw_rc(env, ql_arena_reserve((ql_ctx*)ctx, bytes, &a))) return NULL;
    napi_value r;
    CHECK_NAPI(env, napi_create_external(env, a, NULL, NULL, &r));
    return r;
}

static napi_value js_arena_release(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* a;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &a)) return NULL;
    throw_rc(env, ql_arena_release((ql_arena*)a));
    return NULL;
}

static napi_value js_arena_size(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* a;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &a)) return NULL;
    return make_u64(env, ql_arena_size((ql_arena*)a));
}

/* arenaWrite(arena, off, typedArrayOrBuffer) */
static napi_value js_arena_write(napi_env env, napi_callback_info info)
{
    napi_value argv[3];
    void* a;
    uint64_t off;
    void* data;
    size_t len;
    if (get_args(env, info, 3, argv) || get_ptr(env, argv[0], &a) || get_u64(env, argv[1], &off, 0) ||
        get_bytes(env, argv[2], &data, &len))
        return NULL;
    throw_rc(env, ql_arena_write((ql_arena*)a, off, data, len));
    return NULL;
}

/* arenaRead(arena, off, typedArrayToFill) */
static napi_value js_arena_read(napi_env env, napi_callback_info info)
{
    napi_value argv[3];
    void* a;
    uint64_t off;
    void* data;
    size_t len;
    if (get_args(env, info, 3, argv) || get_ptr(env, argv[0], &a) || get_u64(env, argv[1], &off, 0) ||
        get_bytes(env, argv[2], &data, &len))
        return NULL;
    throw_rc(env, ql_arena_read((ql_arena*)a, off, data, len));
    return NULL;
}

/* ---------------------------------------------------------------------- descriptors, planning */

static napi_value js_gptq_sizes(napi_env env, napi_callback_info info)
{
    napi_value argv[3];
    int32_t K, N, g;
    if (get_args(env, info, 3, argv) || get_i32(env, argv[0], &K) || get_i32(env, argv[1], &N) ||
        get_i32(env, argv[2], &g))
        return NULL;
    uint64_t a, b, c;
    if (throw_rc(env, ql_gptq_sizes(K, N, g, &a, &b, &c))) return NULL;
    napi_value o;
    CHECK_NAPI(env, napi_create_object(env, &o));
    napi_set_named_property(env, o, "qweightBytes", make_u64(env, a));
    napi_set_named_property(env, o, "qzerosBytes", make_u64(env, b));
    napi_set_named_property(env, o, "scalesBytes", make_u64(env, c));
    return o;
}

/* validate(desc, arenaBytes) -> status code (0 ok), does not throw for GPTQ classes */
static napi_value js_validate(napi_env env, napi_callback_info info)
{
    napi_value argv[2];
    ql_gptq_desc d;
    uint64_t bytes;
    if (get_args(env, info, 2, argv) || get_desc(env, argv[0], &d) || get_u64(env, argv[1], &bytes, 0))
        return NULL;
    return make_i32(env, ql_gptq_validate(&d, bytes));
}

static napi_value js_plan_linear(napi_env env, napi_callback_info info)
{
    napi_value argv[4];
    int32_t M, N, K, g;
    if (get_args(env, info, 4, argv) || get_i32(env, argv[0], &M) || get_i32(env, argv[1], &N) ||
        get_i32(env, argv[2], &K) || get_i32(env, argv[3], &g))
        return NULL;
    ql_plan p;
    if (throw_rc(env, ql_plan_linear(M, N, K, g, &p))) return NULL;
    static const char* kinds[] = {"", "gemv_mfma", "gemv_simple", "gemm_mfma", "gemm_simple"};
    napi_value o, s;
    CHECK_NAPI(env, napi_create_object(env, &o));
    CHECK_NAPI(env, napi_create_string_utf8(env, p.kind >= 1 && p.kind <= 4 ? kinds[p.kind] : "?",
                                            NAPI_AUTO_LENGTH, &s));
    napi_set_named_property(env, o, "kind", s);
    napi_set_named_property(env, o, "split", make_i32(env, p.split));
    napi_set_named_property(env, o, "gridX", make_i32(env, p.grid_x));
    napi_set_named_property(env, o, "gridY", make_i32(env, p.grid_y));
    napi_set_named_property(env, o, "block", make_i32(env, p.block));
    napi_set_named_property(env, o, "scratchBytes", make_u64(env, p.scratch_bytes));
    napi_set_named_property(env, o, "refSplit", make_i32(env, p.ref_split));
    return o;
}

static int get_desc_array(napi_env env, napi_value arr, ql_gptq_desc* out, uint32_t* n)
{
    if (napi_get_array_length(env, arr, n) != napi_ok || *n == 0 || *n > 8) {
        napi_throw_type_error(env, "QL_E_INVALID", "expected an array of 1..8 descriptors");
        return 1;
    }
    for (uint32_t i = 0; i < *n; i++) {
        napi_value e;
        if (napi_get_element(env, arr, i, &e) != napi_ok || get_desc(env, e, &out[i])) return 1;
    }
    return 0;
}

static int get_u64_array(napi_env env, napi_value arr, uint64_t* out, uint32_t n)
{
    uint32_t m;
    if (napi_get_array_length(env, arr, &m) != napi_ok || m != n) {
        napi_throw_type_error(env, "QL_E_INVALID", "offset array length mismatch");
        return 1;
    }
    for (uint32_t i = 0; i < n; i++) {
        napi_value e;
        if (napi_get_element(env, arr, i, &e) != napi_ok || get_u64(env, e, &out[i], 0)) return 1;
    }
    return 0;
}

static napi_value js_plan_batch(napi_env env, napi_callback_info info)
{
    napi_value argv[2];
    ql_gptq_desc d[8];
    uint32_t n;
    int32_t M;
    if (get_args(env, info, 2, argv) || get_desc_array(env, argv[0], d, &n) || get_i32(env, argv[1], &M))
        return NULL;
    uint64_t bytes;
    if (throw_rc(env, ql_plan_batch((int32_t)n, d, M, &bytes))) return NULL;
    return make_u64(env, bytes);
}

/* ------------------------------------------------------------------------------------- work */

/* unpack(ctx, desc, weights, out, outOff, f32[, scalesDtype]) */
static napi_value js_unpack(napi_env env, napi_callback_info info)
{
    napi_value argv[6];
    void *ctx, *w, *o;
    ql_gptq_desc d;
    uint64_t off;
    bool f32 = false;
    if (get_args(env, info, 6, argv) || get_ptr(env, argv[0], &ctx) || get_desc(env, argv[1], &d) ||
        get_ptr(env, argv[2], &w) || get_ptr(env, argv[3], &o) || get_u64(env, argv[4], &off, 0))
        return NULL;
    napi_get_value_bool(env, argv[5], &f32);
    /* optional 7th argument: the scales' dtype for the fp32 form (QL_DTYPE_F32: f32 scales) */
    size_t argc = 7;
    napi_value all[7];
    int32_t sdt = QL_DTYPE_F16;
    if (napi_get_cb_info(env, info, &argc, all, NULL, NULL) == napi_ok && argc >= 7) {
        napi_valuetype t;
        if (napi_typeof(env, all[6], &t) == napi_ok && t != napi_undefined && get_i32(env, all[6], &sdt))
            return NULL;
    }
    throw_rc(env, f32 ? ql_unpack_f32_ex((ql_ctx*)ctx, &d, (ql_arena*)w, sdt, (ql_arena*)o, off)
                      : ql_unpack_f16((ql_ctx*)ctx, &d, (ql_arena*)w, (ql_arena*)o, off));
    return NULL;
}

/* linear(ctx, desc, weights, act, xOff, xDtype, M, yOff, scratchOff) */
static napi_value js_linear(napi_env env, napi_callback_info info)
{
    napi_value argv[9];
    void *ctx, *w, *act;
    ql_gptq_desc d;
    uint64_t x_off, y_off, s_off;
    int32_t xdt, M;
    if (get_args(env, info, 9, argv) || get_ptr(env, argv[0], &ctx) || get_desc(env, argv[1], &d) ||
        get_ptr(env, argv[2], &w) || get_ptr(env, argv[3], &act) || get_u64(env, argv[4], &x_off, 0) ||
        get_i32(env, argv[5], &xdt) || get_i32(env, argv[6], &M) || get_u64(env, argv[7], &y_off, 0) ||
        get_u64(env, argv[8], &s_off, 0))
        return NULL;
    throw_rc(env, ql_linear((ql_ctx*)ctx, &d, (ql_arena*)w, (ql_arena*)act, x_off, xdt, M, y_off, s_off));
    return NULL;
}

/* linearBatch(ctx, descs[], weights, act, xOffs[], xDtype, M, yOffs[], scratchOff) */
static napi_value js_linear_batch(napi_env env, napi_callback_info info)
{
    napi_value argv[9];
    void *ctx, *w, *act;
    ql_gptq_desc d[8];
    uint64_t xo[8], yo[8], s_off;
    uint32_t n;
    int32_t xdt, M;
    if (get_args(env, info, 9, argv) || get_ptr(env, argv[0], &ctx) || get_desc_array(env, argv[1], d, &n) ||
        get_ptr(env, argv[2], &w) || get_ptr(env, argv[3], &act) || get_u64_array(env, argv[4], xo, n) ||
        get_i32(env, argv[5], &xdt) || get_i32(env, argv[6], &M) || get_u64_array(env, argv[7], yo, n) ||
        get_u64(env, argv[8], &s_off, 0))
        return NULL;
    throw_rc(env, ql_linear_batch((ql_ctx*)ctx, (int32_t)n, d, (ql_arena*)w, (ql_arena*)act, xo, xdt, M,
                                  yo, s_off));
    return NULL;
}

/* gemvF16w(ctx, weights, wOff, biasOff|null, act, xOff, M, N, K, yOff): fp16-weight GEMV (lm_head) */
static napi_value js_gemv_f16w(napi_env env, napi_callback_info info)
{
    napi_value argv[10];
    void *ctx, *w, *act;
    uint64_t w_off, b_off, x_off, y_off;
    int32_t M, N, K;
    if (get_args(env, info, 10, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[1], &w) ||
        get_u64(env, argv[2], &w_off, 0) || get_u64(env, argv[3], &b_off, 1) || get_ptr(env, argv[4], &act) ||
        get_u64(env, argv[5], &x_off, 0) || get_i32(env, argv[6], &M) || get_i32(env, argv[7], &N) ||
        get_i32(env, argv[8], &K) || get_u64(env, argv[9], &y_off, 0))
        return NULL;
    throw_rc(env, ql_gemv_f16w((ql_ctx*)ctx, (ql_arena*)w, w_off, b_off, (ql_arena*)act, x_off, M, N, K, y_off));
    return NULL;
}

/* embedF16(ctx, weights, embedOff, vocab, D, act, tokensOff, rows, outOff): embedding lookup */
static napi_value js_embed_f16(napi_env env, napi_callback_info info)
{
    napi_value argv[9];
    void *ctx, *w, *act;
    uint64_t e_off, t_off, o_off;
    int32_t vocab, D, rows;
    if (get_args(env, info, 9, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[1], &w) ||
        get_u64(env, argv[2], &e_off, 0) || get_i32(env, argv[3], &vocab) || get_i32(env, argv[4], &D) ||
        get_ptr(env, argv[5], &act) || get_u64(env, argv[6], &t_off, 0) || get_i32(env, argv[7], &rows) ||
        get_u64(env, argv[8], &o_off, 0))
        return NULL;
    throw_rc(env, ql_embed_f16((ql_ctx*)ctx, (ql_arena*)w, e_off, vocab, D, (ql_arena*)act, t_off, rows, o_off));
    return NULL;
}

/* kvStore(ctx, act, srcOff, cache, cacheOff, maxT, rows, rowLen, pos0) */
static napi_value js_kv_store(napi_env env, napi_callback_info info)
{
    napi_value argv[9];
    void *ctx, *act, *cache;
    uint64_t src_off, c_off;
    int32_t max_t, rows, row_len, pos0;
    if (get_args(env, info, 9, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[1], &act) ||
        get_u64(env, argv[2], &src_off, 0) || get_ptr(env, argv[3], &cache) || get_u64(env, argv[4], &c_off, 0) ||
        get_i32(env, argv[5], &max_t) || get_i32(env, argv[6], &rows) || get_i32(env, argv[7], &row_len) ||
        get_i32(env, argv[8], &pos0))
        return NULL;
    throw_rc(env, ql_kv_store((ql_ctx*)ctx, (ql_arena*)act, src_off, (ql_arena*)cache, c_off, max_t, rows, row_len, pos0));
    return NULL;
}

/* attention(ctx, act, qOff, cache, kOff, vOff, maxT, M, nHead, nKvHead, D, pastLen, outOff) */
static napi_value js_attention(napi_env env, napi_callback_info info)
{
    napi_value argv[13];
    void *ctx, *act, *cache;
    uint64_t q_off, k_off, v_off, o_off;
    int32_t max_t, M, H, KV, D, past;
    if (get_args(env, info, 13, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[1], &act) ||
        get_u64(env, argv[2], &q_off, 0) || get_ptr(env, argv[3], &cache) || get_u64(env, argv[4], &k_off, 0) ||
        get_u64(env, argv[5], &v_off, 0) || get_i32(env, argv[6], &max_t) || get_i32(env, argv[7], &M) ||
        get_i32(env, argv[8], &H) || get_i32(env, argv[9], &KV) || get_i32(env, argv[10], &D) ||
        get_i32(env, argv[11], &past) || get_u64(env, argv[12], &o_off, 0))
        return NULL;
    throw_rc(env, ql_attention_decode((ql_ctx*)ctx, (ql_arena*)act, q_off, (ql_arena*)cache, k_off, v_off, max_t,
                                      M, H, KV, D, past, o_off));
    return NULL;
}

/* addRmsNorm(ctx, act, xOff, dOff|null, weights, wOff, eps, M, C, sumOff|null, yOff) */
static napi_value js_add_rmsnorm(napi_env env, napi_callback_info info)
{
    napi_value argv[11];
    void *ctx, *act, *w;
    uint64_t x_off, d_off, w_off, s_off, y_off;
    int32_t M, C;
    double eps;
    if (get_args(env, info, 11, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[1], &act) ||
        get_u64(env, argv[2], &x_off, 0) || get_u64(env, argv[3], &d_off, 1) || get_ptr(env, argv[4], &w) ||
        get_u64(env, argv[5], &w_off, 0))
        return NULL;
    if (napi_get_value_double(env, argv[6], &eps) != napi_ok) {
        napi_throw_type_error(env, "QL_E_INVALID", "eps must be a number");
        return NULL;
    }
    if (get_i32(env, argv[7], &M) || get_i32(env, argv[8], &C) || get_u64(env, argv[9], &s_off, 1) ||
        get_u64(env, argv[10], &y_off, 0))
        return NULL;
    throw_rc(env, ql_add_rmsnorm((ql_ctx*)ctx, (ql_arena*)act, x_off, d_off, (ql_arena*)w, w_off, (float)eps, M, C,
                                 s_off, y_off));
    return NULL;
}

/* siluMul(ctx, act, gateOff, upOff, n, yOff) */
static napi_value js_silu_mul(napi_env env, napi_callback_info info)
{
    napi_value argv[6];
    void *ctx, *act;
    uint64_t g_off, u_off, n, y_off;
    if (get_args(env, info, 6, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[1], &act) ||
        get_u64(env, argv[2], &g_off, 0) || get_u64(env, argv[3], &u_off, 0) || get_u64(env, argv[4], &n, 0) ||
        get_u64(env, argv[5], &y_off, 0))
        return NULL;
    throw_rc(env, ql_silu_mul((ql_ctx*)ctx, (ql_arena*)act, g_off, u_off, (int64_t)n, y_off));
    return NULL;
}

/* unpackBatch(ctx, descs[], w, out, outOffs[]): the whole weight set, ql_unpack_f16_batch */
static napi_value js_unpack_batch(napi_env env, napi_callback_info info)
{
    napi_value argv[5];
    void *ctx, *w, *o;
    uint32_t n = 0, m = 0;
    if (get_args(env, info, 5, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[2], &w) ||
        get_ptr(env, argv[3], &o))
        return NULL;
    if (napi_get_array_length(env, argv[1], &n) != napi_ok || napi_get_array_length(env, argv[4], &m) != napi_ok ||
        n != m) {
        napi_throw_type_error(env, "QL_E_INVALID", "expected descriptor and offset arrays of one length");
        return NULL;
    }
    ql_gptq_desc* d = (ql_gptq_desc*)calloc(n ? n : 1, sizeof *d);
    uint64_t* off = (uint64_t*)calloc(n ? n : 1, sizeof *off);
    int bad = !d || !off;
    for (uint32_t i = 0; i < n && !bad; i++) {
        napi_value e;
        bad = napi_get_element(env, argv[1], i, &e) != napi_ok || get_desc(env, e, &d[i]) ||
              napi_get_element(env, argv[4], i, &e) != napi_ok || get_u64(env, e, &off[i], 0);
    }
    if (!bad) throw_rc(env, ql_unpack_f16_batch((ql_ctx*)ctx, (int32_t)n, d, (ql_arena*)w, (ql_arena*)o, off));
    else if (!d || !off) napi_throw_error(env, "QL_E_INVALID", "out of host memory");
    free(d);
    free(off);
    return NULL;
}

static napi_value js_sync(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* ctx;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &ctx)) return NULL;
    throw_rc(env, ql_sync((ql_ctx*)ctx));
    return NULL;
}

static napi_value js_timer_start(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* ctx;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &ctx)) return NULL;
    throw_rc(env, ql_timer_start((ql_ctx*)ctx));
    return NULL;
}

static napi_value js_timer_stop(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* ctx;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &ctx)) return NULL;
    float ms = 0.f;
    if (throw_rc(env, ql_timer_stop((ql_ctx*)ctx, &ms))) return NULL;
    napi_value r;
    napi_create_double(env, ms, &r);
    return r;
}

static napi_value js_graph_begin(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* ctx;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &ctx)) return NULL;
    throw_rc(env, ql_graph_begin((ql_ctx*)ctx));
    return NULL;
}

static napi_value js_graph_end(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* ctx;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &ctx)) return NULL;
    ql_graph* g = NULL;
    if (throw_rc(env, ql_graph_end((ql_ctx*)ctx, &g))) return NULL;
    napi_value r;
    CHECK_NAPI(env, napi_create_external(env, g, NULL, NULL, &r));
    return r;
}

static napi_value js_graph_launch(napi_env env, napi_callback_info info)
{
    napi_value argv[2];
    void *ctx, *g;
    if (get_args(env, info, 2, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[1], &g)) return NULL;
    throw_rc(env, ql_graph_launch((ql_ctx*)ctx, (ql_graph*)g));
    return NULL;
}

static napi_value js_graph_destroy(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* g;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &g)) return NULL;
    throw_rc(env, ql_graph_destroy((ql_graph*)g));
    return NULL;
}

/* {normWOff|null, normEps, x2Off|null, resOff|null} (any may be absent; null/undefined = no fusion)
   -> ql_seq_fuse */
static int get_fuse(napi_env env, napi_value obj, ql_seq_fuse* f)
{
    napi_valuetype t;
    memset(f, 0, sizeof *f);
    f->norm_w_off = f->x2_off = f->res_off = QL_NONE;
    f->norm_eps = 1e-6f;
    if (napi_typeof(env, obj, &t) != napi_ok) return 1;
    if (t == napi_null || t == napi_undefined) return 0;
    if (t != napi_object) {
        napi_throw_type_error(env, "QL_E_INVALID", "expected a fusion object or null");
        return 1;
    }
    static const char* const names[3] = {"normWOff", "x2Off", "resOff"};
    uint64_t* const dst[3] = {&f->norm_w_off, &f->x2_off, &f->res_off};
    for (int k = 0; k < 3; k++) {
        bool has = false;
        napi_value v;
        if (napi_has_named_property(env, obj, names[k], &has) != napi_ok) return 1;
        if (has && (prop(env, obj, names[k], &v) || get_u64(env, v, dst[k], 1))) return 1;
    }
    bool has = false;
    if (napi_has_named_property(env, obj, "normEps", &has) != napi_ok) return 1;
    if (has) {
        napi_value v;
        double eps;
        if (prop(env, obj, "normEps", &v)) return 1;
        if (napi_get_value_double(env, v, &eps) != napi_ok) {
            napi_throw_type_error(env, "QL_E_INVALID", "normEps must be a number");
            return 1;
        }
        f->norm_eps = (float)eps;
    }
    return 0;
}

/* seqCreate(ctx, descs[], weights, act, xOffs[], xDtype, M, yOffs[], fuse[]?) -> sequence handle;
   with fuse (one entry per linear) the sequence is created by ql_seq_create_fused */
static napi_value js_seq_create(napi_env env, napi_callback_info info)
{
    napi_value argv[9];
    void *ctx, *w, *act;
    int32_t xdt, M;
    uint32_t n, m;
    size_t argc = 9;
    if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok || argc < 8) {
        napi_throw_type_error(env, "QL_E_INVALID", "too few arguments");
        return NULL;
    }
    if (get_ptr(env, argv[0], &ctx)) return NULL;
    if (napi_get_array_length(env, argv[1], &n) != napi_ok || n == 0 || n > 4096) {
        napi_throw_type_error(env, "QL_E_INVALID", "expected an array of 1..4096 descriptors");
        return NULL;
    }
    if (get_ptr(env, argv[2], &w) || get_ptr(env, argv[3], &act) || get_i32(env, argv[5], &xdt) ||
        get_i32(env, argv[6], &M))
        return NULL;
    if (napi_get_array_length(env, argv[4], &m) != napi_ok || m != n ||
        napi_get_array_length(env, argv[7], &m) != napi_ok || m != n) {
        napi_throw_type_error(env, "QL_E_INVALID", "offset arrays must match the descriptors");
        return NULL;
    }
    napi_valuetype ft = napi_undefined;
    if (argc > 8) napi_typeof(env, argv[8], &ft);
    const int fused = ft != napi_undefined && ft != napi_null;
    if (fused && (napi_get_array_length(env, argv[8], &m) != napi_ok || m != n)) {
        napi_throw_type_error(env, "QL_E_INVALID", "fuse must be an array with one entry per descriptor");
        return NULL;
    }
    ql_gptq_desc* d = (ql_gptq_desc*)calloc(n, sizeof(ql_gptq_desc));
    uint64_t* xo = (uint64_t*)calloc(n, sizeof(uint64_t));
    uint64_t* yo = (uint64_t*)calloc(n, sizeof(uint64_t));
    ql_seq_fuse* fz = fused ? (ql_seq_fuse*)calloc(n, sizeof(ql_seq_fuse)) : NULL;
    napi_value result = NULL;
    int bad = !d || !xo || !yo || (fused && !fz);
    for (uint32_t i = 0; i < n && fused && !bad; i++) {
        napi_value e;
        bad = napi_get_element(env, argv[8], i, &e) != napi_ok || get_fuse(env, e, &fz[i]);
    }
    for (uint32_t i = 0; i < n && !bad; i++) {
        napi_value e;
        bad = napi_get_element(env, argv[1], i, &e) != napi_ok || get_desc(env, e, &d[i]);
    }
    if (!bad) bad = get_u64_array(env, argv[4], xo, n) || get_u64_array(env, argv[7], yo, n);
    if (!bad) {
        ql_seq* seq = NULL;
        const int rc = fused ? ql_seq_create_fused((ql_ctx*)ctx, (int32_t)n, d, (ql_arena*)w, (ql_arena*)act, xo,
                                                   xdt, M, yo, fz, &seq)
                             : ql_seq_create((ql_ctx*)ctx, (int32_t)n, d, (ql_arena*)w, (ql_arena*)act, xo,
                                             xdt, M, yo, &seq);
        if (!throw_rc(env, rc)) napi_create_external(env, seq, NULL, NULL, &result);
    }
    free(fz);
    free(d);
    free(xo);
    free(yo);
    return result;
}

static napi_value js_seq_run(napi_env env, napi_callback_info info)
{
    napi_value argv[2];
    void *ctx, *seq;
    if (get_args(env, info, 2, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[1], &seq)) return NULL;
    throw_rc(env, ql_seq_run((ql_ctx*)ctx, (ql_seq*)seq));
    return NULL;
}

static napi_value js_seq_status(napi_env env, napi_callback_info info)
{
    napi_value argv[2];
    void *ctx, *seq;
    if (get_args(env, info, 2, argv) || get_ptr(env, argv[0], &ctx) || get_ptr(env, argv[1], &seq)) return NULL;
    throw_rc(env, ql_seq_status((ql_ctx*)ctx, (ql_seq*)seq));
    return NULL;
}

static napi_value js_seq_info(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* seq;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &seq)) return NULL;
    ql_seq_info si;
    if (throw_rc(env, ql_seq_get_info((ql_seq*)seq, &si))) return NULL;
    napi_value o;
    CHECK_NAPI(env, napi_create_object(env, &o));
    napi_set_named_property(env, o, "linears", make_i32(env, si.linears));
    napi_set_named_property(env, o, "passes", make_i32(env, si.passes));
    napi_set_named_property(env, o, "tiles", make_i32(env, si.tiles));
    napi_set_named_property(env, o, "reduces", make_i32(env, si.reduces));
    napi_set_named_property(env, o, "grid", make_i32(env, si.grid));
    napi_set_named_property(env, o, "maxSplit", make_i32(env, si.max_split));
    napi_set_named_property(env, o, "ldsBytes", make_u64(env, si.lds_bytes));
    napi_set_named_property(env, o, "deviceBytes", make_u64(env, si.device_bytes));
    napi_set_named_property(env, o, "totalUnits", make_u64(env, si.total_units));
    napi_set_named_property(env, o, "busiestUnits", make_u64(env, si.busiest_units));
    napi_value kv, sv;
    napi_create_int32(env, si.kernel, &kv);
    napi_create_int32(env, si.split, &sv);
    napi_set_named_property(env, o, "kernel", kv);
    napi_set_named_property(env, o, "split", sv);
    napi_set_named_property(env, o, "stream", make_i32(env, si.stream));
    napi_set_named_property(env, o, "variant", make_i32(env, si.variant));
    napi_set_named_property(env, o, "launches", make_i32(env, si.launches));
    return o;
}

static napi_value js_seq_destroy(napi_env env, napi_callback_info info)
{
    napi_value argv[1];
    void* seq;
    if (get_args(env, info, 1, argv) || get_ptr(env, argv[0], &seq)) return NULL;
    throw_rc(env, ql_seq_destroy((ql_seq*)seq));
    return NULL;
}

static napi_value init(napi_env env, napi_value exports)
{
    const struct {
        const char* name;
        napi_callback fn;
    } fns[] = {
        {"create", js_create}, {"destroy", js_destroy}, {"deviceInfo", js_device_info},
        {"lastError", js_last_error}, {"arenaReserve", js_arena_reserve},
        {"arenaRelease", js_arena_release}, {"arenaSize", js_arena_size},
        {"arenaWrite", js_arena_write}, {"arenaRead", js_arena_read}, {"gptqSizes", js_gptq_sizes},
        {"validate", js_validate}, {"planLinear", js_plan_linear}, {"planBatch", js_plan_batch},
        {"unpack", js_unpack}, {"unpackBatch", js_unpack_batch}, {"linear", js_linear}, {"linearBatch", js_linear_batch},
        {"sync", js_sync}, {"timerStart", js_timer_start}, {"timerStop", js_timer_stop},
        {"graphBegin", js_graph_begin}, {"graphEnd", js_graph_end},
        {"graphLaunch", js_graph_launch}, {"graphDestroy", js_graph_destroy},
        {"seqCreate", js_seq_create}, {"seqRun", js_seq_run}, {"seqStatus", js_seq_status},
        {"seqInfo", js_seq_info}, {"seqDestroy", js_seq_destroy},
        {"gemvF16w", js_gemv_f16w}, {"embedF16", js_embed_f16}, {"kvStore", js_kv_store}, {"attention", js_attention},
        {"addRmsNorm", js_add_rmsnorm}, {"siluMul", js_silu_mul},
    };
    for (size_t i = 0; i < sizeof fns / sizeof fns[0]; i++) {
        napi_value f;
        if (napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].fn, NULL, &f) != napi_ok ||
            napi_set_named_property(env, exports, fns[i].name, f) != napi_ok)
            return NULL;
    }
    return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
