/*
 * qq_napi.c -- Node-API binding of the C ABI in include/qq_moe.h.
 *
 * A thin layer: typed arrays and ArrayBuffers are passed to the library by
 * pointer (no copies on the JS side), handles are napi externals whose
 * finalizers release the device objects, and every non-zero status becomes a
 * thrown Error carrying qq_last_error(), as the reference throws from
 * matmulGeneric (src/tensor.js:494).
 *
 * Exports (all synchronous, like the JavaScript they replace):
 *   init(device) -> ctx
 *   lastError(ctx | null) -> string
 *   uploadQ80(ctx, bytes, byteOffset, inDim, outDim, nMats) -> tensor
 *       bytes: ArrayBuffer or typed array holding GGUF Q8_0 blocks
 *   matvec(ctx, tensor, mat, x: Float32Array, rows) -> Float32Array(rows*outDim)
 *   moeCreate(ctx, routerBytes, routerOffset, routerType, bias: Float32Array|null,
 *             gate, up, down, H, F, E, K) -> moe
 *   moeForward(ctx, moe, x: Float32Array, hidden: Float32Array, T,
 *              mask: Uint8Array|null, wantProbs) -> {idx, w, probs}
 *       hidden is updated in place; idx Int32Array(T*K), w Float64Array(T*K),
 *       probs Float32Array(T*E) or null
 *   moeSetGating(ctx, moe, gating)       0 = LFM2 sigmoid + bias, 1 = Qwen3 softmax
 *   ggufOpen(path) -> gguf               memory-mapped GGUF reader (include/qq_gguf.h)
 *   ggufTensors(gguf) -> [{name, shape, type, offset, nbytes}]
 *   ggufMoeParams(gguf, block, K, gating) -> {H, F, E, K, gating, routerType, hasBias}
 *   ggufMoeLayer(ctx, gguf, block, K, gating) -> moe (owns its expert tensors)
 *   lfm2Create(ctx, gguf) -> lfm2      whole LFM2 model on the device (include/qq_lfm2.h)
 *   lfm2Info(lfm2) -> {nLayers, nEmbd, nHeads, nHeadKV, headDim, nVocab, nFF, nExperts,
 *                      nExpertsUsed, nDenseLead, lCache, maxCtx, nAttnLayers, eps, ropeFreqBase}
 *   lfm2Forward(ctx, lfm2, token, position, logits: Float32Array|null
 *               [, mask: Uint8Array(nExperts)|null, routes: {idx, w, probs}|null])
 *       one token through the model; logits (nVocab floats) or null (skipLogits);
 *       mask: nonzero = expert skipped in every MoE block (expertMask);
 *       routes: Int32Array(nLayers*K), Float64Array(nLayers*K), Float32Array(nLayers*E)
 *       receive every MoE block's onRouterUpdate payload (dense rows untouched)
 *   lfm2Reset(ctx, lfm2)               zero the KV cache and conv states
 * Device buffers and the device-pointer calls (byte offsets range-checked
 * against the buffer, multiples of 4):
 *   bufAlloc(ctx, nbytes) -> buf       zeroed device memory
 *   bufWrite(ctx, buf, byteOffset, data: ArrayBuffer | typed array)
 *   bufRead(ctx, buf, byteOffset, out: typed array) -> out   waits for enqueued work
 *   synchronize(ctx)
 *   moeForwardDev(ctx, moe, xBuf, xOff, hiddenBuf, hiddenOff, T, mask | null,
 *                 recordBuf | null, recordOff)
 *       hidden += MoE(x), and per row the routing record [K idx | K w | E probs]
 *       as floats (qq_moe_forward_record_dev); enqueued
 *   matvecDev(ctx, tensor, mat, xBuf, xOff, yBuf, yOff, rows)      enqueued
 *   rmsnormDev(ctx, xBuf, xOff, wBuf | null, wOff, outBuf, outOff, T, H, eps)   enqueued
 *   release(handle)    frees a tensor / moe / ctx / gguf / buffer now instead of at GC
 */
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/qq_gguf.h"
#include "../../include/qq_lfm2.h"
#include "../../include/qq_moe.h"

enum { H_CTX = 1, H_TENSOR = 2, H_MOE = 3, H_GGUF = 4, H_LFM2 = 5, H_BUF = 6 };

typedef struct handle {
    int kind;
    void *ptr;           /* qq_ctx*, qq_tensor*, qq_moe*, qq_gguf*, qq_lfm2* or a device buffer (NULL once released) */
    struct handle *ctx;  /* owning context handle (tensor, moe) */
    napi_ref ctx_ref;    /* keeps the context alive while this handle lives */
    napi_ref keep[3];    /* moe: keeps gate/up/down tensors alive */
    int in_dim, out_dim, n_mats;
    int H, E, K;
    int vocab;           /* lfm2 */
    size_t size;         /* buffer: bytes */
} handle;

#define CHECK_NAPI(env, call)                                                        \
    do {                                                                             \
        if ((call) != napi_ok) {                                                     \
            napi_throw_error((env), NULL, "qq_napi: N-API call failed: " #call);     \
            return NULL;                                                             \
        }                                                                            \
    } while (0)

static napi_value throw_qq(napi_env env, const char *what, int rc, qq_ctx *ctx)
{
    char msg[640];
    snprintf(msg, sizeof msg, "%s failed (%d): %s", what, rc, qq_last_error(ctx));
    napi_throw_error(env, NULL, msg);
    return NULL;
}

static void release_handle(napi_env env, handle *h)
{
    if (!h->ptr) return;
    qq_ctx *ctx = h->ctx ? (qq_ctx *)h->ctx->ptr : NULL;
    switch (h->kind) {
    case H_TENSOR: qq_tensor_release(ctx, (qq_tensor *)h->ptr); break;
    case H_MOE: qq_moe_release(ctx, (qq_moe *)h->ptr); break;
    case H_CTX: qq_destroy((qq_ctx *)h->ptr); break;
    case H_GGUF: qq_gguf_close((qq_gguf *)h->ptr); break;
    case H_LFM2: qq_lfm2_release(ctx, (qq_lfm2 *)h->ptr); break;
    case H_BUF: qq_buffer_free(ctx, h->ptr); break;
    }
    h->ptr = NULL;
    for (int i = 0; i < 3; i++)
        if (h->keep[i]) {
            napi_delete_reference(env, h->keep[i]);
            h->keep[i] = NULL;
        }
    if (h->ctx_ref) {
        napi_delete_reference(env, h->ctx_ref);
        h->ctx_ref = NULL;
    }
}

static void finalize_handle(napi_env env, void *data, void *hint)
{
    (void)hint;
    handle *h = (handle *)data;
    release_handle(env, h);
    free(h);
}

static handle *get_handle(napi_env env, napi_value v, int kind)
{
    void *data = NULL;
    napi_valuetype t;
    if (napi_typeof(env, v, &t) != napi_ok || t != napi_external ||
        napi_get_value_external(env, v, &data) != napi_ok || !data) {
        napi_throw_type_error(env, NULL, "qq_napi: expected a handle");
        return NULL;
    }
    handle *h = (handle *)data;
    if (h->kind != kind) {
        napi_throw_type_error(env, NULL, "qq_napi: wrong handle kind");
        return NULL;
    }
    if (!h->ptr) {
        napi_throw_error(env, NULL, "qq_napi: handle already released");
        return NULL;
    }
    return h;
}

static napi_value new_handle(napi_env env, handle *h)
{
    napi_value v;
    if (napi_create_external(env, h, finalize_handle, NULL, &v) != napi_ok) {
        free(h);
        napi_throw_error(env, NULL, "qq_napi: cannot create handle");
        return NULL;
    }
    return v;
}

/* Raw bytes of an ArrayBuffer or of any typed array (its viewed range). */
static int get_bytes(napi_env env, napi_value v, uint8_t **data, size_t *len)
{
    bool is_ab = false, is_ta = false;
    napi_is_arraybuffer(env, v, &is_ab);
    if (is_ab) {
        void *p;
        if (napi_get_arraybuffer_info(env, v, &p, len) != napi_ok) return -1;
        *data = (uint8_t *)p;
        return 0;
    }
    napi_is_typedarray(env, v, &is_ta);
    if (is_ta) {
        napi_typedarray_type tt;
        size_t n, off;
        void *p;
        napi_value ab;
        if (napi_get_typedarray_info(env, v, &tt, &n, &p, &ab, &off) != napi_ok) return -1;
        size_t es = 1;
        switch (tt) {
        case napi_int16_array: case napi_uint16_array: es = 2; break;
        case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
        case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
        default: es = 1;
        }
        *data = (uint8_t *)p;
        *len = n * es;
        return 0;
    }
    return -1;
}

static int get_typed(napi_env env, napi_value v, napi_typedarray_type want, void **data, size_t *n)
{
    bool is_ta = false;
    napi_is_typedarray(env, v, &is_ta);
    if (!is_ta) return -1;
    napi_typedarray_type tt;
    size_t off;
    napi_value ab;
    if (napi_get_typedarray_info(env, v, &tt, n, data, &ab, &off) != napi_ok) return -1;
    return tt == want ? 0 : -1;
}

static int is_nullish(napi_env env, napi_value v)
{
    napi_valuetype t;
    napi_typeof(env, v, &t);
    return t == napi_null || t == napi_undefined;
}

static int get_i32(napi_env env, napi_value v, int32_t *out)
{
    return napi_get_value_int32(env, v, out) == napi_ok ? 0 : -1;
}

#define ARGS(N)                                                               \
    size_t argc = N;                                                          \
    napi_value argv[N];                                                       \
    CHECK_NAPI(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));    \
    if (argc < N) {                                                           \
        napi_throw_type_error(env, NULL, "qq_napi: expected " #N " arguments"); \
        return NULL;                                                          \
    }

static napi_value js_init(napi_env env, napi_callback_info info)
{
    ARGS(1);
    int32_t dev;
    if (get_i32(env, argv[0], &dev)) {
        napi_throw_type_error(env, NULL, "init(device): device must be an integer");
        return NULL;
    }
    qq_ctx *ctx = NULL;
    int rc = qq_init(dev, &ctx);
    if (rc) return throw_qq(env, "qq_init", rc, NULL);
    handle *h = (handle *)calloc(1, sizeof(handle));
    if (!h) {
        qq_destroy(ctx);
        napi_throw_error(env, NULL, "qq_napi: out of memory");
        return NULL;
    }
    h->kind = H_CTX;
    h->ptr = ctx;
    return new_handle(env, h);
}

static napi_value js_last_error(napi_env env, napi_callback_info info)
{
    size_t argc = 1;
    napi_value argv[1], out;
    CHECK_NAPI(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
    qq_ctx *ctx = NULL;
    if (argc >= 1 && !is_nullish(env, argv[0])) {
        handle *h = get_handle(env, argv[0], H_CTX);
        if (!h) return NULL;
        ctx = (qq_ctx *)h->ptr;
    }
    CHECK_NAPI(env, napi_create_string_utf8(env, qq_last_error(ctx), NAPI_AUTO_LENGTH, &out));
    return out;
}

/* child handle that keeps its context's JS handle alive */
static handle *child_of(napi_env env, napi_value ctxv, handle *ch, int kind)
{
    handle *h = (handle *)calloc(1, sizeof(handle));
    if (!h) return NULL;
    h->kind = kind;
    h->ctx = ch;
    if (napi_create_reference(env, ctxv, 1, &h->ctx_ref) != napi_ok) {
        free(h);
        return NULL;
    }
    return h;
}

static napi_value js_upload_q80(napi_env env, napi_callback_info info)
{
    ARGS(6);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    uint8_t *bytes;
    size_t len;
    int32_t off, in_dim, out_dim, n_mats;
    if (get_bytes(env, argv[1], &bytes, &len) || get_i32(env, argv[2], &off) ||
        get_i32(env, argv[3], &in_dim) || get_i32(env, argv[4], &out_dim) || get_i32(env, argv[5], &n_mats) ||
        off < 0 || (size_t)off > len) {
        napi_throw_type_error(env, NULL, "uploadQ80(ctx, bytes, byteOffset, inDim, outDim, nMats)");
        return NULL;
    }
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    qq_tensor *t = NULL;
    int rc = qq_q8_0_upload(ctx, bytes + off, len - off, in_dim, out_dim, n_mats, &t);
    if (rc) return throw_qq(env, "qq_q8_0_upload", rc, ctx);
    handle *h = child_of(env, argv[0], ch, H_TENSOR);
    if (!h) {
        qq_tensor_release(ctx, t);
        napi_throw_error(env, NULL, "qq_napi: out of memory");
        return NULL;
    }
    h->ptr = t;
    h->in_dim = in_dim;
    h->out_dim = out_dim;
    h->n_mats = n_mats;
    return new_handle(env, h);
}

static napi_value js_matvec(napi_env env, napi_callback_info info)
{
    ARGS(5);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    handle *th = get_handle(env, argv[1], H_TENSOR);
    if (!th) return NULL;
    int32_t mat, rows;
    float *x;
    size_t nx;
    if (get_i32(env, argv[2], &mat) || get_typed(env, argv[3], napi_float32_array, (void **)&x, &nx) ||
        get_i32(env, argv[4], &rows) || rows < 0) {
        napi_throw_type_error(env, NULL, "matvec(ctx, tensor, mat, x: Float32Array, rows)");
        return NULL;
    }
    if (nx < (size_t)rows * th->in_dim) {
        napi_throw_range_error(env, NULL, "matvec: input shorter than rows * inDim");
        return NULL;
    }
    napi_value ab, out;
    void *ydata;
    const size_t ny = (size_t)rows * th->out_dim;
    CHECK_NAPI(env, napi_create_arraybuffer(env, ny * 4, &ydata, &ab));
    CHECK_NAPI(env, napi_create_typedarray(env, napi_float32_array, ny, ab, 0, &out));
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_q8_0_matvec(ctx, (qq_tensor *)th->ptr, mat, x, (float *)ydata, rows);
    if (rc) return throw_qq(env, "qq_q8_0_matvec", rc, ctx);
    return out;
}

static napi_value js_moe_create(napi_env env, napi_callback_info info)
{
    ARGS(12);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    uint8_t *rbytes;
    size_t rlen;
    int32_t roff, rtype, H, F, E, K;
    if (get_bytes(env, argv[1], &rbytes, &rlen) || get_i32(env, argv[2], &roff) ||
        get_i32(env, argv[3], &rtype) || get_i32(env, argv[8], &H) || get_i32(env, argv[9], &F) ||
        get_i32(env, argv[10], &E) || get_i32(env, argv[11], &K) || roff < 0 || (size_t)roff > rlen) {
        napi_throw_type_error(env, NULL,
                              "moeCreate(ctx, routerBytes, routerOffset, routerType, bias, gate, up, down, H, F, E, K)");
        return NULL;
    }
    const size_t need = rtype == QQ_TYPE_F32 ? (size_t)E * H * 4 : (size_t)E * ((H + 31) / 32) * 34;
    if (rlen - roff < need) {
        napi_throw_range_error(env, NULL, "moeCreate: router tensor is shorter than [H, E]");
        return NULL;
    }
    float *bias = NULL;
    if (!is_nullish(env, argv[4])) {
        size_t nb;
        if (get_typed(env, argv[4], napi_float32_array, (void **)&bias, &nb) || nb < (size_t)E) {
            napi_throw_type_error(env, NULL, "moeCreate: bias must be a Float32Array of E values or null");
            return NULL;
        }
    }
    handle *g = get_handle(env, argv[5], H_TENSOR);
    if (!g) return NULL;
    handle *u = get_handle(env, argv[6], H_TENSOR);
    if (!u) return NULL;
    handle *d = get_handle(env, argv[7], H_TENSOR);
    if (!d) return NULL;
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    qq_moe *m = NULL;
    int rc = qq_moe_create(ctx, rbytes + roff, rtype, bias, (qq_tensor *)g->ptr, (qq_tensor *)u->ptr,
                           (qq_tensor *)d->ptr, H, F, E, K, &m);
    if (rc) return throw_qq(env, "qq_moe_create", rc, ctx);
    handle *h = child_of(env, argv[0], ch, H_MOE);
    if (!h) {
        qq_moe_release(ctx, m);
        napi_throw_error(env, NULL, "qq_napi: out of memory");
        return NULL;
    }
    h->ptr = m;
    h->H = H;
    h->E = E;
    h->K = K;
    for (int i = 0; i < 3; i++) napi_create_reference(env, argv[5 + i], 1, &h->keep[i]);
    return new_handle(env, h);
}

// qq_moe_set_gating: 0 = LFM2 sigmoid + bias (default), 1 = Qwen3 softmax.
static napi_value js_moe_set_gating(napi_env env, napi_callback_info info)
{
    ARGS(3);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    handle *mh = get_handle(env, argv[1], H_MOE);
    if (!mh) return NULL;
    int32_t gating;
    if (get_i32(env, argv[2], &gating)) {
        napi_throw_type_error(env, NULL, "moeSetGating(ctx, moe, gating)");
        return NULL;
    }
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_moe_set_gating(ctx, (qq_moe *)mh->ptr, gating);
    if (rc) return throw_qq(env, "qq_moe_set_gating", rc, ctx);
    return NULL;
}

static napi_value js_moe_forward(napi_env env, napi_callback_info info)
{
    ARGS(7);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    handle *mh = get_handle(env, argv[1], H_MOE);
    if (!mh) return NULL;
    float *x, *hid;
    size_t nx, nh;
    int32_t T;
    bool want_probs = false;
    if (get_typed(env, argv[2], napi_float32_array, (void **)&x, &nx) ||
        get_typed(env, argv[3], napi_float32_array, (void **)&hid, &nh) || get_i32(env, argv[4], &T) || T < 0 ||
        napi_get_value_bool(env, argv[6], &want_probs) != napi_ok) {
        napi_throw_type_error(env, NULL,
                              "moeForward(ctx, moe, x: Float32Array, hidden: Float32Array, T, mask, wantProbs)");
        return NULL;
    }
    if (nx < (size_t)T * mh->H || nh < (size_t)T * mh->H) {
        napi_throw_range_error(env, NULL, "moeForward: x / hidden shorter than T * H");
        return NULL;
    }
    uint8_t *mask = NULL;
    if (!is_nullish(env, argv[5])) {
        size_t nm;
        if (get_typed(env, argv[5], napi_uint8_array, (void **)&mask, &nm) || nm < (size_t)mh->E) {
            napi_throw_type_error(env, NULL, "moeForward: mask must be a Uint8Array of E entries or null");
            return NULL;
        }
    }
    napi_value res, v_idx, v_w, v_p, ab;
    void *didx, *dw, *dp = NULL;
    CHECK_NAPI(env, napi_create_arraybuffer(env, (size_t)T * mh->K * 4, &didx, &ab));
    CHECK_NAPI(env, napi_create_typedarray(env, napi_int32_array, (size_t)T * mh->K, ab, 0, &v_idx));
    CHECK_NAPI(env, napi_create_arraybuffer(env, (size_t)T * mh->K * 8, &dw, &ab));
    CHECK_NAPI(env, napi_create_typedarray(env, napi_float64_array, (size_t)T * mh->K, ab, 0, &v_w));
    if (want_probs) {
        CHECK_NAPI(env, napi_create_arraybuffer(env, (size_t)T * mh->E * 4, &dp, &ab));
        CHECK_NAPI(env, napi_create_typedarray(env, napi_float32_array, (size_t)T * mh->E, ab, 0, &v_p));
    } else {
        CHECK_NAPI(env, napi_get_null(env, &v_p));
    }
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_moe_forward(ctx, (qq_moe *)mh->ptr, x, hid, T, mask, (int32_t *)didx, (double *)dw, (float *)dp);
    if (rc) return throw_qq(env, "qq_moe_forward", rc, ctx);
    CHECK_NAPI(env, napi_create_object(env, &res));
    CHECK_NAPI(env, napi_set_named_property(env, res, "idx", v_idx));
    CHECK_NAPI(env, napi_set_named_property(env, res, "w", v_w));
    CHECK_NAPI(env, napi_set_named_property(env, res, "probs", v_p));
    return res;
}

static napi_value throw_gguf(napi_env env, const char *what, int rc)
{
    char msg[640];
    snprintf(msg, sizeof msg, "%s failed (%d): %s", what, rc, qq_gguf_last_error());
    napi_throw_error(env, NULL, msg);
    return NULL;
}

static napi_value js_gguf_open(napi_env env, napi_callback_info info)
{
    ARGS(1);
    char path[4096];
    size_t n = 0;
    if (napi_get_value_string_utf8(env, argv[0], path, sizeof path, &n) != napi_ok || n + 1 >= sizeof path) {
        napi_throw_type_error(env, NULL, "ggufOpen(path: string)");
        return NULL;
    }
    qq_gguf *g = NULL;
    int rc = qq_gguf_open(path, &g);
    if (rc) return throw_gguf(env, "qq_gguf_open", rc);
    handle *h = (handle *)calloc(1, sizeof(handle));
    if (!h) {
        qq_gguf_close(g);
        napi_throw_error(env, NULL, "qq_napi: out of memory");
        return NULL;
    }
    h->kind = H_GGUF;
    h->ptr = g;
    return new_handle(env, h);
}

static napi_value set_num(napi_env env, napi_value obj, const char *key, double v)
{
    napi_value x;
    if (napi_create_double(env, v, &x) != napi_ok || napi_set_named_property(env, obj, key, x) != napi_ok)
        return NULL;
    return obj;
}

static napi_value js_gguf_tensors(napi_env env, napi_callback_info info)
{
    ARGS(1);
    handle *gh = get_handle(env, argv[0], H_GGUF);
    if (!gh) return NULL;
    const qq_gguf *g = (const qq_gguf *)gh->ptr;
    qq_gguf_header_info hd;
    int rc = qq_gguf_header(g, &hd);
    if (rc) return throw_gguf(env, "qq_gguf_header", rc);
    napi_value arr;
    CHECK_NAPI(env, napi_create_array_with_length(env, (size_t)hd.tensor_count, &arr));
    for (uint64_t i = 0; i < hd.tensor_count; i++) {
        qq_gguf_tensor t;
        rc = qq_gguf_tensor_info(g, i, &t);
        if (rc) return throw_gguf(env, "qq_gguf_tensor_info", rc);
        napi_value o, name, shape;
        CHECK_NAPI(env, napi_create_object(env, &o));
        CHECK_NAPI(env, napi_create_string_utf8(env, t.name, NAPI_AUTO_LENGTH, &name));
        CHECK_NAPI(env, napi_set_named_property(env, o, "name", name));
        CHECK_NAPI(env, napi_create_array_with_length(env, (size_t)t.n_dims, &shape));
        for (int d = 0; d < t.n_dims && d < 4; d++) {
            napi_value x;
            CHECK_NAPI(env, napi_create_double(env, (double)t.shape[d], &x));
            CHECK_NAPI(env, napi_set_element(env, shape, (uint32_t)d, x));
        }
        CHECK_NAPI(env, napi_set_named_property(env, o, "shape", shape));
        if (!set_num(env, o, "type", t.type) || !set_num(env, o, "offset", (double)t.offset) ||
            !set_num(env, o, "nbytes", (double)t.nbytes)) {
            napi_throw_error(env, NULL, "qq_napi: N-API call failed");
            return NULL;
        }
        CHECK_NAPI(env, napi_set_element(env, arr, (uint32_t)i, o));
    }
    return arr;
}

static napi_value js_gguf_moe_params(napi_env env, napi_callback_info info)
{
    ARGS(4);
    handle *gh = get_handle(env, argv[0], H_GGUF);
    if (!gh) return NULL;
    int32_t block, K, gating;
    if (get_i32(env, argv[1], &block) || get_i32(env, argv[2], &K) || get_i32(env, argv[3], &gating)) {
        napi_throw_type_error(env, NULL, "ggufMoeParams(gguf, block, K, gating)");
        return NULL;
    }
    qq_gguf_moe_info p;
    int rc = qq_gguf_moe_params((const qq_gguf *)gh->ptr, block, K, gating, &p);
    if (rc) return throw_gguf(env, "qq_gguf_moe_params", rc);
    napi_value o;
    CHECK_NAPI(env, napi_create_object(env, &o));
    if (!set_num(env, o, "H", p.H) || !set_num(env, o, "F", p.F) || !set_num(env, o, "E", p.E) ||
        !set_num(env, o, "K", p.K) || !set_num(env, o, "gating", p.gating) ||
        !set_num(env, o, "routerType", p.router_type) || !set_num(env, o, "hasBias", p.has_bias)) {
        napi_throw_error(env, NULL, "qq_napi: N-API call failed");
        return NULL;
    }
    return o;
}

static napi_value js_gguf_moe_layer(napi_env env, napi_callback_info info)
{
    ARGS(5);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    handle *gh = get_handle(env, argv[1], H_GGUF);
    if (!gh) return NULL;
    int32_t block, K, gating;
    if (get_i32(env, argv[2], &block) || get_i32(env, argv[3], &K) || get_i32(env, argv[4], &gating)) {
        napi_throw_type_error(env, NULL, "ggufMoeLayer(ctx, gguf, block, K, gating)");
        return NULL;
    }
    qq_gguf_moe_info p;
    int rc = qq_gguf_moe_params((const qq_gguf *)gh->ptr, block, K, gating, &p);
    if (rc) return throw_gguf(env, "qq_gguf_moe_params", rc);
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    qq_moe *m = NULL;
    rc = qq_gguf_moe_layer(ctx, (const qq_gguf *)gh->ptr, block, K, gating, &m);
    if (rc) return throw_qq(env, "qq_gguf_moe_layer", rc, ctx);
    handle *h = child_of(env, argv[0], ch, H_MOE);
    if (!h) {
        qq_moe_release(ctx, m);
        napi_throw_error(env, NULL, "qq_napi: out of memory");
        return NULL;
    }
    h->ptr = m;
    h->H = p.H;
    h->E = p.E;
    h->K = p.K;
    return new_handle(env, h);
}

static napi_value js_lfm2_create(napi_env env, napi_callback_info info)
{
    ARGS(2);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    handle *gh = get_handle(env, argv[1], H_GGUF);
    if (!gh) return NULL;
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    qq_lfm2 *m = NULL;
    int rc = qq_lfm2_create(ctx, (const qq_gguf *)gh->ptr, &m);
    if (rc) return throw_qq(env, "qq_lfm2_create", rc, ctx);
    handle *h = child_of(env, argv[0], ch, H_LFM2);
    if (!h) {
        qq_lfm2_release(ctx, m);
        napi_throw_error(env, NULL, "qq_napi: out of memory");
        return NULL;
    }
    qq_lfm2_info I;
    qq_lfm2_get_info(m, &I);
    h->ptr = m;
    h->vocab = I.n_vocab;
    return new_handle(env, h);
}

static napi_value js_lfm2_info(napi_env env, napi_callback_info info)
{
    ARGS(1);
    handle *mh = get_handle(env, argv[0], H_LFM2);
    if (!mh) return NULL;
    qq_lfm2_info I;
    qq_lfm2_get_info((const qq_lfm2 *)mh->ptr, &I);
    napi_value o;
    CHECK_NAPI(env, napi_create_object(env, &o));
    const struct {
        const char *k;
        double v;
    } f[] = {{"nLayers", I.n_layers},         {"nEmbd", I.n_embd},         {"nHeads", I.n_heads},
             {"nHeadKV", I.n_head_kv},        {"headDim", I.head_dim},     {"nVocab", I.n_vocab},
             {"nFF", I.n_ff},                 {"nExperts", I.n_experts},   {"nExpertsUsed", I.n_experts_used},
             {"nDenseLead", I.n_dense_lead},  {"lCache", I.l_cache},       {"maxCtx", I.max_ctx},
             {"nAttnLayers", I.n_attn_layers}, {"eps", I.eps},             {"ropeFreqBase", I.rope_freq_base}};
    for (size_t i = 0; i < sizeof f / sizeof f[0]; i++)
        if (!set_num(env, o, f[i].k, f[i].v)) return NULL;
    return o;
}

static napi_value js_lfm2_forward(napi_env env, napi_callback_info info)
{
    // five arguments, and two optional ones (missing ones read as undefined)
    size_t argc = 7;
    napi_value argv[7];
    CHECK_NAPI(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
    if (argc < 5) {
        napi_throw_type_error(env, NULL, "qq_napi: lfm2Forward expects at least 5 arguments");
        return NULL;
    }
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    handle *mh = get_handle(env, argv[1], H_LFM2);
    if (!mh) return NULL;
    int32_t token, pos;
    if (get_i32(env, argv[2], &token) || get_i32(env, argv[3], &pos)) {
        napi_throw_type_error(env, NULL, "lfm2Forward(ctx, lfm2, token, position, logits | null[, mask, routes])");
        return NULL;
    }
    float *logits = NULL;
    if (!is_nullish(env, argv[4])) {
        size_t n;
        if (get_typed(env, argv[4], napi_float32_array, (void **)&logits, &n) || n < (size_t)mh->vocab) {
            napi_throw_type_error(env, NULL, "lfm2Forward: logits must be a Float32Array of nVocab floats or null");
            return NULL;
        }
    }
    qq_lfm2_info I;
    if (qq_lfm2_get_info((qq_lfm2 *)mh->ptr, &I)) {
        napi_throw_error(env, NULL, "lfm2Forward: model info");
        return NULL;
    }
    uint8_t *mask = NULL;
    if (argc > 5 && !is_nullish(env, argv[5])) {
        size_t n;
        if (get_typed(env, argv[5], napi_uint8_array, (void **)&mask, &n) || n < (size_t)I.n_experts) {
            napi_throw_type_error(env, NULL, "lfm2Forward: mask must be a Uint8Array of nExperts bytes or null");
            return NULL;
        }
    }
    int32_t *idx = NULL;
    double *w = NULL;
    float *probs = NULL;
    if (argc > 6 && !is_nullish(env, argv[6])) {
        napi_value vi, vw, vp;
        size_t ni = 0, nw = 0, np = 0;
        const size_t nk = (size_t)I.n_layers * I.n_experts_used, ne = (size_t)I.n_layers * I.n_experts;
        if (napi_get_named_property(env, argv[6], "idx", &vi) != napi_ok ||
            napi_get_named_property(env, argv[6], "w", &vw) != napi_ok ||
            napi_get_named_property(env, argv[6], "probs", &vp) != napi_ok ||
            get_typed(env, vi, napi_int32_array, (void **)&idx, &ni) || ni < nk ||
            get_typed(env, vw, napi_float64_array, (void **)&w, &nw) || nw < nk ||
            get_typed(env, vp, napi_float32_array, (void **)&probs, &np) || np < ne) {
            napi_throw_type_error(env, NULL,
                                  "lfm2Forward: routes must be {idx: Int32Array(nLayers*K), w: Float64Array(nLayers*K), "
                                  "probs: Float32Array(nLayers*nExperts)}");
            return NULL;
        }
    }
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_lfm2_forward_routed(ctx, (qq_lfm2 *)mh->ptr, token, pos, logits, mask, idx, w, probs);
    if (rc) return throw_qq(env, "qq_lfm2_forward", rc, ctx);
    return NULL;
}

static napi_value js_lfm2_reset(napi_env env, napi_callback_info info)
{
    ARGS(2);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    handle *mh = get_handle(env, argv[1], H_LFM2);
    if (!mh) return NULL;
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_lfm2_reset(ctx, (qq_lfm2 *)mh->ptr);
    if (!rc) rc = qq_synchronize(ctx);
    if (rc) return throw_qq(env, "qq_lfm2_reset", rc, ctx);
    return NULL;
}

/* ---- device buffers ---- */

static int get_i64(napi_env env, napi_value v, int64_t *out)
{
    return napi_get_value_int64(env, v, out) == napi_ok ? 0 : -1;
}

/* Device address of bytes [off, off + need) of buffer `v`, range-checked;
 * off must be a multiple of 4 (the buffers hold floats).  NULL with a thrown
 * error when out of range. */
static void *buf_span(napi_env env, napi_value v, napi_value offv, size_t need, const char *what)
{
    handle *h = get_handle(env, v, H_BUF);
    if (!h) return NULL;
    int64_t off;
    if (get_i64(env, offv, &off) || off < 0 || (off & 3) || (uint64_t)off > h->size || need > h->size - (size_t)off) {
        char msg[200];
        snprintf(msg, sizeof msg, "%s: byte range [%lld, +%zu) outside the %zu-byte buffer or unaligned", what,
                 (long long)off, need, h->size);
        napi_throw_range_error(env, NULL, msg);
        return NULL;
    }
    return (char *)h->ptr + off;
}

static napi_value js_buf_alloc(napi_env env, napi_callback_info info)
{
    ARGS(2);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    int64_t n;
    if (get_i64(env, argv[1], &n) || n < 0) {
        napi_throw_type_error(env, NULL, "bufAlloc(ctx, nbytes)");
        return NULL;
    }
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    void *p = NULL;
    int rc = qq_buffer_alloc(ctx, (size_t)n, &p);
    if (rc) return throw_qq(env, "qq_buffer_alloc", rc, ctx);
    handle *h = child_of(env, argv[0], ch, H_BUF);
    if (!h) {
        qq_buffer_free(ctx, p);
        napi_throw_error(env, NULL, "qq_napi: out of memory");
        return NULL;
    }
    h->ptr = p;
    h->size = (size_t)n;
    return new_handle(env, h);
}

/* bufWrite(ctx, buf, byteOffset, data: ArrayBuffer | typed array) */
static napi_value js_buf_write(napi_env env, napi_callback_info info)
{
    ARGS(4);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    uint8_t *data;
    size_t len;
    if (get_bytes(env, argv[3], &data, &len)) {
        napi_throw_type_error(env, NULL, "bufWrite(ctx, buf, byteOffset, data)");
        return NULL;
    }
    void *dst = buf_span(env, argv[1], argv[2], len, "bufWrite");
    if (!dst) return NULL;
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_buffer_write(ctx, dst, data, len);
    if (rc) return throw_qq(env, "qq_buffer_write", rc, ctx);
    return NULL;
}

/* bufRead(ctx, buf, byteOffset, out: typed array) -> out (its whole view is filled) */
static napi_value js_buf_read(napi_env env, napi_callback_info info)
{
    ARGS(4);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    uint8_t *data;
    size_t len;
    bool is_ta = false;
    napi_is_typedarray(env, argv[3], &is_ta);
    if (!is_ta || get_bytes(env, argv[3], &data, &len)) {
        napi_throw_type_error(env, NULL, "bufRead(ctx, buf, byteOffset, out: typed array)");
        return NULL;
    }
    const void *src = buf_span(env, argv[1], argv[2], len, "bufRead");
    if (!src) return NULL;
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_buffer_read(ctx, src, data, len);
    if (rc) return throw_qq(env, "qq_buffer_read", rc, ctx);
    return argv[3];
}

static napi_value js_synchronize(napi_env env, napi_callback_info info)
{
    ARGS(1);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_synchronize(ctx);
    if (rc) return throw_qq(env, "qq_synchronize", rc, ctx);
    return NULL;
}

/* setWaitLimit(ctx, microseconds): qq_set_wait_limit */
static napi_value js_set_wait_limit(napi_env env, napi_callback_info info)
{
    ARGS(2);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int32_t us;
    CHECK_NAPI(env, napi_get_value_int32(env, argv[1], &us));
    int rc = qq_set_wait_limit(ctx, us);
    if (rc) return throw_qq(env, "qq_set_wait_limit", rc, ctx);
    return NULL;
}

/* moeForwardDev(ctx, moe, xBuf, xOff, hiddenBuf, hiddenOff, T, mask | null,
 *               recordBuf | null, recordOff): qq_moe_forward_record_dev, enqueued */
static napi_value js_moe_forward_dev(napi_env env, napi_callback_info info)
{
    ARGS(10);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    handle *mh = get_handle(env, argv[1], H_MOE);
    if (!mh) return NULL;
    int32_t T;
    if (get_i32(env, argv[6], &T) || T < 0) {
        napi_throw_type_error(env, NULL,
                              "moeForwardDev(ctx, moe, xBuf, xOff, hiddenBuf, hiddenOff, T, mask, recordBuf, recordOff)");
        return NULL;
    }
    const size_t rowb = (size_t)T * mh->H * 4;
    const float *x = (const float *)buf_span(env, argv[2], argv[3], rowb, "moeForwardDev x");
    if (!x) return NULL;
    float *hid = (float *)buf_span(env, argv[4], argv[5], rowb, "moeForwardDev hidden");
    if (!hid) return NULL;
    uint8_t *mask = NULL;
    if (!is_nullish(env, argv[7])) {
        size_t n;
        if (get_typed(env, argv[7], napi_uint8_array, (void **)&mask, &n) || n < (size_t)mh->E) {
            napi_throw_type_error(env, NULL, "moeForwardDev: mask must be a Uint8Array of E bytes or null");
            return NULL;
        }
    }
    float *rec = NULL;
    if (!is_nullish(env, argv[8])) {
        rec = (float *)buf_span(env, argv[8], argv[9], (size_t)T * (2 * mh->K + mh->E) * 4, "moeForwardDev record");
        if (!rec) return NULL;
    }
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_moe_forward_record_dev(ctx, (qq_moe *)mh->ptr, x, hid, T, mask, rec);
    if (rc) return throw_qq(env, "qq_moe_forward_record_dev", rc, ctx);
    return NULL;
}

/* matvecDev(ctx, tensor, mat, xBuf, xOff, yBuf, yOff, rows): qq_q8_0_matvec_dev, enqueued */
static napi_value js_matvec_dev(napi_env env, napi_callback_info info)
{
    ARGS(8);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    handle *th = get_handle(env, argv[1], H_TENSOR);
    if (!th) return NULL;
    int32_t mat, rows;
    if (get_i32(env, argv[2], &mat) || get_i32(env, argv[7], &rows) || rows < 0) {
        napi_throw_type_error(env, NULL, "matvecDev(ctx, tensor, mat, xBuf, xOff, yBuf, yOff, rows)");
        return NULL;
    }
    const float *x = (const float *)buf_span(env, argv[3], argv[4], (size_t)rows * th->in_dim * 4, "matvecDev x");
    if (!x) return NULL;
    float *y = (float *)buf_span(env, argv[5], argv[6], (size_t)rows * th->out_dim * 4, "matvecDev y");
    if (!y) return NULL;
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_q8_0_matvec_dev(ctx, (qq_tensor *)th->ptr, mat, x, y, rows);
    if (rc) return throw_qq(env, "qq_q8_0_matvec_dev", rc, ctx);
    return NULL;
}

/* rmsnormDev(ctx, xBuf, xOff, wBuf | null, wOff, outBuf, outOff, T, H, eps): qq_rmsnorm_dev, enqueued */
static napi_value js_rmsnorm_dev(napi_env env, napi_callback_info info)
{
    ARGS(10);
    handle *ch = get_handle(env, argv[0], H_CTX);
    if (!ch) return NULL;
    int32_t T, H;
    double eps;
    if (get_i32(env, argv[7], &T) || get_i32(env, argv[8], &H) || T < 0 || H < 0 ||
        napi_get_value_double(env, argv[9], &eps) != napi_ok) {
        napi_throw_type_error(env, NULL, "rmsnormDev(ctx, xBuf, xOff, wBuf, wOff, outBuf, outOff, T, H, eps)");
        return NULL;
    }
    const size_t rowb = (size_t)T * H * 4;
    const float *x = (const float *)buf_span(env, argv[1], argv[2], rowb, "rmsnormDev x");
    if (!x) return NULL;
    const float *w = NULL;
    if (!is_nullish(env, argv[3])) {
        w = (const float *)buf_span(env, argv[3], argv[4], (size_t)H * 4, "rmsnormDev weight");
        if (!w) return NULL;
    }
    float *out = (float *)buf_span(env, argv[5], argv[6], rowb, "rmsnormDev out");
    if (!out) return NULL;
    qq_ctx *ctx = (qq_ctx *)ch->ptr;
    int rc = qq_rmsnorm_dev(ctx, x, w, out, T, H, eps);
    if (rc) return throw_qq(env, "qq_rmsnorm_dev", rc, ctx);
    return NULL;
}

static napi_value js_release(napi_env env, napi_callback_info info)
{
    ARGS(1);
    void *data = NULL;
    napi_valuetype t;
    if (napi_typeof(env, argv[0], &t) != napi_ok || t != napi_external ||
        napi_get_value_external(env, argv[0], &data) != napi_ok || !data) {
        napi_throw_type_error(env, NULL, "release(handle)");
        return NULL;
    }
    release_handle(env, (handle *)data);
    return NULL;
}

static napi_value module_init(napi_env env, napi_value exports)
{
    const napi_property_descriptor props[] = {
        {"init", NULL, js_init, NULL, NULL, NULL, napi_enumerable, NULL},
        {"lastError", NULL, js_last_error, NULL, NULL, NULL, napi_enumerable, NULL},
        {"uploadQ80", NULL, js_upload_q80, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvec", NULL, js_matvec, NULL, NULL, NULL, napi_enumerable, NULL},
        {"moeCreate", NULL, js_moe_create, NULL, NULL, NULL, napi_enumerable, NULL},
        {"moeSetGating", NULL, js_moe_set_gating, NULL, NULL, NULL, napi_enumerable, NULL},
        {"moeForward", NULL, js_moe_forward, NULL, NULL, NULL, napi_enumerable, NULL},
        {"ggufOpen", NULL, js_gguf_open, NULL, NULL, NULL, napi_enumerable, NULL},
        {"ggufTensors", NULL, js_gguf_tensors, NULL, NULL, NULL, napi_enumerable, NULL},
        {"ggufMoeParams", NULL, js_gguf_moe_params, NULL, NULL, NULL, napi_enumerable, NULL},
        {"ggufMoeLayer", NULL, js_gguf_moe_layer, NULL, NULL, NULL, napi_enumerable, NULL},
        {"lfm2Create", NULL, js_lfm2_create, NULL, NULL, NULL, napi_enumerable, NULL},
        {"lfm2Info", NULL, js_lfm2_info, NULL, NULL, NULL, napi_enumerable, NULL},
        {"lfm2Forward", NULL, js_lfm2_forward, NULL, NULL, NULL, napi_enumerable, NULL},
        {"lfm2Reset", NULL, js_lfm2_reset, NULL, NULL, NULL, napi_enumerable, NULL},
        {"bufAlloc", NULL, js_buf_alloc, NULL, NULL, NULL, napi_enumerable, NULL},
        {"bufWrite", NULL, js_buf_write, NULL, NULL, NULL, napi_enumerable, NULL},
        {"bufRead", NULL, js_buf_read, NULL, NULL, NULL, napi_enumerable, NULL},
        {"synchronize", NULL, js_synchronize, NULL, NULL, NULL, napi_enumerable, NULL},
        {"setWaitLimit", NULL, js_set_wait_limit, NULL, NULL, NULL, napi_enumerable, NULL},
        {"moeForwardDev", NULL, js_moe_forward_dev, NULL, NULL, NULL, napi_enumerable, NULL},
        {"matvecDev", NULL, js_matvec_dev, NULL, NULL, NULL, napi_enumerable, NULL},
        {"rmsnormDev", NULL, js_rmsnorm_dev, NULL, NULL, NULL, napi_enumerable, NULL},
        {"release", NULL, js_release, NULL, NULL, NULL, napi_enumerable, NULL},
    };
    if (napi_define_properties(env, exports, sizeof props / sizeof props[0], props) != napi_ok) return NULL;
    return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, module_init)
