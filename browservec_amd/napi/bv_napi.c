/*
 * N-API binding of libbrowservec_hip.so for Node (the reference's host
 * runtime).  It exposes the C ABI of include/browservec_hip.h one call per
 * function; index.js builds the reference's VectorIndex seam
 * (src/index/flat.ts:24-40) on top of it.  Failed calls throw an Error whose
 * message is bv_last_error(), as the reference throws `new Error(msg)`.
 * Calls are synchronous: the device work of one call is a few hundred
 * microseconds, below the cost of a thread-pool hop.
 */
#define NAPI_VERSION 3
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/browservec_hip.h"

#define CALL(env, expr)                                                  \
    do {                                                                 \
        if ((expr) != napi_ok) {                                         \
            napi_throw_error((env), NULL, "N-API call failed: " #expr); \
            return NULL;                                                 \
        }                                                                \
    } while (0)

static napi_value throw_bv(napi_env env, int rc) {
    static const char *names[] = {"BV_OK",          "BV_E_INVALID", "BV_E_UNSUPPORTED", "BV_E_DEVICE_LOST",
                                  "BV_E_OOM",       "BV_E_HIP",     "BV_E_STATE"};
    const char *msg = bv_last_error();
    char code[24];
    if (rc > 0 && rc < (int)(sizeof names / sizeof names[0])) snprintf(code, sizeof code, "%s", names[rc]);
    else snprintf(code, sizeof code, "BV_E_%d", rc);
    napi_throw_error(env, code, msg && *msg ? msg : "browservec_hip call failed");
    return NULL;
}

static void *get_ptr(napi_env env, napi_value v) {
    void *p = NULL;
    napi_valuetype t;
    if (napi_typeof(env, v, &t) != napi_ok || t != napi_external) return NULL;
    napi_get_value_external(env, v, &p);
    return p;
}

static int get_u32(napi_env env, napi_value v, uint32_t *out) {
    return napi_get_value_uint32(env, v, out) == napi_ok;
}

/* A typed array argument of the expected element type; returns its data and length. */
static void *get_typed(napi_env env, napi_value v, napi_typedarray_type want, size_t *len) {
    bool is;
    if (napi_is_typedarray(env, v, &is) != napi_ok || !is) return NULL;
    napi_typedarray_type t;
    void *data;
    napi_value ab;
    size_t off;
    if (napi_get_typedarray_info(env, v, &t, len, &data, &ab, &off) != napi_ok || t != want) return NULL;
    return data;
}

static napi_value new_typed(napi_env env, napi_typedarray_type t, size_t n, size_t elem, void **data) {
    napi_value ab, arr;
    const size_t bytes = n * elem;
    if (napi_create_arraybuffer(env, bytes > 0 ? bytes : 1, data, &ab) != napi_ok) return NULL;
    if (napi_create_typedarray(env, t, n, ab, 0, &arr) != napi_ok) return NULL;
    return arr;
}

#define ARGS(n)                                                                  \
    size_t argc = (n);                                                           \
    napi_value argv[(n) ? (n) : 1];                                              \
    CALL(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));             \
    if (argc < (n)) {                                                            \
        napi_throw_type_error(env, NULL, "expected " #n " arguments");           \
        return NULL;                                                             \
    }

/* openDevice(ordinal) -> external */
static napi_value open_device(napi_env env, napi_callback_info info) {
    ARGS(1);
    int32_t ord = 0;
    CALL(env, napi_get_value_int32(env, argv[0], &ord));
    bv_device *dev = NULL;
    int rc = bv_device_open(ord, &dev);
    if (rc) return throw_bv(env, rc);
    napi_value out;
    CALL(env, napi_create_external(env, dev, NULL, NULL, &out));
    return out;
}

static napi_value close_device(napi_env env, napi_callback_info info) {
    ARGS(1);
    int rc = bv_device_close((bv_device *)get_ptr(env, argv[0]));
    if (rc) return throw_bv(env, rc);
    return NULL;
}

static napi_value device_lost(napi_env env, napi_callback_info info) {
    ARGS(1);
    int lost = 1;
    int rc = bv_device_is_lost((const bv_device *)get_ptr(env, argv[0]), &lost);
    if (rc) return throw_bv(env, rc);
    napi_value out;
    CALL(env, napi_get_boolean(env, lost != 0, &out));
    return out;
}

static uint32_t field_u32(napi_env env, napi_value obj, const char *name, uint32_t dflt) {
    bool has = false;
    napi_value v;
    uint32_t x = dflt;
    if (napi_has_named_property(env, obj, name, &has) == napi_ok && has &&
        napi_get_named_property(env, obj, name, &v) == napi_ok) {
        napi_valuetype t;
        if (napi_typeof(env, v, &t) == napi_ok && t == napi_number) napi_get_value_uint32(env, v, &x);
    }
    return x;
}

static double field_f64(napi_env env, napi_value obj, const char *name, double dflt) {
    bool has = false;
    napi_value v;
    double x = dflt;
    if (napi_has_named_property(env, obj, name, &has) == napi_ok && has &&
        napi_get_named_property(env, obj, name, &v) == napi_ok) {
        napi_valuetype t;
        if (napi_typeof(env, v, &t) == napi_ok && t == napi_number) napi_get_value_double(env, v, &x);
    }
    return x;
}

/* createIndex(dev, {kind, dim, metric, bits, scorer, seed, rounds, chunkRows,
 *                   nlist, nprobe, sampleSize, trainSize, iters, ivfSeed, targetRecall}) -> external */
static napi_value create_index(napi_env env, napi_callback_info info) {
    ARGS(2);
    bv_index_desc d;
    memset(&d, 0, sizeof d);
    d.size = sizeof d;
    d.kind = field_u32(env, argv[1], "kind", BV_KIND_FLAT);
    d.dim = field_u32(env, argv[1], "dim", 0);
    d.metric = field_u32(env, argv[1], "metric", BV_METRIC_COSINE);
    d.bits = field_u32(env, argv[1], "bits", 0);
    d.scorer = field_u32(env, argv[1], "scorer", BV_SCORER_ASYM);
    d.has_seed = field_u32(env, argv[1], "hasSeed", 0);
    d.seed = field_u32(env, argv[1], "seed", 0);
    d.rounds = field_u32(env, argv[1], "rounds", 0);
    d.chunk_rows = field_u32(env, argv[1], "chunkRows", 0);
    d.nlist = field_u32(env, argv[1], "nlist", 0);
    d.nprobe = field_u32(env, argv[1], "nprobe", 0);
    d.sample_size = field_u32(env, argv[1], "sampleSize", 0);
    d.train_size = field_u32(env, argv[1], "trainSize", 0);
    d.iters = field_u32(env, argv[1], "iters", 0);
    d.has_ivf_seed = field_u32(env, argv[1], "hasIvfSeed", 0);
    d.ivf_seed = field_u32(env, argv[1], "ivfSeed", 0);
    d.target_recall = (float)field_f64(env, argv[1], "targetRecall", -1.0);
    bv_index *idx = NULL;
    int rc = bv_index_create((bv_device *)get_ptr(env, argv[0]), &d, &idx);
    if (rc) return throw_bv(env, rc);
    napi_value out;
    CALL(env, napi_create_external(env, idx, NULL, NULL, &out));
    return out;
}

static napi_value destroy_index(napi_env env, napi_callback_info info) {
    ARGS(1);
    int rc = bv_index_destroy((bv_index *)get_ptr(env, argv[0]));
    if (rc) return throw_bv(env, rc);
    return NULL;
}

static napi_value index_size(napi_env env, napi_callback_info info) {
    ARGS(1);
    uint64_t rows = 0;
    int rc = bv_index_size((const bv_index *)get_ptr(env, argv[0]), &rows);
    if (rc) return throw_bv(env, rc);
    napi_value out;
    CALL(env, napi_create_double(env, (double)rows, &out));
    return out;
}

/* append(idx, Float32Array data, count) */
static napi_value append(napi_env env, napi_callback_info info) {
    ARGS(3);
    size_t n = 0;
    const float *data = (const float *)get_typed(env, argv[1], napi_float32_array, &n);
    uint32_t count = 0;
    if (!data || !get_u32(env, argv[2], &count)) {
        napi_throw_type_error(env, NULL, "append(idx, Float32Array, count)");
        return NULL;
    }
    int rc = bv_index_append((bv_index *)get_ptr(env, argv[0]), data, n, count);
    if (rc) return throw_bv(env, rc);
    return NULL;
}

/* Result object {rows: Uint32Array, scores: Float32Array, counts: Uint32Array}. */
static napi_value result(napi_env env, size_t nq, size_t k, uint32_t **rows, float **scores, uint32_t **counts,
                         napi_value *r, napi_value *s, napi_value *c) {
    *r = new_typed(env, napi_uint32_array, nq * k, 4, (void **)rows);
    *s = new_typed(env, napi_float32_array, nq * k, 4, (void **)scores);
    *c = new_typed(env, napi_uint32_array, nq, 4, (void **)counts);
    if (!*r || !*s || !*c) return NULL;
    napi_value obj;
    if (napi_create_object(env, &obj) != napi_ok) return NULL;
    napi_set_named_property(env, obj, "rows", *r);
    napi_set_named_property(env, obj, "scores", *s);
    napi_set_named_property(env, obj, "counts", *c);
    return obj;
}

/* query(idx, Float32Array q, k) / queryMasked(idx, q, k, Uint32Array mask) */
static napi_value query_common(napi_env env, napi_callback_info info, int masked) {
    size_t argc = 4;
    napi_value argv[4];
    CALL(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
    size_t qn = 0, mn = 0;
    const float *q = argc > 1 ? (const float *)get_typed(env, argv[1], napi_float32_array, &qn) : NULL;
    uint32_t k = 0;
    const uint32_t *mask = NULL;
    if (masked && argc > 3) mask = (const uint32_t *)get_typed(env, argv[3], napi_uint32_array, &mn);
    if (!q || argc < 3 || !get_u32(env, argv[2], &k) || (masked && !mask)) {
        napi_throw_type_error(env, NULL, masked ? "queryMasked(idx, Float32Array, k, Uint32Array)"
                                                : "query(idx, Float32Array, k)");
        return NULL;
    }
    uint32_t *rows, *counts;
    float *scores;
    napi_value r, s, c;
    napi_value obj = result(env, 1, k, &rows, &scores, &counts, &r, &s, &c);
    if (!obj) return NULL;
    bv_index *idx = (bv_index *)get_ptr(env, argv[0]);
    int rc = masked ? bv_index_query_masked(idx, q, k, mask, mn, rows, scores, counts)
                    : bv_index_query(idx, q, k, rows, scores, counts);
    if (rc) return throw_bv(env, rc);
    return obj;
}
static napi_value query(napi_env env, napi_callback_info info) { return query_common(env, info, 0); }
static napi_value query_masked(napi_env env, napi_callback_info info) { return query_common(env, info, 1); }

/* queryBatch(idx, Float32Array packed, n, k) */
static napi_value query_batch(napi_env env, napi_callback_info info) {
    ARGS(4);
    size_t qn = 0;
    const float *q = (const float *)get_typed(env, argv[1], napi_float32_array, &qn);
    uint32_t nq = 0, k = 0;
    if (!q || !get_u32(env, argv[2], &nq) || !get_u32(env, argv[3], &k)) {
        napi_throw_type_error(env, NULL, "queryBatch(idx, Float32Array, n, k)");
        return NULL;
    }
    uint32_t *rows, *counts;
    float *scores;
    napi_value r, s, c;
    napi_value obj = result(env, nq, k, &rows, &scores, &counts, &r, &s, &c);
    if (!obj) return NULL;
    int rc = bv_index_query_batch((bv_index *)get_ptr(env, argv[0]), q, nq, k, rows, scores, counts);
    if (rc) return throw_bv(env, rc);
    return obj;
}

/* search(idx, Float32Array queries, n, fetch, k): top-fetch by code score, exact re-rank to k */
static napi_value search(napi_env env, napi_callback_info info) {
    ARGS(5);
    size_t qn = 0;
    const float *q = (const float *)get_typed(env, argv[1], napi_float32_array, &qn);
    uint32_t nq = 0, fetch = 0, k = 0;
    if (!q || !get_u32(env, argv[2], &nq) || !get_u32(env, argv[3], &fetch) || !get_u32(env, argv[4], &k)) {
        napi_throw_type_error(env, NULL, "search(idx, Float32Array, n, fetch, k)");
        return NULL;
    }
    uint32_t *rows, *counts;
    float *scores;
    napi_value r, s, c;
    napi_value obj = result(env, nq, k, &rows, &scores, &counts, &r, &s, &c);
    if (!obj) return NULL;
    int rc = bv_index_search((bv_index *)get_ptr(env, argv[0]), q, nq, fetch, k, rows, scores, counts);
    if (rc) return throw_bv(env, rc);
    return obj;
}

/* rerank(idx, Float32Array q, Uint32Array candidates, k) */
static napi_value rerank(napi_env env, napi_callback_info info) {
    ARGS(4);
    size_t qn = 0, cn = 0;
    const float *q = (const float *)get_typed(env, argv[1], napi_float32_array, &qn);
    const uint32_t *cand = (const uint32_t *)get_typed(env, argv[2], napi_uint32_array, &cn);
    uint32_t k = 0;
    if (!q || !cand || !get_u32(env, argv[3], &k)) {
        napi_throw_type_error(env, NULL, "rerank(idx, Float32Array, Uint32Array, k)");
        return NULL;
    }
    uint32_t *rows, *counts;
    float *scores;
    napi_value r, s, c;
    napi_value obj = result(env, 1, k, &rows, &scores, &counts, &r, &s, &c);
    if (!obj) return NULL;
    int rc = bv_index_rerank((bv_index *)get_ptr(env, argv[0]), q, cand, (uint32_t)cn, k, rows, scores, counts);
    if (rc) return throw_bv(env, rc);
    return obj;
}

static napi_value set_nprobe(napi_env env, napi_callback_info info) {
    ARGS(2);
    uint32_t n = 0;
    get_u32(env, argv[1], &n);
    int rc = bv_index_set_nprobe((bv_index *)get_ptr(env, argv[0]), n);
    if (rc) return throw_bv(env, rc);
    return NULL;
}

static napi_value stats(napi_env env, napi_callback_info info) {
    ARGS(1);
    bv_index_stats st;
    memset(&st, 0, sizeof st);
    int rc = bv_index_get_stats((bv_index *)get_ptr(env, argv[0]), &st);
    if (rc) return throw_bv(env, rc);
    napi_value obj, v;
    CALL(env, napi_create_object(env, &obj));
#define NUM(name, x)                                   \
    CALL(env, napi_create_double(env, (double)(x), &v)); \
    CALL(env, napi_set_named_property(env, obj, name, v))
    NUM("rows", st.rows);
    NUM("dim", st.dim);
    NUM("paddedDim", st.padded_dim);
    NUM("wordsPerRow", st.words_per_row);
    NUM("bits", st.bits);
    NUM("chunkCount", st.chunk_count);
    NUM("lastQueryMs", st.last_query_ms);
    NUM("lastQueryGpuMs", st.last_query_gpu_ms);
    NUM("deviceBytes", st.device_bytes);
    NUM("nlist", st.nlist);
    NUM("nprobe", st.nprobe);
    NUM("buildMs", st.build_ms);
    NUM("tunedRecall", st.tuned_recall);
#undef NUM
    return obj;
}

static napi_value last_error(napi_env env, napi_callback_info info) {
    (void)info;
    napi_value out;
    const char *m = bv_last_error();
    CALL(env, napi_create_string_utf8(env, m ? m : "", NAPI_AUTO_LENGTH, &out));
    return out;
}

static napi_value init(napi_env env, napi_value exports) {
    static const struct {
        const char *name;
        napi_callback fn;
    } fns[] = {
        {"openDevice", open_device},   {"closeDevice", close_device}, {"deviceLost", device_lost},
        {"createIndex", create_index}, {"destroyIndex", destroy_index}, {"size", index_size},
        {"append", append},            {"query", query},              {"queryMasked", query_masked},
        {"queryBatch", query_batch},   {"search", search},            {"rerank", rerank},
        {"setNprobe", set_nprobe},     {"stats", stats},              {"lastError", last_error},
    };
    for (size_t i = 0; i < sizeof fns / sizeof fns[0]; ++i) {
        napi_value f;
        if (napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].fn, NULL, &f) != napi_ok) return NULL;
        if (napi_set_named_property(env, exports, fns[i].name, f) != napi_ok) return NULL;
    }
    napi_value v;
    napi_create_uint32(env, (uint32_t)bv_abi_version(), &v);
    napi_set_named_property(env, exports, "abiVersion", v);
    return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
