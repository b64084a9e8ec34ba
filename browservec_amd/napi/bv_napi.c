/*
 * N-API binding of libbrowservec_hip.so for Node (the reference's host
 * runtime).  It exposes the C ABI of include/browservec_hip.h one call per
 * function; index.js builds the reference's VectorIndex seam
 * (src/index/flat.ts:24-40) on top of it.
 *
 * Calls that do device work (append, build, every query) run as
 * napi_async_work on libuv's thread pool and return a Promise, so a 4M-row
 * append or an IVF build does not block the event loop; the library
 * serializes calls on one index.  Input typed arrays are held by references
 * until the work completes, and results are written straight into typed
 * arrays created before the work is queued.  A failed call rejects (or, for
 * the synchronous calls, throws) an Error whose message is bv_last_error()
 * and whose `code` is the BV_E_* name, as the reference throws
 * `new Error(msg)`.  Query lengths are checked here against the index
 * dimension before any pointer reaches the library.
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

static const char *code_name(int rc) {
    static const char *names[] = {"BV_OK", "BV_E_INVALID", "BV_E_UNSUPPORTED", "BV_E_DEVICE_LOST",
                                  "BV_E_OOM", "BV_E_HIP", "BV_E_STATE"};
    if (rc > 0 && rc < (int)(sizeof names / sizeof names[0])) return names[rc];
    return "BV_E_UNKNOWN";
}

static napi_value throw_bv(napi_env env, int rc) {
    const char *msg = bv_last_error();
    napi_throw_error(env, code_name(rc), msg && *msg ? msg : "browservec_hip call failed");
    return NULL;
}

/* An index handle: the library object plus its (immutable) dimension, so
 * lengths are checked without a library call.  `pending` counts queued
 * device calls; destroy() on a handle with calls in flight marks it dead and
 * the last call's completion destroys the index (all on the main thread). */
typedef struct {
    bv_index *idx;
    bv_graph *graph; /* a graph searcher's handle has graph set and idx NULL */
    uint32_t dim;
    uint32_t pending;
    int dead;
} index_handle;

static void *get_ptr(napi_env env, napi_value v) {
    void *p = NULL;
    napi_valuetype t;
    if (napi_typeof(env, v, &t) != napi_ok || t != napi_external) return NULL;
    napi_get_value_external(env, v, &p);
    return p;
}

static index_handle *get_index(napi_env env, napi_value v) {
    index_handle *h = (index_handle *)get_ptr(env, v);
    return h && h->idx && !h->dead ? h : NULL;
}

static index_handle *get_graph(napi_env env, napi_value v) {
    index_handle *h = (index_handle *)get_ptr(env, v);
    return h && h->graph && !h->dead ? h : NULL;
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

static napi_value length_error(napi_env env, size_t want, size_t got) {
    char msg[96];
    snprintf(msg, sizeof msg, "expected %zu floats, got %zu", want, got);
    napi_throw_type_error(env, NULL, msg);
    return NULL;
}

/* ---- asynchronous device calls --------------------------------------------- */
typedef enum {
    OP_APPEND, OP_QUERY, OP_QUERY_MASKED, OP_QUERY_BATCH, OP_SEARCH, OP_RERANK, OP_BUILD, OP_SAVE, OP_LOAD,
    OP_ROWS, OP_ROWS_MASKED, OP_GRAPH_SEARCH
} op_kind;

typedef struct {
    napi_async_work work;
    napi_deferred deferred;
    op_kind op;
    index_handle *h;
    bv_index *idx;
    napi_ref keep[3];   /* input arrays and the index handle, held until completion */
    napi_ref result;    /* result object (queries), or NULL */
    const float *data;
    size_t n_floats;
    uint64_t count;
    const uint32_t *aux; /* mask words or candidate rows */
    size_t n_aux;
    uint32_t nq, k, fetch;
    uint32_t *rows, *counts;
    float *scores;
    const void *section;  /* loadSection input */
    void *saved;          /* saveSection output (malloc'd; copied to JS on completion) */
    uint64_t section_size;
    int rc;
    char msg[512];
} job;

static void job_execute(napi_env env, void *data) {
    (void)env;
    job *j = (job *)data;
    switch (j->op) {
    case OP_APPEND: j->rc = bv_index_append(j->idx, j->data, j->n_floats, j->count); break;
    case OP_QUERY: j->rc = bv_index_query(j->idx, j->data, j->k, j->rows, j->scores, j->counts); break;
    case OP_QUERY_MASKED:
        j->rc = bv_index_query_masked(j->idx, j->data, j->k, j->aux, j->n_aux, j->rows, j->scores, j->counts);
        break;
    case OP_QUERY_BATCH: j->rc = bv_index_query_batch(j->idx, j->data, j->nq, j->k, j->rows, j->scores, j->counts); break;
    case OP_SEARCH:
        j->rc = bv_index_search(j->idx, j->data, j->nq, j->fetch, j->k, j->rows, j->scores, j->counts);
        break;
    case OP_RERANK:
        j->rc = bv_index_rerank(j->idx, j->data, j->aux, (uint32_t)j->n_aux, j->k, j->rows, j->scores, j->counts);
        break;
    case OP_ROWS:
        j->rc = bv_index_query_rows(j->idx, j->data, j->aux, j->n_aux, j->k, j->rows, j->scores, j->counts);
        break;
    case OP_ROWS_MASKED:
        j->rc = bv_index_query_rows_masked(j->idx, j->data, j->aux, j->n_aux, j->k, j->rows, j->scores, j->counts);
        break;
    case OP_GRAPH_SEARCH:
        j->rc = bv_graph_search(j->h->graph, j->data, j->nq, j->k, j->fetch, (uint32_t)j->count, j->rows, j->scores,
                                j->counts);
        break;
    case OP_BUILD: j->rc = bv_index_build(j->idx); break;
    case OP_SAVE: {
        uint64_t size = 0;
        j->rc = bv_index_save_section(j->idx, NULL, 0, &size);
        if (j->rc) break;
        j->saved = malloc(size ? size : 1);
        if (!j->saved) {
            j->rc = BV_E_OOM;
            snprintf(j->msg, sizeof j->msg, "out of host memory");
            return;
        }
        j->section_size = size;
        j->rc = bv_index_save_section(j->idx, j->saved, size, &size);
        break;
    }
    case OP_LOAD:
        j->rc = bv_index_load_section(j->idx, j->data, j->n_floats, j->count, j->section, j->section_size);
        break;
    }
    /* the message is thread-local: copy it on this thread */
    if (j->rc) snprintf(j->msg, sizeof j->msg, "%s", bv_last_error());
}

static void job_complete(napi_env env, napi_status status, void *data) {
    job *j = (job *)data;
    napi_value v;
    if (status != napi_ok && !j->rc) {
        j->rc = BV_E_STATE;
        snprintf(j->msg, sizeof j->msg, "async work was cancelled");
    }
    if (j->rc) {
        napi_value msg, code, err;
        napi_create_string_utf8(env, j->msg[0] ? j->msg : "browservec_hip call failed", NAPI_AUTO_LENGTH, &msg);
        napi_create_string_utf8(env, code_name(j->rc), NAPI_AUTO_LENGTH, &code);
        napi_create_error(env, code, msg, &err);
        napi_reject_deferred(env, j->deferred, err);
    } else if (j->op == OP_SAVE) {
        void *dst = NULL;
        napi_value ab;
        if (napi_create_arraybuffer(env, j->section_size, &dst, &ab) == napi_ok &&
            napi_create_typedarray(env, napi_uint8_array, j->section_size, ab, 0, &v) == napi_ok) {
            memcpy(dst, j->saved, j->section_size);
            napi_resolve_deferred(env, j->deferred, v);
        } else {
            napi_value msg, err;
            napi_create_string_utf8(env, "out of memory for the index section", NAPI_AUTO_LENGTH, &msg);
            napi_create_error(env, NULL, msg, &err);
            napi_reject_deferred(env, j->deferred, err);
        }
    } else {
        if (j->result) napi_get_reference_value(env, j->result, &v);
        else napi_get_undefined(env, &v);
        napi_resolve_deferred(env, j->deferred, v);
    }
    free(j->saved);
    for (int i = 0; i < 3; ++i)
        if (j->keep[i]) napi_delete_reference(env, j->keep[i]);
    if (j->result) napi_delete_reference(env, j->result);
    napi_delete_async_work(env, j->work);
    index_handle *h = j->h;
    free(j);
    if (--h->pending == 0 && h->dead && h->idx) {
        bv_index_destroy(h->idx);
        h->idx = NULL;
    }
    if (h->pending == 0 && h->dead && h->graph) {
        bv_graph_destroy(h->graph);
        h->graph = NULL;
    }
}

/* Queues the job and returns its promise.  `handle` (the index external)
 * stays referenced until completion, so the index outlives the work. */
static napi_value queue(napi_env env, job *j, napi_value handle, const char *name) {
    napi_value promise, res;
    if (napi_create_reference(env, handle, 1, &j->keep[2]) != napi_ok ||
        napi_create_promise(env, &j->deferred, &promise) != napi_ok ||
        napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &res) != napi_ok ||
        napi_create_async_work(env, NULL, res, job_execute, job_complete, j, &j->work) != napi_ok ||
        napi_queue_async_work(env, j->work) != napi_ok) {
        for (int i = 0; i < 3; ++i)
            if (j->keep[i]) napi_delete_reference(env, j->keep[i]);
        if (j->result) napi_delete_reference(env, j->result);
        free(j);
        napi_throw_error(env, NULL, "could not queue the device call");
        return NULL;
    }
    j->h->pending++;
    return promise;
}

static job *new_job(napi_env env, op_kind op, index_handle *h) {
    (void)env;
    job *j = (job *)calloc(1, sizeof(job));
    if (j) {
        j->op = op;
        j->h = h;
        j->idx = h->idx;
    }
    return j;
}

/* Result object {rows: Uint32Array, scores: Float32Array, counts: Uint32Array},
 * referenced by the job until it completes. */
static int job_result(napi_env env, job *j, size_t nq, size_t k) {
    napi_value r, s, c, obj;
    r = new_typed(env, napi_uint32_array, nq * k, 4, (void **)&j->rows);
    s = new_typed(env, napi_float32_array, nq * k, 4, (void **)&j->scores);
    c = new_typed(env, napi_uint32_array, nq, 4, (void **)&j->counts);
    if (!r || !s || !c || napi_create_object(env, &obj) != napi_ok) return 0;
    napi_set_named_property(env, obj, "rows", r);
    napi_set_named_property(env, obj, "scores", s);
    napi_set_named_property(env, obj, "counts", c);
    return napi_create_reference(env, obj, 1, &j->result) == napi_ok;
}

static int keep(napi_env env, job *j, int slot, napi_value v) {
    return napi_create_reference(env, v, 1, &j->keep[slot]) == napi_ok;
}

/* ---- device ------------------------------------------------------------------ */
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

/* debugInject(dev, what): host-side failure flags (BV_INJECT_*). */
static napi_value debug_inject(napi_env env, napi_callback_info info) {
    ARGS(2);
    uint32_t what = 0;
    get_u32(env, argv[1], &what);
    int rc = bv_debug_inject((bv_device *)get_ptr(env, argv[0]), (int)what);
    if (rc) return throw_bv(env, rc);
    return NULL;
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

/* The handle's finalizer: an index the script dropped without destroy(); calls in
 * flight hold a reference to the handle, so none is pending here. */
static void index_finalize(napi_env env, void *data, void *hint) {
    (void)env;
    (void)hint;
    index_handle *h = (index_handle *)data;
    if (h->idx) bv_index_destroy(h->idx);
    free(h);
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
    d.ivf_incremental = field_u32(env, argv[1], "incremental", 0);
    bv_index *idx = NULL;
    int rc = bv_index_create((bv_device *)get_ptr(env, argv[0]), &d, &idx);
    if (rc) return throw_bv(env, rc);
    index_handle *h = (index_handle *)calloc(1, sizeof *h);
    if (!h) {
        bv_index_destroy(idx);
        napi_throw_error(env, "BV_E_OOM", "out of host memory");
        return NULL;
    }
    h->idx = idx;
    h->dim = d.dim;
    napi_value out;
    CALL(env, napi_create_external(env, h, index_finalize, NULL, &out));
    return out;
}

static napi_value destroy_index(napi_env env, napi_callback_info info) {
    ARGS(1);
    index_handle *h = get_index(env, argv[0]);
    if (!h) return NULL;
    h->dead = 1;
    if (h->pending) return NULL;  /* the last call in flight destroys it */
    int rc = bv_index_destroy(h->idx);
    h->idx = NULL;
    if (rc) return throw_bv(env, rc);
    return NULL;
}

static napi_value index_size(napi_env env, napi_callback_info info) {
    ARGS(1);
    index_handle *h = get_index(env, argv[0]);
    uint64_t rows = 0;
    int rc = bv_index_size(h ? h->idx : NULL, &rows);
    if (rc) return throw_bv(env, rc);
    napi_value out;
    CALL(env, napi_create_double(env, (double)rows, &out));
    return out;
}

/* append(idx, Float32Array data, count) -> Promise<void> */
static napi_value append(napi_env env, napi_callback_info info) {
    ARGS(3);
    index_handle *h = get_index(env, argv[0]);
    size_t n = 0;
    const float *data = (const float *)get_typed(env, argv[1], napi_float32_array, &n);
    uint32_t count = 0;
    if (!h || !data || !get_u32(env, argv[2], &count)) {
        napi_throw_type_error(env, NULL, "append(idx, Float32Array, count)");
        return NULL;
    }
    /* the reference's check and message (src/index/flat.ts:96-98) */
    if (n != (size_t)count * h->dim) {
        char msg[96];
        snprintf(msg, sizeof msg, "expected %zu floats, got %zu", (size_t)count * h->dim, n);
        napi_throw_error(env, "BV_E_INVALID", msg);
        return NULL;
    }
    job *j = new_job(env, OP_APPEND, h);
    if (!j || !keep(env, j, 0, argv[1])) {
        free(j);
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    j->data = data;
    j->n_floats = n;
    j->count = count;
    return queue(env, j, argv[0], "browservec.append");
}

/* build(idx) -> Promise<void>: the IVF build now (queries build on demand). */
static napi_value build(napi_env env, napi_callback_info info) {
    ARGS(1);
    index_handle *h = get_index(env, argv[0]);
    if (!h) {
        napi_throw_type_error(env, NULL, "build(idx)");
        return NULL;
    }
    job *j = new_job(env, OP_BUILD, h);
    if (!j) {
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    return queue(env, j, argv[0], "browservec.build");
}

/* saveSection(idx) -> Promise<Uint8Array>: the index section of a snapshot
 * (codes, scales, IVF state). */
static napi_value save_section(napi_env env, napi_callback_info info) {
    ARGS(1);
    index_handle *h = get_index(env, argv[0]);
    if (!h) {
        napi_throw_type_error(env, NULL, "saveSection(idx)");
        return NULL;
    }
    job *j = new_job(env, OP_SAVE, h);
    if (!j) {
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    return queue(env, j, argv[0], "browservec.saveSection");
}

/* loadSection(idx, Float32Array rows, count, Uint8Array section) -> Promise<void>:
 * fills an empty index from a snapshot's rows and its index section. */
static napi_value load_section(napi_env env, napi_callback_info info) {
    ARGS(4);
    index_handle *h = get_index(env, argv[0]);
    size_t n = 0, nb = 0;
    const float *data = (const float *)get_typed(env, argv[1], napi_float32_array, &n);
    uint32_t count = 0;
    const void *sec = get_typed(env, argv[3], napi_uint8_array, &nb);
    if (!h || (!data && n) || !get_u32(env, argv[2], &count) || !sec) {
        napi_throw_type_error(env, NULL, "loadSection(idx, Float32Array, count, Uint8Array)");
        return NULL;
    }
    if (n != (size_t)count * h->dim) return length_error(env, (size_t)count * h->dim, n);
    job *j = new_job(env, OP_LOAD, h);
    if (!j || !keep(env, j, 0, argv[1]) || !keep(env, j, 1, argv[3])) {
        free(j);
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    j->data = data;
    j->n_floats = n;
    j->count = count;
    j->section = sec;
    j->section_size = nb;
    return queue(env, j, argv[0], "browservec.loadSection");
}

/* query(idx, Float32Array q, k) / queryMasked(idx, q, k, Uint32Array mask) -> Promise<result> */
static napi_value query_common(napi_env env, napi_callback_info info, int masked) {
    size_t argc = 4;
    napi_value argv[4];
    CALL(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
    size_t qn = 0, mn = 0;
    index_handle *h = argc > 0 ? get_index(env, argv[0]) : NULL;
    const float *q = argc > 1 ? (const float *)get_typed(env, argv[1], napi_float32_array, &qn) : NULL;
    uint32_t k = 0;
    const uint32_t *mask = NULL;
    if (masked && argc > 3) mask = (const uint32_t *)get_typed(env, argv[3], napi_uint32_array, &mn);
    if (!h || !q || argc < 3 || !get_u32(env, argv[2], &k) || (masked && !mask)) {
        napi_throw_type_error(env, NULL, masked ? "queryMasked(idx, Float32Array, k, Uint32Array)"
                                                : "query(idx, Float32Array, k)");
        return NULL;
    }
    if (qn != h->dim) return length_error(env, h->dim, qn);
    job *j = new_job(env, masked ? OP_QUERY_MASKED : OP_QUERY, h);
    if (!j || !keep(env, j, 0, argv[1]) || (masked && !keep(env, j, 1, argv[3])) || !job_result(env, j, 1, k)) {
        free(j);
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    j->data = q;
    j->k = k;
    j->aux = mask;
    j->n_aux = mn;
    return queue(env, j, argv[0], "browservec.query");
}
static napi_value query(napi_env env, napi_callback_info info) { return query_common(env, info, 0); }
static napi_value query_masked(napi_env env, napi_callback_info info) { return query_common(env, info, 1); }

/* queryBatch(idx, Float32Array packed, n, k) / search(idx, packed, n, fetch, k) -> Promise<result> */
static napi_value batch_common(napi_env env, napi_callback_info info, int with_fetch) {
    size_t argc = 5;
    napi_value argv[5];
    CALL(env, napi_get_cb_info(env, info, &argc, argv, NULL, NULL));
    size_t qn = 0;
    index_handle *h = argc > 0 ? get_index(env, argv[0]) : NULL;
    const float *q = argc > 1 ? (const float *)get_typed(env, argv[1], napi_float32_array, &qn) : NULL;
    uint32_t nq = 0, fetch = 0, k = 0;
    const size_t need = with_fetch ? 5 : 4;
    if (!h || !q || argc < need || !get_u32(env, argv[2], &nq) ||
        (with_fetch && !get_u32(env, argv[3], &fetch)) || !get_u32(env, argv[need - 1], &k)) {
        napi_throw_type_error(env, NULL, with_fetch ? "search(idx, Float32Array, n, fetch, k)"
                                                    : "queryBatch(idx, Float32Array, n, k)");
        return NULL;
    }
    if (qn != (size_t)nq * h->dim) return length_error(env, (size_t)nq * h->dim, qn);
    job *j = new_job(env, with_fetch ? OP_SEARCH : OP_QUERY_BATCH, h);
    if (!j || !keep(env, j, 0, argv[1]) || !job_result(env, j, nq, k)) {
        free(j);
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    j->data = q;
    j->nq = nq;
    j->fetch = fetch;
    j->k = k;
    return queue(env, j, argv[0], with_fetch ? "browservec.search" : "browservec.queryBatch");
}
static napi_value query_batch(napi_env env, napi_callback_info info) { return batch_common(env, info, 0); }
static napi_value search(napi_env env, napi_callback_info info) { return batch_common(env, info, 1); }

/* rerank(idx, Float32Array q, Uint32Array candidates, k) -> Promise<result> */
static napi_value rerank(napi_env env, napi_callback_info info) {
    ARGS(4);
    size_t qn = 0, cn = 0;
    index_handle *h = get_index(env, argv[0]);
    const float *q = (const float *)get_typed(env, argv[1], napi_float32_array, &qn);
    const uint32_t *cand = (const uint32_t *)get_typed(env, argv[2], napi_uint32_array, &cn);
    uint32_t k = 0;
    if (!h || !q || !cand || !get_u32(env, argv[3], &k)) {
        napi_throw_type_error(env, NULL, "rerank(idx, Float32Array, Uint32Array, k)");
        return NULL;
    }
    if (qn != h->dim) return length_error(env, h->dim, qn);
    job *j = new_job(env, OP_RERANK, h);
    if (!j || !keep(env, j, 0, argv[1]) || !keep(env, j, 1, argv[2]) || !job_result(env, j, 1, k)) {
        free(j);
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    j->data = q;
    j->aux = cand;
    j->n_aux = cn;
    j->k = k;
    return queue(env, j, argv[0], "browservec.rerank");
}

/* queryRows(idx, Float32Array q, Uint32Array rows, k) and
 * queryRowsMasked(idx, Float32Array q, Uint32Array maskWords, k) -> Promise<result>:
 * queryRowsExact's exact scores of the listed (or masked-in) rows and their top k */
static napi_value rows_common(napi_env env, napi_callback_info info, int masked) {
    ARGS(4);
    size_t qn = 0, an = 0;
    index_handle *h = get_index(env, argv[0]);
    const float *q = (const float *)get_typed(env, argv[1], napi_float32_array, &qn);
    const uint32_t *aux = (const uint32_t *)get_typed(env, argv[2], napi_uint32_array, &an);
    uint32_t k = 0;
    if (!h || !q || !aux || !get_u32(env, argv[3], &k)) {
        napi_throw_type_error(env, NULL, masked ? "queryRowsMasked(idx, Float32Array, Uint32Array, k)"
                                                : "queryRows(idx, Float32Array, Uint32Array, k)");
        return NULL;
    }
    if (qn != h->dim) return length_error(env, h->dim, qn);
    job *j = new_job(env, masked ? OP_ROWS_MASKED : OP_ROWS, h);
    if (!j || !keep(env, j, 0, argv[1]) || !keep(env, j, 1, argv[2]) || !job_result(env, j, 1, k)) {
        free(j);
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    j->data = q;
    j->aux = aux;
    j->n_aux = an;
    j->k = k;
    return queue(env, j, argv[0], masked ? "browservec.queryRowsMasked" : "browservec.queryRows");
}
static napi_value query_rows(napi_env env, napi_callback_info info) { return rows_common(env, info, 0); }
static napi_value query_rows_masked(napi_env env, napi_callback_info info) { return rows_common(env, info, 1); }

/* ---- graph search (HNSWGpuSearcher) --------------------------------------- */
/* graphCreate(device, {dim, metric, degree}) -> external */
static napi_value graph_create(napi_env env, napi_callback_info info) {
    ARGS(2);
    bv_device *dev = (bv_device *)get_ptr(env, argv[0]);
    const uint32_t dim = field_u32(env, argv[1], "dim", 0);
    const uint32_t metric = field_u32(env, argv[1], "metric", BV_METRIC_COSINE);
    const uint32_t degree = field_u32(env, argv[1], "degree", 0);
    bv_graph *g = NULL;
    int rc = bv_graph_create(dev, dim, metric, degree, &g);
    if (rc) return throw_bv(env, rc);
    index_handle *h = (index_handle *)calloc(1, sizeof(index_handle));
    if (!h) {
        bv_graph_destroy(g);
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    h->graph = g;
    h->dim = dim;
    napi_value out;
    CALL(env, napi_create_external(env, h, NULL, NULL, &out));
    return out;
}

/* graphAppend(g, Float32Array rows, count) (synchronous, as the reference's) */
static napi_value graph_append(napi_env env, napi_callback_info info) {
    ARGS(3);
    size_t n = 0;
    index_handle *h = get_graph(env, argv[0]);
    const float *d = (const float *)get_typed(env, argv[1], napi_float32_array, &n);
    uint32_t count = 0;
    if (!h || !d || !get_u32(env, argv[2], &count)) {
        napi_throw_type_error(env, NULL, "graphAppend(g, Float32Array, count)");
        return NULL;
    }
    int rc = bv_graph_append(h->graph, d, n, count);
    if (rc) return throw_bv(env, rc);
    return NULL;
}

/* graphUpload(g, Uint32Array links, rows) */
static napi_value graph_upload(napi_env env, napi_callback_info info) {
    ARGS(3);
    size_t n = 0;
    index_handle *h = get_graph(env, argv[0]);
    const uint32_t *l = (const uint32_t *)get_typed(env, argv[1], napi_uint32_array, &n);
    uint32_t rows = 0;
    if (!h || !l || !get_u32(env, argv[2], &rows)) {
        napi_throw_type_error(env, NULL, "graphUpload(g, Uint32Array, rows)");
        return NULL;
    }
    int rc = bv_graph_upload(h->graph, l, rows);
    if (rc) return throw_bv(env, rc);
    return NULL;
}

/* graphSearch(g, Float32Array queries, n, k, ef, entry) -> Promise<result> */
static napi_value graph_search(napi_env env, napi_callback_info info) {
    ARGS(6);
    size_t qn = 0;
    index_handle *h = get_graph(env, argv[0]);
    const float *q = (const float *)get_typed(env, argv[1], napi_float32_array, &qn);
    uint32_t n = 0, k = 0, ef = 0, entry = 0;
    if (!h || !q || !get_u32(env, argv[2], &n) || !get_u32(env, argv[3], &k) || !get_u32(env, argv[4], &ef) ||
        !get_u32(env, argv[5], &entry)) {
        napi_throw_type_error(env, NULL, "graphSearch(g, Float32Array, n, k, ef, entry)");
        return NULL;
    }
    if (qn < (size_t)n * h->dim) return length_error(env, (size_t)n * h->dim, qn);
    job *j = (job *)calloc(1, sizeof(job));
    if (!j || !keep(env, j, 0, argv[1]) || !job_result(env, j, n, k)) {
        free(j);
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    j->op = OP_GRAPH_SEARCH;
    j->h = h;
    j->data = q;
    j->nq = n;
    j->k = k;
    j->fetch = ef;
    j->count = entry;
    return queue(env, j, argv[0], "browservec.graphSearch");
}

static napi_value graph_destroy(napi_env env, napi_callback_info info) {
    ARGS(1);
    index_handle *h = get_graph(env, argv[0]);
    if (!h) return NULL;
    h->dead = 1;
    if (h->pending) return NULL;  /* the search in flight destroys it */
    bv_graph_destroy(h->graph);
    h->graph = NULL;
    return NULL;
}

static napi_value set_nprobe(napi_env env, napi_callback_info info) {
    ARGS(2);
    index_handle *h = get_index(env, argv[0]);
    uint32_t n = 0;
    get_u32(env, argv[1], &n);
    int rc = bv_index_set_nprobe(h ? h->idx : NULL, n);
    if (rc) return throw_bv(env, rc);
    return NULL;
}

static napi_value stats(napi_env env, napi_callback_info info) {
    ARGS(1);
    index_handle *h = get_index(env, argv[0]);
    bv_index_stats st;
    memset(&st, 0, sizeof st);
    int rc = bv_index_get_stats(h ? h->idx : NULL, &st);
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
    NUM("buildExactRows", st.build_exact_rows);
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
        {"openDevice", open_device},   {"closeDevice", close_device},   {"deviceLost", device_lost},
        {"debugInject", debug_inject}, {"createIndex", create_index},   {"destroyIndex", destroy_index},
        {"size", index_size},          {"append", append},              {"build", build},
        {"query", query},              {"queryMasked", query_masked},   {"queryBatch", query_batch},
        {"search", search},            {"rerank", rerank},              {"setNprobe", set_nprobe},
        {"queryRows", query_rows},     {"queryRowsMasked", query_rows_masked},
        {"graphCreate", graph_create}, {"graphAppend", graph_append},    {"graphUpload", graph_upload},
        {"graphSearch", graph_search}, {"graphDestroy", graph_destroy},
        {"stats", stats},              {"lastError", last_error},
        {"saveSection", save_section}, {"loadSection", load_section},
    };
    for (size_t i = 0; i < sizeof fns / sizeof fns[0]; ++i) {
        napi_value f;
        if (napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].fn, NULL, &f) != napi_ok) return NULL;
        if (napi_set_named_property(env, exports, fns[i].name, f) != napi_ok) return NULL;
    }
    napi_value v;
    napi_create_uint32(env, (uint32_t)bv_abi_version(), &v);
    napi_set_named_property(env, exports, "abiVersion", v);
    napi_create_uint32(env, BV_INJECT_LOST, &v);
    napi_set_named_property(env, exports, "INJECT_LOST", v);
    napi_create_uint32(env, BV_INJECT_APPEND_OOM, &v);
    napi_set_named_property(env, exports, "INJECT_APPEND_OOM", v);
    return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
