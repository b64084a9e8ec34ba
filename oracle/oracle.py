"""CPU oracle for BrowserVec's search path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker (or as the timed CPU
baseline).  The shipped library never calls it.

The arithmetic lives in ``bv_oracle.c`` (built by ``oracle/Makefile`` into
``liboracle.so``); this module adds numpy-friendly wrappers and the IVF
orchestration glue.  Each function cites the reference file:line it restates.

Parity pins (the check that would fail on a plausible transcription mistake):

===========================  =================================================
function                     pinned by
===========================  =================================================
mulberry32 / random_signs    (1) JS-engine cross-check: tests/golden/js_vectors.json
                             written by tests/golden/make_js_vectors.js under
                             node's own Math.imul / >>> / Float32Array
                             semantics; (2) determinism, [0,1) range and mean
                             (tests/unit/prng.test.ts:4-37)
pad_to_pow2                  table from tests/unit/rotator.test.ts:18-28
fwht                         unit impulse -> all ones; H.H = n.I; brute-force
                             Hadamard matrix product (exact for small ints)
rotator / rotate             orthonormality (<Ra,Rb> = <a,b>); f64 FWHT
                             restatement within 1e-6; JS-engine vectors
quantize_row8/4/1            codec.test.ts KATs ([0.5,-2.5,1,0] -> scale 2.5,
                             zero row -> scale 1, zeros -> 0xffffffff);
                             round-trip <= step/2; rounding boundaries at
                             exact n+0.5 (ties up, -0.5 -> 0); JS vectors
normalize / dot_row / l2     store.test.ts KAT ([3,4] -> [0.6,0.8]); long
                             double brute force within 1 ulp f32
scan_f32/q8/q4/q1            long-double brute force of the dequantized
                             product, relative 1e-6
scan_hamming / int8sym       Python big-int brute force (exact)
wasm_dot / wasm_l2           scalar lane emulation, bit-exact
topk_ref / merge_partials    topk.test.ts KATs + full sort on random input;
                             the [5,5,7] tie example
topk_canonical               full sort by (score desc, row asc)
kmeans pieces                kmeans.test.ts KATs (updateCentroids ->
                             [1,1,10,10], normalizeRows([3,4,0,0]))
random_init_centroids        JS-engine vectors of the rows picked
                             (Math.floor(rng() * count), seeds up to 4096 lists)
update_centroids             JS-engine Float32Array run on a sample whose
                             sequential f32 sums differ from f64 sums, with an
                             empty cluster re-seeded and normalizeRows after
Reservoir                    JS-engine slot sequences; first cap slots are the
                             identity, admission probability cap/(i+1) and
                             final inclusion cap/n within 5 sd over 6000 seeds
assign_f32 (order 1)         brute-force argmax; the AVX2 path equals the
                             scalar fmaf chain (order 2), ties included
choose_nprobe / pick_tune    ivfTune.test.ts tables
probe_scores                 long double brute force within 1 ulp f32
graph_search / graph_hits    a connected graph searched with ef >= its rows
                             returns the brute-force top-k of the same f32
                             element-order distances (every row visited);
                             dedup keeps the first slot of an id; seeds
                             (graph_entries) against hand-computed rows;
                             the shader's lane races and reduction tie order
                             are restated in one fixed order: parity unpinned
                             beyond tie-free cases
===========================  =================================================
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

u32p = ctypes.POINTER(ctypes.c_uint32)
f32p = ctypes.POINTER(ctypes.c_float)
f64p = ctypes.POINTER(ctypes.c_double)
i32p = ctypes.POINTER(ctypes.c_int32)
u64p = ctypes.POINTER(ctypes.c_uint64)

DEFAULT_SEED = 0x9E3779B9
IVF_SEED = 0x51ED270B


def build() -> str:
    """Compile liboracle.so from bv_oracle.c (gcc is in the image)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    sig = {
        "bvo_mulberry32_next": (ctypes.c_uint32, [u32p]),
        "bvo_mulberry32_draw": (ctypes.c_double, [u32p]),
        "bvo_mulberry32_stream": (None, [ctypes.c_uint32, ctypes.c_uint64, f64p]),
        "bvo_random_signs": (None, [ctypes.c_uint32, ctypes.c_uint32, f32p]),
        "bvo_pad_to_pow2": (ctypes.c_uint32, [ctypes.c_uint32]),
        "bvo_fwht": (None, [f32p, ctypes.c_uint32]),
        "bvo_round_seed": (ctypes.c_uint32, [ctypes.c_uint32, ctypes.c_uint32]),
        "bvo_rotator_signs": (None, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, f32p]),
        "bvo_rotate": (None, [f32p, ctypes.c_uint32, f32p, ctypes.c_uint32, f32p]),
        "bvo_quantize_row8": (ctypes.c_float, [f32p, ctypes.c_uint32, u32p]),
        "bvo_quantize_row4": (ctypes.c_float, [f32p, ctypes.c_uint32, u32p]),
        "bvo_quantize_row1": (ctypes.c_float, [f32p, ctypes.c_uint32, u32p]),
        "bvo_dequant_row8": (None, [u32p, ctypes.c_uint32, ctypes.c_float, f32p]),
        "bvo_dequant_row4": (None, [u32p, ctypes.c_uint32, ctypes.c_float, f32p]),
        "bvo_dequant_row1": (None, [u32p, ctypes.c_uint32, ctypes.c_float, f32p]),
        "bvo_encode": (ctypes.c_int, [f32p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.c_uint32, ctypes.c_uint32, u32p, f32p, f32p]),
        "bvo_normalize": (None, [f32p, ctypes.c_uint32]),
        "bvo_normalize_many": (None, [f32p, ctypes.c_uint64, ctypes.c_uint32]),
        "bvo_dot_row": (ctypes.c_double, [f32p, f32p, ctypes.c_uint32]),
        "bvo_l2_row": (ctypes.c_double, [f32p, f32p, ctypes.c_uint32]),
        "bvo_rerank_scores": (None, [f32p, ctypes.c_uint32, f32p, u32p, ctypes.c_uint32, f32p]),
        "bvo_scan_f32": (None, [f32p, ctypes.c_uint64, ctypes.c_uint32, f32p, ctypes.c_uint32, f32p]),
        "bvo_scan_q8": (None, [u32p, f32p, ctypes.c_uint64, ctypes.c_uint32, f32p, u32p, f32p]),
        "bvo_scan_q4": (None, [u32p, f32p, ctypes.c_uint64, ctypes.c_uint32, f32p, u32p, f32p]),
        "bvo_scan_q1": (None, [u32p, f32p, ctypes.c_uint64, ctypes.c_uint32, f32p, u32p, f32p]),
        "bvo_query_bits": (None, [f32p, ctypes.c_uint32, u32p]),
        "bvo_scan_hamming": (None, [u32p, ctypes.c_uint64, ctypes.c_uint32, u32p, u32p, i32p]),
        "bvo_scan_int8sym": (None, [u32p, ctypes.c_uint64, ctypes.c_uint32, u32p, u32p, i32p]),
        "bvo_dot_exact": (None, [f32p, f32p, ctypes.c_uint64, ctypes.c_uint32, f64p, f64p]),
        "bvo_wasm_dot": (None, [f32p, f32p, f32p, ctypes.c_uint64, ctypes.c_uint32]),
        "bvo_wasm_l2": (None, [f32p, f32p, f32p, ctypes.c_uint64, ctypes.c_uint32]),
        "bvo_wasm_dot_scalar": (None, [f32p, f32p, f32p, ctypes.c_uint64, ctypes.c_uint32]),
        "bvo_topk_ref": (ctypes.c_uint32, [f32p, ctypes.c_uint32, ctypes.c_uint32, u32p, f32p]),
        "bvo_merge_partials": (ctypes.c_uint32, [f32p, u32p, ctypes.c_uint32, ctypes.c_uint32,
                                                 ctypes.c_uint32, u32p, f32p]),
        "bvo_topk_canonical": (ctypes.c_uint32, [f32p, u32p, ctypes.c_uint32, ctypes.c_uint32,
                                                 ctypes.c_float, u32p, f32p]),
        "bvo_normalize_rows": (None, [f32p, ctypes.c_uint32, ctypes.c_uint32]),
        "bvo_random_init_centroids": (None, [f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                             ctypes.c_uint32, f32p]),
        "bvo_update_centroids": (None, [f32p, ctypes.c_uint32, u32p, f32p, ctypes.c_uint32,
                                        ctypes.c_uint32, ctypes.c_uint32, i32p]),
        "bvo_assign_f32": (None, [f32p, ctypes.c_uint32, f32p, ctypes.c_uint32, ctypes.c_uint32,
                                  ctypes.c_uint32, u32p]),
        "bvo_assign_quant": (None, [u32p, f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                    f32p, ctypes.c_uint32, u32p]),
        "bvo_probe_scores": (None, [f32p, ctypes.c_uint32, ctypes.c_uint32, f32p, f32p]),
        "bvo_reservoir_slot": (ctypes.c_int64, [ctypes.c_uint32, u64p, u64p, u32p]),
        "bvo_build_csr": (None, [u32p, ctypes.c_uint64, ctypes.c_uint32, i32p, i32p]),
        "bvo_choose_nprobe": (ctypes.c_uint32, [u32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_double, f64p]),
        "bvo_pick_tune_queries": (ctypes.c_uint32, [ctypes.c_uint32, ctypes.c_uint32, u32p]),
        "bvo_graph_search": (None, [f32p, ctypes.c_uint32, ctypes.c_int, u32p, ctypes.c_uint32, ctypes.c_uint32,
                                    ctypes.c_uint32, f32p, ctypes.c_uint32, u32p, ctypes.c_uint32, ctypes.c_uint32,
                                    ctypes.c_uint32, f32p, u32p]),
        "bvo_graph_entries": (ctypes.c_uint32, [ctypes.c_uint32, ctypes.c_uint32, u32p]),
        "bvo_graph_hits": (ctypes.c_uint32, [f32p, u32p, ctypes.c_uint32, ctypes.c_uint32, u32p, f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = _load()


def _p(a: np.ndarray | None, t):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(t)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint32)


# --------------------------------------------------------------------- prng
def mulberry32_stream(seed: int, n: int) -> np.ndarray:
    """n successive mulberry32(seed)() draws as f64 (src/quant/prng.ts:5-14)."""
    out = np.empty(n, dtype=np.float64)
    _lib.bvo_mulberry32_stream(seed & 0xFFFFFFFF, n, _p(out, f64p))
    return out


def random_signs(n: int, seed: int) -> np.ndarray:
    """randomSigns (src/quant/prng.ts:17-22)."""
    out = np.empty(n, dtype=np.float32)
    _lib.bvo_random_signs(n, seed & 0xFFFFFFFF, _p(out, f32p))
    return out


def uniform_vectors(rows: int, dim: int, seed: int, scale: float = 1.0, normalize: bool = False) -> np.ndarray:
    """The reference tests' generator: f32(rng()*2-1) per coordinate
    (tests/browser/helpers.ts:15-25), optionally times `scale` in f64 before
    the f32 store (tests/unit/codec.test.ts:12-17)."""
    d = mulberry32_stream(seed, rows * dim)
    v = ((d * 2.0 - 1.0) * scale).astype(np.float32).reshape(rows, dim)
    if normalize:
        normalize_rows_store(v)
    return v


# ------------------------------------------------------------------ rotator
def pad_to_pow2(n: int) -> int:
    """padToPow2 (src/quant/rotator.ts:17-21)."""
    return int(_lib.bvo_pad_to_pow2(n))


def fwht(a) -> np.ndarray:
    """fwht (src/quant/rotator.ts:24-36), returns a transformed copy."""
    a = _f32(a).copy()
    _lib.bvo_fwht(_p(a, f32p), a.size)
    return a


def round_seed(seed: int, r: int) -> int:
    return int(_lib.bvo_round_seed(seed & 0xFFFFFFFF, r))


def rotator_signs(dim: int, seed: int = DEFAULT_SEED, rounds: int = 2) -> np.ndarray:
    """Rotator constructor's per-round +-1/sqrt(P) vectors (rotator.ts:44-58)."""
    P = pad_to_pow2(dim)
    s = np.empty((max(rounds, 1), P), dtype=np.float32)
    _lib.bvo_rotator_signs(dim, seed & 0xFFFFFFFF, rounds, _p(s, f32p))
    return s[:rounds]


def rotate(x, dim: int | None = None, seed: int = DEFAULT_SEED, rounds: int = 2) -> np.ndarray:
    """Rotator.rotateInto for each row of x (rotator.ts:61-70)."""
    x = _f32(np.atleast_2d(x))
    dim = x.shape[1] if dim is None else dim
    P = pad_to_pow2(dim)
    signs = np.ascontiguousarray(rotator_signs(dim, seed, rounds)) if rounds else np.zeros((1, P), np.float32)
    out = np.empty((x.shape[0], P), dtype=np.float32)
    for i in range(x.shape[0]):
        _lib.bvo_rotate(_p(np.ascontiguousarray(x[i]), f32p), dim, _p(signs, f32p), rounds, _p(out[i], f32p))
    return out


# ------------------------------------------------------------------- codecs
def quantize_row(x, bits: int = 8):
    """quantizeRow / quantizeRow4 / quantizeRow1 (src/quant/codec.ts)."""
    x = _f32(x)
    n = x.size
    per = {8: 4, 4: 8, 1: 32}[bits]
    if n % per:
        raise ValueError(f"paddedDim must be a multiple of {per}")
    words = np.zeros(n // per, dtype=np.uint32)
    fn = {8: _lib.bvo_quantize_row8, 4: _lib.bvo_quantize_row4, 1: _lib.bvo_quantize_row1}[bits]
    scale = fn(_p(x, f32p), n, _p(words, u32p))
    return words, np.float32(scale)


def dequant_row(words, scale: float, bits: int = 8) -> np.ndarray:
    words = _u32(words)
    per = {8: 4, 4: 8, 1: 32}[bits]
    out = np.empty(words.size * per, dtype=np.float32)
    fn = {8: _lib.bvo_dequant_row8, 4: _lib.bvo_dequant_row4, 1: _lib.bvo_dequant_row1}[bits]
    fn(_p(words, u32p), words.size, float(scale), _p(out, f32p))
    return out


def encode(data, dim: int, bits: int = 8, seed: int = DEFAULT_SEED, rounds: int = 2, want_rotated: bool = False):
    """BatchEncoder.encode (src/quant/encode.ts:54-78)."""
    data = _f32(data).reshape(-1)
    count = data.size // dim
    P = pad_to_pow2(dim)
    wpr = P // {8: 4, 4: 8, 1: 32}[bits]
    words = np.zeros((count, wpr), dtype=np.uint32)
    scales = np.zeros(count, dtype=np.float32)
    rot = np.zeros((count, P), dtype=np.float32) if want_rotated else None
    _lib.bvo_encode(_p(data, f32p), count, dim, seed & 0xFFFFFFFF, rounds, bits, _p(words, u32p),
                    _p(scales, f32p), _p(rot, f32p))
    return words, scales, rot


# -------------------------------------------------------------------- store
def normalize(v) -> np.ndarray:
    """normalizeInPlace (src/store/store.ts:209-217) on a copy."""
    v = _f32(v).copy()
    _lib.bvo_normalize(_p(v, f32p), v.size)
    return v


def normalize_rows_store(m: np.ndarray) -> np.ndarray:
    """normalizeInPlace applied to every row of m, in place."""
    assert m.dtype == np.float32 and m.flags["C_CONTIGUOUS"]
    _lib.bvo_normalize_many(_p(m, f32p), m.shape[0], m.shape[1])
    return m


def dot_row(row, q) -> float:
    """Store.dotRow (src/store/store.ts:114-130), the f64 result."""
    row, q = _f32(row), _f32(q)
    return float(_lib.bvo_dot_row(_p(row, f32p), _p(q, f32p), row.size))


def l2_row(row, q) -> float:
    """Store.l2Row (src/store/store.ts:137-160), the f64 result."""
    row, q = _f32(row), _f32(q)
    return float(_lib.bvo_l2_row(_p(row, f32p), _p(q, f32p), row.size))


def rerank_scores(rows: np.ndarray, q, cand) -> np.ndarray:
    """rerankExact's f32(dotRow) per candidate (src/index.ts:583-594)."""
    rows, q, cand = _f32(rows), _f32(q), _u32(cand)
    out = np.empty(cand.size, dtype=np.float32)
    _lib.bvo_rerank_scores(_p(rows, f32p), rows.shape[1], _p(q, f32p), _p(cand, u32p), cand.size, _p(out, f32p))
    return out


# -------------------------------------------------------------------- scans
def scan_f32(corpus, q, metric: str = "cosine") -> np.ndarray:
    """fp32 distance kernel scores (src/engine/wgsl/distance.ts:24-191)."""
    corpus, q = _f32(corpus), _f32(q)
    out = np.empty(corpus.shape[0], dtype=np.float32)
    _lib.bvo_scan_f32(_p(corpus, f32p), corpus.shape[0], corpus.shape[1], _p(q, f32p),
                      2 if metric == "l2" else 0, _p(out, f32p))
    return out


def scan_quant(codes, scales, q_rot, bits: int, cand=None) -> np.ndarray:
    """distanceQ8 / Q4 / Q1 asymmetric scores (src/engine/wgsl/distanceQ*.ts)."""
    codes, scales, q_rot = _u32(codes), _f32(scales), _f32(q_rot)
    cand = None if cand is None else _u32(cand)
    n = codes.shape[0] if cand is None else cand.size
    P = q_rot.size
    out = np.empty(n, dtype=np.float32)
    fn = {8: _lib.bvo_scan_q8, 4: _lib.bvo_scan_q4, 1: _lib.bvo_scan_q1}[bits]
    fn(_p(codes, u32p), _p(scales, f32p), n, P, _p(q_rot, f32p), _p(cand, u32p), _p(out, f32p))
    return out


def query_bits(q_rot) -> np.ndarray:
    q_rot = _f32(q_rot)
    out = np.empty(q_rot.size // 32, dtype=np.uint32)
    _lib.bvo_query_bits(_p(q_rot, f32p), q_rot.size, _p(out, u32p))
    return out


def scan_hamming(codes, P: int, qbits, cand=None) -> np.ndarray:
    codes, qbits = _u32(codes), _u32(qbits)
    cand = None if cand is None else _u32(cand)
    n = codes.shape[0] if cand is None else cand.size
    out = np.empty(n, dtype=np.int32)
    _lib.bvo_scan_hamming(_p(codes, u32p), n, P, _p(qbits, u32p), _p(cand, u32p), _p(out, i32p))
    return out


def scan_int8sym(codes, P: int, qcodes, cand=None) -> np.ndarray:
    codes, qcodes = _u32(codes), _u32(qcodes)
    cand = None if cand is None else _u32(cand)
    n = codes.shape[0] if cand is None else cand.size
    out = np.empty(n, dtype=np.int32)
    _lib.bvo_scan_int8sym(_p(codes, u32p), n, P, _p(qcodes, u32p), _p(cand, u32p), _p(out, i32p))
    return out


def dot_exact(a, b):
    """long double sum_i a_i b_i and sum_i |a_i b_i| per row of a."""
    a, b = _f32(np.atleast_2d(a)), _f32(b)
    dot = np.empty(a.shape[0]); mag = np.empty(a.shape[0])
    _lib.bvo_dot_exact(_p(a, f32p), _p(b, f32p), a.shape[0], a.shape[1], _p(dot, f64p), _p(mag, f64p))
    return dot, mag


# ----------------------------------------------------- CPU baseline (wasm)
def wasm_scan(corpus, q, metric: str = "cosine", scalar: bool = False) -> np.ndarray:
    """Lane-exact restatement of kernel.wat dot / l2 (src/fallback/kernel.wat:6-83)."""
    corpus, q = _f32(corpus), _f32(q)
    out = np.empty(corpus.shape[0], dtype=np.float32)
    if scalar:
        fn = _lib.bvo_wasm_dot_scalar
    else:
        fn = _lib.bvo_wasm_l2 if metric == "l2" else _lib.bvo_wasm_dot
    fn(_p(corpus, f32p), _p(q, f32p), _p(out, f32p), corpus.shape[0], corpus.shape[1])
    return out


# -------------------------------------------------------------------- top-k
def topk_ref(scores, k: int):
    """topK with the reference's tie semantics (src/index/flat.ts:217-239)."""
    scores = _f32(scores)
    n = scores.size
    m = min(k, n)
    rows = np.empty(max(m, 1), dtype=np.uint32); out = np.empty(max(m, 1), dtype=np.float32)
    c = _lib.bvo_topk_ref(_p(scores, f32p), n, k, _p(rows, u32p), _p(out, f32p))
    return rows[:c].copy(), out[:c].copy()


def merge_partials(scores, rows, n: int, k: int):
    """mergePartials (src/index/gpuTopk.ts:160-189)."""
    scores, rows = _f32(scores), _u32(rows)
    m = max(min(k, n), 1)
    r = np.empty(m, dtype=np.uint32); s = np.empty(m, dtype=np.float32)
    c = _lib.bvo_merge_partials(_p(scores, f32p), _p(rows, u32p), scores.size, n, k, _p(r, u32p), _p(s, f32p))
    return r[:c].copy(), s[:c].copy()


def topk_canonical(scores, k: int, ids=None, floor: float = -np.inf):
    """Top-k ordered by (score desc, row asc); entries <= floor dropped."""
    scores = _f32(scores)
    ids = None if ids is None else _u32(ids)
    n = scores.size
    m = max(min(k, n), 1)
    r = np.empty(m, dtype=np.uint32); s = np.empty(m, dtype=np.float32)
    c = _lib.bvo_topk_canonical(_p(scores, f32p), _p(ids, u32p), n, k, float(floor), _p(r, u32p), _p(s, f32p))
    return r[:c].copy(), s[:c].copy()


# ------------------------------------------------------------------ k-means
def normalize_rows(m) -> np.ndarray:
    """normalizeRows (src/index/kmeans.ts:211-219) on a copy."""
    m = _f32(np.atleast_2d(m)).copy()
    _lib.bvo_normalize_rows(_p(m, f32p), m.shape[0], m.shape[1])
    return m


def random_init_centroids(sample, nlist: int, seed: int) -> np.ndarray:
    """randomInitCentroids (src/index/kmeans.ts:154-170)."""
    sample = _f32(sample)
    out = np.empty((nlist, sample.shape[1]), dtype=np.float32)
    _lib.bvo_random_init_centroids(_p(sample, f32p), sample.shape[0], nlist, sample.shape[1], seed & 0xFFFFFFFF,
                                   _p(out, f32p))
    return out


def update_centroids(sample, assign, centroids, seed: int):
    """updateCentroids (src/index/kmeans.ts:177-209); returns (centroids, counts)."""
    sample, assign = _f32(sample), _u32(assign)
    c = _f32(centroids).copy()
    counts = np.empty(c.shape[0], dtype=np.int32)
    _lib.bvo_update_centroids(_p(sample, f32p), sample.shape[0], _p(assign, u32p), _p(c, f32p), c.shape[0],
                              c.shape[1], seed & 0xFFFFFFFF, _p(counts, i32p))
    return c, counts


def assign_f32(rows, centroids, order: int = 0) -> np.ndarray:
    """argmax-dot assignment (src/engine/wgsl/assign.ts:31-58); order 0 = the
    reference kernel's dot4 groups, 1 = one sequential FMA chain (vectorized
    across centroids when the CPU has AVX2 + FMA), 2 = the same chain on the
    scalar path."""
    rows, centroids = _f32(rows), _f32(centroids)
    out = np.empty(rows.shape[0], dtype=np.uint32)
    _lib.bvo_assign_f32(_p(rows, f32p), rows.shape[0], _p(centroids, f32p), centroids.shape[0], rows.shape[1],
                        order, _p(out, u32p))
    return out


def assign_quant(codes, scales, P: int, bits: int, centroids) -> np.ndarray:
    """Quantized assignment (assignQ8.ts / assignQ4.ts / assignQ1.ts)."""
    codes, scales, centroids = _u32(codes), _f32(scales), _f32(centroids)
    out = np.empty(codes.shape[0], dtype=np.uint32)
    _lib.bvo_assign_quant(_p(codes, u32p), _p(scales, f32p), codes.shape[0], P, bits, _p(centroids, f32p),
                          centroids.shape[0], _p(out, u32p))
    return out


def probe_scores(centroids, rq) -> np.ndarray:
    """pickProbes' f32 scores (src/index/ivfquant.ts:495-511)."""
    centroids, rq = _f32(centroids), _f32(rq)
    out = np.empty(centroids.shape[0], dtype=np.float32)
    _lib.bvo_probe_scores(_p(centroids, f32p), centroids.shape[0], centroids.shape[1], _p(rq, f32p), _p(out, f32p))
    return out


def build_csr(cluster, nlist: int):
    """CSR lists (src/index/ivfquant.ts:297-305)."""
    cluster = _u32(cluster)
    offset = np.empty(nlist + 1, dtype=np.int32)
    rows = np.empty(max(cluster.size, 1), dtype=np.int32)
    _lib.bvo_build_csr(_p(cluster, u32p), cluster.size, nlist, _p(offset, i32p), _p(rows, i32p))
    return offset, rows[: cluster.size]


def choose_nprobe(ranks, nlist: int, target: float):
    """chooseNprobe (src/index/ivfTune.ts:31-42) -> (nprobe, recall)."""
    ranks = _u32(ranks)
    rec = ctypes.c_double(0.0)
    n = _lib.bvo_choose_nprobe(_p(ranks, u32p), ranks.size, nlist, float(target), ctypes.byref(rec))
    return int(n), float(rec.value)


def pick_tune_queries(filled: int, want: int):
    out = np.empty(max(want, 1), dtype=np.uint32)
    n = _lib.bvo_pick_tune_queries(filled, want, _p(out, u32p))
    return [int(x) for x in out[:n]]


class Reservoir:
    """Reservoir sampler (src/index/ivfquant.ts:112-124, 235-245)."""

    def __init__(self, cap: int, seed: int):
        self.cap = cap
        self.filled = ctypes.c_uint64(0)
        self.seen = ctypes.c_uint64(0)
        self.rng = ctypes.c_uint32(seed & 0xFFFFFFFF)

    def slot(self) -> int:
        return int(_lib.bvo_reservoir_slot(self.cap, ctypes.byref(self.filled), ctypes.byref(self.seen),
                                           ctypes.byref(self.rng)))


# ------------------------------------------------------------- graph search
GRAPH_EF = 256
GRAPH_EMPTY = 0xFFFFFFFF


def graph_entries(entry: int, graph_rows: int) -> np.ndarray:
    """HNSWGpuSearcher.search's seed rows (src/index/hnswGpu.ts:142-150)."""
    out = np.empty(8, np.uint32)
    n = _lib.bvo_graph_entries(int(entry) & 0xFFFFFFFF, int(graph_rows), _p(out, u32p))
    return out[:n].copy()


def graph_search(corpus, graph, queries, entries, ef: int, iter_cap: int, l2: bool = False):
    """The beam-search shader (src/engine/wgsl/graphSearch.ts:62-259), lanes in
    lane order: (dist [nq, 256], id [nq, 256]) beams.  graph: [graph_rows, K]
    adjacency over the first graph_rows rows of corpus."""
    corpus, queries = _f32(corpus), _f32(np.atleast_2d(queries))
    graph, entries = _u32(graph), _u32(entries)
    nq, dim = queries.shape
    K = graph.shape[1]
    dist = np.empty((nq, GRAPH_EF), np.float32)
    ids = np.empty((nq, GRAPH_EF), np.uint32)
    _lib.bvo_graph_search(_p(corpus, f32p), dim, 1 if l2 else 0, _p(graph, u32p), K, graph.shape[0],
                          corpus.shape[0], _p(queries, f32p), nq, _p(entries, u32p), entries.size, int(ef),
                          int(iter_cap), _p(dist, f32p), _p(ids, u32p))
    return dist, ids


def graph_hits(dist, ids, ef_active: int, k: int):
    """The searcher's dedup + stable sort + top-k of one beam
    (src/index/hnswGpu.ts:191-203): (rows, scores)."""
    dist, ids = _f32(dist), _u32(ids)
    rows = np.empty(max(k, 1), np.uint32)
    scores = np.empty(max(k, 1), np.float32)
    n = _lib.bvo_graph_hits(_p(dist, f32p), _p(ids, u32p), int(ef_active), int(k), _p(rows, u32p), _p(scores, f32p))
    return rows[:n].copy(), scores[:n].copy()
