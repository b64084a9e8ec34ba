"""GPU parity: the HIP path against the CPU oracle on identical seeded inputs.

Bars (stated per check):
  * codes, scales, rotated queries, Hamming / int8-symmetric scores,
    re-rank scores and top-k selection over the device's own scores:
    bit-exact;
  * fp32 scan scores: |gpu - oracle| <= 1e-5 * sum_i |term_i| (REL_TOL);
  * top-k ID sets vs the oracle: identical except rows within the score
    tolerance of the k-th score (near-ties).
"""

import numpy as np
import pytest

from oracle import oracle as o
from tests.helpers import (REL_TOL, assert_fetch_rerank, assert_scores_close, assert_topk_near, clustered, gaussian,
                           need_gpu, quant_magnitude, say)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    from browservec_amd import DeviceContext

    c = DeviceContext(0)
    yield c
    c.destroy()


def _special_rows(dim):
    rows = [np.zeros(dim, np.float32)]
    t = np.full(dim, 1e-9, np.float32)
    t[0] = 1.0
    rows.append(t)  # tiny coordinates: exercises the sequential 1-bit sum
    e = np.zeros(dim, np.float32)
    e[dim // 2] = -1.0
    rows.append(e)
    d = np.full(dim, 3e-39, np.float32)  # subnormal coordinates
    d[1::3] = -1e-45
    rows.append(d)
    n = np.linspace(-1, 1, dim, dtype=np.float32)
    n[dim // 3] = np.nan  # NaN never raises the max; NaN codes store as 0
    rows.append(n)
    f = np.linspace(1, -1, dim, dtype=np.float32)
    f[1] = np.inf  # infinite scale: finite coordinates code to 0
    rows.append(f)
    return np.stack(rows)


ENCODE_CASES = [(100, 8), (100, 4), (100, 1), (384, 8), (384, 4), (384, 1), (768, 8), (768, 4), (768, 1),
                (1024, 8), (1024, 1), (48, 8), (40, 8), (33, 1), (2000, 8), (2000, 1)]


@pytest.mark.parametrize("dim,bits", ENCODE_CASES)
def test_encode_bit_exact(ctx, dim, bits):
    from browservec_amd import QuantIndex

    say("encode", dim, bits)
    data = np.concatenate([gaussian(257, dim, 7 + dim), o.uniform_vectors(40, dim, 3), _special_rows(dim)])
    idx = QuantIndex(ctx, dim, seed=o.DEFAULT_SEED, rounds=2, bits=bits)
    idx.append(data[:100], 100)
    idx.append(data[100:], data.shape[0] - 100)  # second append: offsets
    words, scales = idx.export_codes()
    want_w, want_s, _ = o.encode(data, dim, bits)
    assert np.array_equal(words, want_w)
    assert np.array_equal(scales.view(np.uint32), want_s.view(np.uint32))
    q = gaussian(1, dim, 99)[0]
    assert np.array_equal(idx.export_rotated_query(q).view(np.uint32), o.rotate(q, dim)[0].view(np.uint32))
    idx.destroy()


def test_encode_seed_and_rounds(ctx):
    from browservec_amd import QuantIndex

    say("encode seed/rounds")
    data = gaussian(64, 200, 5)
    for seed, rounds in ((12345, 1), (99, 3)):
        idx = QuantIndex(ctx, 200, seed=seed, rounds=rounds, bits=8)
        idx.append(data, 64)
        w, s = idx.export_codes()
        ww, ss, _ = o.encode(data, 200, 8, seed=seed, rounds=rounds)
        assert np.array_equal(w, ww) and np.array_equal(s, ss)
        idx.destroy()


# 1-bit asym covers every layout path of the bit-plane scan: P = 128 (one
# unit, query layout built by its own kernel), 512 and 1024 (built inside the
# scan), 2048 (own kernel, 16 lanes per row); P = 64 keeps the plain fp32 sum
SCAN_CASES = [(768, 8, "asym"), (384, 8, "asym"), (768, 4, "asym"), (1024, 4, "asym"), (768, 1, "asym"),
              (1024, 1, "asym"), (100, 1, "asym"), (400, 1, "asym"), (2000, 1, "asym"), (48, 1, "asym"),
              (1024, 1, "hamming"), (768, 8, "int8sym"), (2048, 8, "asym")]


@pytest.mark.parametrize("dim,bits,scorer", SCAN_CASES)
def test_quant_scan_scores_and_topk(ctx, dim, bits, scorer):
    from browservec_amd import QuantIndex

    say("quant scan", dim, bits, scorer)
    n = 6000
    data = clustered(n, dim, 64, 0.1, dim + bits)
    idx = QuantIndex(ctx, dim, bits=bits, scorer=scorer)
    idx.append(data, n)
    codes, scales = idx.export_codes()
    P = idx.padded_dim
    for qi, q in enumerate(data[[5, 777]] + gaussian(2, dim, 3, normalize=False) * 0.05):
        q = o.normalize(q)
        dense = idx.export_scores(q)
        q_rot = o.rotate(q, dim)[0]
        if scorer == "hamming":
            want = o.scan_hamming(codes, P, o.query_bits(q_rot)).astype(np.float32)
            assert np.array_equal(dense, want)
            tol = 0.0
        elif scorer == "int8sym":
            qc, _ = o.quantize_row(q_rot, 8)
            want = o.scan_int8sym(codes, P, qc).astype(np.float32)
            assert np.array_equal(dense, want)
            tol = 0.0
        else:
            want = o.scan_quant(codes, scales, q_rot, bits)
            mag = quant_magnitude(codes, scales, q_rot, bits)
            assert_scores_close(dense, want, mag, f"q{qi}")
            tol = 2 * REL_TOL * float(mag.max())
        for k in (1, 10, 100, 250):
            hits = idx.query(q, k)
            rows = np.array([h.row for h in hits], np.uint32)
            sc = np.array([h.score for h in hits], np.float32)
            # selection over the device's own scores is exact and canonical
            er, es = o.topk_canonical(dense, k)
            assert np.array_equal(rows, er), (k, rows[:5], er[:5])
            assert np.array_equal(sc.view(np.uint32), es.view(np.uint32))
            assert_topk_near(rows, want, k, tol, f"k={k}")
    idx.destroy()


@pytest.mark.parametrize("dim,metric", [(768, "cosine"), (768, "dot"), (768, "l2"), (384, "cosine"),
                                        (67, "cosine"), (67, "l2"), (100, "dot"), (1024, "l2"), (3, "l2")])
def test_flat_scan(ctx, dim, metric):
    from browservec_amd import FlatIndex

    say("flat", dim, metric)
    n = 5000
    data = gaussian(n, dim, dim, normalize=(metric == "cosine"))
    idx = FlatIndex(ctx, dim, metric)
    idx.append(data, n)
    for qi in range(3):
        q = gaussian(1, dim, 1000 + qi, normalize=(metric == "cosine"))[0]
        dense = idx.export_scores(q)
        want = o.scan_f32(data, q, metric)
        if metric == "l2":
            d = data.astype(np.float64) - q
            mag = (d * d).sum(1)
        else:
            _, mag = o.dot_exact(data, q)
        assert_scores_close(dense, want, mag, f"{metric} q{qi}")
        for k in (1, 10, 64):
            hits = idx.query(q, k)
            rows = np.array([h.row for h in hits], np.uint32)
            er, _ = o.topk_canonical(dense, k)
            assert np.array_equal(rows, er)
            assert_topk_near(rows, want, k, 2 * REL_TOL * float(mag.max()), metric)
    idx.destroy()


def test_flat_matches_wasm_baseline_top10(ctx):
    """Config-1 shape scaled to the test budget: 20,000 x 384 cosine, the GPU
    top-10 IDs equal the CPU baseline's (kernel.wat restatement) except
    near-ties."""
    from browservec_amd import FlatIndex

    say("flat vs wasm baseline")
    data = gaussian(20000, 384, 1)
    qs = gaussian(20, 384, 2)
    idx = FlatIndex(ctx, 384, "cosine")
    idx.append(data, 20000)
    for q in qs:
        base = o.wasm_scan(data, q)
        hits = idx.query(q, 10)
        assert_topk_near([h.row for h in hits], base, 10, 2e-5)
    idx.destroy()


def test_rerank_bit_exact(ctx):
    from browservec_amd import QuantIndex

    say("rerank")
    dim = 768
    data = gaussian(3000, dim, 11)
    idx = QuantIndex(ctx, dim, bits=8)
    idx.append(data, 3000)
    q = gaussian(1, dim, 12)[0]
    cand = np.random.default_rng(0).choice(3000, 300, replace=False).astype(np.uint32)
    hits = idx.rerank(q, cand, 50)
    want = o.rerank_scores(data, q, cand)
    er, es = o.topk_canonical(want, 50, ids=cand)
    assert [h.row for h in hits] == er.tolist()
    assert np.array_equal(np.array([h.score for h in hits], np.float32).view(np.uint32), es.view(np.uint32))
    # odd dimension: scalar tail after the four accumulators
    idx2 = QuantIndex(ctx, 771, bits=8)
    d2 = gaussian(500, 771, 13)
    idx2.append(d2, 500)
    q2 = gaussian(1, 771, 14)[0]
    c2 = np.arange(0, 500, 3, dtype=np.uint32)
    h2 = idx2.rerank(q2, c2, 20)
    w2 = o.rerank_scores(d2, q2, c2)
    r2, s2 = o.topk_canonical(w2, 20, ids=c2)
    assert [h.row for h in h2] == r2.tolist()
    assert np.array_equal(np.array([h.score for h in h2], np.float32), s2)
    idx.destroy()
    idx2.destroy()


@pytest.mark.parametrize("bits,fetch", [(8, 100), (4, 200), (1, 200)])
def test_search_fetch_then_rerank(ctx, bits, fetch):
    """The quantized query path: approximate top-fetch by code score, exact f64
    re-rank, top-10 (src/index.ts:414-418)."""
    from browservec_amd import QuantIndex

    say("search", bits, fetch)
    dim, n = 768, 20000
    data = clustered(n, dim, 128, 0.1, 21)
    idx = QuantIndex(ctx, dim, bits=bits)
    idx.append(data, n)
    codes, scales = idx.export_codes()
    qs = data[[3, 4000, 19999]] + gaussian(3, dim, 22, normalize=False) * 0.05
    qs = np.stack([o.normalize(q) for q in qs])
    rows, scores, cnt = idx.search(qs, fetch, 10)
    for i, q in enumerate(qs):
        assert cnt[i] == 10
        q_rot = o.rotate(q, dim)[0]
        approx = o.scan_quant(codes, scales, q_rot, bits)
        mag = quant_magnitude(codes, scales, q_rot, bits)
        # every returned score is the exact f64 dotRow of that row
        exact = o.rerank_scores(data, q, rows[i])
        assert np.array_equal(scores[i].view(np.uint32), exact.view(np.uint32))
        # and the result is the oracle pipeline's (top-fetch by code score,
        # exact re-rank, canonical top-10) up to near-ties at the fetch boundary
        tol = 2 * REL_TOL * max(float(mag.max()), float(np.abs(approx).max()))
        assert_fetch_rerank(rows[i], scores[i], approx, np.arange(n), lambda rr: o.rerank_scores(data, q, rr),
                            fetch, 10, tol, what=f"bits {bits} query {i}")
    idx.destroy()


def test_masked_queries(ctx):
    from browservec_amd import FlatIndex, QuantIndex

    say("masked")
    dim, n = 384, 7000
    data = gaussian(n, dim, 31)
    rng = np.random.default_rng(4)
    keep = rng.random(n) < 0.3
    words = np.zeros((n + 31) // 32, np.uint32)
    for r in np.nonzero(keep)[0]:
        words[r >> 5] |= np.uint32(1 << (r & 31))
    for idx in (FlatIndex(ctx, dim, "cosine"), QuantIndex(ctx, dim, bits=8), QuantIndex(ctx, dim, bits=1)):
        idx.append(data, n)
        q = gaussian(1, dim, 32)[0]
        dense = idx.export_scores(q)
        hits = idx.query_masked(q, 50, words)
        rows = np.array([h.row for h in hits], np.uint32)
        assert keep[rows].all()
        er, _ = o.topk_canonical(dense[keep], 50, ids=np.nonzero(keep)[0].astype(np.uint32))
        assert np.array_equal(rows, er)
        # fewer matching rows than k: only the matching rows come back
        few = np.zeros_like(words)
        few[0] = 0b1011
        hits = idx.query_masked(q, 10, few)
        assert sorted(h.row for h in hits) == [0, 1, 3]
        idx.destroy()


def test_edge_cases(ctx):
    from browservec_amd import FlatIndex, QuantIndex, _lib
    from browservec_amd._lib import BVError

    say("edges")
    idx = FlatIndex(ctx, 16, "cosine")
    assert idx.query(np.ones(16, np.float32), 5) == []  # empty index -> []
    with pytest.raises(BVError, match="expected 32 floats, got 31"):
        idx.append(np.ones(31, np.float32), 2)
    x = gaussian(7, 16, 1)
    idx.append(x, 7)
    hits = idx.query(x[2], 10)  # k > n
    assert len(hits) == 7 and hits[0].row == 2
    assert idx.query(x[2], 0) == []
    # exact duplicates: ties ordered by row
    dup = np.repeat(gaussian(1, 16, 9), 12, axis=0)
    idx2 = FlatIndex(ctx, 16, "dot")
    idx2.append(np.concatenate([gaussian(5, 16, 2), dup]), 17)
    hits = idx2.query(dup[0], 12)
    assert [h.row for h in hits] == list(range(5, 17))
    # fetch beyond the fused top-k capacity falls back to dense selection
    idx3 = QuantIndex(ctx, 64, bits=8)
    d3 = gaussian(3000, 64, 5)
    idx3.append(d3, 3000)
    q = gaussian(1, 64, 6)[0]
    hits = idx3.query(q, 1500)
    er, _ = o.topk_canonical(idx3.export_scores(q), 1500)
    assert [h.row for h in hits] == er.tolist()
    # the reference's rejections
    with pytest.raises(BVError) as e:
        QuantIndex(ctx, 64, bits=8, metric="l2")
    assert e.value.code == _lib.BV_E_UNSUPPORTED
    for i in (idx, idx2, idx3):
        i.destroy()


@pytest.mark.parametrize("bits", [8, 1])
def test_batch_equals_singles(ctx, bits):
    from browservec_amd import QuantIndex

    say("batch", bits)
    dim = 256
    data = gaussian(4000, dim, 41)
    idx = QuantIndex(ctx, dim, bits=bits)
    idx.append(data, 4000)
    qs = gaussian(70, dim, 42)
    batch = idx.query_batch(qs, 70, 15)
    for i in range(70):
        assert batch[i] == idx.query(qs[i], 15)
    rows, scores, cnt = idx.search(qs, 60, 10)
    for i in (0, 33, 69):
        r1, s1, _ = idx.search(qs[i:i + 1], 60, 10)
        assert np.array_equal(rows[i], r1[0]) and np.array_equal(scores[i], s1[0])
    idx.destroy()


def test_browservec_api(ctx):
    """BrowserVec orchestration over the native index: create / addBatch /
    query / queryBatch / delete / filter, against exact brute force
    (tests/browser/gpu.test.ts:14-112 restated)."""
    from browservec_amd import BrowserVec

    say("BrowserVec")
    dim = 64
    vecs = o.uniform_vectors(1000, dim, 1)
    for quant_bits in (0, 8):
        db = BrowserVec.create(dimension=dim, metric="cosine", quantBits=quant_bits)
        db.add_batch([{"id": f"v{i}", "vector": vecs[i], "metadata": {"even": i % 2 == 0}} for i in range(1000)])
        normed = vecs.copy()
        o.normalize_rows_store(normed)
        q = o.uniform_vectors(1, dim, 77)[0]
        qn = o.normalize(q)
        exact = np.array([o.dot_row(normed[i], qn) for i in range(1000)], np.float32)
        want, _ = o.topk_canonical(exact, 10)
        res = db.query(q, k=10)
        got = [int(r["id"][1:]) for r in res]
        if quant_bits == 0:
            assert_topk_near(got, exact, 10, 2e-5)
        else:
            assert len(set(got) & set(want.tolist())) >= 9  # recall floor (gpu.test.ts:158-184)
        batch = db.query_batch([q, q], k=10)
        assert batch[0] == batch[1] == res
        db.delete(res[0]["id"])
        res2 = db.query(q, k=10)
        assert res[0]["id"] not in [r["id"] for r in res2] and len(res2) == 10
        filt = db.query(q, k=5, filter=lambda m: m is not None and m["even"])
        assert all(int(r["id"][1:]) % 2 == 0 for r in filt) and len(filt) == 5
        # 499 matching rows take queryRowsExact: exact dotRow scores, top 5
        even = np.array([i for i in range(0, 1000, 2) if f"v{i}" != res[0]["id"]], np.uint32)
        wr, ws = o.topk_canonical(exact[even], 5, even)
        assert [int(r["id"][1:]) for r in filt] == wr.tolist()
        assert [r["score"] for r in filt] == ws.tolist()
        st = db.stats()
        assert st["count"] == 999 and st["deleted"] == 1
        db.destroy()


@pytest.mark.parametrize("bits", [8, 0])
def test_topk_when_best_rows_share_a_workgroup(ctx, bits):
    """The 300 best rows sit next to each other, so one workgroup holds far
    more of the top-k than its local list keeps; the merge must rescan it and
    still return the exact top-k of the device's scores."""
    from browservec_amd import FlatIndex, QuantIndex

    say("concentrated top-k", bits)
    dim, n = 256, 100_000
    rng = np.random.default_rng(8)
    q = gaussian(1, dim, 81)[0]
    data = gaussian(n, dim, 82)
    near = q[None, :] + 0.02 * rng.standard_normal((300, dim)).astype(np.float32)
    o.normalize_rows_store(near)
    data[1000:1300] = near
    idx = QuantIndex(ctx, dim, bits=8) if bits else FlatIndex(ctx, dim, "cosine")
    idx.append(data, n)
    dense = idx.export_scores(q)
    for k in (100, 250, 17):
        hits = idx.query(q, k)
        er, es = o.topk_canonical(dense, k)
        assert [h.row for h in hits] == er.tolist(), k
    if bits:
        rows, scores, cnt = idx.search(q[None], 200, 10)
        exact = o.rerank_scores(data, q, rows[0])
        assert np.array_equal(exact, scores[0])
        assert set(rows[0].tolist()) <= set(range(1000, 1300))
    idx.destroy()


def _mixture_1m(n, dim, nclusters, sigma, seed):
    """The headline workload's corpus shape: unit-norm centres + sigma N(0,1),
    rows normalized (generated in blocks to bound host memory)."""
    rng = np.random.default_rng(seed)
    centres = rng.standard_normal((nclusters, dim), dtype=np.float32)
    o.normalize_rows_store(centres)
    x = np.empty((n, dim), np.float32)
    for s in range(0, n, 100_000):
        e = min(n, s + 100_000)
        lab = rng.integers(0, nclusters, e - s)
        x[s:e] = centres[lab] + sigma * rng.standard_normal((e - s, dim), dtype=np.float32)
    return o.normalize_rows_store(x)


def test_int8_1m_rows_fetch_rerank_matches_oracle(ctx):
    """1,000,000 x 768 int8 (P = 1024), fetch 100 -> exact re-rank -> top 10:
    the headline shape, where the grid reaches its workgroup cap and the
    dynamic share of the rows is handed out by tickets.  Single queries equal
    the oracle pipeline (top 100 by code score, exact re-rank, canonical top
    10) up to fetch-boundary near-ties; an eight-query batch (matrix-core
    path) equals the single queries bit for bit.  The same at fetch 1024 and
    k 32, where the scan's grid and bound take their large-fetch forms."""
    from browservec_amd import QuantIndex

    n, dim, fetch, k = 1_000_000, 768, 100, 10
    say("1M x 768 int8: data")
    data = _mixture_1m(n, dim, 1024, 0.1, 0xB5EC0101)
    idx = QuantIndex(ctx, dim, bits=8)
    idx.append(data, n)
    say("1M x 768 int8: codes")
    for r0 in (0, 499_000, n - 1000):  # sampled blocks bit-exact against the oracle's encode
        w, sc = idx.export_codes(r0, 1000)
        ww, ss, _ = o.encode(data[r0:r0 + 1000], dim, 8)
        assert np.array_equal(w, ww) and np.array_equal(sc.view(np.uint32), ss.view(np.uint32)), r0
    words, scales = idx.export_codes()
    rng = np.random.default_rng(0xB5EC0102)
    pick = rng.integers(0, n, 8)
    qs = data[pick] + 0.05 * rng.standard_normal((8, dim), dtype=np.float32)
    qs = np.stack([o.normalize(q) for q in qs]).astype(np.float32)
    singles = [idx.search(qs[i:i + 1], fetch, k) for i in range(8)]
    say("1M x 768 int8: batch of 8")
    br, bs, bc = idx.search(qs, fetch, k)
    for i in range(8):
        r1, s1, c1 = singles[i]
        assert bc[i] == c1[0] == k
        assert np.array_equal(br[i], r1[0]) and np.array_equal(bs[i].view(np.uint32), s1[0].view(np.uint32)), i
    smax = float(scales.max())
    for i in range(4):
        say("1M x 768 int8: oracle query", i)
        rq = o.rotate(qs[i], dim)[0]
        approx = o.scan_quant(words, scales, rq, 8)
        tol = 2 * REL_TOL * smax * float(np.abs(rq.astype(np.float64)).sum())
        r1, s1, _ = singles[i]
        assert_fetch_rerank(r1[0], s1[0], approx, np.arange(n), lambda rr, q=qs[i]: o.rerank_scores(data, q, rr),
                            fetch, k, tol, what=f"1M query {i}")
        if i < 2:
            # fetch 1024, k 32: the per-wave lists leave room for one workgroup
            # per CU (a smaller grid) and the waves publish their four best
            # lane maxima, so the threshold helper still forms its bound
            say("1M x 768 int8: fetch 1024, query", i)
            rw, sw, cw = idx.search(qs[i:i + 1], 1024, 32)
            assert cw[0] == 32
            assert_fetch_rerank(rw[0], sw[0], approx, np.arange(n),
                                lambda rr, q=qs[i]: o.rerank_scores(data, q, rr), 1024, 32, tol,
                                what=f"1M query {i} fetch 1024")
    say("1M x 768 int8: batch of 8, fetch 1024")
    wide = [idx.search(qs[i:i + 1], 1024, 32) for i in range(8)]
    br, bs, bc = idx.search(qs, 1024, 32)
    for i in range(8):
        r1, s1, c1 = wide[i]
        assert bc[i] == c1[0] == 32
        assert np.array_equal(br[i], r1[0]) and np.array_equal(bs[i].view(np.uint32), s1[0].view(np.uint32)), i
    idx.destroy()


@pytest.mark.parametrize("kind", ["int8", "ivf_int8", "int4_no_rerank"])
def test_browservec_query_batch_takes_one_batched_search(ctx, kind):
    """BrowserVec.queryBatch on a quantized or IVF store answers the batch
    with one device search() call, not a loop of query(), and returns per
    query exactly what query() returns (ids, order and score bits), with
    tombstones skipped and an nprobe option applied to the whole batch
    (src/index.ts:402-421, 473-517)."""
    from browservec_amd import BrowserVec

    say("queryBatch batched", kind)
    dim, n, nq = 96, 6000, 40
    data = clustered(n, dim, 40, 0.1, seed=171)
    if kind == "ivf_int8":
        db = BrowserVec.create(dimension=dim, quantBits=8, ann={"type": "ivf", "nlist": 24, "iters": 3, "nprobe": 4})
    else:
        db = BrowserVec.create(dimension=dim, quantBits=8 if kind == "int8" else 4)
    db.add_vectors([f"v{i}" for i in range(n)], data)
    qs = data[np.random.default_rng(172).integers(0, n, nq)] + 0.05 * gaussian(nq, dim, 173, normalize=False)
    db.delete("v17")
    opts = {"rerank": False} if kind == "int4_no_rerank" else {}
    if kind == "ivf_int8":
        opts["nprobe"] = 6
    calls = {"search": 0, "query": 0}
    search, query = db.index.search, db.query

    def counted_search(*a, **kw):
        calls["search"] += 1
        return search(*a, **kw)

    def counted_query(*a, **kw):
        calls["query"] += 1
        return query(*a, **kw)

    db.index.search, db.query = counted_search, counted_query
    batch = db.query_batch(list(qs), k=10, **opts)
    assert calls == {"search": 1, "query": 0}, calls
    db.index.search, db.query = search, query
    if kind == "ivf_int8":
        assert db.index.stats()["nprobe"] == 4  # the override was consumed by the batch
    for i in range(nq):
        single = db.query(qs[i], k=10, **opts)
        assert len(single) == 10 and "v17" not in [r["id"] for r in single]
        assert [r["id"] for r in batch[i]] == [r["id"] for r in single], i
        assert (np.array([r["score"] for r in batch[i]], np.float32).view(np.uint32).tolist() ==
                np.array([r["score"] for r in single], np.float32).view(np.uint32).tolist()), i
    db.destroy()


def test_1bit_asym_large_fetch_matches_oracle(ctx):
    """600,000 x 1024 1-bit asymmetric codes, fetch 1024 -> exact re-rank ->
    top 32 (the reference's re-rank factor 32 at k 32): the bit-plane scan's
    lists and re-score table leave LDS for one workgroup per CU, so the grid
    shrinks to what the device holds and each wave publishes its four best
    lane maxima.  Single queries equal the oracle pipeline (top 1024 by the
    dequantized product, exact re-rank, canonical top 32) up to
    fetch-boundary near-ties, as does fetch 320 (k 10); a batch equals the
    single queries bit for bit."""
    from browservec_amd import QuantIndex

    n, dim = 600_000, 1024
    say("600k x 1024 1-bit asym: data")
    data = _mixture_1m(n, dim, 1024, 0.1, 0xB5EC0201)
    idx = QuantIndex(ctx, dim, bits=1, scorer="asym")
    idx.append(data, n)
    words, scales = idx.export_codes()
    rng = np.random.default_rng(0xB5EC0202)
    pick = rng.integers(0, n, 8)
    qs = data[pick] + 0.05 * rng.standard_normal((8, dim), dtype=np.float32)
    qs = np.stack([o.normalize(q) for q in qs]).astype(np.float32)
    for fetch, k in ((1024, 32), (320, 10)):
        singles = [idx.search(qs[i:i + 1], fetch, k) for i in range(8)]
        say("600k x 1024 1-bit asym: batch of 8, fetch", fetch)
        br, bs, bc = idx.search(qs, fetch, k)
        for i in range(8):
            r1, s1, c1 = singles[i]
            assert bc[i] == c1[0] == k
            assert np.array_equal(br[i], r1[0]) and np.array_equal(bs[i].view(np.uint32), s1[0].view(np.uint32)), i
        for i in range(2):
            say("600k x 1024 1-bit asym: oracle query", i, "fetch", fetch)
            rq = o.rotate(qs[i], dim)[0]
            approx = o.scan_quant(words, scales, rq, 1)
            # every 1-bit code dequantizes to +-1: sum_i |deq_i q_i| * scale
            tol = 2 * REL_TOL * float(np.abs(scales.astype(np.float64)).max()) * float(
                np.abs(rq.astype(np.float64)).sum())
            r1, s1, _ = singles[i]
            assert_fetch_rerank(r1[0], s1[0], approx, np.arange(n),
                                lambda rr, q=qs[i]: o.rerank_scores(data, q, rr), fetch, k, tol,
                                what=f"1-bit query {i} fetch {fetch}")
    idx.destroy()
