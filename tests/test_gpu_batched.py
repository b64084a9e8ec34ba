"""Query batches on the matrix-core paths against the same queries run one at
a time through the fused single-query scan (src/index.ts:473-517: a batch
must answer exactly as its queries would alone).  int8 / int4 keys are formed
by the same f64 combine of exact int32 level dots in both paths; fp32 batches
re-score the matrix-core survivors with the single-query arithmetic.  Rows
and score bits must be identical, including re-ranked scores."""

import numpy as np
import pytest

from oracle import oracle as o
from tests.helpers import clustered, gaussian, need_gpu, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    from browservec_amd import DeviceContext

    c = DeviceContext(0)
    yield c
    c.destroy()


def singles_equal(idx, qs, fetch, k):
    rows, scores, cnt = idx.search(qs, fetch, k)
    for i in range(qs.shape[0]):
        r1, s1, c1 = idx.search(qs[i:i + 1], fetch, k)
        assert cnt[i] == c1[0], i
        assert np.array_equal(rows[i, :cnt[i]], r1[0, :c1[0]]), i
        assert np.array_equal(scores[i, :cnt[i]].view(np.uint32), s1[0, :c1[0]].view(np.uint32)), i
    return rows, scores, cnt


@pytest.mark.parametrize("bits,dim,n,nq", [(8, 768, 40000, 70), (8, 20, 20000, 9), (8, 100, 3000, 64),
                                           (4, 1024, 40000, 40), (4, 100, 20000, 9)])
def test_batched_search_equals_singles(ctx, bits, dim, n, nq):
    from browservec_amd import QuantIndex

    say("batched", bits, dim, n, nq)
    data = clustered(n, dim, 50, 0.1, seed=7 + dim)
    idx = QuantIndex(ctx, dim, bits=bits)
    idx.append(data, n)
    qs = data[np.arange(nq) * (n // nq)] + gaussian(nq, dim, 9, normalize=False) * 0.05
    qs = np.stack([o.normalize(q) for q in qs]).astype(np.float32)
    rows, scores, cnt = singles_equal(idx, qs, 100, 10)
    # the re-ranked scores are Store.dotRow of the returned rows
    for i in (0, nq - 1):
        exact = o.rerank_scores(data, qs[i], rows[i, :cnt[i]])
        assert np.array_equal(scores[i, :cnt[i]].view(np.uint32), exact.view(np.uint32))
    batch = idx.query_batch(qs, nq, 20)
    for i in range(nq):
        assert batch[i] == idx.query(qs[i], 20), i
    idx.destroy()


def test_batched_int8_query_blocks_and_appends(ctx):
    """int8 batches above the sample size score each row on the first query
    level alone, 128 queries per workgroup, with a bound from the row's code
    norm: 300 queries (three blocks, the last partial) over rows appended in
    three calls (the norms of each append's rows), dot metric with rows of
    varied norm, still equal to single queries."""
    from browservec_amd import QuantIndex

    dim, n, nq = 256, 60000, 300
    say("batched int8 blocks/appends")
    data = clustered(n, dim, 80, 0.1, seed=61)
    data = data * np.random.default_rng(62).uniform(0.25, 4.0, (n, 1)).astype(np.float32)
    idx = QuantIndex(ctx, dim, bits=8, metric="dot")
    idx.append(data[:17000], 17000)
    idx.append(data[17000:17001], 1)
    idx.append(data[17001:], n - 17001)
    qs = (data[np.arange(nq) * 199] + gaussian(nq, dim, 63, normalize=False) * 0.05).astype(np.float32)
    singles_equal(idx, qs, 100, 10)
    idx.destroy()


def test_batched_int8_near_duplicates(ctx):
    """Groups of eight rows within a small perturbation of each other: their
    level-one bounds overlap the query's bound, so whole groups are kept and
    the exact re-score must order them as single queries do."""
    from browservec_amd import QuantIndex

    dim, n, nq = 768, 40000, 24
    say("batched int8 near-duplicates")
    base = clustered(n // 8, dim, 40, 0.1, seed=64)
    rng = np.random.default_rng(65)
    data = np.repeat(base, 8, axis=0) + rng.standard_normal((n, dim)).astype(np.float32) * np.float32(1e-4)
    data = np.stack([o.normalize(r) for r in data]).astype(np.float32)
    idx = QuantIndex(ctx, dim, bits=8)
    idx.append(data, n)
    qs = (data[np.arange(nq) * 1601] + gaussian(nq, dim, 66, normalize=False) * 0.03).astype(np.float32)
    qs = np.stack([o.normalize(q) for q in qs]).astype(np.float32)
    singles_equal(idx, qs, 100, 10)
    idx.destroy()


def test_batched_large_fetch(ctx):
    from browservec_amd import QuantIndex

    dim, n, nq = 64, 40000, 16
    say("batched fetch 1000")
    data = gaussian(n, dim, 21)
    idx = QuantIndex(ctx, dim, bits=8)
    idx.append(data, n)
    qs = gaussian(nq, dim, 22)
    singles_equal(idx, qs, 1000, 10)
    batch = idx.query_batch(qs, nq, 1000)
    for i in (0, 7, 15):
        assert batch[i] == idx.query(qs[i], 1000), i
    idx.destroy()


def test_batched_overflow_falls_back(ctx):
    """Sampled rows (every second row here) all score low while the other
    rows all sit next to the queries: the sample's bound admits every
    unsampled row, the append buffer overflows, and those queries must still
    answer exactly as alone."""
    from browservec_amd import QuantIndex

    dim, n, nq = 64, 40000, 8
    say("batched overflow")
    rng = np.random.default_rng(5)
    qs = np.abs(gaussian(nq, dim, 31))  # queries in the positive orthant
    qs /= np.linalg.norm(qs, axis=1, keepdims=True)
    data = -np.abs(gaussian(n, dim, 32))  # even (sampled) rows: negative scores
    odd = np.arange(1, n, 2)
    near = np.abs(qs[odd % nq] + rng.standard_normal((odd.size, dim)).astype(np.float32) * 0.01)
    data[odd] = near / np.linalg.norm(near, axis=1, keepdims=True)  # odd rows: scores near 1
    idx = QuantIndex(ctx, dim, bits=8)
    idx.append(data.astype(np.float32), n)
    singles_equal(idx, qs.astype(np.float32), 100, 10)
    idx.destroy()


@pytest.mark.parametrize("scorer", ["asym", "hamming"])
def test_batched_1bit_overflow_falls_back(ctx, scorer):
    """The overflow case of test_batched_overflow_falls_back on 1-bit codes:
    the sampled rows score low, every unsampled row can reach the bound,
    the kept lists overflow and those queries run alone (for the asymmetric
    scorer after the exact bound raises), still equal to single queries."""
    from browservec_amd import QuantIndex

    dim, n, nq = 128, 40000, 8
    say("batched 1-bit overflow", scorer)
    rng = np.random.default_rng(15)
    qs = np.abs(gaussian(nq, dim, 41))
    qs /= np.linalg.norm(qs, axis=1, keepdims=True)
    data = -np.abs(gaussian(n, dim, 42))
    odd = np.arange(1, n, 2)
    near = np.abs(qs[odd % nq] + rng.standard_normal((odd.size, dim)).astype(np.float32) * 0.01)
    data[odd] = near / np.linalg.norm(near, axis=1, keepdims=True)
    idx = QuantIndex(ctx, dim, bits=1, scorer=scorer)
    idx.append(data.astype(np.float32), n)
    singles_equal(idx, qs.astype(np.float32), 100, 10)
    idx.destroy()


def f32_singles_equal(idx, qs, k):
    """queryBatch rows and score bits equal query() of each vector."""
    nq = qs.shape[0]
    batch = idx.query_batch(qs, nq, k)
    for i in range(nq):
        single = idx.query(qs[i], k)
        assert [h.row for h in batch[i]] == [h.row for h in single], i
        assert np.array_equal(np.float32([h.score for h in batch[i]]).view(np.uint32),
                              np.float32([h.score for h in single]).view(np.uint32)), i
    return batch


@pytest.mark.parametrize("metric,dim,n,nq", [("cosine", 768, 40000, 40), ("dot", 96, 30000, 9),
                                             ("l2", 768, 40000, 33), ("l2", 128, 20000, 64),
                                             ("cosine", 64, 5000, 33)])
def test_batched_f32_equals_singles(ctx, metric, dim, n, nq):
    """fp32 batches: the matrix-core pass (its own summation order) only
    prefilters, with a slack that bounds its difference from the single-query
    scan's score; the survivors are re-scored by the single-query arithmetic,
    so rows and score bits equal query() of each vector (src/index.ts:477-501
    with gpu.test.ts:96-112's ID equality).  Scores stay within 1e-5 of the
    oracle's fp32 score (relative to |x||q|, or (|x|+|q|)^2 for l2)."""
    from browservec_amd import FlatIndex

    say("batched f32", metric, dim, n, nq)
    data = clustered(n, dim, 50, 0.15, seed=3 + dim)
    if metric != "cosine":  # rows of varied norm
        data = data * np.random.default_rng(dim).uniform(0.5, 2.0, (n, 1)).astype(np.float32)
    idx = FlatIndex(ctx, dim, metric)
    idx.append(data, n)
    qs = gaussian(nq, dim, 17 + dim)
    if metric == "l2":  # queries near rows, so the nearest distances are small
        qs = (data[np.arange(nq) * 7] + 0.01 * qs).astype(np.float32)
    k = 20
    batch = f32_singles_equal(idx, qs, k)
    norms = np.linalg.norm(data.astype(np.float64), axis=1)
    for i in (0, nq - 1):
        exact = o.scan_f32(data, qs[i], "l2" if metric == "l2" else "cosine")
        qn = np.linalg.norm(qs[i].astype(np.float64))
        mag = (norms + qn) ** 2 if metric == "l2" else norms * qn
        rows = np.array([h.row for h in batch[i]])
        got = np.float64([h.score for h in batch[i]])
        assert len(rows) == k
        assert np.all(np.abs(got - exact[rows]) <= 1e-5 * mag[rows] + 1e-7), i
    idx.destroy()


def test_batched_f32_near_duplicates(ctx):
    """Groups of rows within float rounding of each other (the ties the
    prefilter's slack must keep): batch rows and score bits still equal
    single queries."""
    from browservec_amd import FlatIndex

    dim, n, nq = 128, 40000, 16
    say("batched f32 near-duplicates")
    base = gaussian(n // 8, dim, 41)
    rng = np.random.default_rng(42)
    data = np.repeat(base, 8, axis=0) + rng.standard_normal((n, dim)).astype(np.float32) * np.float32(1e-7)
    data = np.stack([o.normalize(r) for r in data]).astype(np.float32)
    data[::8] = np.repeat(base, 1, axis=0)  # exact duplicates of the group leaders' source rows
    idx = FlatIndex(ctx, dim, "cosine")
    idx.append(data, n)
    qs = (data[np.arange(nq) * 997] + gaussian(nq, dim, 43, normalize=False) * 0.02).astype(np.float32)
    f32_singles_equal(idx, qs, 30)
    idx.destroy()


def test_batched_f32_overflow_falls_back(ctx):
    """Sampled rows all far from the queries, the rest all near: the kept
    rows overflow their buffer and those queries run the full fused scan,
    still equal to single queries."""
    from browservec_amd import FlatIndex

    dim, n, nq = 64, 40000, 8
    say("batched f32 overflow")
    rng = np.random.default_rng(6)
    qs = np.abs(gaussian(nq, dim, 33))
    qs /= np.linalg.norm(qs, axis=1, keepdims=True)
    data = -np.abs(gaussian(n, dim, 34))
    odd = np.arange(1, n, 2)
    near = np.abs(qs[odd % nq] + rng.standard_normal((odd.size, dim)).astype(np.float32) * 0.01)
    data[odd] = near / np.linalg.norm(near, axis=1, keepdims=True)
    idx = FlatIndex(ctx, dim, "cosine")
    idx.append(data.astype(np.float32), n)
    f32_singles_equal(idx, qs.astype(np.float32), 10)
    idx.destroy()


@pytest.mark.parametrize("n", [1, 5, 300])
def test_batched_tiny_corpus(ctx, n):
    """Corpora smaller than one row tile: rows past the end are clamped on
    load and dropped, k clamps to the row count, and batch results equal
    single queries."""
    from browservec_amd import FlatIndex, QuantIndex

    dim, nq = 64, 9
    say("batched tiny", n)
    data = gaussian(n, dim, 70 + n)
    qs = gaussian(nq, dim, 71 + n)
    quant = QuantIndex(ctx, dim, bits=8)
    quant.append(data, n)
    rows, scores, cnt = quant.search(qs, 8, 3)
    for i in range(nq):
        r1, s1, c1 = quant.search(qs[i:i + 1], 8, 3)
        assert cnt[i] == c1[0] == min(3, n)
        assert np.array_equal(rows[i, :cnt[i]], r1[0, :c1[0]])
        assert np.array_equal(scores[i, :cnt[i]].view(np.uint32), s1[0, :c1[0]].view(np.uint32))
    quant.destroy()
    flat = FlatIndex(ctx, dim, "cosine")
    flat.append(data, n)
    batch = f32_singles_equal(flat, qs, 4)
    for i in range(nq):
        exact = o.scan_f32(data, qs[i], "cosine")
        assert len(batch[i]) == min(4, n)
        for h in batch[i]:
            assert abs(h.score - float(exact[h.row])) <= 1e-5 * float(np.linalg.norm(data[h.row])) + 1e-7
    flat.destroy()


@pytest.mark.parametrize("dim,n,nq", [(256, 40000, 33), (1024, 30000, 300), (128, 20000, 9)])
def test_batched_hamming_equals_singles(ctx, dim, n, nq):
    """Hamming batches run the int8 first-level pass over the +1 / -1
    expansion of the 1-bit codes: the int8 dot of two +1 / -1 rows is
    P - 2 * popcount(a ^ b), so the keys are the single-query scan's exact
    Hamming similarities; rows and scores equal the same queries run alone,
    with and without the re-rank, across appends (the expansion follows
    them), with duplicate rows tying."""
    from browservec_amd import QuantIndex

    say("batched hamming", dim, n, nq)
    data = clustered(n, dim, 40, 0.1, seed=dim + 3)
    data[n // 2:n // 2 + 200] = data[:200]  # ties: identical codes
    idx = QuantIndex(ctx, dim, bits=1, scorer="hamming")
    idx.append(data[:n - 2000], n - 2000)
    qs = data[np.arange(nq) * (n // nq)] + gaussian(nq, dim, 4, normalize=False) * 0.05
    qs = np.stack([o.normalize(q) for q in qs]).astype(np.float32)
    singles_equal(idx, qs, 200, 10)
    idx.append(data[n - 2000:], 2000)
    rows, scores, cnt = singles_equal(idx, qs, 0, 50)
    # the scores are Hamming similarities of the codes: integers in [-P, P]
    P = idx.padded_dim
    assert np.all(scores[:, :1] == np.round(scores[:, :1])) and np.all(np.abs(scores[:, 0]) <= P)
    batch = idx.query_batch(qs, nq, 20)
    for i in range(nq):
        assert batch[i] == idx.query(qs[i], 20), i
    idx.destroy()


@pytest.mark.parametrize("dim,n,nq", [(1024, 40000, 64), (256, 30000, 33), (100, 20000, 9)])
def test_batched_1bit_asym_equals_singles(ctx, dim, n, nq):
    """1-bit asymmetric batches (the reference's distanceQ1 scorer) run the
    int8 first-level pass over the +1 / -1 expansion with the rotated query's
    int8 level one: the score scale * sum_i (bit_i ? x_i : -x_i) lies within
    scale * (|x - s1 q1|_1 + the f32 summation slack) of scale * s1 * D, D
    the level-one dot; the rows that can still reach a query's fetch get
    their exact keys from q1p_exact_rows, in the single-query scan's own
    layout (4 and 8 lanes per row at these dimensions).  Rows and score
    bits equal the same queries run alone, with and without the re-rank,
    across appends (the expansion follows them), with duplicate rows
    tying."""
    from browservec_amd import QuantIndex

    say("batched 1-bit asym", dim, n, nq)
    data = clustered(n, dim, 40, 0.1, seed=dim + 5)
    data[n // 2:n // 2 + 200] = data[:200]  # ties: identical codes and scales
    idx = QuantIndex(ctx, dim, bits=1)
    idx.append(data[:n - 2000], n - 2000)
    qs = data[np.arange(nq) * (n // nq)] + gaussian(nq, dim, 6, normalize=False) * 0.05
    qs = np.stack([o.normalize(q) for q in qs]).astype(np.float32)
    singles_equal(idx, qs, 200, 10)
    idx.append(data[n - 2000:], 2000)
    rows, scores, cnt = singles_equal(idx, qs, 0, 50)
    # the approximate scores are the oracle's distanceQ1 scores of those rows
    words, sc = idx.export_codes()
    for i in (0, nq - 1):
        q_rot = o.rotate(qs[i], dim)[0]
        want = o.scan_quant(words, sc, q_rot, 1, cand=rows[i, :cnt[i]].astype(np.uint32))
        mag = np.abs(sc[rows[i, :cnt[i]]].astype(np.float64)) * float(np.abs(q_rot.astype(np.float64)).sum())
        assert np.all(np.abs(scores[i, :cnt[i]].astype(np.float64) - want) <= 1e-5 * mag + 1e-30), i
    batch = idx.query_batch(qs, nq, 20)
    for i in range(nq):
        assert batch[i] == idx.query(qs[i], 20), i
    idx.destroy()
