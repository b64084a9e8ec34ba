"""Selection for any k and the exact scan of listed rows.

- k above the fused top-k's 1024 (flat.ts:217-239 takes any k): every row's
  scan score, then a device sort; the rows and score bits equal the oracle's
  canonical top-k over the same scores.
- queryRowsExact (src/index.ts:445-464) on the device: Store.dotRow /
  Store.l2Row (store.ts:114-160) of each listed row, bit for bit, and their
  canonical top-k; the mask form builds the same list on the device.
"""

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


def hits_arrays(hits):
    return (np.array([h.row for h in hits], np.int64),
            np.array([h.score for h in hits], np.float32))


def check_canonical(hits, scores, k, ids=None):
    want_r, want_s = o.topk_canonical(scores, k, ids)
    got_r, got_s = hits_arrays(hits)
    assert got_r.size == want_r.size
    assert np.array_equal(got_r, want_r.astype(np.int64))
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))


def mask_of(sel, n):
    words = np.zeros((n + 31) // 32, np.uint32)
    for r in np.nonzero(sel)[0]:
        words[r >> 5] |= np.uint32(1 << (int(r) & 31))
    return words


@pytest.mark.parametrize("kind,metric,dim,n", [("quant8", "cosine", 128, 30000), ("flat", "dot", 96, 20000),
                                               ("flat", "l2", 40, 9000), ("quant4", "cosine", 64, 12000)])
def test_large_k_matches_canonical_top_k(ctx, kind, metric, dim, n):
    from browservec_amd import FlatIndex, QuantIndex

    say("large k", kind, metric, dim, n)
    data = clustered(n, dim, 50, 0.1, seed=dim + n)
    if metric == "cosine":
        o.normalize_rows_store(data)
    idx = FlatIndex(ctx, dim, metric) if kind == "flat" else QuantIndex(ctx, dim, bits=int(kind[-1]))
    idx.append(data, n)
    qs = gaussian(3, dim, 9)
    for qi, k in ((0, 1025), (1, 4096), (2, n + 50)):
        sc = idx.export_scores(qs[qi])
        check_canonical(idx.query(qs[qi], k), sc, k)
    # masked, k beyond the matching rows and beyond 1024
    rng = np.random.default_rng(5)
    sel = rng.random(n) < 0.3
    words = mask_of(sel, n)
    sc = idx.export_scores(qs[0])
    ids = np.nonzero(sel)[0].astype(np.uint32)
    for k in (2000, int(sel.sum()) + 10):
        check_canonical(idx.query_masked(qs[0], k, words), sc[ids], k, ids)
    # batches loop the same path
    got = idx.query_batch(qs[:2].reshape(-1), 2, 1500)
    for i in range(2):
        check_canonical(got[i], idx.export_scores(qs[i]), 1500)
    idx.destroy()


def exact_scores(data, q, rows, metric):
    fn = o.l2_row if metric == "l2" else o.dot_row
    return np.array([fn(data[r], q) for r in rows], dtype=np.float64).astype(np.float32)


@pytest.mark.parametrize("kind,metric,dim,n", [("flat", "l2", 37, 5000), ("flat", "dot", 96, 8000),
                                               ("flat", "cosine", 768, 3000), ("quant8", "cosine", 100, 6000),
                                               ("ivf", "dot", 64, 4000), ("ivfquant", "cosine", 48, 4000)])
def test_query_rows_exact(ctx, kind, metric, dim, n):
    from browservec_amd import FlatIndex, IVFIndex, IVFQuantIndex, QuantIndex
    from browservec_amd._lib import BVError

    say("query rows", kind, metric, dim, n)
    data = clustered(n, dim, 40, 0.1, seed=3 * dim + n)
    if metric == "cosine":
        o.normalize_rows_store(data)
    if kind == "flat":
        idx = FlatIndex(ctx, dim, metric)
    elif kind == "quant8":
        idx = QuantIndex(ctx, dim, bits=8)
    elif kind == "ivf":
        idx = IVFIndex(ctx, dim, metric=metric, ivf={"nlist": 8, "iters": 2})
    else:
        idx = IVFQuantIndex(ctx, dim, bits=8, ivf={"nlist": 8, "iters": 2})
    idx.append(data, n)
    rng = np.random.default_rng(dim)
    q = gaussian(1, dim, 17)[0]
    if metric == "cosine":
        q = o.normalize_rows_store(q[None].copy())[0]
    # duplicate rows in the corpus make exact score ties, ordered by row
    data2 = data[:50].copy()
    idx.append(data2, 50)
    full = np.concatenate([data, data2])
    for m, k in ((1, 1), (200, 10), (min(n, 4096), 100), (min(n, 12000), 3000), (300, 1000)):
        rows = rng.choice(n + 50, size=m, replace=False).astype(np.uint32)
        if m >= 300:  # both copies of the duplicated rows, in shuffled order
            rows = np.union1d(rows[:m - 100], np.r_[0:50, n:n + 50]).astype(np.uint32)
            rng.shuffle(rows)
        want = exact_scores(full, q, rows, metric)
        check_canonical(idx.query_rows(q, rows, k), want, k, rows)
        # the mask form over the same rows (list order does not matter)
        sel = np.zeros(n + 50, bool)
        sel[rows] = True
        words = mask_of(sel, n + 50)
        check_canonical(idx.query_rows_masked(q, k, words), want, k, rows)
    # the reference's topK picks the same rows when no scores tie
    rows = rng.choice(n, size=500, replace=False).astype(np.uint32)
    rows.sort()
    want = exact_scores(full, q, rows, metric)
    if np.unique(want).size == want.size:
        ref_pos, ref_s = o.topk_ref(want, 20)
        got_r, got_s = hits_arrays(idx.query_rows(q, rows, 20))
        assert np.array_equal(got_r, rows[ref_pos].astype(np.int64))
        assert np.array_equal(got_s.view(np.uint32), ref_s.view(np.uint32))
    # edges: empty list, k = 0, a short mask, mask bits past the rows, a bad row
    assert idx.query_rows(q, np.empty(0, np.uint32), 10) == []
    assert idx.query_rows(q, rows, 0) == []
    short = np.full(3, 0xFFFFFFFF, np.uint32)
    check_canonical(idx.query_rows_masked(q, 500, short), exact_scores(full, q, np.arange(96), metric), 500,
                    np.arange(96, dtype=np.uint32))
    wide = np.full((n + 50 + 31) // 32 + 4, 0xFFFFFFFF, np.uint32)
    allr = np.arange(n + 50, dtype=np.uint32)
    check_canonical(idx.query_rows_masked(q, 7, wide), exact_scores(full, q, allr, metric), 7, allr)
    with pytest.raises(BVError, match="out of range"):
        idx.query_rows(q, np.array([3, n + 50], np.uint32), 5)
    idx.destroy()


def test_browservec_ivf_filters_take_the_exact_device_scan(ctx):
    """BrowserVec.query on an IVF store (src/index.ts:372-395): a filter that
    matches few rows, and a selective one matching more than 4096 rows, both
    return queryRowsExact's answer -- the exact top k of the matching rows --
    now scored on the device; a near-total filter over-fetches through the
    index and post-filters."""
    from browservec_amd import BrowserVec

    say("BrowserVec IVF filters")
    dim, n = 48, 12000
    vecs = clustered(n, dim, 30, 0.1, seed=4)
    db = BrowserVec.create(dimension=dim, metric="cosine", quantBits=8, ann={"nlist": 16, "iters": 2, "nprobe": 2})
    db.add_batch([{"id": f"v{i}", "vector": vecs[i], "metadata": {"m": i % 7}} for i in range(n)])
    normed = vecs.copy()
    o.normalize_rows_store(normed)
    q = gaussian(1, dim, 23)[0]
    qn = o.normalize(q)
    exact = np.array([o.dot_row(normed[i], qn) for i in range(n)], np.float32)
    for keep, k in ((lambda m: m["m"] == 3, 10), (lambda m: m["m"] != 0 and m["m"] != 1, 25)):
        match = np.array([i for i in range(n) if keep({"m": i % 7})], np.uint32)
        assert match.size <= 4096 or n - match.size > max(2 * k, 256)
        res = db.query(q, k=k, filter=keep)
        wr, ws = o.topk_canonical(exact[match], k, match)
        assert [int(r["id"][1:]) for r in res] == wr.tolist()
        assert [r["score"] for r in res] == ws.tolist()
    res = db.query(q, k=10, filter=lambda m: m["m"] != 5 or True)  # every row: the index path
    assert len(res) == 10
    db.destroy()


@pytest.mark.parametrize("bits", [8, 0])
def test_ivf_large_k(ctx, bits):
    """IVF queries with k above 1024 (ivfquant.ts:459-527 takes any k): every
    candidate of the probed lists scored by the scan, then a device sort;
    the canonical top-k of the scan scores over exactly the probed rows, and
    the first 1024 equal the fused query's answer at k = 1024."""
    from browservec_amd import IVFIndex, IVFQuantIndex

    say("ivf large k", bits)
    dim, n = 64, 20000
    data = clustered(n, dim, 40, 0.1, seed=31 + bits)
    ivf = {"nlist": 32, "iters": 2, "nprobe": 6}
    idx = IVFQuantIndex(ctx, dim, bits=bits, ivf=ivf) if bits else IVFIndex(ctx, dim, ivf=ivf)
    idx.append(data, n)
    cen, off, lrows = idx.export_ivf()
    qs = gaussian(3, dim, 32)
    for i, k in enumerate((1500, 4000, n)):
        rq = o.rotate(qs[i], dim)[0] if bits else qs[i]
        probes, _ = o.topk_canonical(o.probe_scores(cen, rq), 6)
        rows = np.sort(np.concatenate([lrows[off[c]:off[c + 1]] for c in probes])).astype(np.uint32)
        sc = idx.export_scores(qs[i])
        got = idx.query(qs[i], k)
        check_canonical(got, sc[rows], k, rows)
        if rows.size >= 1024:
            small = idx.query(qs[i], 1024)
            assert [(h.row, h.score) for h in got[:1024]] == [(h.row, h.score) for h in small]
    idx.destroy()
