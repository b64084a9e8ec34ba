"""IVF parity on the device: the k-means build (reservoir, init, Lloyd
iterations, final assignment, CSR lists) against the oracle's restatement of
src/index/ivfquant.ts / ivf.ts / kmeans.ts, and IVF queries (probes, list
gather, scan, exact re-rank) against the oracle pipeline."""

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


def dequant_f32(words, scales, bits, P):
    """The device assignment's row values: unpack4x8snorm(b) * scale (int8),
    signed nibble * (scale * f32(1/7)) (int4), f32 arithmetic throughout."""
    n = words.shape[0]
    if bits == 8:
        b = words.view(np.uint8).reshape(n, -1)[:, :P].view(np.int8).astype(np.float32)
        u = np.maximum(b / np.float32(127.0), np.float32(-1.0))
        return (u * scales[:, None]).astype(np.float32)
    w = words.astype(np.uint64)
    shifts = np.arange(8, dtype=np.uint64) * 4
    nib = ((w[:, :, None] >> shifts) & 0xF).astype(np.int32).reshape(n, -1)[:, :P]
    sig = (nib - 16 * (nib >> 3)).astype(np.float32)
    inv7 = (scales * (np.float32(1.0) / np.float32(7.0))).astype(np.float32)
    return (sig * inv7[:, None]).astype(np.float32)


def reference_build(data, dim, bits, ivf, seed=o.DEFAULT_SEED):
    """The reference's IVF build restated on the oracle (test infrastructure)."""
    n = data.shape[0]
    quant = bits > 0
    cap = max(1024, ivf.get("sampleSize") or 50000)
    ivf_seed = ivf.get("seed")
    if quant:
        rseed = ((ivf_seed if ivf_seed is not None else seed) ^ 0x85EBCA6B) & 0xFFFFFFFF
        words, scales, rot = o.encode(data, dim, bits, seed, want_rotated=True)
        src = rot
    else:
        rseed = ivf_seed if ivf_seed is not None else o.IVF_SEED
        words = scales = None
        src = data
    res = o.Reservoir(cap, rseed)
    sample = np.zeros((cap, src.shape[1]), np.float32)
    sample_row = np.zeros(cap, np.int64)
    for i in range(n):
        s = res.slot()
        if s >= 0:
            sample[s] = src[i]
            sample_row[s] = i
    filled = min(n, cap)
    if ivf.get("nlist"):
        nlist = max(1, min(ivf["nlist"], n))
    else:
        nlist = max(1, min(min(4096, max(16, int(np.floor(np.sqrt(n) + 0.5)))), n))
    train = min(filled, ivf.get("trainSize") or 16384)
    kseed = ivf_seed if ivf_seed is not None else o.IVF_SEED
    iters = ivf.get("iters") or 8
    T = np.ascontiguousarray(sample[:train])
    cen = o.random_init_centroids(T, nlist, kseed)
    for it in range(iters):
        a = o.assign_f32(T, cen, order=1)
        cen, _ = o.update_centroids(T, a, cen, (kseed + it + 1) & 0xFFFFFFFF)
    if quant:
        P = src.shape[1]
        final = o.assign_f32(dequant_f32(words, scales, bits, P), cen, order=1)
    else:
        final = o.assign_f32(data, cen, order=1)
    off, rows = o.build_csr(final, nlist)
    return dict(cen=cen, off=off, rows=rows, final=final, words=words, scales=scales, nlist=nlist,
                src=src, filled=filled, sample_row=sample_row[:filled])


CASES = [(8, 96, {"nlist": 24, "iters": 4}), (4, 128, {"nlist": 16, "iters": 3, "seed": 77}),
         (0, 96, {"nlist": 20, "iters": 4}), (0, 100, {"iters": 2, "sampleSize": 1500, "trainSize": 1200})]


@pytest.mark.parametrize("bits,dim,ivf", CASES)
def test_ivf_build_matches_oracle(ctx, bits, dim, ivf):
    from browservec_amd import IVFIndex, IVFQuantIndex

    say("ivf build", bits, dim, ivf)
    n = 6000
    data = clustered(n, dim, 40, 0.08, seed=90 + bits)
    data[11] = 0.0  # a zero row (int8: scale 0, which the matrix-core assignment leaves to the exact one)
    data[12] = data[4000]  # a duplicate row
    idx = IVFQuantIndex(ctx, dim, bits=bits, ivf=ivf) if bits else IVFIndex(ctx, dim, ivf=ivf)
    idx.append(data[:2500], 2500)  # two appends: the reservoir carries over
    idx.append(data[2500:], n - 2500)
    cen, off, rows = idx.export_ivf()
    ref = reference_build(data, dim, bits, ivf)
    assert cen.shape[0] == ref["nlist"]
    assert np.array_equal(cen.view(np.uint32), ref["cen"].view(np.uint32)), "centroids differ"
    assert np.array_equal(off.astype(np.int64), ref["off"].astype(np.int64)), "list offsets differ"
    assert np.array_equal(rows.astype(np.int64), ref["rows"].astype(np.int64)), "list rows differ"
    if bits:
        # against the reference kernels' own dot4 order: equal except near-ties
        P = cen.shape[1]
        ref_assign = o.assign_quant(ref["words"], ref["scales"], P, bits, ref["cen"])
        diff = np.nonzero(ref_assign != ref["final"])[0]
        V = dequant_f32(ref["words"], ref["scales"], bits, P).astype(np.float64)
        for r in diff:
            s = V[r] @ ref["cen"].astype(np.float64).T
            assert abs(s[ref_assign[r]] - s[ref["final"][r]]) <= 1e-5 * np.abs(V[r]).sum(), r
    st = idx.stats()
    assert st["nlist"] == ref["nlist"] and st["nprobe"] == max(1, int(np.floor(ref["nlist"] * 0.05 + 0.5)))
    if bits == 8:  # the final assignment ran on the matrix cores: it decided most rows itself
        assert 1 <= st["build_exact_rows"] < n // 2, st["build_exact_rows"]
    else:
        assert st["build_exact_rows"] == n
    idx.destroy()


@pytest.mark.parametrize("bits", [8, 0])
def test_ivf_search_matches_oracle_pipeline(ctx, bits):
    """Probes, gathered lists, scan and exact re-rank (ivfquant.ts:466-527)."""
    from browservec_amd import IVFIndex, IVFQuantIndex

    dim, n, nprobe, fetch = 96, 12000, 5, 40
    ivf = {"nlist": 32, "iters": 3, "nprobe": nprobe}
    say("ivf search", bits)
    data = clustered(n, dim, 48, 0.1, seed=123 + bits)
    idx = IVFQuantIndex(ctx, dim, bits=bits, ivf=ivf) if bits else IVFIndex(ctx, dim, ivf=ivf)
    idx.append(data, n)
    cen, off, lrows = idx.export_ivf()
    qs = data[[5, 777, 11111]] + gaussian(3, dim, 7, normalize=False) * 0.05
    qs = np.stack([o.normalize(q) for q in qs])
    rows, scores, cnt = idx.search(qs, fetch, 10) if bits else (None, None, None)
    flat_hits = [idx.query(q, 10) for q in qs]
    for i, q in enumerate(qs):
        rq = o.rotate(q, dim)[0] if bits else q
        probes, _ = o.topk_canonical(o.probe_scores(cen, rq), nprobe)
        cand = np.concatenate([lrows[off[c]:off[c + 1]] for c in probes]).astype(np.uint32)
        if bits:
            words, scales = idx_codes(idx)
            approx = o.scan_quant(words, scales, rq, bits, cand=cand)
            mag = quant_magnitude(words[cand], scales[cand], rq, bits)
            # query(): the approximate top-10 of the probed lists by code score
            got = np.array([h.row for h in flat_hits[i]])
            assert set(got.tolist()) <= set(cand.tolist())
            want, ws = o.topk_canonical(approx, 10, ids=cand)
            kth = float(ws[-1])
            pos = {int(r): j for j, r in enumerate(cand)}
            for r in set(got.tolist()) ^ set(want.tolist()):
                assert abs(float(approx[pos[r]]) - kth) <= 2 * REL_TOL * mag.max(), r
            # search(): the oracle pipeline over the probed lists (top-fetch by
            # code score, exact re-rank, canonical top-10), up to fetch-boundary
            # near-ties
            assert cnt[i] == 10
            tol = 2 * REL_TOL * max(float(mag.max()), float(np.abs(approx).max()))
            assert_fetch_rerank(rows[i], scores[i], approx, cand, lambda rr: o.rerank_scores(data, q, rr), fetch, 10,
                                tol, what=f"ivf query {i}")
        else:
            exact = o.scan_f32(data[cand], q)
            want, ws = o.topk_canonical(exact, 10, ids=cand)
            got = [h.row for h in flat_hits[i]]
            kth = float(ws[-1])
            pos = {int(r): j for j, r in enumerate(cand)}
            for r in set(got) ^ set(want.tolist()):
                assert abs(float(exact[pos[r]]) - kth) <= 1e-5, r
    idx.destroy()


def idx_codes(idx):
    words = np.empty((idx.size, idx.words_per_row), np.uint32)
    scales = np.empty(idx.size, np.float32)
    from browservec_amd import _lib as L
    from browservec_amd.index import _ptr

    L.check(idx.lib.bv_index_export_codes(idx.handle, 0, idx.size, _ptr(words), _ptr(scales)))
    return words, scales


def test_ivf_masked_and_nprobe_override(ctx):
    """Masked IVF scans keep only rows whose bit is set; a per-query nprobe
    override is consumed by one query (ivfquant.ts:487-491)."""
    from browservec_amd import IVFQuantIndex

    dim, n = 64, 8000
    say("ivf masked")
    data = clustered(n, dim, 30, 0.1, seed=5)
    idx = IVFQuantIndex(ctx, dim, bits=8, ivf={"nlist": 20, "iters": 2, "nprobe": 4})
    idx.append(data, n)
    rng = np.random.default_rng(3)
    keep = rng.random(n) < 0.4
    words = np.zeros((n + 31) // 32, np.uint32)
    for r in np.nonzero(keep)[0]:
        words[r >> 5] |= np.uint32(1 << (int(r) & 31))
    q = data[100]
    hits = idx.query_masked(q, 10, words)
    assert hits and all(keep[h.row] for h in hits)
    idx.set_nprobe(20)  # every list: the masked query sees every kept row
    hits_all = idx.query_masked(q, 10, words)
    cen, off, lrows = idx.export_ivf()
    words_c, scales = idx_codes(idx)
    rq = o.rotate(q, dim)[0]
    approx = o.scan_quant(words_c, scales, rq, 8)
    mag = quant_magnitude(words_c, scales, rq, 8)
    tol = 2 * REL_TOL * max(float(mag.max()), float(np.abs(approx).max()))
    approx[~keep] = -np.inf
    got = [h.row for h in hits_all]
    assert len(got) == 10
    assert_topk_near(got, approx, 10, tol, what="masked ivf, every list")
    assert_scores_close([h.score for h in hits_all], approx[got], mag[got], "masked ivf scores")
    # the order is the device scores' canonical order
    keys = [(h.score, -h.row) for h in hits_all]
    assert keys == sorted(keys, reverse=True)
    # the override was consumed: the next query uses nprobe 4 again
    assert idx.stats()["nprobe"] == 4
    idx.destroy()


def reference_tune(data, dim, bits, ref, target):
    """ivfquant.ts:322-344 / ivf.ts:269-291 on the oracle: evenly spaced
    reservoir rows as queries, the exhaustive top k+1 in the index's own
    scores, the probe rank of each hit's list (first hit skipped),
    chooseNprobe."""
    n = data.shape[0]
    k = min(10, n - 1)
    ranks = []
    for si in o.pick_tune_queries(ref["filled"], 32):
        r = int(ref["sample_row"][si])
        rq = ref["src"][r]  # the sample row: rotated (quantized kinds) or raw (fp32)
        if bits:
            scores = o.scan_quant(ref["words"], ref["scales"], rq, bits)
        else:
            scores = o.scan_f32(data, rq)
        gt, _ = o.topk_canonical(scores, k + 1)
        order, _ = o.topk_canonical(o.probe_scores(ref["cen"], rq), ref["nlist"])
        rank = np.empty(ref["nlist"], np.int64)
        rank[order] = np.arange(ref["nlist"])
        ranks += [int(rank[ref["final"][g]]) for g in gt[1:]]
    return o.choose_nprobe(ranks, ref["nlist"], target)


@pytest.mark.parametrize("bits,target", [(8, 0.9), (0, 0.95), (4, 0.8)])
def test_ivf_tune_matches_oracle(ctx, bits, target):
    """targetRecall tuning (ivfTune.ts:31-42): the tuned nprobe and its
    estimated recall equal the oracle's restatement of the reference's tune;
    an explicit nprobe disables tuning."""
    from browservec_amd import IVFIndex, IVFQuantIndex

    dim, n = 96, 6000
    ivf = {"nlist": 24, "iters": 4, "targetRecall": target}
    say("ivf tune", bits, target)
    data = clustered(n, dim, 40, 0.2, seed=31 + bits)
    idx = IVFQuantIndex(ctx, dim, bits=bits, ivf=ivf) if bits else IVFIndex(ctx, dim, ivf=ivf)
    idx.append(data, n)
    idx.build()
    ref = reference_build(data, dim, bits, ivf)
    want_np, want_rec = reference_tune(data, dim, bits, ref, target)
    st = idx.stats()
    assert st["nprobe"] == want_np, (st["nprobe"], want_np, want_rec)
    assert np.float32(st["tuned_recall"]) == np.float32(want_rec), (st["tuned_recall"], want_rec)
    idx.destroy()
    fixed_ivf = dict(ivf, nprobe=3)
    fixed = IVFQuantIndex(ctx, dim, bits=bits, ivf=fixed_ivf) if bits else IVFIndex(ctx, dim, ivf=fixed_ivf)
    fixed.append(data, n)
    fixed.build()
    assert fixed.stats()["nprobe"] == 3 and fixed.stats()["tuned_recall"] < 0
    fixed.destroy()


def probed_rows(cen, off, lrows, q, nprobe):
    probes, _ = o.topk_canonical(o.probe_scores(cen, q), nprobe)
    return set(np.concatenate([lrows[off[c]:off[c + 1]] for c in probes]).tolist())


def test_ivf_probe_selection_many_lists(ctx):
    """pickProbes at 1024 lists (ivfquant.ts:495-517): the sampled bound
    (nprobe <= 64) and the bisection (nprobe > 64) both pick the oracle's
    probe set.  k covers every candidate, so a query returns exactly the rows
    of the lists it probed; single queries with a one-query override, then a
    batch of 300 queries (more than one query per prefix run; eight-query
    probe tiles, the last one partial)."""
    from browservec_amd import IVFIndex

    dim, n = 128, 8192
    say("ivf probes 1024 lists")
    data = clustered(n, dim, 256, 0.2, seed=41)
    idx = IVFIndex(ctx, dim, ivf={"nlist": 1024, "iters": 2, "nprobe": 48})
    idx.append(data, n)
    cen, off, lrows = idx.export_ivf()
    assert cen.shape[0] == 1024
    qs = gaussian(300, dim, 42)
    for i, nprobe in enumerate([1, 16, 32, 64, 65, 80]):
        want = probed_rows(cen, off, lrows, qs[i], nprobe)
        assert len(want) <= 1024
        idx.set_nprobe(nprobe)
        got = {h.row for h in idx.query(qs[i], 1024)}
        assert got == want, nprobe
    batch = idx.query_batch(qs, qs.shape[0], 1024)
    for i in range(qs.shape[0]):
        want = probed_rows(cen, off, lrows, qs[i], 48)
        assert len(want) <= 1024
        assert {h.row for h in batch[i]} == want, i
    idx.destroy()


def test_ivf_probe_scores_widest_query(ctx):
    """The widest query the scans serve (4096 floats) fills the probe
    kernel's LDS staging; the probe set equals pickProbes'."""
    from browservec_amd import IVFIndex

    dim, n = 4096, 64
    say("ivf probes dim 4096")
    data = clustered(n, dim, 8, 0.3, seed=43)
    idx = IVFIndex(ctx, dim, ivf={"nlist": 8, "iters": 2, "nprobe": 3})
    idx.append(data, n)
    cen, off, lrows = idx.export_ivf()
    for i, q in enumerate(gaussian(3, dim, 44)):
        got = {h.row for h in idx.query(q, n)}
        assert got == probed_rows(cen, off, lrows, q, 3), i
    idx.destroy()


def test_ivf_lazy_build_inside_a_query(ctx):
    """The first query after an append builds the lists (ivfquant.ts:461)
    and, with targetRecall and no nprobe, tunes nprobe before it scans.
    Whatever entry point triggers that build (query, search, search_device),
    its results equal those of an index built explicitly first, and the
    tuned nprobe equals the oracle's."""
    import torch

    from browservec_amd import IVFQuantIndex

    dim, n = 96, 6000
    ivf = {"nlist": 24, "iters": 4, "targetRecall": 0.9}
    say("ivf lazy build")
    data = clustered(n, dim, 40, 0.2, seed=33)
    qs = np.stack([o.normalize(q) for q in data[[3, 2000, 4500]] + gaussian(3, dim, 34, normalize=False) * 0.05])
    qs = qs.astype(np.float32)

    def fresh():
        idx = IVFQuantIndex(ctx, dim, bits=8, ivf=ivf)
        idx.append(data, n)
        return idx

    ref_idx = fresh()
    ref_idx.build()
    want_q = ref_idx.query(qs[0], 10)
    want_rows, want_scores, want_cnt = ref_idx.search(qs, 40, 10)
    ref = reference_build(data, dim, 8, ivf)
    want_np, _ = reference_tune(data, dim, 8, ref, 0.9)
    assert ref_idx.stats()["nprobe"] == want_np

    a = fresh()
    assert a.query(qs[0], 10) == want_q
    assert a.stats()["nprobe"] == want_np
    b = fresh()
    rows, scores, cnt = b.search(qs, 40, 10)
    assert np.array_equal(rows, want_rows) and np.array_equal(scores.view(np.uint32), want_scores.view(np.uint32))
    c = fresh()
    d_q = torch.from_numpy(qs).cuda()
    d_rows = torch.empty(3, 10, dtype=torch.int32, device="cuda")
    d_sc = torch.empty(3, 10, dtype=torch.float32, device="cuda")
    d_n = torch.empty(3, dtype=torch.int32, device="cuda")
    c.search_device(d_q.data_ptr(), 3, 40, 10, d_rows.data_ptr(), d_sc.data_ptr(), d_n.data_ptr())
    c.sync()
    assert np.array_equal(d_rows.cpu().numpy().view(np.uint32), want_rows)
    assert np.array_equal(d_sc.cpu().numpy().view(np.uint32), want_scores.view(np.uint32))
    for idx in (ref_idx, a, b, c):
        idx.destroy()


@pytest.mark.parametrize("bits", [8, 0])
def test_ivf_incremental_append(ctx, bits):
    """Incremental mode (src/index/ivfquant.ts:216-233,462 rebuilds after
    every append instead): rows appended after a build are assigned to the
    current centroids with the final-assignment arithmetic and extend the
    lists, centroids unchanged; an explicit build then retrains over the
    reservoir and equals the reference-mode index's lists."""
    from browservec_amd import IVFIndex, IVFQuantIndex

    dim, n0, n1 = 64, 4000, 1500
    ivf = {"nlist": 16, "iters": 3, "nprobe": 4, "sampleSize": 2048}
    say("ivf incremental", bits)
    data = clustered(n0 + n1, dim, 24, 0.1, seed=77 + bits)
    make = (lambda o: IVFQuantIndex(ctx, dim, bits=bits, ivf=o)) if bits else (lambda o: IVFIndex(ctx, dim, ivf=o))
    inc = make(dict(ivf, incremental=True))
    ref = make(ivf)
    for x in (inc, ref):
        x.append(data[:n0], n0)
        x.build()
    cen0, off0, rows0 = inc.export_ivf()
    inc.append(data[n0:], n1)
    ref.append(data[n0:], n1)
    cen1, off1, rows1 = inc.export_ivf()  # no rebuild: the lists were extended
    assert np.array_equal(cen1.view(np.uint32), cen0.view(np.uint32))
    old = np.empty(n0, np.int64)
    for c in range(off0.size - 1):
        old[rows0[off0[c]:off0[c + 1]]] = c
    if bits:
        words, scales = idx_codes(inc)
        new = o.assign_quant(words[n0:], scales[n0:], cen0.shape[1], bits, cen0)
        V = dequant_f32(words[n0:], scales[n0:], bits, cen0.shape[1]).astype(np.float64)
    else:
        new = o.assign_f32(data[n0:], cen0)
        V = data[n0:].astype(np.float64)
    got = np.empty(n0 + n1, np.int64)
    for c in range(off1.size - 1):
        seg = rows1[off1[c]:off1[c + 1]]
        assert np.all(np.diff(seg.astype(np.int64)) > 0), c  # rows ascending within a list
        got[seg] = c
    assert np.array_equal(got[:n0], old)  # old rows keep their lists
    for r in np.nonzero(got[n0:] != new)[0]:  # new rows: the oracle's assignment, up to near-ties
        s = V[r] @ cen0.astype(np.float64).T
        assert abs(s[got[n0 + r]] - s[new[r]]) <= 1e-5 * np.abs(V[r]).sum(), r
    q = data[[10, n0 + 20]]
    for qq in q:  # queries run on the extended lists without a rebuild
        assert [h.row for h in inc.query(qq, 10)] and inc.stats()["nlist"] == 16
    inc.build()  # retrain: the reference's lists
    for a, b in zip(inc.export_ivf(), ref.export_ivf()):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for qq in q:
        assert [(h.row, h.score) for h in inc.query(qq, 10)] == [(h.row, h.score) for h in ref.query(qq, 10)]
    inc.destroy()
    ref.destroy()


@pytest.mark.parametrize("dim,n,nq,ivf", [(96, 12000, 40, {"nlist": 32, "iters": 3, "nprobe": 5}),
                                          (768, 20000, 300, {"nlist": 64, "iters": 2, "nprobe": 9}),
                                          (64, 3000, 9, {"nlist": 16, "iters": 2, "nprobe": 16})])
@pytest.mark.parametrize("bits", [8, 4])
def test_ivf_batches_list_major_equal_singles(ctx, dim, n, nq, ivf, bits):
    """IVF int8 and int4 batches read every probed list once for all the queries
    probing it (list-major) and write each row's single-query key at its
    candidate position: rows and score bits equal the same queries run one at
    a time, with and without the re-rank, also with every list probed."""
    from browservec_amd import IVFQuantIndex

    say("ivf list-major batch", bits, dim, n, nq)
    data = clustered(n, dim, 48, 0.1, seed=dim + nq)
    idx = IVFQuantIndex(ctx, dim, bits=bits, ivf=ivf)
    idx.append(data, n)
    qs = data[np.arange(nq) * (n // nq)] + gaussian(nq, dim, 11, normalize=False) * 0.05
    qs = np.stack([o.normalize(q) for q in qs]).astype(np.float32)
    for fetch, k in ((40, 10), (0, 25)):
        rows, scores, cnt = idx.search(qs, fetch, k)
        for i in range(nq):
            r1, s1, c1 = idx.search(qs[i:i + 1], fetch, k)
            assert cnt[i] == c1[0], i
            assert np.array_equal(rows[i, :cnt[i]], r1[0, :c1[0]]), i
            assert np.array_equal(scores[i, :cnt[i]].view(np.uint32), s1[0, :c1[0]].view(np.uint32)), i
    m = min(16, nq)
    batch = idx.query_batch(qs[:m], m, 30)
    for i in range(m):
        assert batch[i] == idx.query(qs[i], 30), i
    idx.destroy()
