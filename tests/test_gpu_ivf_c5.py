"""IVF int8 at the shape of the 4M x 768 IVF workload: padded dimension 1024
(dim 768), 4096 lists, nprobe 32, fetch 40 -> 10.

The build, probes, gather and list scan are compared with the oracle's
restatement of src/index/ivfquant.ts / kmeans.ts on 40,000 rows (a train
sample of 8,192 and two Lloyd iterations keep the oracle's assignment to
seconds); the 4,000,000-row, 20-iteration build is checked by what the
mathematics fixes: unit centroids, lists that partition the rows in
ascending order, every sampled row in the list of the centroid the oracle's
assignment arithmetic picks for its codes, and a bit-identical rebuild."""

import numpy as np
import pytest

from oracle import oracle as o
from tests.helpers import REL_TOL, assert_fetch_rerank, clustered, gaussian, need_gpu, say
from tests.test_gpu_ivf import dequant_f32, reference_build

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    from browservec_amd import DeviceContext

    c = DeviceContext(0)
    yield c
    c.destroy()


def device_search(idx, qs, fetch, k):
    """bv_index_search_device over the whole batch in one call (no host
    chunking), so multi-query candidate offsets and batched probe tiles run."""
    import torch

    nq = qs.shape[0]
    d_q = torch.from_numpy(np.ascontiguousarray(qs, np.float32)).cuda()
    rows = torch.empty(nq, k, dtype=torch.int32, device="cuda")
    scores = torch.empty(nq, k, dtype=torch.float32, device="cuda")
    cnt = torch.empty(nq, dtype=torch.int32, device="cuda")
    idx.search_device(d_q.data_ptr(), nq, fetch, k, rows.data_ptr(), scores.data_ptr(), cnt.data_ptr())
    idx.sync()
    return rows.cpu().numpy().view(np.uint32), scores.cpu().numpy(), cnt.cpu().numpy()


def test_ivf_4096_lists_p1024_matches_oracle(ctx):
    from browservec_amd import IVFQuantIndex

    dim, n, nq = 768, 40000, 300
    ivf = {"nlist": 4096, "iters": 2, "trainSize": 8192, "nprobe": 32}
    say("ivf 4096 lists P=1024 build", n)
    data = clustered(n, dim, 4096, 0.15, seed=501)
    idx = IVFQuantIndex(ctx, dim, bits=8, ivf=ivf)
    idx.append(data[:15000], 15000)  # two appends: the reservoir carries over
    idx.append(data[15000:], n - 15000)
    cen, off, lrows = idx.export_ivf()
    ref = reference_build(data, dim, 8, ivf)
    assert cen.shape == (4096, 1024)
    assert np.array_equal(cen.view(np.uint32), ref["cen"].view(np.uint32)), "centroids differ"
    assert np.array_equal(off.astype(np.int64), ref["off"].astype(np.int64)), "list offsets differ"
    assert np.array_equal(lrows.astype(np.int64), ref["rows"].astype(np.int64)), "list rows differ"
    # the final assignment took the int8 matrix-core pass: most rows decided there
    assert idx.stats()["build_exact_rows"] < n // 2

    say("ivf 4096 lists probes", nq)
    rng = np.random.default_rng(502)
    qs = data[rng.integers(0, n, nq)] + gaussian(nq, dim, 503, normalize=False) * 0.05
    qs = np.stack([o.normalize(q) for q in qs]).astype(np.float32)
    # pickProbes' scores: the 300-query batch (eight-query probe tiles) equals
    # single queries bit for bit, and both equal the oracle's f64 strided dot
    ps = idx.export_probe_scores(qs)
    # calls of fewer than eight queries take the one-query kernel
    ps1 = np.concatenate([idx.export_probe_scores(qs[s:s + 7]) for s in range(0, nq, 7)])
    assert np.array_equal(ps.view(np.uint32), ps1.view(np.uint32))
    rq = np.stack([o.rotate(q, dim)[0] for q in qs])
    for i in (0, 1, 7, 8, 150, nq - 1):
        assert np.array_equal(ps[i].view(np.uint32), idx.export_probe_scores(qs[i:i + 1])[0].view(np.uint32)), i
        assert np.array_equal(ps[i].view(np.uint32), o.probe_scores(cen, rq[i]).view(np.uint32)), i

    # probes + gather: k covers every candidate, so each query returns exactly
    # the rows of the 32 lists the oracle's pickProbes chooses
    rows, _, cnt = device_search(idx, qs, 0, 1024)
    for i in range(nq):
        probes, _ = o.topk_canonical(ps[i], 32)
        want = np.concatenate([lrows[off[c]:off[c + 1]] for c in probes])
        assert want.size <= 1024
        assert cnt[i] == want.size and set(rows[i, :cnt[i]].tolist()) == set(want.tolist()), i

    # the P = 1024 indexed scan, fetch 40 -> exact re-rank to 10: every query
    # of the batch (list-major path) and a few one at a time (fused scan, the
    # short tail) equal the oracle pipeline over the probed lists: top 40 by
    # code score, exact re-rank, canonical top 10, up to fetch-boundary
    # near-ties
    words = np.empty((n, idx.words_per_row), np.uint32)
    scales = np.empty(n, np.float32)
    for s0 in range(0, n, 10000):
        w, sc = idx.export_codes(s0, min(10000, n - s0))
        words[s0:s0 + w.shape[0]], scales[s0:s0 + w.shape[0]] = w, sc
    rows, scores, cnt = device_search(idx, qs, 40, 10)
    singles = {i: device_search(idx, qs[i:i + 1], 40, 10) for i in (0, 99, nq - 1)}
    for i in range(nq):
        probes, _ = o.topk_canonical(ps[i], 32)
        cand = np.concatenate([lrows[off[c]:off[c + 1]] for c in probes]).astype(np.uint32)
        approx = o.scan_quant(words, scales, rq[i], 8, cand=cand)
        tol = 2 * REL_TOL * float(scales[cand].max()) * float(np.abs(rq[i].astype(np.float64)).sum())
        assert cnt[i] == 10, i
        ex = lambda rr, q=qs[i]: o.rerank_scores(data, q, rr)  # noqa: E731
        assert_fetch_rerank(rows[i], scores[i], approx, cand, ex, 40, 10, tol, what=f"batch query {i}")
        if i in singles:
            r1, s1, c1 = singles[i]
            assert c1[0] == 10
            assert_fetch_rerank(r1[0], s1[0], approx, cand, ex, 40, 10, tol, what=f"single query {i}")
    idx.destroy()


def test_ivf_full_shape_build_properties(ctx):
    """4,000,000 x 768, 4096 lists, 20 Lloyd iterations on the 16,384-row
    sample: checked by properties the build must hold at full size."""
    import torch

    from browservec_amd import IVFQuantIndex

    n, dim, nlist = 4_000_000, 768, 4096
    say("ivf full shape build", n, dim, nlist)
    g = torch.Generator(device="cuda").manual_seed(0xB5EC0005)
    centres = torch.randn(nlist, dim, generator=g, device="cuda")
    centres /= centres.norm(dim=1, keepdim=True)
    x = torch.empty(n, dim, device="cuda")
    for s in range(0, n, 1 << 18):
        e = min(n, s + (1 << 18))
        lab = torch.randint(0, nlist, (e - s,), generator=g, device="cuda")
        blk = centres[lab] + 0.15 * torch.randn(e - s, dim, generator=g, device="cuda")
        x[s:e] = blk / blk.norm(dim=1, keepdim=True)
    torch.cuda.synchronize()
    ivf = {"nlist": nlist, "iters": 20, "nprobe": 32}
    built = []
    for rep in range(2):
        idx = IVFQuantIndex(ctx, dim, bits=8, ivf=ivf)
        idx.append_device(x.data_ptr(), n)
        idx.build()
        built.append((idx, idx.export_ivf()))
    del x
    torch.cuda.empty_cache()
    (idx, (cen, off, lrows)), (idx2, (cen2, off2, lrows2)) = built
    # a rebuild from the same rows is bit-identical
    assert np.array_equal(cen.view(np.uint32), cen2.view(np.uint32))
    assert np.array_equal(off, off2) and np.array_equal(lrows, lrows2)
    idx2.destroy()
    # spherical centroids: unit norm to f32 rounding
    norms = np.linalg.norm(cen.astype(np.float64), axis=1)
    assert np.all(np.abs(norms - 1.0) <= 1e-6), float(np.abs(norms - 1.0).max())
    # CSR: the lists partition the rows, ascending within each list
    assert off[0] == 0 and off[-1] == n and np.all(np.diff(off.astype(np.int64)) >= 0)
    assert np.array_equal(np.sort(lrows), np.arange(n, dtype=np.uint32))
    seg = np.repeat(np.arange(nlist), np.diff(off.astype(np.int64)))
    inside = seg[1:] == seg[:-1]
    assert np.all(lrows[1:][inside] > lrows[:-1][inside])
    # final assignment: sampled rows sit in the list of the centroid the
    # oracle's assignment picks for their codes (the same FMA chain)
    rng = np.random.default_rng(7)
    sample = np.sort(rng.choice(n, 1500, replace=False))
    list_of = np.empty(n, np.int64)
    list_of[lrows] = seg
    words = np.empty((sample.size, idx.words_per_row), np.uint32)
    scales = np.empty(sample.size, np.float32)
    for j, r in enumerate(sample):
        w, s = idx.export_codes(int(r), 1)
        words[j], scales[j] = w[0], s[0]
    want = o.assign_f32(dequant_f32(words, scales, 8, 1024), cen, order=1)
    assert np.array_equal(list_of[sample], want.astype(np.int64))
    idx.destroy()
