"""Graph beam search (HNSW layer 0): HNSWGpuSearcher (src/index/hnswGpu.ts:
28-244) with the shader's best-first beam (src/engine/wgsl/graphSearch.ts:
62-259), against the oracle's restatement with the shader's lanes in lane
order: raw beams bit for bit (distances and ids, slot by slot), and the
searcher's seeds, dedup and top-k."""

import numpy as np
import pytest

from oracle import oracle as o
from tests.helpers import clustered, gaussian, need_gpu, say

pytestmark = pytest.mark.gpu
EMPTY = 0xFFFFFFFF


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    from browservec_amd import DeviceContext

    c = DeviceContext(0)
    yield c
    c.destroy()


def knn_graph(x, K, metric, seed, holes=0.0):
    """Fixed-degree adjacency: each row's K nearest (f64 scores, self
    excluded, blockwise), a fraction of slots emptied."""
    n = x.shape[0]
    x64 = x.astype(np.float64)
    g = np.empty((n, K), np.uint32)
    for s in range(0, n, 1024):
        blk = x64[s:s + 1024]
        if metric == "l2":
            sc = -(np.sum(blk * blk, 1)[:, None] - 2 * blk @ x64.T + np.sum(x64 * x64, 1)[None, :])
        else:
            sc = blk @ x64.T
        sc[np.arange(blk.shape[0]), np.arange(s, s + blk.shape[0])] = -np.inf
        g[s:s + blk.shape[0]] = np.argsort(-sc, axis=1, kind="stable")[:, :K]
    if holes:
        rng = np.random.default_rng(seed)
        g[rng.random(g.shape) < holes] = EMPTY
    return g


@pytest.mark.parametrize("metric,dim,n,K,ef,holes", [("dot", 48, 3000, 16, 64, 0.0), ("l2", 37, 2500, 24, 40, 0.1),
                                                     ("cosine", 128, 4000, 32, 256, 0.0),
                                                     ("dot", 96, 2000, 64, 100, 0.2)])
def test_beams_equal_the_oracle(ctx, metric, dim, n, K, ef, holes):
    from browservec_amd import GraphSearcher

    say("graph beams", metric, dim, n, K, ef)
    x = clustered(n, dim, 40, 0.2, seed=dim + K)
    if metric == "cosine":
        o.normalize_rows_store(x)
    g = knn_graph(x, K, metric, seed=K, holes=holes)
    gs = GraphSearcher(ctx, dim, metric, K)
    gs.append(x[:n // 2], n // 2)
    gs.append(x[n // 2:], n - n // 2)
    gs.upload_graph(g, n)
    qs = gaussian(20, dim, 5 + dim)
    if metric == "cosine":
        qs = o.normalize_rows_store(qs.copy())
    e = o.graph_entries(17, n)
    for iters in (ef, 5):
        d_gpu, i_gpu = gs.search_beams(qs, e, ef, iters)
        d_cpu, i_cpu = o.graph_search(x, g, qs, e, ef, iters, l2=(metric == "l2"))
        assert np.array_equal(i_gpu, i_cpu)
        assert np.array_equal(d_gpu.view(np.uint32), d_cpu.view(np.uint32))
    # the searcher: seeds from the entry, width max(ef, k), dedup, sort, k
    for k in (10, ef + 7, 300):
        hits = gs.search(qs, qs.shape[0], k, ef, 17)
        efa = min(max(ef, k), 256)
        d_cpu, i_cpu = o.graph_search(x, g, qs, e, efa, efa, l2=(metric == "l2"))
        for i in range(qs.shape[0]):
            want_r, want_s = o.graph_hits(d_cpu[i], i_cpu[i], efa, k)
            assert [h.row for h in hits[i]] == want_r.tolist(), (k, i)
            assert np.array_equal(np.float32([h.score for h in hits[i]]).view(np.uint32), want_s.view(np.uint32))
    gs.destroy()


def test_partial_adjacency_bad_ids_and_shedding(ctx):
    """An adjacency that covers only the first rows (the rest have no
    neighbours), ids past the corpus (skipped), duplicate seeds, and a wide
    beam on a degree-64 graph whose visits overflow the 2048-slot visited
    table (shed ids come back unseen)."""
    from browservec_amd import GraphSearcher

    say("graph edge cases")
    dim, n, K = 32, 6000, 64
    x = gaussian(n, dim, 61)
    g = knn_graph(x, K, "dot", seed=3)
    g[::7, 5] = n + 11  # past the corpus
    gs = GraphSearcher(ctx, dim, "dot", K)
    gs.append(x, n)
    gs.upload_graph(g[:4000], 4000)  # rows 4000.. have no neighbours
    qs = gaussian(16, dim, 62)
    e = np.array([3, 3, 4100, 5999, n + 5, 0], np.uint32)
    d_gpu, i_gpu = gs.search_beams(qs, e, 256, 256)
    d_cpu, i_cpu = o.graph_search(x, g[:4000], qs, e, 256, 256)
    assert np.array_equal(i_gpu, i_cpu) and np.array_equal(d_gpu.view(np.uint32), d_cpu.view(np.uint32))
    live = i_cpu[i_cpu != EMPTY]
    assert live.size > 0
    gs.destroy()


def test_recall_and_errors(ctx):
    from browservec_amd import GraphSearcher
    from browservec_amd._lib import BVError

    say("graph recall")
    dim, n, K = 64, 8000, 32
    x = clustered(n, dim, 64, 0.15, seed=9)
    o.normalize_rows_store(x)
    g = knn_graph(x, K, "cosine", seed=1)
    gs = GraphSearcher(ctx, dim, "cosine", K)
    gs.append(x, n)
    gs.upload_graph(g, n)
    qs = o.normalize_rows_store((x[:50] + 0.05 * gaussian(50, dim, 3, normalize=False)).astype(np.float32))
    hits = gs.search(qs, 50, 10, 64, 0)
    truth = np.argsort(-(qs.astype(np.float64) @ x.astype(np.float64).T), axis=1)[:, :10]
    rec = np.mean([len({h.row for h in hits[i]} & set(truth[i].tolist())) / 10 for i in range(50)])
    assert rec >= 0.9, rec
    with pytest.raises(BVError, match="degree"):
        GraphSearcher(ctx, dim, "cosine", 65)
    with pytest.raises(BVError, match=f"expected {dim} floats"):
        gs.append(x[0, :dim - 1], 1)
    empty = GraphSearcher(ctx, dim, "cosine", K)
    with pytest.raises(BVError, match="adjacency"):
        empty.search(qs[:1], 1, 10, 64, 0)
    empty.destroy()
    gs.destroy()
