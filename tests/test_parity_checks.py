"""The strict fetch -> re-rank check itself (CPU): it accepts the oracle
pipeline's answer and rejects permuted, substituted, truncated and
mis-scored answers."""

import numpy as np
import pytest

from oracle import oracle as o
from tests.helpers import assert_fetch_rerank, fetch_window


def _case(seed, n=5000, fetch=100, k=10):
    rng = np.random.default_rng(seed)
    approx = rng.standard_normal(n).astype(np.float32)
    # exact scores correlated with the approximate ones, so the fetch matters
    exact = (approx + 0.3 * rng.standard_normal(n)).astype(np.float32)
    cand, _ = o.topk_canonical(approx, fetch)
    want, ws = o.topk_canonical(exact[cand], k, ids=cand)
    return approx, exact, want, ws


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_accepts_the_oracle_pipeline(seed):
    approx, exact, want, ws = _case(seed)
    assert_fetch_rerank(want, ws, approx, np.arange(approx.size), lambda r: exact[r], 100, 10, 0.0)


def test_rejects_wrong_answers():
    approx, exact, want, ws = _case(4)
    ids = np.arange(approx.size)
    ex = lambda r: exact[r]  # noqa: E731
    # permuted
    pr, ps = want.copy(), ws.copy()
    pr[[0, 1]], ps[[0, 1]] = pr[[1, 0]], ps[[1, 0]]
    with pytest.raises(AssertionError):
        assert_fetch_rerank(pr, ps, approx, ids, ex, 100, 10, 0.0)
    # a row from outside the fetch replaces the last one
    sure, maybe = fetch_window(approx, ids, 100, 0.0)
    outside = next(r for r in np.argsort(-exact) if r not in set(sure.tolist()) | set(maybe.tolist()))
    sr = np.concatenate([want[:-1], [outside]]).astype(np.uint32)
    ss = exact[sr]
    order = np.lexsort((sr, -ss.astype(np.float64)))
    with pytest.raises(AssertionError):
        assert_fetch_rerank(sr[order], ss[order], approx, ids, ex, 100, 10, 0.0)
    # a fetched row that does not make the top 10 replaces one that does
    cand, _ = o.topk_canonical(approx, 100)
    worse = next(int(r) for r in cand[::-1] if int(r) not in set(want.tolist()))
    sr = np.concatenate([want[:4], want[5:], [worse]]).astype(np.uint32)
    ss = exact[sr]
    order = np.lexsort((sr, -ss.astype(np.float64)))
    with pytest.raises(AssertionError):
        assert_fetch_rerank(sr[order], ss[order], approx, ids, ex, 100, 10, 0.0)
    # too few rows
    with pytest.raises(AssertionError):
        assert_fetch_rerank(want[:9], ws[:9], approx, ids, ex, 100, 10, 0.0)
    # a score that is not the exact score
    bad = ws.copy()
    bad[3] = np.nextafter(bad[3], np.float32(np.inf))
    with pytest.raises(AssertionError):
        assert_fetch_rerank(want, bad, approx, ids, ex, 100, 10, 0.0)


def test_near_tie_at_the_fetch_boundary_is_allowed():
    approx, exact, want, ws = _case(5)
    ids = np.arange(approx.size)
    cand, cs = o.topk_canonical(approx, 100)
    # a row just outside the fetch whose approximate score is within the
    # tolerance of the 100th: a scan with slightly different scores may fetch
    # it instead of the 100th
    nxt, _ = o.topk_canonical(approx, 101)
    r101, r100 = int(nxt[100]), int(cand[99])
    tol = float(cs[99] - approx[r101]) * 1.01 + 1e-12
    alt = [int(r) for r in cand if int(r) != r100] + [r101]
    alt = np.array(alt, np.uint32)
    wr, wsc = o.topk_canonical(exact[alt], 10, ids=alt)
    assert_fetch_rerank(wr, wsc, approx, ids, lambda r: exact[r], 100, 10, tol)
