"""Shared helpers for the parity tests (not collected by pytest)."""

from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import oracle as o

REL_TOL = 1e-5  # fp32 scores: |gpu - oracle| <= 1e-5 * sum_i |term_i|


def need_gpu():
    try:
        import torch

        ok = torch.cuda.is_available()
    except Exception:
        ok = False
    if not ok:
        pytest.skip("no HIP device")


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def gaussian(rows: int, dim: int, seed: int, normalize: bool = True) -> np.ndarray:
    x = np.random.default_rng(seed).standard_normal((rows, dim)).astype(np.float32)
    if normalize:
        o.normalize_rows_store(x)
    return x


def clustered(rows: int, dim: int, nclusters: int, sigma: float, seed: int) -> np.ndarray:
    """Gaussian mixture: unit-norm centres + sigma * N(0,1), then normalized."""
    rng = np.random.default_rng(seed)
    centres = rng.standard_normal((nclusters, dim)).astype(np.float32)
    o.normalize_rows_store(centres)
    lab = rng.integers(0, nclusters, rows)
    x = (centres[lab] + sigma * rng.standard_normal((rows, dim)).astype(np.float32)).astype(np.float32)
    o.normalize_rows_store(x)
    return x


def dequant_matrix(codes: np.ndarray, bits: int) -> np.ndarray:
    """Dequantized code values without the row scale (f64), rows x P."""
    if bits == 8:
        b = codes.view(np.uint8).astype(np.int8).astype(np.float64)
        return np.maximum(b / 127.0, -1.0)
    if bits == 4:
        w = codes.astype(np.uint64)
        shifts = np.arange(8, dtype=np.uint64) * 4
        nib = ((w[:, :, None] >> shifts) & 0xF).astype(np.int64)
        nib = np.where(nib > 7, nib - 16, nib).astype(np.float64)
        return nib.reshape(codes.shape[0], -1)
    w = codes.astype(np.uint64)
    shifts = np.arange(32, dtype=np.uint64)
    bit = ((w[:, :, None] >> shifts) & 1).astype(np.float64)
    return (bit * 2 - 1).reshape(codes.shape[0], -1)


def quant_magnitude(codes, scales, q_rot, bits) -> np.ndarray:
    """sum_i |deq_i * q_i| * scale per row: the scale of a dot product's
    rounding error, used for the 1e-5 relative tolerance."""
    d = dequant_matrix(codes, bits)
    m = np.abs(d) @ np.abs(q_rot.astype(np.float64))
    s = np.abs(scales.astype(np.float64)) * ((1.0 / 7.0) if bits == 4 else 1.0)
    return m * s


def assert_scores_close(got, want, mag, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bound = REL_TOL * np.maximum(np.asarray(mag, np.float64), np.abs(want))
    bad = np.nonzero(err > bound)[0]
    assert bad.size == 0, f"{what}: {bad.size} scores beyond tolerance, e.g. row {bad[:5]} err {err[bad[:5]]}"


def assert_topk_near(got_rows, ref_scores, k, tol_abs, what=""):
    """The device's top-k ID set equals the oracle's top-k, except for rows
    whose oracle score is within tol_abs of the oracle's k-th score."""
    ref_scores = np.asarray(ref_scores, np.float32)
    want_rows, want_s = o.topk_canonical(ref_scores, k)
    got = set(int(r) for r in got_rows)
    want = set(int(r) for r in want_rows)
    assert len(got) == len(got_rows), f"{what}: duplicate rows"
    if got == want:
        return
    kth = float(want_s[-1]) if len(want_s) else 0.0
    for r in got ^ want:
        assert abs(float(ref_scores[r]) - kth) <= tol_abs, (
            f"{what}: row {r} differs (score {ref_scores[r]}, k-th {kth})")


def fetch_window(approx, ids, fetch: int, tol: float):
    """The oracle pipeline's fetch (src/index.ts:414-418): the top-`fetch`
    rows by approximate score, ties by row.  Returns (sure, maybe): `sure`
    holds the rows whose approximate score exceeds the fetch-th score by more
    than tol (every scan whose scores are within tol / 2 of the oracle's
    fetches them), `maybe` the rows within tol of it (a fetch-boundary
    near-tie: such a scan may or may not fetch them).  Every other row is
    fetched by no such scan."""
    approx = np.asarray(approx, np.float64)
    ids = np.asarray(ids, np.int64)
    nf = min(fetch, ids.size)
    order = np.lexsort((ids, -approx))
    kth = approx[order[nf - 1]]
    sure = ids[approx > kth + tol]
    maybe = ids[np.abs(approx - kth) <= tol]
    return sure, maybe


def assert_fetch_rerank(got_rows, got_scores, approx, ids, exact_fn, fetch: int, k: int, tol: float, what=""):
    """A fetch -> exact re-rank -> top-k answer equals the oracle pipeline's
    (top-`fetch` by approximate score, exact re-rank, canonical top-k by
    exact score and row), allowing only fetch-boundary near-ties: rows whose
    approximate score is within tol of the fetch-th may be in or out of the
    fetch.  exact_fn(rows) gives the oracle's exact f32 scores.  Fails on a
    wrong order, a row outside the fetch window, a score that is not the
    exact score, or a fetched row that beats the last row returned."""
    got_rows = [int(r) for r in got_rows]
    sure, maybe = fetch_window(approx, ids, fetch, tol)
    nf = min(fetch, np.asarray(ids).size)
    assert len(got_rows) == min(k, nf), f"{what}: {len(got_rows)} rows, want {min(k, nf)}"
    assert len(set(got_rows)) == len(got_rows), f"{what}: duplicate rows"
    allowed = set(sure.tolist()) | set(maybe.tolist())
    out = [r for r in got_rows if r not in allowed]
    assert not out, f"{what}: rows {out} are outside the oracle's fetch window"
    ex = exact_fn(np.array(got_rows, np.uint32))
    got_scores = np.asarray(got_scores, np.float32)
    assert np.array_equal(got_scores.view(np.uint32), ex.view(np.uint32)), f"{what}: scores are not the exact scores"
    keys = [(float(s), -r) for s, r in zip(ex, got_rows)]
    assert keys == sorted(keys, reverse=True), f"{what}: rows not in (score desc, row asc) order"
    rest = np.array(sorted(set(sure.tolist()) - set(got_rows)), np.uint32)
    if rest.size and len(got_rows) == k:
        er = exact_fn(rest)
        last = keys[-1]
        beat = [int(r) for r, s in zip(rest, er) if (float(s), -int(r)) > last]
        assert not beat, f"{what}: fetched rows {beat[:5]} beat the last row returned"
