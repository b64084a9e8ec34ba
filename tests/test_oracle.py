"""Pins the CPU oracle before it is trusted as the checker.

Sources of truth, in order of strength:
  * known answers from the reference's own unit tests (file:line cited);
  * tests/golden/js_vectors.json, written under node's V8 by
    tests/golden/make_js_vectors.js -- exact JS-number semantics;
  * closed forms and independent brute force (numpy f64, long double, Python
    integers), chosen so a dropped term, wrong sign or transposed index fails.
"""

import json
import os

import numpy as np
import pytest

from oracle import oracle as o

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "js_vectors.json")


@pytest.fixture(scope="module")
def js():
    with open(GOLDEN) as f:
        return json.load(f)


def bits_to_f32(bits):
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


def f32_bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ------------------------------------------------------------------ prng
def test_mulberry32_matches_js_engine(js):
    for case in js["mulberry32"]:
        got = o.mulberry32_stream(case["seed"], len(case["draws"]))
        assert np.array_equal(got, np.asarray(case["draws"], dtype=np.float64)), case["seed"]


def test_mulberry32_properties():
    # tests/unit/prng.test.ts:4-37: determinism, range, mean
    a = o.mulberry32_stream(42, 100)
    assert np.array_equal(a, o.mulberry32_stream(42, 100))
    assert not np.array_equal(o.mulberry32_stream(1, 20), o.mulberry32_stream(2, 20))
    r = o.mulberry32_stream(0xDEADBEEF, 10_000)
    assert r.min() >= 0 and r.max() < 1
    m = o.mulberry32_stream(7, 50_000).mean()
    assert 0.48 < m < 0.52


def test_random_signs_match_js_engine(js):
    for case in js["signs"]:
        assert o.round_seed(o.DEFAULT_SEED, case["round"]) == case["seed"]
        got = f32_bits(o.random_signs(64, case["seed"]))
        assert np.array_equal(got, np.asarray(case["bits"], dtype=np.uint32))


def test_round_seed_closed_form():
    # (seed ^ (0x9e3779b9 * (r+1))) >>> 0 with the product reduced mod 2^32
    for seed in (0, 1, 0x9E3779B9, 0xFFFFFFFF):
        for r in range(5):
            assert o.round_seed(seed, r) == (seed ^ ((0x9E3779B9 * (r + 1)) % 2**32))
    assert o.round_seed(0, 1) == 0x3C6EF372


# -------------------------------------------------------------- rotator
def test_pad_to_pow2_table():
    # tests/unit/rotator.test.ts:18-28
    for n, p in [(1, 4), (4, 4), (5, 8), (384, 512), (768, 1024), (1024, 1024), (1536, 2048)]:
        assert o.pad_to_pow2(n) == p


def test_fwht_unit_impulse_and_involution():
    v = np.zeros(8, np.float32)
    v[0] = 1
    assert np.array_equal(o.fwht(v), np.ones(8, np.float32))  # rotator.test.ts:40-46
    rng = np.random.default_rng(0)
    x = rng.integers(-50, 50, size=64).astype(np.float32)  # small ints: exact in f32
    assert np.array_equal(o.fwht(o.fwht(x)), x * 64)


def test_fwht_matches_hadamard_matrix():
    n = 32
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    rng = np.random.default_rng(1)
    x = rng.integers(-1000, 1000, size=n).astype(np.float32)
    assert np.array_equal(o.fwht(x).astype(np.float64), H @ x.astype(np.float64))


def test_rotation_matches_js_engine(js):
    for case in js["rotate"]:
        x = bits_to_f32(case["input"])
        got = o.rotate(x, case["dim"], case["seed"], case["rounds"])[0]
        assert np.array_equal(f32_bits(got), np.asarray(case["output"], dtype=np.uint32)), case["dim"]


def test_rotation_orthonormal_and_close_to_f64():
    # rotator.test.ts:50-60, plus an independent f64 restatement
    dim = 100
    a = o.uniform_vectors(1, dim, 2)[0]
    b = o.uniform_vectors(1, dim, 3)[0]
    ra = o.rotate(a, dim, 12345)[0]
    rb = o.rotate(b, dim, 12345)[0]
    assert abs(float(ra.astype(np.float64) @ rb) - float(a.astype(np.float64) @ b)) < 1e-5
    assert abs(float(ra.astype(np.float64) @ ra) - float(a.astype(np.float64) @ a)) < 1e-5
    P = o.pad_to_pow2(dim)
    signs = o.rotator_signs(dim, 12345, 2).astype(np.float64)
    x = np.zeros(P)
    x[:dim] = a
    H = np.array([[1.0]])
    while H.shape[0] < P:
        H = np.block([[H, H], [H, -H]])
    for r in range(2):
        x = H @ (x * signs[r])
    assert np.max(np.abs(x - ra)) <= 1e-6 * np.max(np.abs(x))


def test_rotator_signs_scaled():
    s = o.rotator_signs(768, o.DEFAULT_SEED, 2)
    assert s.shape == (2, 1024)
    assert set(np.unique(s).tolist()) == {-1 / 32, 1 / 32}  # exactly +-2^-5
    s512 = o.rotator_signs(384, 1, 2)
    assert np.all(np.abs(s512) == np.float32(1 / np.sqrt(512)))


# ---------------------------------------------------------------- codecs
def test_codecs_match_js_engine(js):
    for case in js["codec"]:
        x = bits_to_f32(case["input"])
        for bits, key in ((8, "q8"), (4, "q4"), (1, "q1")):
            want = case[key]
            if want is None:
                continue
            words, scale = o.quantize_row(x, bits)
            assert np.array_equal(words, np.asarray(want["words"], dtype=np.uint32)), (key, x.size)
            assert int(f32_bits(scale)) == want["scale_f32"], key


def test_codec_known_answers():
    # tests/unit/codec.test.ts:30-47, 99-103
    w, s = o.quantize_row([0.5, -2.5, 1, 0], 8)
    assert s == np.float32(2.5)
    # codes: round(0.2*127)=25, -127, round(0.4*127)=51, 0
    assert w[0] == (25 | (0x81 << 8) | (51 << 16) | (0 << 24))
    back = o.dequant_row(w, s, 8)
    assert abs(back[1] + 2.5) < 1e-4
    w, s = o.quantize_row(np.zeros(16, np.float32), 8)
    assert s == 1 and not w.any()
    w, s = o.quantize_row(np.zeros(32, np.float32), 1)
    assert w[0] == 0xFFFFFFFF
    with pytest.raises(ValueError, match="multiple of 4"):
        o.quantize_row(np.zeros(7, np.float32), 8)
    with pytest.raises(ValueError, match="multiple of 8"):
        o.quantize_row(np.zeros(12, np.float32), 4)
    with pytest.raises(ValueError, match="multiple of 32"):
        o.quantize_row(np.zeros(48, np.float32), 1)


@pytest.mark.parametrize("bits,levels", [(8, 127), (4, 7)])
def test_codec_round_trip_bound(bits, levels):
    # codec.test.ts:20-28, 55-63
    v = o.uniform_vectors(1, 64, 1 if bits == 8 else 3, scale=3.0)[0]
    w, s = o.quantize_row(v, bits)
    back = o.dequant_row(w, s, bits)
    step = float(s) / levels
    assert np.all(np.abs(back.astype(np.float64) - v) <= step / 2 + 1e-6)


def test_codec_rounding_ties_go_up():
    # Inputs whose scaled value is exactly k + 0.5 in f64: x = (k+0.5)/127 * scale
    # with scale = 1 (max element 1.0).  Math.round sends ties toward +inf.
    ks = np.arange(-126, 126)
    x = np.concatenate([[1.0], (ks + 0.5) / 127.0]).astype(np.float32)
    x = x[: (x.size // 4) * 4]
    w, s = o.quantize_row(x, 8)
    assert s == 1.0
    codes = w.view(np.uint8).astype(np.int8).astype(np.int64)
    # expected: compute in f64 exactly as the reference does, with ties up
    y = x.astype(np.float64) * (1.0 / 1.0) * 127.0
    r = np.floor(y)
    r = np.where(y - r >= 0.5, r + 1, r)
    assert np.array_equal(codes, np.clip(r, -127, 127).astype(np.int64))


def test_codec_1bit_scale_is_sequential_mean():
    v = o.uniform_vectors(1, 64, 5, scale=3.0)[0]
    w, s = o.quantize_row(v, 1)
    acc = 0.0
    for x in v.astype(np.float64):
        acc += abs(x)
    assert s == np.float32(acc / 64)
    back = o.dequant_row(w, s, 1)
    assert np.array_equal(np.sign(back), np.where(v >= 0, 1, -1).astype(np.float32))


def test_encode_equals_rotate_then_quantize():
    # tests/unit/encode.test.ts:15-46
    for bits in (8, 4, 1):
        dim = 48 if bits == 8 else 40
        data = o.uniform_vectors(5, dim, 1)
        words, scales, rot = o.encode(data, dim, bits, seed=11, want_rotated=True)
        r = o.rotate(data, dim, 11, 2)
        assert np.array_equal(rot, r)
        for i in range(5):
            w, s = o.quantize_row(r[i], bits)
            assert np.array_equal(words[i], w) and scales[i] == s
    # wordsPerRow at dim 384: 128/64/16 (encode.test.ts:48-53)
    for bits, wpr in ((8, 128), (4, 64), (1, 16)):
        w, _, _ = o.encode(np.zeros((1, 384), np.float32), 384, bits)
        assert w.shape[1] == wpr


# ---------------------------------------------------------------- store
def test_store_arithmetic_matches_js_engine(js):
    for case in js["store"]:
        a, q = bits_to_f32(case["a"]), bits_to_f32(case["q"])
        assert o.dot_row(a, q) == case["dot"]
        assert o.l2_row(a, q) == case["l2"]
        assert int(f32_bits(np.float32(o.dot_row(a, q)))) == case["dot_f32"]
        assert np.array_equal(f32_bits(o.normalize(a)), np.asarray(case["normalized"], dtype=np.uint32))


def test_store_known_answers_and_long_double():
    n = o.normalize([3, 4])  # store.test.ts:5-14
    assert abs(n[0] - 0.6) < 1e-6 and abs(n[1] - 0.8) < 1e-6
    assert not o.normalize(np.zeros(4, np.float32)).any()
    a = o.uniform_vectors(1, 771, 9)[0]
    q = o.uniform_vectors(1, 771, 10)[0]
    d, _ = o.dot_exact(a, q)
    assert abs(o.dot_row(a, q) - d[0]) <= 1e-12 * 771
    assert np.float32(o.dot_row(a, q)) == np.float32(d[0]) or abs(np.float32(o.dot_row(a, q)) - d[0]) < 1e-6


# ------------------------------------------------------------------ scans
def _dequant_dot(codes, scales, P, bits, q):
    deq = np.stack([o.dequant_row(codes[i], 1.0, bits) for i in range(codes.shape[0])]).astype(np.float64)
    if bits == 8:
        deq = np.stack([np.maximum(((codes[i].view(np.uint8).astype(np.int8)).astype(np.float64)) / 127.0, -1)
                        for i in range(codes.shape[0])])
    exact = (deq @ q.astype(np.float64)) * scales.astype(np.float64)
    mag = (np.abs(deq) @ np.abs(q.astype(np.float64))) * np.abs(scales.astype(np.float64))
    return exact, mag


@pytest.mark.parametrize("bits", [8, 4, 1])
def test_quant_scans_vs_f64_brute_force(bits):
    dim = 96
    data = o.uniform_vectors(50, dim, 3, normalize=True)
    codes, scales, _ = o.encode(data, dim, bits)
    q = o.rotate(o.uniform_vectors(1, dim, 4, normalize=True)[0], dim)[0]
    got = o.scan_quant(codes, scales, q, bits)
    exact, mag = _dequant_dot(codes, scales, 128, bits, q)
    assert np.all(np.abs(got - exact) <= 1e-6 * np.maximum(mag, 1e-30))
    # indexed mode reads cand[i]
    cand = np.array([7, 3, 3, 49], np.uint32)
    assert np.array_equal(o.scan_quant(codes, scales, q, bits, cand), got[cand])


@pytest.mark.parametrize("metric", ["cosine", "l2"])
def test_f32_scan_vs_long_double(metric):
    for dim in (64, 67):
        data = o.uniform_vectors(40, dim, 5)
        q = o.uniform_vectors(1, dim, 6)[0]
        got = o.scan_f32(data, q, metric)
        if metric == "l2":
            d = data.astype(np.float64) - q
            exact = -(d * d).sum(1)
            mag = -exact
        else:
            exact, mag = o.dot_exact(data, q)
        assert np.all(np.abs(got - exact) <= 1e-6 * np.maximum(np.abs(mag), 1e-30))


def test_hamming_and_int8sym_vs_integer_brute_force():
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 2**32, size=(30, 32), dtype=np.uint64).astype(np.uint32)
    qb = rng.integers(0, 2**32, size=32, dtype=np.uint64).astype(np.uint32)
    got = o.scan_hamming(codes, 1024, qb)
    for i in range(30):
        pc = sum(bin(int(c) ^ int(b)).count("1") for c, b in zip(codes[i], qb))
        assert got[i] == 1024 - 2 * pc
    c8 = rng.integers(-127, 128, size=(20, 64)).astype(np.int8)
    q8 = rng.integers(-127, 128, size=64).astype(np.int8)
    got = o.scan_int8sym(c8.view(np.uint32).reshape(20, 16), 64, q8.view(np.uint32))
    want = [sum(int(a) * int(b) for a, b in zip(c8[i], q8)) for i in range(20)]
    assert got.tolist() == want


def test_query_bits_rule():
    q = np.array([0.0, -0.0, 1.0, -1.0] + [np.nan] + [0.5] * 27, np.float32)
    b = o.query_bits(q)[0]
    assert b & 1 and b & 2 and b & 4 and not b & 8 and not b & 16


# ------------------------------------------------------- wasm baseline
@pytest.mark.parametrize("dim", [384, 767, 3])
def test_wasm_sse_equals_scalar_lane_emulation(dim):
    data = o.uniform_vectors(64, dim, 11)
    q = o.uniform_vectors(1, dim, 12)[0]
    assert np.array_equal(f32_bits(o.wasm_scan(data, q)), f32_bits(o.wasm_scan(data, q, scalar=True)))
    exact, mag = o.dot_exact(data, q)
    assert np.all(np.abs(o.wasm_scan(data, q) - exact) <= 1e-6 * mag)
    d = data.astype(np.float64) - q
    assert np.allclose(o.wasm_scan(data, q, "l2"), -(d * d).sum(1), rtol=1e-5)


# ----------------------------------------------------------------- top-k
def test_topk_known_answers(js):
    for case in js["topk"]:
        rows, _ = o.topk_ref(np.asarray(case["scores"], np.float32), case["k"])
        assert rows.tolist() == case["rows"], case["scores"][:6]
    rows, _ = o.topk_ref([3, 1, 2], 10)  # topk.test.ts:31-35
    assert rows.tolist() == [0, 2, 1]
    assert o.topk_ref([1, 2], 0)[0].size == 0
    rows, s = o.topk_ref([-5, -1, -3], 2)
    assert rows.tolist() == [1, 2] and s.tolist() == [-1, -3]


def test_topk_matches_full_sort():
    # topk.test.ts:16-30 (distinct scores -> order fully determined)
    d = o.mulberry32_stream(1, 3000)
    off = 0
    for n, k in ((100, 10), (1000, 1), (1000, 50), (17, 17)):
        s = (d[off:off + n] * 200 - 100).astype(np.float32)
        off += n
        rows, sc = o.topk_ref(s, k)
        want = np.argsort(-s.astype(np.float64), kind="stable")[:k]
        assert rows.tolist() == want.tolist()
        crow, _ = o.topk_canonical(s, k)
        assert crow.tolist() == want.tolist()


def test_topk_canonical_ties_and_floor():
    s = np.array([5, 5, 7, -0.0, 0.0, -3.4e38], np.float32)
    rows, _ = o.topk_canonical(s, 2)
    assert rows.tolist() == [2, 0]  # canonical: lower row among ties
    rows, _ = o.topk_ref(s[:3], 2)
    assert rows.tolist() == [2, 1]  # reference semantics evict the lower row
    rows, _ = o.topk_canonical(s, 10, floor=-3.39e38)
    assert rows.tolist() == [2, 0, 1, 3, 4]  # -0 ties +0, order by row
    ids = np.array([10, 9, 8, 7, 6, 5], np.uint32)
    rows, _ = o.topk_canonical(s, 2, ids=ids)
    assert rows.tolist() == [8, 9]


def test_merge_partials_skips_fillers():
    scores = np.array([3, 2, -3.4e38, 9, 1, 0.5], np.float32)
    rows = np.array([0, 1, 2, 300, 4, 5], np.uint32)
    r, s = o.merge_partials(scores, rows, n=10, k=3)
    # row 300 >= n is dropped; the f32 filler (> f64 -3.4e38) survives the
    # score test but sorts last
    assert r.tolist() == [0, 1, 4]


# --------------------------------------------------------------- k-means
def test_kmeans_known_answers():
    # kmeans.test.ts:94-103 (normalizeRows) and 115-123 (updateCentroids, no
    # normalization there -- checked against the un-normalized mean here)
    m = o.normalize_rows(np.array([[3, 4], [0, 0]], np.float32))
    assert np.allclose(m, [[0.6, 0.8], [0, 0]], atol=1e-6)
    sample = np.array([[0, 0], [2, 2], [10, 10]], np.float32)
    c, counts = o.update_centroids(sample, [0, 0, 1], np.zeros((2, 2), np.float32), seed=1)
    assert counts.tolist() == [2, 1]
    assert np.allclose(c, o.normalize_rows(np.array([[1, 1], [10, 10]], np.float32)))
    # empty cluster re-seeded from a sample row (kmeans.test.ts:125-135)
    sample = np.array([[1, 2], [3, 4]], np.float32)
    c, counts = o.update_centroids(sample, [0, 0], np.zeros((2, 2), np.float32), seed=5)
    assert counts.tolist() == [2, 0]
    seeds = o.normalize_rows(sample)
    assert any(np.array_equal(c[1], seeds[i]) for i in range(2))


def test_random_init_picks_match_js_engine(js):
    """The rows randomInitCentroids copies (kmeans.ts:154-170), pinned by the
    picks V8 computed: each sample row is a distinct unit vector (angle
    2*pi*r/count), so the row behind every centroid is recoverable."""
    for case in js["init_picks"]:
        count, nlist = case["count"], case["nlist"]
        ang = 2 * np.pi * np.arange(count) / count
        sample = np.stack([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
        cen = o.random_init_centroids(sample, nlist, case["seed"])
        got = np.argmax(cen.astype(np.float64) @ sample.astype(np.float64).T, axis=1)
        assert got.tolist() == case["picks"], case["seed"]


def test_update_centroids_matches_js_engine(js):
    """updateCentroids (kmeans.ts:177-209) against V8's Float32Array run on a
    sample whose sequential f32 column sums differ from the f64 sums (a large
    value absorbs later small ones), with an empty cluster re-seeded from the
    sample and normalizeRows after."""
    m = js["mean_update"]
    assert m["col0_f32_sum"] != m["col0_f64_sum"]  # the fixture separates the two
    sample = bits_to_f32(m["sample"]).reshape(m["count"], m["dim"])
    cen_in = bits_to_f32(m["centroids_in"]).reshape(m["nlist"], m["dim"])
    got, counts = o.update_centroids(sample, np.array(m["assign"], np.uint32), cen_in, m["seed"])
    assert np.array_equal(f32_bits(got).reshape(-1), np.asarray(m["centroids_out"], np.uint32))
    assert counts.tolist() == [int(np.sum(np.array(m["assign"]) == c)) for c in range(m["nlist"])]
    # an f64 accumulation gives a different centroid 0: the check separates them
    f64 = sample[np.array(m["assign"]) == 0].astype(np.float64).sum(axis=0) / counts[0]
    f64 = (f64 / np.linalg.norm(f64)).astype(np.float32)
    assert not np.array_equal(f32_bits(f64), f32_bits(got[0]))


def test_assign_argmax_lowest_index_wins():
    rows = np.array([[1, 0, 0, 0]], np.float32)
    cents = np.array([[0, 1, 0, 0], [1, 0, 0, 0], [1, 0, 0, 0]], np.float32)
    assert o.assign_f32(rows, cents, 0).tolist() == [1]
    assert o.assign_f32(rows, cents, 1).tolist() == [1]
    rng = np.random.default_rng(2)
    x = rng.standard_normal((50, 16)).astype(np.float32)
    c = rng.standard_normal((7, 16)).astype(np.float32)
    want = np.argmax(x.astype(np.float64) @ c.T.astype(np.float64), axis=1)
    assert np.array_equal(o.assign_f32(x, c, 0), want)
    assert np.array_equal(o.assign_f32(x, c, 1), want)


def test_assign_vector_path_equals_scalar_chain():
    """The AVX2 assignment (eight centroids per lane group, four groups in
    flight) runs each lane's fmaf chain exactly as the scalar loop: equal
    assignments, including ties between duplicated centroids and a centroid
    count that leaves partial lane groups."""
    rng = np.random.default_rng(12)
    x = rng.standard_normal((300, 96)).astype(np.float32)
    c = rng.standard_normal((37, 96)).astype(np.float32)
    c[20] = c[3]
    c[36] = c[3]
    x[:10] = c[3]
    a1 = o.assign_f32(x, c, 1)
    assert np.array_equal(a1, o.assign_f32(x, c, 2))
    assert np.all(a1[:10] == 3)


def test_probe_scores_vs_long_double():
    c = o.uniform_vectors(9, 64, 1, normalize=True)
    q = o.uniform_vectors(1, 64, 2)[0]
    got = o.probe_scores(c, q)
    exact, _ = o.dot_exact(c, q)
    assert np.array_equal(got, exact.astype(np.float32)) or np.all(np.abs(got - exact) < 1e-6)


def test_csr_and_tuning_tables():
    off, rows = o.build_csr([2, 0, 2, 1, 0], 3)
    assert off.tolist() == [0, 2, 3, 5] and rows.tolist() == [1, 4, 3, 0, 2]
    ranks = [0, 0, 0, 0, 0, 0, 1, 1, 1, 7]  # ivfTune.test.ts:9-16
    assert o.choose_nprobe(ranks, 16, 0.5) == (1, 0.6)
    assert o.choose_nprobe(ranks, 16, 0.9) == (2, 0.9)
    assert o.choose_nprobe(ranks, 16, 0.95) == (8, 1.0)
    assert o.choose_nprobe([0, 4], 5, 1) == (5, 1.0)
    assert o.choose_nprobe([], 16, 0.95) == (16, 1.0)
    assert o.choose_nprobe([], 0, 0.95) == (1, 1.0)
    assert o.choose_nprobe([0, 1, 1, 3], 8, 0.75) == (2, 0.75)
    assert o.pick_tune_queries(5, 32) == [0, 1, 2, 3, 4]
    p = o.pick_tune_queries(1000, 32)
    assert len(set(p)) == 32 and p == sorted(p) and max(p) < 1000


def test_reservoir_matches_js_engine(js):
    """Slots of the IVF reservoir (ivfquant.ts:114-124, 235-245) pinned by
    V8's run of the same recurrence (Math.floor of the f64 product)."""
    for case in js["reservoir"]:
        res = o.Reservoir(case["cap"], (case["seed"] ^ 0x85EBCA6B) & 0xFFFFFFFF)
        assert [res.slot() for _ in range(case["n"])] == case["slots"], case["seed"]


def test_reservoir_is_a_uniform_sample():
    """What the mathematics fixes for reservoir sampling: the first `cap`
    rows fill slots 0..cap-1 in order; row i >= cap is admitted with
    probability cap/(i+1) (a `seen` for `seen + 1` slip gives cap/i, 1.0 at
    i = cap); and after n rows every row is in the sample with probability
    cap/n.  Frequencies over 6000 seeds must sit within 5 standard
    deviations of those values."""
    cap, n, trials = 8, 48, 6000
    admit = np.zeros(n)
    held = np.zeros(n)
    for seed in range(trials):
        res = o.Reservoir(cap, (seed * 2654435761) & 0xFFFFFFFF)
        owner = [-1] * cap
        for i in range(n):
            s = res.slot()
            if i < cap:
                assert s == i
            if s >= 0:
                admit[i] += 1
                owner[s] = i
        for r in owner:
            held[r] += 1
    for i in range(cap, n):
        p = cap / (i + 1)
        sd = np.sqrt(p * (1 - p) / trials)
        assert abs(admit[i] / trials - p) <= 5 * sd, (i, admit[i] / trials, p)
    p = cap / n
    sd = np.sqrt(p * (1 - p) / trials)
    assert np.all(np.abs(held / trials - p) <= 5 * sd), held / trials


def _knn_graph(x, K, metric):
    """Fixed-degree kNN adjacency by brute force (f64 scores), self excluded."""
    if metric == "l2":
        s = -((x[:, None, :].astype(np.float64) - x[None, :, :]) ** 2).sum(-1)
    else:
        s = x.astype(np.float64) @ x.astype(np.float64).T
    np.fill_diagonal(s, -np.inf)
    g = np.argsort(-s, axis=1, kind="stable")[:, :K].astype(np.uint32)
    g[:, -1] = (np.arange(x.shape[0]) + 1) % x.shape[0]  # a ring: every row reachable
    return g


@pytest.mark.parametrize("metric", ["dot", "l2"])
def test_graph_search_visits_everything_when_ef_covers_the_graph(metric):
    """With ef at least the row count (and an iteration cap that high) the
    beam expands every reachable row, so the searcher's hits are the
    brute-force top-k of the shader's own distance arithmetic: f32, element
    order, each product and sum rounded (graphSearch.ts:101-109)."""
    rng = np.random.default_rng(3)
    n, dim, K = 200, 12, 8
    x = rng.standard_normal((n, dim)).astype(np.float32)
    g = _knn_graph(x, K, metric)
    q = rng.standard_normal((4, dim)).astype(np.float32)
    e = o.graph_entries(7, n)
    dist, ids = o.graph_search(x, g, q, e, 256, 256, l2=(metric == "l2"))
    for i in range(4):
        if metric == "l2":
            d = (x - q[i]).astype(np.float32)
            brute = np.cumsum(d * d, axis=1, dtype=np.float32)[:, -1]
            score = -brute
        else:
            score = np.cumsum(x * q[i], axis=1, dtype=np.float32)[:, -1]
        live = ids[i][ids[i] != o.GRAPH_EMPTY]
        assert live.size == np.unique(live).size  # the visited set keeps ids unique here
        rows, sc = o.graph_hits(dist[i], ids[i], 256, 10)
        want_r, want_s = o.topk_canonical(score, 10)
        assert np.array_equal(sc.view(np.uint32), want_s.view(np.uint32))
        assert set(rows.tolist()) == set(want_r.tolist())


def test_graph_entries_and_hits_known_answers():
    # seeds: the entry, then floor((i + 1) * rows / (extra + 1)) % rows
    assert o.graph_entries(0, 500).tolist() == [0, 62, 125, 187, 250, 312, 375, 437]
    assert o.graph_entries(3, 4).tolist() == [3, 0, 1, 2, 3]
    assert o.graph_entries(0, 1).tolist() == [0, 0]
    # dedup keeps an id's first slot; ties keep slot order; k cuts
    dist = np.full(256, 3.4e38, np.float32)
    ids = np.full(256, o.GRAPH_EMPTY, np.uint32)
    dist[:5] = [-1.0, -3.0, -1.0, -2.0, -3.0]
    ids[:5] = [10, 11, 12, 11, 13]
    rows, sc = o.graph_hits(dist, ids, 256, 3)
    assert rows.tolist() == [11, 13, 10] and sc.tolist() == [3.0, 3.0, 1.0]
