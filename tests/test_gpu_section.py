"""Index sections (src/persist/format.ts:1-22; src/index.ts:673-700 re-encodes
and re-trains on load): an index filled from a snapshot's rows and a saved
section must be the saved index -- the same codes, scales and IVF lists, the
same answers bit for bit, and the same state after further appends."""

import numpy as np
import pytest

from tests.helpers import clustered, gaussian, need_gpu, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    from browservec_amd import DeviceContext

    c = DeviceContext(0)
    yield c
    c.destroy()


def same_answers(a, b, qs, fetch, k):
    if not getattr(a, "bits", 0):
        fetch = 0  # fp32 kinds: the scan's own scores, no re-rank
    ra, sa, ca = a.search(qs, fetch, k)
    rb, sb, cb = b.search(qs, fetch, k)
    assert np.array_equal(ca, cb)
    for i in range(qs.shape[0]):
        assert np.array_equal(ra[i, :ca[i]], rb[i, :cb[i]]), i
        assert np.array_equal(sa[i, :ca[i]].view(np.uint32), sb[i, :cb[i]].view(np.uint32)), i


def make(ctx, kind, dim):
    from browservec_amd import FlatIndex, IVFIndex, IVFQuantIndex, QuantIndex

    if kind == "quant8":
        return QuantIndex(ctx, dim, bits=8, seed=1234)
    if kind == "quant1":
        return QuantIndex(ctx, dim, bits=1)
    if kind == "ivfquant":
        return IVFQuantIndex(ctx, dim, bits=8, ivf={"nlist": 16, "iters": 3, "nprobe": 4, "sampleSize": 1024})
    if kind == "ivfinc":  # incremental lists: appends after the load extend them as on the saved index
        return IVFQuantIndex(ctx, dim, bits=4, ivf={"nlist": 10, "iters": 2, "nprobe": 3, "incremental": True})
    if kind == "ivf":
        return IVFIndex(ctx, dim, ivf={"nlist": 12, "iters": 2, "nprobe": 3})
    return FlatIndex(ctx, dim, "dot")


@pytest.mark.parametrize("kind,dim,n", [("quant8", 100, 20000), ("quant1", 200, 3000), ("ivfquant", 64, 6000),
                                        ("ivfinc", 80, 4000), ("ivf", 48, 5000), ("flat", 96, 20000)])
def test_section_round_trip(ctx, kind, dim, n):
    say("section", kind, dim, n)
    data = clustered(n + 700, dim, 30, 0.1, seed=dim + n)
    a = make(ctx, kind, dim)
    a.append(data[:n // 3], n // 3)
    a.append(data[n // 3:n], n - n // 3)
    qs = (data[np.arange(40) * 37] + gaussian(40, dim, 5, normalize=False) * 0.05).astype(np.float32)
    same_answers(a, a, qs[:2], 50, 10)  # builds IVF lists before the save
    sec = a.save_section()
    b = make(ctx, kind, dim)
    b.load_section(data[:n], n, sec)
    assert b.size == n
    if kind.startswith("quant") or kind in ("ivfquant", "ivfinc"):
        wa, sa = a.export_codes()
        wb, sb = b.export_codes()
        assert np.array_equal(wa, wb) and np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
    if kind.startswith("ivf"):
        for x, y in zip(a.export_ivf(), b.export_ivf()):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    same_answers(a, b, qs, 50, 10)
    # a second save of the loaded index is byte-identical
    assert b.save_section() == sec
    # appends continue exactly as on the saved index (reservoir, lists)
    a.append(data[n:], 700)
    b.append(data[n:], 700)
    same_answers(a, b, qs, 50, 10)
    if kind.startswith("ivf"):
        for x, y in zip(a.export_ivf(), b.export_ivf()):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    a.destroy()
    b.destroy()


def test_section_errors(ctx):
    from browservec_amd import QuantIndex
    from browservec_amd._lib import BVError

    say("section errors")
    dim, n = 64, 500
    data = gaussian(n, dim, 3)
    a = QuantIndex(ctx, dim, bits=8)
    a.append(data, n)
    sec = a.save_section()
    other = QuantIndex(ctx, dim, bits=8, seed=7)  # another rotation seed
    with pytest.raises(BVError, match="different configuration"):
        other.load_section(data, n, sec)
    b = QuantIndex(ctx, dim, bits=8)
    with pytest.raises(BVError, match="truncated|bytes, expected"):
        b.load_section(data, n, sec[:100])
    with pytest.raises(BVError, match="holds 500 rows"):
        b.load_section(data[:10], 10, sec)
    with pytest.raises(BVError, match="expected 32000 floats"):
        b.load_section(data[:10], n, sec)
    assert b.size == 0  # nothing loaded by the failed calls
    b.load_section(data, n, sec)
    with pytest.raises(BVError, match="empty index"):
        b.load_section(data, n, sec)
    for x in (a, other, b):
        x.destroy()
