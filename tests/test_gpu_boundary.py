"""Error paths of the drop-in boundary, forced from the host
(bv_debug_inject sets flags only; no kernel is made to fail).

  * device loss (src/engine/device.ts:68-76): every later call fails with
    the reference's message "GPU device lost; re-create the store"
    (src/index/flat.ts:137) and the row count stays as it was;
  * a failed append allocation (src/index/quant.ts:129-140 appends are
    all-or-nothing): the index, its reservoir included, is unchanged, and a
    retried append gives the same index as if the failure never happened;
  * an append that fails after its rows were encoded: the reservoir sample
    and the incrementally extended IVF lists are unchanged too."""

import numpy as np
import pytest

from tests.helpers import clustered, gaussian, need_gpu, say

pytestmark = pytest.mark.gpu


def test_device_lost_fails_every_call_and_keeps_rows():
    need_gpu()
    from browservec_amd import DeviceContext, FlatIndex, QuantIndex
    from browservec_amd import _lib as L

    say("inject lost")
    ctx = DeviceContext(0)
    data = gaussian(500, 64, 1)
    flat = FlatIndex(ctx, 64, "cosine")
    flat.append(data, 500)
    quant = QuantIndex(ctx, 64, bits=8)
    quant.append(data, 500)
    assert not ctx.lost
    ctx.debug_inject("lost")
    assert ctx.lost
    for idx in (flat, quant):
        with pytest.raises(L.BVError) as e:
            idx.query(data[0], 5)
        assert e.value.code == L.BV_E_DEVICE_LOST and str(e.value) == "GPU device lost; re-create the store"
        with pytest.raises(L.BVError) as e:
            idx.append(data[:10], 10)
        assert e.value.code == L.BV_E_DEVICE_LOST
        assert idx.size == 500
    with pytest.raises(L.BVError):
        quant.search(data[:2], 10, 5)
    flat.destroy()
    quant.destroy()
    ctx.destroy()


def test_failed_append_leaves_the_index_unchanged():
    need_gpu()
    from browservec_amd import DeviceContext, IVFQuantIndex
    from browservec_amd import _lib as L

    say("inject append oom")
    ctx = DeviceContext(0)
    dim, n = 96, 6000
    ivf = {"nlist": 24, "iters": 3, "sampleSize": 1024}  # the reservoir replaces rows after 1024
    data = clustered(n, dim, 40, 0.1, seed=61)
    a = IVFQuantIndex(ctx, dim, bits=8, ivf=ivf)
    a.append(data[:3000], 3000)
    ctx.debug_inject("append_oom")
    with pytest.raises(L.BVError) as e:
        a.append(data[3000:], n - 3000)
    assert e.value.code == L.BV_E_OOM
    assert a.size == 3000
    a.append(data[3000:], n - 3000)  # the retry succeeds
    b = IVFQuantIndex(ctx, dim, bits=8, ivf=ivf)
    b.append(data[:3000], 3000)
    b.append(data[3000:], n - 3000)
    ca, oa, ra = a.export_ivf()
    cb, ob, rb = b.export_ivf()
    assert np.array_equal(ca.view(np.uint32), cb.view(np.uint32))
    assert np.array_equal(oa, ob) and np.array_equal(ra, rb)
    wa, sa = a.export_codes()
    wb, sb = b.export_codes()
    assert np.array_equal(wa, wb) and np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
    a.destroy()
    b.destroy()
    ctx.destroy()


@pytest.mark.parametrize("kind", ["quant8", "quant8_768", "flat", "ivf8"])
def test_two_query_streams_equal_one(kind):
    """bv_index_set_query_streams(2): consecutive search_device calls
    alternate between two streams and overlap; every call's rows and score
    bits equal the one-stream answers, an append between calls waits for
    the queries in flight and the next queries see the new rows."""
    need_gpu()
    import torch
    from browservec_amd import DeviceContext, FlatIndex, IVFQuantIndex, QuantIndex

    # (two streams run the register-lean build of the int8 scan: 768
    # dimensions is the 1024-code layout of the 1M x 768 workload)
    dim, n, nq = (768 if kind == "quant8_768" else 256), 60000, 24
    say("two query streams", kind)
    ctx = DeviceContext(0)
    data = gaussian(n, dim, 91)
    if kind == "ivf8":  # (each stream has its own probe and candidate buffers)
        idx = IVFQuantIndex(ctx, dim, bits=8, ivf={"nlist": 64, "nprobe": 8})
    else:
        idx = QuantIndex(ctx, dim, bits=8) if kind.startswith("quant8") else FlatIndex(ctx, dim, "cosine")
    idx.append(data[:n], n)
    q = torch.from_numpy(gaussian(nq, dim, 92)).cuda()
    fetch = 40 if kind != "flat" else 0

    def run(streams):
        idx.set_query_streams(streams)
        rows = torch.zeros(nq, 10, dtype=torch.int32, device="cuda")
        sc = torch.zeros(nq, 10, dtype=torch.float32, device="cuda")
        cnt = torch.zeros(nq, dtype=torch.int32, device="cuda")
        for i in range(nq):  # one query per call, each with its own outputs
            idx.search_device(q[i].data_ptr(), 1, fetch, 10, rows[i].data_ptr(), sc[i].data_ptr(), cnt[i].data_ptr())
        idx.sync()
        return rows.cpu().numpy(), sc.cpu().numpy(), cnt.cpu().numpy()

    r1, s1, c1 = run(1)
    for streams in (3, 4, 2):  # (two is left set for the append below)
        r2, s2, c2 = run(streams)
        assert np.array_equal(r1, r2) and np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
        assert np.array_equal(c1, c2)
    # an append while queries are in flight on both streams
    rows = torch.zeros(4, 10, dtype=torch.int32, device="cuda")
    sc = torch.zeros(4, 10, dtype=torch.float32, device="cuda")
    cnt = torch.zeros(4, dtype=torch.int32, device="cuda")
    for i in range(2):
        idx.search_device(q[i].data_ptr(), 1, fetch, 10, rows[i].data_ptr(), sc[i].data_ptr(), cnt[i].data_ptr())
    near = np.repeat(q[2:3].cpu().numpy(), 3000, axis=0)  # copies of query 2
    idx.append(near, 3000)
    for i in range(2, 4):
        idx.search_device(q[i].data_ptr(), 1, fetch, 10, rows[i].data_ptr(), sc[i].data_ptr(), cnt[i].data_ptr())
    idx.sync()
    got = rows.cpu().numpy()
    assert np.array_equal(got[:2], r1[:2])
    assert (got[2] >= n).all()  # the appended copies of query 2 win its top 10
    idx.set_query_streams(1)
    idx.destroy()
    ctx.destroy()


@pytest.mark.parametrize("bits", [8, 0])
def test_late_append_failure_leaves_sample_and_lists_unchanged(bits):
    """An append that fails after its rows were uploaded and encoded (a host
    append staged through pinned buffers in two chunks, failing after both)
    leaves the IVF reservoir's slots and state and the incrementally
    extended lists as they were: the index still answers from its old lists,
    and after the retried append both its extended lists and a rebuild from
    its reservoir equal those of an index whose append never failed."""
    need_gpu()
    from browservec_amd import DeviceContext, IVFIndex, IVFQuantIndex
    from browservec_amd import _lib as L

    say("inject append late", bits)
    ctx = DeviceContext(0)
    dim, n0, n1 = 96, 3000, 200_000  # 200,000 x 96 fp32 = 73 MiB: two staged chunks
    ivf = {"nlist": 24, "iters": 3, "sampleSize": 1024, "incremental": True}
    data = clustered(n0 + n1, dim, 40, 0.1, seed=62)

    def make():
        return IVFQuantIndex(ctx, dim, bits=bits, ivf=ivf) if bits else IVFIndex(ctx, dim, ivf=ivf)

    a = make()
    a.append(data[:n0], n0)
    a.build()  # lists current: the next append extends them
    cen0, off0, rows0 = a.export_ivf()
    hits0 = [h.row for h in a.query(data[7], 10)]
    ctx.debug_inject("append_late")
    with pytest.raises(L.BVError) as e:
        a.append(data[n0:], n1)
    assert e.value.code == L.BV_E_HIP and a.size == n0
    cen1, off1, rows1 = a.export_ivf()
    assert np.array_equal(cen0.view(np.uint32), cen1.view(np.uint32))
    assert np.array_equal(off0, off1) and np.array_equal(rows0, rows1)
    assert [h.row for h in a.query(data[7], 10)] == hits0
    a.append(data[n0:], n1)  # the retry succeeds
    b = make()
    b.append(data[:n0], n0)
    b.build()
    b.append(data[n0:], n1)
    for stage in ("extended lists", "rebuild from the reservoir"):
        ca, oa, ra = a.export_ivf()
        cb, ob, rb = b.export_ivf()
        assert np.array_equal(ca.view(np.uint32), cb.view(np.uint32)), stage
        assert np.array_equal(oa, ob) and np.array_equal(ra, rb), stage
        a.build()
        b.build()
    a.destroy()
    b.destroy()
    ctx.destroy()
