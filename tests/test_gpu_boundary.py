"""Error paths of the drop-in boundary, forced from the host
(bv_debug_inject sets flags only; no kernel is made to fail).

  * device loss (src/engine/device.ts:68-76): every later call fails with
    the reference's message "GPU device lost; re-create the store"
    (src/index/flat.ts:137) and the row count stays as it was;
  * a failed append allocation (src/index/quant.ts:129-140 appends are
    all-or-nothing): the index, its reservoir included, is unchanged, and a
    retried append gives the same index as if the failure never happened."""

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
