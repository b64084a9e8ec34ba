"""Host appends larger than one 64 MiB staging chunk go through pinned
buffers on a copy stream, chunk by chunk, overlapped with the encode of the
previous chunk (VectorIndex.append, flat.ts:37, quant.ts:129-140,
ivfquant.ts:216-233).  The index they build equals the one a single device
copy builds: the same rows, codes, scales, reservoir and lists."""

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


@pytest.mark.parametrize("kind", ["quant8", "flat", "ivfquant", "ivf"])
def test_staged_host_append_equals_device_append(ctx, kind):
    import torch
    from browservec_amd import FlatIndex, IVFIndex, IVFQuantIndex, QuantIndex

    dim = 768
    n = 50_000  # 147 MiB: chunks of 21,845 rows, the last one ragged
    say("staged append", kind, n, dim)
    data = clustered(n, dim, 64, 0.1, seed=71)
    ivf = {"nlist": 24, "iters": 2, "nprobe": 4, "sampleSize": 20000}

    def make():
        if kind == "quant8":
            return QuantIndex(ctx, dim, bits=8)
        if kind == "ivfquant":
            return IVFQuantIndex(ctx, dim, bits=8, ivf=ivf)
        if kind == "ivf":
            return IVFIndex(ctx, dim, ivf=ivf)
        return FlatIndex(ctx, dim, "dot")

    host, dev = make(), make()
    host.append(data[:1000], 1000)  # a small append first: the staged one starts mid-index
    host.append(data[1000:], n - 1000)
    d = torch.from_numpy(data).cuda()
    dev.append_device(d[:1000].data_ptr(), 1000)
    dev.append_device(d[1000:].data_ptr(), n - 1000)
    torch.cuda.synchronize()
    assert host.size == dev.size == n
    qs = gaussian(4, dim, 72)
    if kind in ("quant8", "ivfquant"):
        wa, sa = host.export_codes()
        wb, sb = dev.export_codes()
        assert np.array_equal(wa, wb) and np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
    if kind.startswith("ivf"):
        for x, y in zip(host.export_ivf(), dev.export_ivf()):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    for q in qs:
        assert [(h.row, h.score) for h in host.query(q, 20)] == [(h.row, h.score) for h in dev.query(q, 20)]
    # the stored rows themselves (exact re-scores read them)
    rows = np.array([0, 999, 1000, 21844, 22845, 43690, n - 1], np.uint32)
    a = host.query_rows(qs[0], rows, len(rows))
    b = dev.query_rows(qs[0], rows, len(rows))
    assert [(h.row, h.score) for h in a] == [(h.row, h.score) for h in b]
    if kind == "quant8":  # a pinned source skips the staging buffers
        pin = make()
        pin.append(torch.from_numpy(data).pin_memory().numpy(), n)
        wc, sc = pin.export_codes()
        assert np.array_equal(wc, wb) and np.array_equal(sc.view(np.uint32), sb.view(np.uint32))
        pin.destroy()
    host.destroy()
    dev.destroy()
