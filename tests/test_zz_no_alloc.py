"""bv_index_search_device_noalloc (the entry point for callers that cannot
allocate device memory) against bv_index_search_device on the same inputs:
rows, score bits and counts equal, on consecutive calls that lay the shared
scratch out differently (the second call smaller), and a request beyond the
scratch limit is refused with BV_E_INVALID."""

import numpy as np
import pytest

from oracle import oracle as o
from tests.helpers import clustered, gaussian, need_gpu, say

pytestmark = pytest.mark.gpu


def run(idx, fn, qs, fetch, k):
    import torch

    nq = qs.shape[0]
    d_q = torch.from_numpy(np.ascontiguousarray(qs, np.float32)).cuda()
    rows = torch.full((nq, k), -1, dtype=torch.int32, device="cuda")
    scores = torch.zeros(nq, k, dtype=torch.float32, device="cuda")
    cnt = torch.zeros(nq, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    fn(d_q.data_ptr(), nq, fetch, k, rows.data_ptr(), scores.data_ptr(), cnt.data_ptr())
    idx.sync()
    return rows.cpu().numpy(), scores.cpu().numpy().view(np.uint32), cnt.cpu().numpy()


def same(idx, qs, fetch, k):
    want = run(idx, idx.search_device, qs, fetch, k)
    got = run(idx, idx.search_device_noalloc, qs, fetch, k)
    for w, g in zip(want, got):
        assert np.array_equal(w, g)
    return got


def test_noalloc_equals_search_device():
    need_gpu()
    from browservec_amd import DeviceContext, FlatIndex, QuantIndex
    from browservec_amd import _lib as L

    ctx = DeviceContext(0)
    say("noalloc int8 20000x768 nq 6 fetch 100")
    big = clustered(20000, 768, 64, 0.1, seed=81)
    a = QuantIndex(ctx, 768, bits=8)
    a.append(big, big.shape[0])
    qa = np.stack([o.normalize(q) for q in big[[1, 500, 9000, 12345, 17000, 19999]] +
                   gaussian(6, 768, 82, normalize=False) * 0.05]).astype(np.float32)
    rows, scores, cnt = same(a, qa, 100, 10)
    assert np.all(cnt == 10)
    exact = o.rerank_scores(big, qa[0], rows[0].astype(np.uint32))
    assert np.array_equal(scores[0], exact.view(np.uint32))

    say("noalloc int4 3000x100 nq 3 fetch 40 (smaller, right after)")
    small = clustered(3000, 100, 16, 0.1, seed=83)
    b = QuantIndex(ctx, 100, bits=4)
    b.append(small, small.shape[0])
    same(b, gaussian(3, 100, 84), 40, 5)

    say("noalloc fp32 l2 5000x64 nq 2")
    c = FlatIndex(ctx, 64, "l2")
    c.append(gaussian(5000, 64, 85), 5000)
    same(c, gaussian(2, 64, 86), 0, 7)

    say("noalloc beyond the scratch limit")
    with pytest.raises(L.BVError) as e:
        run(a, a.search_device_noalloc, np.repeat(qa, 20, axis=0), 1000, 10)
    assert e.value.code == L.BV_E_INVALID and "scratch" in str(e.value)
    # the index still answers after the refusal
    same(a, qa[:2], 100, 10)
    for idx in (a, b, c):
        idx.destroy()
    ctx.destroy()
