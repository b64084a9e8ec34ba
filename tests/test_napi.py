"""The Node (N-API) binding: the addon loads in node, exposes the VectorIndex
seam, and fails cleanly without a device.  The GPU half runs queries from
node and requires results identical to the Python binding's."""

import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from tests.helpers import gaussian, clustered, need_gpu, say

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "browservec_amd", "lib", "browservec_napi.node")
MODULE = os.path.join(ROOT, "browservec_amd", "napi", "index.js")


def run_node(script: str, timeout: int = 120) -> subprocess.CompletedProcess:
    node = shutil.which("node")
    if node is None:
        pytest.skip("node is not installed")
    if not os.path.exists(ADDON):
        pytest.fail(f"{ADDON} is not built (python -m browservec_amd.build)")
    return subprocess.run([node, "-e", script], capture_output=True, text=True, timeout=timeout)


def test_addon_exports_the_seam():
    r = run_node(f"""
const m = require({json.dumps(MODULE)});
const proto = Object.getOwnPropertyNames(m.HipIndex.prototype);
console.log(JSON.stringify({{abi: m.abiVersion, proto: proto, native: Object.keys(m.native)}}));
""")
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["abi"] == 1
    for member in ("size", "append", "query", "queryMasked", "queryBatch", "setNprobe", "destroy", "rerankExact",
                   "search"):
        assert member in out["proto"], member
    for fn in ("openDevice", "createIndex", "append", "query", "queryMasked", "queryBatch", "search", "rerank"):
        assert fn in out["native"], fn


def test_addon_argument_errors_and_no_device_message():
    r = run_node(f"""
const m = require({json.dumps(MODULE)});
const out = {{}};
try {{ m.native.query(null, 3, 1); }} catch (e) {{ out.typeErr = e.constructor.name; }}
if (!process.env.HIP_VISIBLE_DEVICES_PROBE) {{
  try {{ const c = new m.HipDeviceContext(0); out.opened = true; c.destroy(); }}
  catch (e) {{ out.code = e.code; out.message = e.message; }}
}}
console.log(JSON.stringify(out));
""")
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["typeErr"] == "TypeError"
    if not out.get("opened"):
        assert out["code"].startswith("BV_E_") and out["message"]


NODE_SEARCH = """
const fs = require('fs');
const m = require(%(module)s);
function f32(p) { const b = fs.readFileSync(p); return new Float32Array(b.buffer, b.byteOffset, b.length / 4); }
const rows = f32(%(rows)s), qs = f32(%(queries)s);
const dim = %(dim)d, n = %(n)d, nq = %(nq)d;
(async () => {
  const ctx = new m.HipDeviceContext(0);
  const out = {};
  const flat = m.buildIndex(ctx, dim, 'cosine', 0);
  flat.append(rows, n);
  out.flatSize = flat.size;
  out.flat = await flat.queryBatch(qs, nq, 10);
  const quant = m.buildIndex(ctx, dim, 'cosine', 8, {});
  quant.append(rows, n);
  out.approx = await quant.query(qs.subarray(0, dim), 40);
  out.search = await quant.search(qs, nq, 40, 10);
  out.rerank = await quant.rerankExact(qs.subarray(0, dim), out.approx, 10);
  const ivf = m.buildIndex(ctx, dim, 'cosine', 8, {}, {nlist: 16, iters: 3, nprobe: 4});
  ivf.append(rows, n);
  out.ivf = await ivf.queryBatch(qs, nq, 10);
  out.ivfStats = [ivf.nlist, ivf.nprobe];
  try { m.buildIndex(ctx, dim, 'l2', 0, {}, {}); } catch (e) { out.ivfL2 = e.message; }
  flat.destroy(); quant.destroy(); ivf.destroy(); ctx.destroy();
  console.log(JSON.stringify(out));
})().catch((e) => { console.error(e.code, e.message); process.exit(3); });
"""


@pytest.mark.gpu
def test_node_results_equal_python_binding(tmp_path):
    need_gpu()
    from browservec_amd import DeviceContext, FlatIndex, IVFQuantIndex, QuantIndex

    dim, n, nq = 96, 3000, 4
    say("napi", dim, n, nq)
    x = clustered(n, dim, 40, 0.1, seed=11)
    q = gaussian(nq, dim, seed=12)
    (tmp_path / "rows.f32").write_bytes(x.tobytes())
    (tmp_path / "q.f32").write_bytes(q.tobytes())
    r = run_node(NODE_SEARCH % {"module": json.dumps(MODULE), "rows": json.dumps(str(tmp_path / "rows.f32")),
                                "queries": json.dumps(str(tmp_path / "q.f32")), "dim": dim, "n": n, "nq": nq})
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["flatSize"] == n

    ctx = DeviceContext(0)
    try:
        flat = FlatIndex(ctx, dim, "cosine")
        flat.append(x, n)
        quant = QuantIndex(ctx, dim, bits=8)
        quant.append(x, n)

        def same(hits_js, hits_py):
            assert [h["row"] for h in hits_js] == [h.row for h in hits_py]
            assert np.array_equal(np.float32([h["score"] for h in hits_js]), np.float32([h.score for h in hits_py]))

        py_flat = flat.query_batch(q, nq, 10)
        for i in range(nq):
            same(out["flat"][i], py_flat[i])
        py_approx = quant.query(q[0], 40)
        same(out["approx"], py_approx)
        rows, scores, cnt = quant.search(q, 40, 10)
        for i in range(nq):
            assert [h["row"] for h in out["search"][i]] == rows[i, :cnt[i]].tolist()
            assert np.array_equal(np.float32([h["score"] for h in out["search"][i]]), scores[i, :cnt[i]])
        same(out["rerank"], quant.rerank(q[0], [h.row for h in py_approx], 10))
        ivf = IVFQuantIndex(ctx, dim, bits=8, ivf={"nlist": 16, "iters": 3, "nprobe": 4})
        ivf.append(x, n)
        py_ivf = ivf.query_batch(q, nq, 10)
        for i in range(nq):
            same(out["ivf"][i], py_ivf[i])
        assert out["ivfStats"] == [16, 4]
        assert out["ivfL2"] == "IVF supports metric cosine/dot only (l2 is later work)"
        ivf.destroy()
        flat.destroy()
        quant.destroy()
    finally:
        ctx.destroy()
