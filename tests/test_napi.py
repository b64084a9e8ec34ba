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
    """Each class carries the duck-typed members of its reference
    counterpart, and no others that would change BrowserVec's path:
    queryMasked only on flat / quantized (flat.ts:128, quant.ts:174),
    queryBatch only on flat fp32 (whose batch equals single queries),
    setNprobe and the IVF getters only on IVF (ivf.ts:123-150,
    ivfquant.ts:151-212), ingestMode on quantized kinds."""
    r = run_node(f"""
const m = require({json.dumps(MODULE)});
const has = (C) => ['size', 'append', 'query', 'queryMasked', 'queryBatch', 'setNprobe', 'destroy', 'search',
  'rerankExact', 'chunkCount', 'nlist', 'nprobe', 'tunedRecall', 'trainMode', 'ingestMode', 'build',
  'saveSection', 'loadSection', 'queryRowsExact', 'queryRowsMasked']
  .filter((k) => k in C.prototype);
console.log(JSON.stringify({{abi: m.abiVersion, native: Object.keys(m.native),
  flat: has(m.HipFlatIndex), quant: has(m.HipQuantIndex), ivf: has(m.HipIvfIndex),
  ivfquant: has(m.HipIvfQuantIndex)}}));
""")
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["abi"] == 1
    common = {"size", "append", "query", "destroy", "search", "rerankExact", "chunkCount", "saveSection",
              "loadSection", "queryRowsExact", "queryRowsMasked"}
    assert set(out["flat"]) == common | {"queryMasked", "queryBatch"}
    assert set(out["quant"]) == common | {"queryMasked", "ingestMode"}
    ivf = common | {"setNprobe", "nlist", "nprobe", "tunedRecall", "trainMode", "build"}
    assert set(out["ivf"]) == ivf
    assert set(out["ivfquant"]) == ivf | {"ingestMode"}
    for fn in ("openDevice", "debugInject", "createIndex", "append", "build", "query", "queryMasked", "queryBatch",
               "search", "rerank", "saveSection", "loadSection", "queryRows", "queryRowsMasked", "graphCreate",
               "graphAppend", "graphUpload", "graphSearch", "graphDestroy"):
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
  const pending = flat.append(rows, n);
  out.appendIsPromise = pending instanceof Promise;
  await pending;
  out.flatSize = flat.size;
  out.flat = await flat.queryBatch(qs, nq, 10);
  try { await flat.query(qs.subarray(0, dim - 1), 5); } catch (e) { out.shortQuery = [e.constructor.name, e.message]; }
  try { await flat.queryBatch(qs.subarray(0, dim * 2), 3, 5); } catch (e) { out.shortBatch = e.message; }
  try { await flat.append(rows.subarray(0, dim + 1), 1); } catch (e) { out.badAppend = [e.code, e.message]; }
  const quant = m.buildIndex(ctx, dim, 'cosine', 8, {});
  out.ingestBefore = quant.ingestMode;
  await quant.append(rows, n);
  out.ingestAfter = quant.ingestMode;
  out.approx = await quant.query(qs.subarray(0, dim), 40);
  out.search = await quant.search(qs, nq, 40, 10);
  out.rerank = await quant.rerankExact(qs.subarray(0, dim), out.approx, 10);
  out.rows = await quant.queryRowsExact(qs.subarray(0, dim), [5, 17, 2000, 40, 999, 2999], 4);
  out.rowsMasked = await flat.queryRowsMasked(qs.subarray(dim, 2 * dim), 6, new Uint32Array([0xf0f0f0f0, 0x1, 0x80000000]));
  try { await quant.queryRowsExact(qs.subarray(0, dim), [1, n], 2); } catch (e) { out.rowsBad = [e.code, e.message]; }
  const ivf = m.buildIndex(ctx, dim, 'cosine', 8, {}, {nlist: 16, iters: 3, nprobe: 4});
  await ivf.append(rows, n);
  out.trainBefore = ivf.trainMode;
  out.ivf = [];
  for (let i = 0; i < nq; i++) out.ivf.push(await ivf.query(qs.subarray(i * dim, (i + 1) * dim), 10));
  out.trainAfter = ivf.trainMode;
  out.ivfStats = [ivf.nlist, ivf.nprobe];
  // a snapshot's index section: the loaded index answers as the saved one
  const sec = await ivf.saveSection();
  out.sectionIsBytes = sec instanceof Uint8Array && sec.length > 0;
  const ivf2 = m.buildIndex(ctx, dim, 'cosine', 8, {}, {nlist: 16, iters: 3, nprobe: 4});
  await ivf2.loadSection(rows, n, sec);
  out.loadedTrain = ivf2.trainMode;
  out.ivfLoaded = [];
  for (let i = 0; i < nq; i++) out.ivfLoaded.push(await ivf2.query(qs.subarray(i * dim, (i + 1) * dim), 10));
  try { await ivf2.loadSection(rows, n, sec); } catch (e) { out.loadTwice = [e.code, e.message]; }
  ivf2.destroy();
  try { m.buildIndex(ctx, dim, 'l2', 0, {}, {}); } catch (e) { out.ivfL2 = e.message; }
  // the graph searcher: a ring adjacency of degree 4 over the rows
  const gsr = new m.HipGraphSearcher(ctx, dim, 'cosine', 4);
  gsr.append(rows, n);
  const links = new Uint32Array(n * 4);
  for (let r = 0; r < n; r++) for (let j = 0; j < 4; j++) links[r * 4 + j] = (r + j + 1) %% n;
  gsr.uploadGraph(links, n);
  out.graph = await gsr.search(qs, nq, 5, 32, 0);
  try { new m.HipGraphSearcher(ctx, dim, 'cosine', 65); } catch (e) { out.graphDegree = [e.code, e.message]; }
  gsr.destroy();
  // a destroy while a call is in flight: the call still completes
  const q2 = quant.query(qs.subarray(0, dim), 5);
  quant.destroy();
  out.inflight = (await q2).length;
  // the device-lost path, forced from the host
  ctx.debugInject('lost');
  out.lost = ctx.lost;
  try { await flat.query(qs.subarray(0, dim), 5); } catch (e) { out.lostErr = [e.code, e.message]; }
  out.sizeAfterLost = flat.size;
  flat.destroy(); ivf.destroy(); ctx.destroy();
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
    assert out["flatSize"] == n and out["appendIsPromise"]
    assert out["shortQuery"] == ["TypeError", f"expected {dim} floats, got {dim - 1}"]
    assert out["shortBatch"] == f"expected {3 * dim} floats, got {2 * dim}"
    assert out["badAppend"] == ["BV_E_INVALID", f"expected {dim} floats, got {dim + 1}"]
    assert out["ingestBefore"] == "pending" and out["ingestAfter"] == "device"
    assert out["trainBefore"] == "pending" and out["trainAfter"] == "device"
    assert out["inflight"] == 5
    assert out["lost"] is True
    assert out["lostErr"] == ["BV_E_DEVICE_LOST", "GPU device lost; re-create the store"]
    assert out["sizeAfterLost"] == n
    assert out["sectionIsBytes"] and out["loadedTrain"] == "device"
    assert out["ivfLoaded"] == out["ivf"]
    assert out["loadTwice"] == ["BV_E_STATE", "a section loads into an empty index"]

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
            same(out["flat"][i], flat.query(q[i], 10))
        py_approx = quant.query(q[0], 40)
        same(out["approx"], py_approx)
        rows, scores, cnt = quant.search(q, 40, 10)
        for i in range(nq):
            assert [h["row"] for h in out["search"][i]] == rows[i, :cnt[i]].tolist()
            assert np.array_equal(np.float32([h["score"] for h in out["search"][i]]), scores[i, :cnt[i]])
        same(out["rerank"], quant.rerank(q[0], [h.row for h in py_approx], 10))
        same(out["rows"], quant.query_rows(q[0], [5, 17, 2000, 40, 999, 2999], 4))
        same(out["rowsMasked"], flat.query_rows_masked(q[1], 6, np.array([0xF0F0F0F0, 1, 0x80000000], np.uint32)))
        assert out["rowsBad"] == ["BV_E_INVALID", f"a listed row is out of range (the index holds {n} rows)"]
        ivf = IVFQuantIndex(ctx, dim, bits=8, ivf={"nlist": 16, "iters": 3, "nprobe": 4})
        ivf.append(x, n)
        for i in range(nq):
            same(out["ivf"][i], ivf.query(q[i], 10))
        assert out["ivfStats"] == [16, 4]
        assert out["ivfL2"] == "IVF supports metric cosine/dot only (l2 is later work)"
        from browservec_amd import GraphSearcher

        gs = GraphSearcher(ctx, dim, "cosine", 4)
        gs.append(x, n)
        gs.upload_graph(np.array([[(r + j + 1) % n for j in range(4)] for r in range(n)], np.uint32), n)
        py_graph = gs.search(q, nq, 5, 32, 0)
        for i in range(nq):
            same(out["graph"][i], py_graph[i])
        assert out["graphDegree"][0] == "BV_E_UNSUPPORTED" and "degree" in out["graphDegree"][1]
        gs.destroy()
        ivf.destroy()
        flat.destroy()
        quant.destroy()
    finally:
        ctx.destroy()


NODE_QUERY_BATCH = """
const fs = require('fs');
const m = require(%(module)s);
function f32(p) { const b = fs.readFileSync(p); return new Float32Array(b.buffer, b.byteOffset, b.length / 4); }
const rows = f32(%(rows)s), qs = f32(%(queries)s);
const dim = %(dim)d, n = %(n)d, nq = %(nq)d;
const RERANK_FACTOR = 4;  // BrowserVec's default for int8 / int4 (src/index.ts:236-250)
// The tombstone skip and stop-at-k of BrowserVec.query / queryBatch (src/index.ts:424-435, 505-515).
function post(hits, k, deleted) {
  const out = [];
  for (const h of hits) {
    if (deleted.has(h.row)) continue;
    out.push({row: h.row, score: h.score});
    if (out.length === k) break;
  }
  return out;
}
// BrowserVec.query's quantized path with the one-call search (src/index.ts:402-421).
async function queryOne(index, q, k, opts, deleted) {
  const total = index.size;
  const kEff = Math.min(total, k + deleted.size);
  const doRerank = opts.rerank !== undefined ? opts.rerank : RERANK_FACTOR > 1;
  const fetch = doRerank ? Math.min(total, Math.max(kEff, kEff * RERANK_FACTOR)) : kEff;
  if (opts.nprobe !== undefined && 'setNprobe' in index) index.setNprobe(opts.nprobe);
  const batch = await index.search(q, 1, doRerank ? fetch : 0, kEff);
  return post(batch[0], k, deleted);
}
// The queryBatch branch the integration adds (src/index.ts:473-517): one search() call.
async function queryBatch(index, packed, count, k, opts, deleted) {
  const total = index.size;
  const kEff = Math.min(total, k + deleted.size);
  const doRerank = opts.rerank !== undefined ? opts.rerank : RERANK_FACTOR > 1;
  const fetch = doRerank ? Math.min(total, Math.max(kEff, kEff * RERANK_FACTOR)) : kEff;
  if (kEff === 0 || fetch > 1024) throw new Error('falls back to the query() loop');
  if (opts.nprobe !== undefined && 'setNprobe' in index) index.setNprobe(opts.nprobe);
  const batch = await index.search(packed, count, doRerank ? fetch : 0, kEff);
  return batch.map((hits) => post(hits, k, deleted));
}
(async () => {
  const ctx = new m.HipDeviceContext(0);
  const out = {};
  const cases = [['int8', 8, null, {}], ['ivf_int8', 8, {nlist: 24, iters: 3, nprobe: 4}, {nprobe: 6}],
                 ['int4_no_rerank', 4, null, {rerank: false}]];
  for (const [name, bits, ann, opts] of cases) {
    const index = ann ? m.buildIndex(ctx, dim, 'cosine', bits, {}, ann) : m.buildIndex(ctx, dim, 'cosine', bits, {});
    await index.append(rows, n);
    const deleted = new Set([17]);
    let calls = 0;
    const search = index.search.bind(index);
    index.search = (...a) => { calls += 1; return search(...a); };
    const batch = await queryBatch(index, qs, nq, 10, opts, deleted);
    const batchCalls = calls;
    const singles = [];
    for (let i = 0; i < nq; i++) singles.push(await queryOne(index, qs.subarray(i * dim, (i + 1) * dim), 10, opts, deleted));
    out[name] = {batch: batch, singles: singles, batchCalls: batchCalls, nprobeAfter: ann ? index.nprobe : null};
    index.destroy();
  }
  ctx.destroy();
  console.log(JSON.stringify(out));
})().catch((e) => { console.error(e.code, e.message); process.exit(3); });
"""


@pytest.mark.gpu
def test_node_query_batch_branch_takes_one_search(tmp_path):
    """The queryBatch branch INTEGRATION.md adds to BrowserVec, run in node
    over the addon: a quantized or IVF store's batch is one search() call,
    and every query's rows, order and score bits equal query()'s one-call
    search with the same kEff / fetch / re-rank / nprobe rules and the same
    tombstone skip (src/index.ts:402-436, 473-517)."""
    need_gpu()
    dim, n, nq = 96, 6000, 24
    say("napi queryBatch", dim, n, nq)
    x = clustered(n, dim, 40, 0.1, seed=181)
    q = x[np.random.default_rng(182).integers(0, n, nq)] + 0.05 * gaussian(nq, dim, seed=183, normalize=False)
    q = q.astype(np.float32)
    (tmp_path / "rows.f32").write_bytes(x.tobytes())
    (tmp_path / "q.f32").write_bytes(q.tobytes())
    r = run_node(NODE_QUERY_BATCH % {"module": json.dumps(MODULE), "rows": json.dumps(str(tmp_path / "rows.f32")),
                                     "queries": json.dumps(str(tmp_path / "q.f32")), "dim": dim, "n": n,
                                     "nq": nq})
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    for name in ("int8", "ivf_int8", "int4_no_rerank"):
        res = out[name]
        assert res["batchCalls"] == 1, name
        for i in range(nq):
            b, s = res["batch"][i], res["singles"][i]
            assert len(b) == 10 and 17 not in [h["row"] for h in b], (name, i)
            assert [h["row"] for h in b] == [h["row"] for h in s], (name, i)
            assert (np.float32([h["score"] for h in b]).view(np.uint32).tolist() ==
                    np.float32([h["score"] for h in s]).view(np.uint32).tolist()), (name, i)
    assert out["ivf_int8"]["nprobeAfter"] == 4  # the override was consumed by one call
