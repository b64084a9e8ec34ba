'use strict';
// Node host side of the MI355X search path: the reference's VectorIndex seam
// (src/index/flat.ts:24-40) and DeviceContext (src/engine/device.ts:3-9)
// implemented over libbrowservec_hip.so through the N-API addon
// (bv_napi.c).  A reference build swaps its WebGPU FlatIndex / QuantIndex /
// IVFIndex / IVFQuantIndex for these classes inside buildIndex
// (src/index.ts:105-142); BrowserVec and everything above the seam stay as
// they are.
//
// Each class carries exactly the duck-typed members its reference
// counterpart has, because BrowserVec picks its code path by their presence
// (src/index.ts:389-394, 477-481, 718-748):
//   - queryMasked on flat and quantized indexes only (IVF filters go through
//     BrowserVec's exact scan or over-fetch, as in the reference);
//   - queryBatch on flat fp32 indexes only, whose batches return exactly the
//     single-query results (an addition: the reference's WebGPU FlatIndex
//     has no queryBatch; its queryBatch is HNSW's, hnsw.ts:166); quantized
//     and IVF batches go through search() in one call, with query()'s
//     re-rank and nprobe rules, in the branch the integration adds to
//     BrowserVec.queryBatch (a queryBatch member would skip the re-rank);
//   - setNprobe / nlist / nprobe / tunedRecall / trainMode on IVF kinds,
//     ingestMode on quantized kinds, chunkCount everywhere.
// search() (approximate top-fetch + exact re-rank in one device call),
// rerankExact(), queryRowsExact() / queryRowsMasked() (BrowserVec's exact
// filtered scan, src/index.ts:445-464, on the device rows) and
// saveSection() / loadSection() (a snapshot section that skips re-encoding
// and re-training on load) are extras a caller may use explicitly.
const path = require('path');

const native = require(path.join(__dirname, '..', 'lib', 'browservec_napi.node'));

const KIND = { flat: 0, quant: 1, ivf: 2, ivfquant: 3 };
const METRIC = { cosine: 0, dot: 1, l2: 2 };
const SCORER = { asym: 0, hamming: 1, int8sym: 2 };

// DeviceContext: the HIP device, with the `lost` flag the reference polls.
class HipDeviceContext {
  constructor(ordinal) {
    this.handle = native.openDevice(ordinal === undefined ? 0 : ordinal);
  }
  get lost() {
    return this.handle === null || native.deviceLost(this.handle);
  }
  // Test hook: force the device-lost state (or a failed allocation on the
  // next append) from the host; no device work happens.
  debugInject(what) {
    native.debugInject(this.handle, what === 'lost' ? native.INJECT_LOST : native.INJECT_APPEND_OOM);
  }
  destroy() {
    if (this.handle !== null) {
      native.closeDevice(this.handle);
      this.handle = null;
    }
  }
}

function toHits(res, qi, k) {
  const n = res.counts[qi];
  const out = new Array(n);
  for (let j = 0; j < n; j++) out[j] = { row: res.rows[qi * k + j], score: res.scores[qi * k + j] };
  return out;
}

function f32(a) {
  return a instanceof Float32Array ? a : Float32Array.from(a);
}

function batchHits(res, n, k) {
  const out = [];
  for (let i = 0; i < n; i++) out.push(toHits(res, i, k));
  return out;
}

// Members every index kind has (VectorIndex plus chunkCount and the extras).
class HipIndex {
  constructor(ctx, dim, metric, kind, opts) {
    const o = opts || {};
    const ivf = o.ivf || null;
    this.dim = dim;
    this.metric = metric || 'cosine';
    this.bits = o.bits || 0;
    this.handle = native.createIndex(ctx.handle, {
      kind: kind,
      dim: dim,
      metric: METRIC[this.metric],
      bits: this.bits,
      scorer: SCORER[o.scorer || 'asym'],
      hasSeed: o.seed === undefined ? 0 : 1,
      seed: o.seed === undefined ? 0 : o.seed >>> 0,
      rounds: o.rounds || 0,
      chunkRows: o.chunkRows || 0,
      nlist: ivf && ivf.nlist ? ivf.nlist : 0,
      nprobe: ivf && ivf.nprobe ? ivf.nprobe : 0,
      sampleSize: ivf && ivf.sampleSize ? ivf.sampleSize : 0,
      trainSize: ivf && ivf.trainSize ? ivf.trainSize : 0,
      iters: ivf && ivf.iters ? ivf.iters : 0,
      hasIvfSeed: ivf && ivf.seed !== undefined ? 1 : 0,
      ivfSeed: ivf && ivf.seed !== undefined ? ivf.seed >>> 0 : 0,
      targetRecall: ivf && ivf.targetRecall !== undefined ? ivf.targetRecall : -1,
      incremental: ivf && ivf.incremental ? 1 : 0,
    });
  }
  get size() {
    return native.size(this.handle);
  }
  // append(data, count): `data` holds count*dim prepared floats; the rows
  // are copied and encoded on the device off the event loop (await it, as
  // BrowserVec awaits the reference's async appends).
  append(data, count) {
    return native.append(this.handle, f32(data), count);
  }
  query(q, k) {
    return native.query(this.handle, f32(q), k).then((res) => toHits(res, 0, k));
  }
  // BrowserVec.query's quantized path in one device call: approximate
  // top-`fetch`, exact Store.dotRow re-rank to k (src/index.ts:402-421).
  search(packed, n, fetch, k) {
    return native.search(this.handle, f32(packed), n, fetch, k).then((res) => batchHits(res, n, k));
  }
  // rerankExact (src/index.ts:583-594) against the rows kept on the device.
  rerankExact(q, candidates, k) {
    const rows = Uint32Array.from(candidates.map(function (h) { return h.row; }));
    return native.rerank(this.handle, f32(q), rows, k).then((res) => toHits(res, 0, k));
  }
  // queryRowsExact (src/index.ts:445-464): Store.dotRow / Store.l2Row of
  // each listed row, bit for bit, and their top k as {row, score} (rows in
  // the index's numbering, ties ordered by row).
  queryRowsExact(q, rows, k) {
    const r = rows instanceof Uint32Array ? rows : Uint32Array.from(rows);
    return native.queryRows(this.handle, f32(q), r, k).then((res) => toHits(res, 0, k));
  }
  // The same over the rows whose mask bit is set (the row list is built on
  // the device): a selective filter of any size.
  queryRowsMasked(q, k, maskWords) {
    const m = maskWords instanceof Uint32Array ? maskWords : Uint32Array.from(maskWords);
    return native.queryRowsMasked(this.handle, f32(q), m, k).then((res) => toHits(res, 0, k));
  }
  // Snapshot index section (codes, scales, IVF state): a load from the
  // snapshot's rows plus this section skips re-encoding and re-training
  // (the reference re-derives them, src/index.ts:673-700).
  saveSection() {
    return native.saveSection(this.handle);
  }
  // Fills this empty index; the descriptor must match the saved index.
  loadSection(data, count, section) {
    return native.loadSection(this.handle, f32(data), count,
      section instanceof Uint8Array ? section : new Uint8Array(section));
  }
  get chunkCount() {
    return native.stats(this.handle).chunkCount;
  }
  stats() {
    return native.stats(this.handle);
  }
  destroy() {
    if (this.handle !== null) {
      native.destroyIndex(this.handle);
      this.handle = null;
    }
  }
}

function queryMasked(q, k, maskWords) {
  const m = maskWords instanceof Uint32Array ? maskWords : Uint32Array.from(maskWords);
  return native.queryMasked(this.handle, f32(q), k, m).then((res) => toHits(res, 0, k));
}

// FlatIndex (src/index/flat.ts:42): exact fp32 scans.
class HipFlatIndex extends HipIndex {
  constructor(ctx, dim, metric, opts) {
    super(ctx, dim, metric, KIND.flat, Object.assign({}, opts, { bits: 0 }));
  }
  queryMasked(q, k, maskWords) {
    return queryMasked.call(this, q, k, maskWords);
  }
  // One device call for the batch; every query's rows and score bits equal
  // those of query() on the same vector.
  queryBatch(packed, n, k) {
    return native.queryBatch(this.handle, f32(packed), n, k).then((res) => batchHits(res, n, k));
  }
}

// QuantIndex (src/index/quant.ts:21): rotate + quantize on the device.
class HipQuantIndex extends HipIndex {
  constructor(ctx, dim, metric, opts) {
    super(ctx, dim, metric, KIND.quant, opts);
  }
  queryMasked(q, k, maskWords) {
    return queryMasked.call(this, q, k, maskWords);
  }
  // where rotate + quantize runs (src/index/quant.ts:115-118): on the device
  get ingestMode() {
    return this.size > 0 ? 'device' : 'pending';
  }
}

// IVFIndex (src/index/ivf.ts:51) / IVFQuantIndex (src/index/ivfquant.ts:33).
class HipIvfIndex extends HipIndex {
  constructor(ctx, dim, metric, opts) {
    super(ctx, dim, metric, (opts && opts.bits) ? KIND.ivfquant : KIND.ivf, opts);
  }
  setNprobe(n) {
    native.setNprobe(this.handle, n || 0);
  }
  // The build now (queries after an append build on demand, ivfquant.ts:461).
  build() {
    return native.build(this.handle);
  }
  // IVF getters (src/index.ts:718-748); 0 before a build.
  get nlist() {
    return native.stats(this.handle).nlist;
  }
  get nprobe() {
    return native.stats(this.handle).nprobe;
  }
  // estimated recall@10 at the tuned nprobe; undefined unless tuning ran
  get tunedRecall() {
    const r = native.stats(this.handle).tunedRecall;
    return r < 0 ? undefined : r;
  }
  // where the k-means mean update ran (src/index/ivf.ts:133-135)
  get trainMode() {
    return native.stats(this.handle).nlist > 0 ? 'device' : 'pending';
  }
}

class HipIvfQuantIndex extends HipIvfIndex {
  get ingestMode() {
    return this.size > 0 ? 'device' : 'pending';
  }
}

// buildIndex (src/index.ts:105-142) for the kinds this library serves:
// flat and quantized scans, and IVF over either, with the reference's
// rejections and messages.  HNSW is the reference's CPU graph index and
// stays there.
function buildIndex(ctx, dim, metric, quantBits, quant, ann, chunkRows) {
  const bits = quantBits || 0;
  const q = quant || {};
  const opts = { bits: bits, seed: q.seed, rounds: q.rounds, scorer: q.scorer, chunkRows: chunkRows, ivf: ann || null };
  if (ann && ann.type === 'hnsw') throw new Error('HNSW indexes are not served by this library');
  if (ann) {
    if (metric === 'l2') throw new Error('IVF supports metric cosine/dot only (l2 is later work)');
    if (bits === 8 || bits === 4 || bits === 1) return new HipIvfQuantIndex(ctx, dim, metric, opts);
    if (bits === 0) return new HipIvfIndex(ctx, dim, metric, opts);
    throw new Error(`quantBits ${bits} not supported with ann`);
  }
  if (bits === 0) return new HipFlatIndex(ctx, dim, metric, opts);
  if (bits === 8 || bits === 4 || bits === 1) {
    if (metric === 'l2') {
      throw new Error('quantized mode supports metric cosine/dot only (l2 quantization is later work)');
    }
    return new HipQuantIndex(ctx, dim, metric, opts);
  }
  throw new Error(`quantBits ${bits} not supported (ships 0, 1, 4, 8)`);
}

// HNSWGpuSearcher (src/index/hnswGpu.ts:28-244) on the device: the HNSW
// index (its CPU graph build) hands over corpus rows and the layer-0
// adjacency; search() beam-searches a query batch in one launch.
class HipGraphSearcher {
  constructor(ctx, dim, metric, degree) {
    this.dim = dim;
    this.degree = degree;
    this.handle = native.graphCreate(ctx.handle, { dim, metric: METRIC[metric], degree });
    this.rows = 0;
    this.graphRows = 0;
  }
  get maxRows() {
    return 0xfffffffe;
  }
  append(data, count) {
    native.graphAppend(this.handle, f32(data), count);
    this.rows += count;
  }
  uploadGraph(links, rows) {
    native.graphUpload(this.handle, links instanceof Uint32Array ? links : Uint32Array.from(links), rows);
    this.graphRows = rows;
  }
  get uploadedRows() {
    return this.graphRows;
  }
  search(queries, nQ, k, ef, entry) {
    return native.graphSearch(this.handle, f32(queries), nQ, k, ef, entry >>> 0).then((res) => batchHits(res, nQ, k));
  }
  destroy() {
    if (this.handle !== null) {
      native.graphDestroy(this.handle);
      this.handle = null;
    }
  }
}

module.exports = {
  HipDeviceContext, HipIndex, HipFlatIndex, HipQuantIndex, HipIvfIndex, HipIvfQuantIndex, HipGraphSearcher,
  buildIndex,
  native, abiVersion: native.abiVersion,
};
