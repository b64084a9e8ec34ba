'use strict';
// Node host side of the MI355X search path: the reference's VectorIndex seam
// (src/index/flat.ts:24-40) and DeviceContext (src/engine/device.ts:3-9)
// implemented over libbrowservec_hip.so through the N-API addon
// (bv_napi.c).  A reference build swaps its WebGPU FlatIndex / QuantIndex
// for HipIndex inside buildIndex (src/index.ts:105-142); BrowserVec and
// everything above the seam stay as they are.
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

// FlatIndex (src/index/flat.ts:42) and QuantIndex (src/index/quant.ts:21)
// on the device: same members, same results order (score desc, row asc).
class HipIndex {
  constructor(ctx, dim, metric, opts) {
    const o = opts || {};
    const bits = o.bits || 0;
    this.dim = dim;
    this.metric = metric || 'cosine';
    this.bits = bits;
    const ivf = o.ivf || null;
    this.isIvf = ivf !== null;
    this.handle = native.createIndex(ctx.handle, {
      kind: ivf ? (bits ? KIND.ivfquant : KIND.ivf) : (bits ? KIND.quant : KIND.flat),
      dim: dim,
      metric: METRIC[this.metric],
      bits: bits,
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
    });
  }
  get size() {
    return native.size(this.handle);
  }
  // append(data, count): `data` holds count*dim prepared floats.
  append(data, count) {
    native.append(this.handle, f32(data), count);
  }
  query(q, k) {
    return Promise.resolve(toHits(native.query(this.handle, f32(q), k), 0, k));
  }
  queryMasked(q, k, maskWords) {
    const m = maskWords instanceof Uint32Array ? maskWords : Uint32Array.from(maskWords);
    return Promise.resolve(toHits(native.queryMasked(this.handle, f32(q), k, m), 0, k));
  }
  queryBatch(packed, n, k) {
    const res = native.queryBatch(this.handle, f32(packed), n, k);
    const out = [];
    for (let i = 0; i < n; i++) out.push(toHits(res, i, k));
    return Promise.resolve(out);
  }
  // BrowserVec.query's quantized path in one device call: approximate
  // top-`fetch`, exact Store.dotRow re-rank to k (src/index.ts:402-421).
  search(packed, n, fetch, k) {
    const res = native.search(this.handle, f32(packed), n, fetch, k);
    const out = [];
    for (let i = 0; i < n; i++) out.push(toHits(res, i, k));
    return Promise.resolve(out);
  }
  // rerankExact (src/index.ts:583-594) against the rows kept on the device.
  rerankExact(q, candidates, k) {
    const rows = Uint32Array.from(candidates.map(function (h) { return h.row; }));
    return Promise.resolve(toHits(native.rerank(this.handle, f32(q), rows, k), 0, k));
  }
  setNprobe(n) {
    native.setNprobe(this.handle, n || 0);
  }
  get chunkCount() {
    return native.stats(this.handle).chunkCount;
  }
  // IVF getters (src/index.ts:718-748); 0 for flat kinds and before a build.
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

// buildIndex (src/index.ts:105-142) for the kinds this library serves:
// flat and quantized scans, and IVF over either.  HNSW is the reference's
// CPU graph index and stays there.
function buildIndex(ctx, dim, metric, quantBits, quant, ann, chunkRows) {
  if (ann && ann.type === 'hnsw') throw new Error('HNSW indexes are not served by this library');
  if (ann && metric === 'l2') throw new Error('IVF supports metric cosine/dot only (l2 is later work)');
  const q = quant || {};
  return new HipIndex(ctx, dim, metric, {
    bits: quantBits || 0,
    seed: q.seed,
    rounds: q.rounds,
    scorer: q.scorer,
    chunkRows: chunkRows,
    ivf: ann || null,
  });
}

module.exports = { HipDeviceContext, HipIndex, buildIndex, native, abiVersion: native.abiVersion };
