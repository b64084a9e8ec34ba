// Writes tests/golden/js_vectors.json: golden vectors for the parts of the
// search path whose exact bits depend on JavaScript number semantics
// (Math.imul, >>>, |0, Math.round, Float32Array stores, f64 accumulation).
//
// This is an independent implementation written for this repository (not the
// reference's code) and run under node's V8, the engine family the reference
// runs on.  It follows the algorithms of:
//   src/quant/prng.ts:5-22      mulberry32, randomSigns
//   src/quant/rotator.ts:17-78  padToPow2, fwht, Rotator
//   src/quant/codec.ts:22-154   quantizeRow / quantizeRow4 / quantizeRow1
//   src/store/store.ts:114-217  dotRow, l2Row, normalizeInPlace
//   src/index/flat.ts:217-239   topK (tie semantics)
//   src/index/ivfquant.ts:114-124,235-245  the reservoir sampler's slots
//   src/index/kmeans.ts:154-219 random init picks, the Float32Array mean
//                               update, normalizeRows
// The oracle (oracle/bv_oracle.c) must reproduce every value bit for bit.
//
// Usage: node tests/golden/make_js_vectors.js > tests/golden/js_vectors.json
'use strict';

function makeRng(seed) {
  var state = seed >>> 0;
  return function () {
    state = (state + 0x6d2b79f5) | 0;
    var x = Math.imul(state ^ (state >>> 15), state | 1);
    x = (x + Math.imul(x ^ (x >>> 7), x | 61)) ^ x;
    return ((x ^ (x >>> 14)) >>> 0) / 4294967296;
  };
}

function signVector(n, seed) {
  var rng = makeRng(seed);
  var v = new Float32Array(n);
  for (var i = 0; i < n; i++) v[i] = rng() < 0.5 ? -1 : 1;
  return v;
}

function pow2Pad(n) {
  var p = 4;
  while (p < n) p *= 2;
  return p;
}

function hadamardInPlace(a) {
  var n = a.length;
  for (var h = 1; h < n; h *= 2) {
    for (var blk = 0; blk < n; blk += 2 * h) {
      for (var j = blk; j < blk + h; j++) {
        var u = a[j];
        var w = a[j + h];
        a[j] = u + w;
        a[j + h] = u - w;
      }
    }
  }
}

function makeRotation(dim, seed, rounds) {
  var P = pow2Pad(dim);
  var inv = 1 / Math.sqrt(P);
  var tables = [];
  for (var r = 0; r < rounds; r++) {
    var s = signVector(P, (seed ^ (0x9e3779b9 * (r + 1))) >>> 0);
    for (var i = 0; i < P; i++) s[i] = s[i] * inv;
    tables.push(s);
  }
  return function (src) {
    var out = new Float32Array(P);
    for (var i = 0; i < src.length; i++) out[i] = src[i];
    for (var r = 0; r < rounds; r++) {
      var s = tables[r];
      for (var i = 0; i < P; i++) out[i] = out[i] * s[i];
      hadamardInPlace(out);
    }
    return out;
  };
}

function codeOf(x, levels) {
  var c = x;
  if (c < -1) c = -1;
  if (c > 1) c = 1;
  var b = Math.round(c * levels);
  if (b < -levels) b = -levels;
  if (b > levels) b = levels;
  return b;
}

function quant8(v) {
  var m = 0;
  for (var i = 0; i < v.length; i++) { var a = Math.abs(v[i]); if (a > m) m = a; }
  var scale = m > 0 ? m : 1;
  var inv = 1 / scale;
  var words = new Uint32Array(v.length / 4);
  for (var g = 0; g < words.length; g++) {
    var w = 0;
    for (var j = 0; j < 4; j++) w |= (codeOf(v[4 * g + j] * inv, 127) & 0xff) << (8 * j);
    words[g] = w >>> 0;
  }
  return { words: Array.from(words), scale: scale };
}

function quant4(v) {
  var m = 0;
  for (var i = 0; i < v.length; i++) { var a = Math.abs(v[i]); if (a > m) m = a; }
  var scale = m > 0 ? m : 1;
  var inv = 1 / scale;
  var words = new Uint32Array(v.length / 8);
  for (var g = 0; g < words.length; g++) {
    var w = 0;
    for (var j = 0; j < 8; j++) w |= (codeOf(v[8 * g + j] * inv, 7) & 0xf) << (4 * j);
    words[g] = w >>> 0;
  }
  return { words: Array.from(words), scale: scale };
}

function quant1(v) {
  var t = 0;
  for (var i = 0; i < v.length; i++) t += Math.abs(v[i]);
  var scale = t > 0 ? t / v.length : 1;
  var words = new Uint32Array(v.length / 32);
  for (var g = 0; g < words.length; g++) {
    var w = 0;
    for (var j = 0; j < 32; j++) if (v[32 * g + j] >= 0) w |= 1 << j;
    words[g] = w >>> 0;
  }
  return { words: Array.from(words), scale: scale };
}

function unitNormalize(v) {
  var s = 0;
  for (var i = 0; i < v.length; i++) s += v[i] * v[i];
  var nrm = Math.sqrt(s);
  if (nrm > 0) { var inv = 1 / nrm; for (var i = 0; i < v.length; i++) v[i] = v[i] * inv; }
}

function dot4way(x, y) {
  var n = x.length, lim = n - (n % 4);
  var s0 = 0, s1 = 0, s2 = 0, s3 = 0, i = 0;
  for (; i < lim; i += 4) {
    s0 += x[i] * y[i]; s1 += x[i + 1] * y[i + 1]; s2 += x[i + 2] * y[i + 2]; s3 += x[i + 3] * y[i + 3];
  }
  var acc = s0 + s1 + s2 + s3;
  for (; i < n; i++) acc += x[i] * y[i];
  return acc;
}

function negSq4way(x, y) {
  var n = x.length, lim = n - (n % 4);
  var s0 = 0, s1 = 0, s2 = 0, s3 = 0, i = 0;
  for (; i < lim; i += 4) {
    var d0 = x[i] - y[i], d1 = x[i + 1] - y[i + 1], d2 = x[i + 2] - y[i + 2], d3 = x[i + 3] - y[i + 3];
    s0 += d0 * d0; s1 += d1 * d1; s2 += d2 * d2; s3 += d3 * d3;
  }
  var acc = s0 + s1 + s2 + s3;
  for (; i < n; i++) { var d = x[i] - y[i]; acc += d * d; }
  return -acc;
}

function selectTop(scores, k) {
  var lim = Math.min(k, scores.length);
  if (lim <= 0) return [];
  var h = [];
  for (var row = 0; row < scores.length; row++) {
    var sc = scores[row];
    if (h.length < lim) {
      h.push({ row: row, score: sc });
      if (h.length === lim) h.sort(function (a, b) { return a.score - b.score; });
    } else if (sc > h[0].score) {
      h[0] = { row: row, score: sc };
      for (var i = 0; i + 1 < h.length && h[i].score > h[i + 1].score; i++) {
        var t = h[i]; h[i] = h[i + 1]; h[i + 1] = t;
      }
    }
  }
  return h.sort(function (a, b) { return b.score - a.score; });
}

function f32bits(arr) {
  return Array.from(new Uint32Array(new Float32Array(arr).buffer));
}

function uniformVec(n, seed, mul) {
  var rng = makeRng(seed);
  var v = new Float32Array(n);
  for (var i = 0; i < n; i++) v[i] = (rng() * 2 - 1) * mul;
  return v;
}

var out = { generator: 'tests/golden/make_js_vectors.js', node: process.version };

// mulberry32 streams
out.mulberry32 = [0, 1, 42, 7, 0xdeadbeef, 0x9e3779b9, 0xffffffff].map(function (seed) {
  var rng = makeRng(seed);
  var draws = [];
  for (var i = 0; i < 64; i++) draws.push(rng());
  return { seed: seed >>> 0, draws: draws };
});

// signs for the default rotation seed, round 0 and 1
out.signs = [0, 1].map(function (r) {
  var seed = (0x9e3779b9 ^ (0x9e3779b9 * (r + 1))) >>> 0;
  return { round: r, seed: seed, bits: f32bits(signVector(64, seed)) };
});

// rotations (dim, seed, rounds) of uniform vectors
out.rotate = [[6, 1, 2, 7], [100, 12345, 2, 2], [384, 99, 2, 4], [768, 0x9e3779b9, 2, 11], [64, 1, 3, 5]].map(
  function (c) {
    var v = uniformVec(c[0], c[3], 1);
    return { dim: c[0], seed: c[1] >>> 0, rounds: c[2], vec_seed: c[3], input: f32bits(v),
             output: f32bits(makeRotation(c[0], c[1] >>> 0, c[2])(v)) };
  });

// codecs on uniform*3 vectors, rotated rows, and hand-made boundary rows
var codecInputs = [];
codecInputs.push(f32bits(uniformVec(64, 1, 3)));
codecInputs.push(f32bits(makeRotation(768, 0x9e3779b9, 2)(uniformVec(768, 21, 1))));
codecInputs.push(f32bits(new Float32Array([0.5, -2.5, 1, 0, 0, 0, 0, 0])));
// values whose scaled code lands on x.5 boundaries: v/127*(k+0.5) with max 1
var b = new Float32Array(256);
b[0] = 1;
for (var i = 1; i < 256; i++) b[i] = ((i % 2 ? 1 : -1) * (((i * 37) % 127) + 0.5)) / 127;
codecInputs.push(f32bits(b));
var b4 = new Float32Array(64);
b4[0] = -1;
for (var i = 1; i < 64; i++) b4[i] = ((i % 2 ? -1 : 1) * ((i % 7) + 0.5)) / 7;
codecInputs.push(f32bits(b4));
// non-finite and subnormal rows: NaN never raises the max, an infinite max
// scales every finite value to 0, NaN codes store as 0
var nf = uniformVec(64, 5, 1);
nf[3] = NaN; nf[17] = 1e-45; nf[40] = -3e-39;
codecInputs.push(f32bits(nf));
var inf = uniformVec(64, 6, 1);
inf[9] = Infinity; inf[50] = NaN;
codecInputs.push(f32bits(inf));
var sub = new Float32Array(64);
for (var i = 0; i < 64; i++) sub[i] = (i % 3 ? 1 : -1) * 1e-45 * (1 + (i % 11));
sub[5] = 3e-39;
codecInputs.push(f32bits(sub));
codecInputs.push(f32bits(makeRotation(64, 0x9e3779b9, 2)(sub)));
out.rotate.push({ dim: 64, seed: 0x9e3779b9, rounds: 2, vec_seed: -1, input: f32bits(sub),
                  output: f32bits(makeRotation(64, 0x9e3779b9, 2)(sub)) });
out.rotate.push({ dim: 64, seed: 0x9e3779b9, rounds: 2, vec_seed: -1, input: f32bits(inf),
                  output: f32bits(makeRotation(64, 0x9e3779b9, 2)(inf)) });
out.codec = codecInputs.map(function (bits) {
  var v = new Float32Array(new Uint32Array(bits).buffer);
  var r = { input: bits, q8: quant8(v), q4: null, q1: null };
  if (v.length % 8 === 0) r.q4 = quant4(v);
  if (v.length % 32 === 0) r.q1 = quant1(v);
  r.q8.scale_f32 = f32bits([r.q8.scale])[0];
  if (r.q4) r.q4.scale_f32 = f32bits([r.q4.scale])[0];
  if (r.q1) r.q1.scale_f32 = f32bits([r.q1.scale])[0];
  return r;
});

// Math.round boundary probes (the quantizer's rounding primitive)
out.js_round = [0.5, -0.5, 1.5, -1.5, 2.5, 0.49999999999999994, -0.49999999999999994, 126.5, -126.5, 3.4999999999999996]
  .map(function (x) { return { x: x, round: Math.round(x) }; });

// store arithmetic
out.store = [[768, 31], [100, 32], [7, 33], [1024, 34]].map(function (c) {
  var a = uniformVec(c[0], c[1], 1);
  var q = uniformVec(c[0], c[1] + 1000, 1);
  var an = a.slice(); unitNormalize(an);
  return { dim: c[0], a: f32bits(a), q: f32bits(q), normalized: f32bits(an), dot: dot4way(a, q), l2: negSq4way(a, q),
           dot_f32: f32bits([dot4way(a, q)])[0] };
});

// topK tie semantics
out.topk = [
  { scores: [5, 5, 7], k: 2 },
  { scores: [1, 1, 1, 0], k: 3 },
  { scores: [3, 1, 2], k: 10 },
  { scores: [2, 2, 2, 2, 3, 3, 1, 2, 3], k: 4 },
].map(function (c) {
  var r = selectTop(new Float32Array(c.scores), c.k);
  return { scores: c.scores, k: c.k, rows: r.map(function (h) { return h.row; }) };
});
var rs = uniformVec(200, 77, 3);
for (var i = 0; i < 200; i += 3) rs[i] = rs[0];
out.topk.push({ scores: Array.from(rs), k: 25, rows: selectTop(rs, 25).map(function (h) { return h.row; }) });

// reservoir: the slot each appended row takes (-1: not sampled) for a
// sampler of capacity `cap` seeded (seed ^ 0x85ebca6b) >>> 0
function reservoirSlots(cap, seed, n) {
  var rng = makeRng((seed ^ 0x85ebca6b) >>> 0);
  var filled = 0, seen = 0, slots = [];
  for (var i = 0; i < n; i++) {
    if (filled < cap) {
      slots.push(filled);
      filled++;
    } else {
      var j = Math.floor(rng() * (seen + 1));
      slots.push(j < cap ? j : -1);
    }
    seen++;
  }
  return slots;
}
out.reservoir = [[1024, 0x9e3779b9, 3000], [1024, 7, 5000], [1500, 0x51ed270b, 4000]].map(function (c) {
  return { cap: c[0], seed: c[1] >>> 0, n: c[2], slots: reservoirSlots(c[0], c[1] >>> 0, c[2]) };
});

// random init: the sample row each centroid copies
out.init_picks = [[0x51ed270b, 16, 1200], [77, 4096, 8192], [12345, 24, 6000]].map(function (c) {
  var rng = makeRng(c[0]);
  var picks = [];
  for (var i = 0; i < c[1]; i++) picks.push(Math.floor(rng() * c[2]));
  return { seed: c[0] >>> 0, nlist: c[1], count: c[2], picks: picks };
});

// mean update with Float32Array sums: values chosen so that the sequential
// f32 sums differ from f64 sums (a large value absorbs small ones), plus an
// empty cluster re-seeded from the sample, then normalizeRows
function meanUpdate(sample, count, dim, assign, centroids, nlist, seed) {
  var sums = new Float32Array(nlist * dim);
  var counts = new Int32Array(nlist);
  for (var r = 0; r < count; r++) {
    var c = assign[r];
    for (var i = 0; i < dim; i++) sums[c * dim + i] += sample[r * dim + i];
    counts[c]++;
  }
  var rng = makeRng(seed);
  for (var c2 = 0; c2 < nlist; c2++) {
    if (counts[c2] === 0) {
      var pick = Math.floor(rng() * count);
      for (var i2 = 0; i2 < dim; i2++) centroids[c2 * dim + i2] = sample[pick * dim + i2];
    } else {
      var inv = 1 / counts[c2];
      for (var i3 = 0; i3 < dim; i3++) centroids[c2 * dim + i3] = sums[c2 * dim + i3] * inv;
    }
  }
  for (var r2 = 0; r2 < nlist; r2++) {
    var s = 0;
    for (var i4 = 0; i4 < dim; i4++) s += centroids[r2 * dim + i4] * centroids[r2 * dim + i4];
    var iv = 1 / (Math.sqrt(s) || 1);
    for (var i5 = 0; i5 < dim; i5++) centroids[r2 * dim + i5] *= iv;
  }
  return centroids;
}
(function () {
  var dim = 4, nlist = 3, count = 9;
  var sample = new Float32Array(count * dim);
  var u = uniformVec(count * dim, 91, 1);
  for (var i = 0; i < count * dim; i++) sample[i] = u[i];
  // cluster 0: one large value followed by many small ones in each column
  sample[0] = 16777216; sample[1] = 1; sample[2] = 3.0000002; sample[3] = -8388608;
  for (var r = 1; r < 6; r++) { sample[r * dim] = 1; sample[r * dim + 1] = 1e-8; sample[r * dim + 2] = 1.1920929e-7; sample[r * dim + 3] = 0.75; }
  var assign = new Uint32Array([0, 0, 0, 0, 0, 0, 2, 2, 0]);  // cluster 1 stays empty
  var cen = new Float32Array(nlist * dim);
  var before = f32bits(cen);
  out.mean_update = { dim: dim, nlist: nlist, count: count, seed: 4242, sample: f32bits(sample),
                      assign: Array.from(assign), centroids_in: before,
                      centroids_out: f32bits(meanUpdate(sample, count, dim, assign, cen, nlist, 4242)) };
  var s64 = 0;
  for (var r3 = 0; r3 < count; r3++) if (assign[r3] === 0) s64 += sample[r3 * dim];
  var acc = new Float32Array(1);
  for (var r4 = 0; r4 < count; r4++) if (assign[r4] === 0) acc[0] += sample[r4 * dim];
  out.mean_update.col0_f64_sum = s64;
  out.mean_update.col0_f32_sum = acc[0];
})();

process.stdout.write(JSON.stringify(out));
