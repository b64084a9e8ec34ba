"""Index classes behind the reference's ``VectorIndex`` seam.

``FlatIndex`` / ``QuantIndex`` mirror src/index/flat.ts:42-211 and
src/index/quant.ts:21-258: same constructor knowledge (dim, metric, bits,
seed, rounds, chunkRows), same ``size`` / ``append`` / ``query`` /
``queryMasked`` / ``destroy`` surface and error messages, with every byte of
corpus and every scan living on the MI355X through libbrowservec_hip.so.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib as L


@dataclass(frozen=True)
class FlatHit:
    """One result (src/index/flat.ts:24-27): row id and score (higher = closer)."""

    row: int
    score: float


def _ptr(a: np.ndarray | None):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _check_len(a: np.ndarray, want: int) -> None:
    """The library reads exactly `want` floats: refuse any other length before
    a pointer reaches it (the reference's message, src/index/flat.ts:96-98)."""
    if a.size != want:
        raise L.BVError(L.BV_E_INVALID, f"expected {want} floats, got {a.size}")


class DeviceContext:
    """The engine's DeviceContext (src/engine/device.ts:3-9) over a HIP device."""

    def __init__(self, ordinal: int = 0):
        self.lib = L.load()
        h = ctypes.c_void_p()
        L.check(self.lib.bv_device_open(ordinal, ctypes.byref(h)))
        self.handle = h

    @property
    def lost(self) -> bool:
        v = ctypes.c_int(0)
        L.check(self.lib.bv_device_is_lost(self.handle, ctypes.byref(v)))
        return bool(v.value)

    def info(self) -> dict:
        name = ctypes.create_string_buffer(256)
        cu = ctypes.c_uint32()
        hbm = ctypes.c_uint64()
        L.check(self.lib.bv_device_info(self.handle, name, 256, ctypes.byref(cu), ctypes.byref(hbm)))
        return {"name": name.value.decode(), "cu_count": cu.value, "hbm_bytes": hbm.value}

    def debug_inject(self, what: str) -> None:
        """Force the device-lost state ('lost'), a failed allocation on the
        next append ('append_oom') or a failure of the next append after its
        rows are encoded ('append_late') from the host; no device work is made
        to fail."""
        L.check(self.lib.bv_debug_inject(self.handle, {"lost": 1, "append_oom": 2, "append_late": 3}[what]))

    def destroy(self) -> None:
        if self.handle:
            self.lib.bv_device_close(self.handle)
            self.handle = None


class NativeIndex:
    """Common native-index plumbing; subclasses fix the index kind."""

    kind = L.KIND_FLAT

    def __init__(self, ctx: DeviceContext, dim: int, metric: str = "cosine", bits: int = 0,
                 seed: int | None = None, rounds: int = 2, chunk_rows: int | None = None,
                 scorer: str = "asym", ivf: dict | None = None):
        self.ctx = ctx
        self.lib = ctx.lib
        self.dim = int(dim)
        self.metric = metric
        self.bits = bits
        d = L.IndexDesc()
        d.size = ctypes.sizeof(L.IndexDesc)
        d.kind = self.kind
        d.dim = self.dim
        if metric not in L.METRICS:
            raise L.BVError(L.BV_E_INVALID, f"unknown metric {metric}")
        d.metric = L.METRICS[metric]
        d.bits = bits
        d.scorer = L.SCORERS[scorer]
        if seed is not None:
            d.seed = seed & 0xFFFFFFFF
            d.has_seed = 1
        d.rounds = rounds
        d.chunk_rows = chunk_rows or 0
        d.target_recall = -1.0
        ivf = ivf or {}
        d.nlist = ivf.get("nlist") or 0
        d.nprobe = ivf.get("nprobe") or 0
        d.sample_size = ivf.get("sampleSize") or 0
        d.train_size = ivf.get("trainSize") or 0
        d.iters = ivf.get("iters") or 0
        if ivf.get("seed") is not None:
            d.ivf_seed = ivf["seed"] & 0xFFFFFFFF
            d.has_ivf_seed = 1
        if ivf.get("targetRecall") is not None:
            d.target_recall = float(ivf["targetRecall"])
        d.ivf_incremental = 1 if ivf.get("incremental") else 0
        h = ctypes.c_void_p()
        L.check(self.lib.bv_index_create(ctx.handle, ctypes.byref(d), ctypes.byref(h)))
        self.handle = h

    # -- VectorIndex -------------------------------------------------------
    @property
    def size(self) -> int:
        v = ctypes.c_uint64()
        L.check(self.lib.bv_index_size(self.handle, ctypes.byref(v)))
        return v.value

    def append(self, data, count: int) -> None:
        data = _f32(data).reshape(-1)
        L.check(self.lib.bv_index_append(self.handle, _ptr(data), data.size, int(count)))

    def query(self, q, k: int) -> list[FlatHit]:
        q = _f32(q).reshape(-1)
        _check_len(q, self.dim)
        rows = np.empty(max(k, 1), np.uint32)
        scores = np.empty(max(k, 1), np.float32)
        n = ctypes.c_uint32()
        L.check(self.lib.bv_index_query(self.handle, _ptr(q), int(k), _ptr(rows), _ptr(scores), ctypes.byref(n)))
        return [FlatHit(int(rows[i]), float(scores[i])) for i in range(n.value)]

    def query_masked(self, q, k: int, mask_words) -> list[FlatHit]:
        q = _f32(q).reshape(-1)
        _check_len(q, self.dim)
        m = np.ascontiguousarray(mask_words, dtype=np.uint32)
        rows = np.empty(max(k, 1), np.uint32)
        scores = np.empty(max(k, 1), np.float32)
        n = ctypes.c_uint32()
        L.check(self.lib.bv_index_query_masked(self.handle, _ptr(q), int(k), _ptr(m), m.size, _ptr(rows),
                                               _ptr(scores), ctypes.byref(n)))
        return [FlatHit(int(rows[i]), float(scores[i])) for i in range(n.value)]

    def query_rows(self, q, rows, k: int) -> list[FlatHit]:
        """queryRowsExact (src/index.ts:445-464) on the device: the exact
        scores of the listed rows (Store.dotRow, or Store.l2Row under l2) and
        their top k, as (row, score)."""
        q = _f32(q).reshape(-1)
        _check_len(q, self.dim)
        lst = np.ascontiguousarray(rows, dtype=np.uint32).reshape(-1)
        return self._rows_call(self.lib.bv_index_query_rows, q, lst, k)

    def query_rows_masked(self, q, k: int, mask_words) -> list[FlatHit]:
        """query_rows over the rows whose mask bit is set; the row list is
        built on the device."""
        q = _f32(q).reshape(-1)
        _check_len(q, self.dim)
        m = np.ascontiguousarray(mask_words, dtype=np.uint32).reshape(-1)
        return self._rows_call(self.lib.bv_index_query_rows_masked, q, m, k)

    def _rows_call(self, fn, q, arr, k):
        out_rows = np.empty(max(k, 1), np.uint32)
        scores = np.empty(max(k, 1), np.float32)
        n = ctypes.c_uint32()
        L.check(fn(self.handle, _ptr(q), _ptr(arr) if arr.size else None, arr.size, int(k), _ptr(out_rows),
                   _ptr(scores), ctypes.byref(n)))
        return [FlatHit(int(out_rows[i]), float(scores[i])) for i in range(n.value)]

    def query_batch(self, packed, n: int, k: int) -> list[list[FlatHit]]:
        packed = _f32(packed).reshape(-1)
        _check_len(packed, int(n) * self.dim)
        rows = np.empty((n, max(k, 1)), np.uint32)
        scores = np.empty((n, max(k, 1)), np.float32)
        cnt = np.empty(max(n, 1), np.uint32)
        L.check(self.lib.bv_index_query_batch(self.handle, _ptr(packed), int(n), int(k), _ptr(rows),
                                              _ptr(scores), _ptr(cnt)))
        return [[FlatHit(int(rows[i, j]), float(scores[i, j])) for j in range(cnt[i])] for i in range(n)]

    def destroy(self) -> None:
        if getattr(self, "handle", None):
            self.lib.bv_index_destroy(self.handle)
            self.handle = None

    # -- extras ------------------------------------------------------------
    def set_nprobe(self, n: int | None) -> None:
        L.check(self.lib.bv_index_set_nprobe(self.handle, int(n or 0)))

    def search(self, queries, fetch: int, k: int):
        """Approximate top-`fetch` then exact f64 re-rank to top-`k`, on the
        device (BrowserVec.query's quantized path, src/index.ts:414-418).
        Returns (rows[nq,k], scores[nq,k], counts[nq])."""
        qs = _f32(queries)
        if qs.size % self.dim:
            _check_len(qs, (qs.size // self.dim + 1) * self.dim)
        qs = qs.reshape(-1, self.dim)
        nq = qs.shape[0]
        rows = np.empty((nq, max(k, 1)), np.uint32)
        scores = np.empty((nq, max(k, 1)), np.float32)
        cnt = np.empty(max(nq, 1), np.uint32)
        L.check(self.lib.bv_index_search(self.handle, _ptr(qs), nq, int(fetch), int(k), _ptr(rows), _ptr(scores),
                                          _ptr(cnt)))
        return rows[:, :k], scores[:, :k], cnt[:nq]

    def rerank(self, q, cand, k: int) -> list[FlatHit]:
        """BrowserVec.rerankExact on the device (src/index.ts:583-594)."""
        q = _f32(q).reshape(-1)
        _check_len(q, self.dim)
        c = np.ascontiguousarray(cand, dtype=np.uint32)
        rows = np.empty(max(k, 1), np.uint32)
        scores = np.empty(max(k, 1), np.float32)
        n = ctypes.c_uint32()
        L.check(self.lib.bv_index_rerank(self.handle, _ptr(q), _ptr(c), c.size, int(k), _ptr(rows), _ptr(scores),
                                         ctypes.byref(n)))
        return [FlatHit(int(rows[i]), float(scores[i])) for i in range(n.value)]

    def stats(self) -> dict:
        s = L.IndexStats()
        L.check(self.lib.bv_index_get_stats(self.handle, ctypes.byref(s)))
        return {f: getattr(s, f) for f, _ in L.IndexStats._fields_}

    @property
    def chunk_count(self) -> int:
        return self.stats()["chunk_count"]

    def export_scores(self, q) -> np.ndarray:
        q = _f32(q).reshape(-1)
        _check_len(q, self.dim)
        out = np.empty(self.size, np.float32)
        L.check(self.lib.bv_index_export_scores(self.handle, _ptr(q), _ptr(out)))
        return out

    # quantized kinds (QuantIndex, IVFQuantIndex): parity exports
    def export_codes(self, row0: int = 0, count: int | None = None):
        count = self.size - row0 if count is None else count
        words = np.empty((count, self.words_per_row), np.uint32)
        scales = np.empty(count, np.float32)
        L.check(self.lib.bv_index_export_codes(self.handle, row0, count, _ptr(words), _ptr(scales)))
        return words, scales

    def export_rotated_query(self, q) -> np.ndarray:
        q = _f32(q).reshape(-1)
        _check_len(q, self.dim)
        out = np.empty(self.padded_dim, np.float32)
        L.check(self.lib.bv_index_export_rotated_query(self.handle, _ptr(q), _ptr(out)))
        return out

    def save_section(self) -> bytes:
        """The index section of a snapshot: codes, scales and IVF state, so a
        load skips re-encoding and re-training."""
        size = ctypes.c_uint64(0)
        L.check(self.lib.bv_index_save_section(self.handle, None, 0, ctypes.byref(size)))
        buf = np.empty(size.value, np.uint8)
        L.check(self.lib.bv_index_save_section(self.handle, _ptr(buf), size.value, ctypes.byref(size)))
        return buf.tobytes()

    def load_section(self, data, count: int, section: bytes) -> None:
        """Fills this empty index from a snapshot's rows and a saved section."""
        data = _f32(data).reshape(-1)
        sec = np.frombuffer(section, np.uint8)
        L.check(self.lib.bv_index_load_section(self.handle, _ptr(data), data.size, int(count), _ptr(sec), sec.size))

    # device-resident entry points (pointers are integers, e.g. tensor.data_ptr())
    def append_device(self, d_ptr: int, count: int) -> None:
        L.check(self.lib.bv_index_append_device(self.handle, ctypes.c_void_p(d_ptr), int(count)))

    def search_device(self, d_q: int, nq: int, fetch: int, k: int, d_rows: int, d_scores: int, d_n: int) -> None:
        L.check(self.lib.bv_index_search_device(self.handle, ctypes.c_void_p(d_q), int(nq), int(fetch), int(k),
                                                ctypes.c_void_p(d_rows), ctypes.c_void_p(d_scores),
                                                ctypes.c_void_p(d_n)))

    def search_device_noalloc(self, d_q: int, nq: int, fetch: int, k: int, d_rows: int, d_scores: int,
                              d_n: int) -> None:
        """search_device without any device allocation (library-owned scratch)."""
        L.check(self.lib.bv_index_search_device_noalloc(self.handle, ctypes.c_void_p(d_q), int(nq), int(fetch),
                                                        int(k), ctypes.c_void_p(d_rows), ctypes.c_void_p(d_scores),
                                                        ctypes.c_void_p(d_n)))

    def sync(self) -> None:
        L.check(self.lib.bv_index_sync(self.handle))

    def set_query_streams(self, n: int) -> None:
        """1 to 4 streams for search_device's single queries (2 or more:
        consecutive calls take the streams in turn and overlap; each call in
        flight needs its own outputs)."""
        L.check(self.lib.bv_index_set_query_streams(self.handle, int(n)))

    def stream_ptr(self) -> int:
        s = ctypes.c_void_p()
        L.check(self.lib.bv_index_stream(self.handle, ctypes.byref(s)))
        return s.value or 0

    def kernel_timing(self, enable: bool):
        ms = ctypes.c_double()
        n = ctypes.c_uint64()
        L.check(self.lib.bv_index_kernel_timing(self.handle, 1 if enable else 0, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class FlatIndex(NativeIndex):
    """Exact fp32 flat index (src/index/flat.ts:42-211)."""

    kind = L.KIND_FLAT

    def __init__(self, ctx, dim, metric="cosine", chunk_rows=None):
        super().__init__(ctx, dim, metric, 0, chunk_rows=chunk_rows)


class QuantIndex(NativeIndex):
    """TurboQuant flat index (src/index/quant.ts:21-258): rotate + quantize on
    the device at append; asymmetric scans (or the Hamming / int8 scorers)."""

    kind = L.KIND_QUANT

    def __init__(self, ctx, dim, seed=0x9E3779B9, rounds=2, bits=8, chunk_rows=None, scorer="asym",
                 metric="cosine"):
        super().__init__(ctx, dim, metric, bits, seed=seed, rounds=rounds, chunk_rows=chunk_rows, scorer=scorer)
        st = self.stats()
        self.padded_dim = st["padded_dim"]
        self.words_per_row = st["words_per_row"]

    @property
    def ingest_mode(self) -> str:
        """ingestMode (src/index/quant.ts:115-118): where rotate+quantize ran,
        'pending' before the first append."""
        return "device" if self.size else "pending"

class IVFIndex(NativeIndex):
    """IVF over fp32 rows (src/index/ivf.ts:51): spherical k-means lists,
    probes by exact dot with the centroids, scan of the probed lists."""

    kind = L.KIND_IVF
    is_ivf = True  # BrowserVec filters IVF queries by over-fetching (src/index.ts:389-394)

    def __init__(self, ctx, dim, metric="cosine", ivf: dict | None = None, chunk_rows=None):
        super().__init__(ctx, dim, metric, 0, chunk_rows=chunk_rows, ivf=ivf)

    def build(self) -> None:
        L.check(self.lib.bv_index_build(self.handle))

    @property
    def train_mode(self) -> str:
        """trainMode (src/index/ivf.ts:133-135): where the k-means mean update
        ran, 'pending' before a build."""
        return "device" if self.stats()["nlist"] else "pending"

    def export_ivf(self):
        """(centroids [nlist, D], list offsets [nlist+1], list rows [rows]):
        the lists a query would probe now."""
        L.check(self.lib.bv_index_export_ivf(self.handle, None, None, None))  # builds stale lists
        st = self.stats()
        nlist = st["nlist"]
        D = st["padded_dim"] if self.bits else self.dim
        cen = np.empty((nlist, D), np.float32)
        off = np.empty(nlist + 1, np.uint32)
        rows = np.empty(max(self.size, 1), np.uint32)
        L.check(self.lib.bv_index_export_ivf(self.handle, _ptr(cen), _ptr(off), _ptr(rows)))
        return cen, off, rows[: self.size]

    def export_probe_scores(self, queries) -> np.ndarray:
        """pickProbes' score of every centroid for each query, [nq, nlist]."""
        qs = _f32(queries)
        _check_len(qs, qs.size // self.dim * self.dim if qs.size else self.dim)
        qs = qs.reshape(-1, self.dim)
        self.build()
        out = np.empty((qs.shape[0], self.stats()["nlist"]), np.float32)
        L.check(self.lib.bv_index_export_probe_scores(self.handle, _ptr(qs), qs.shape[0], _ptr(out)))
        return out


class IVFQuantIndex(IVFIndex):
    """IVF over TurboQuant codes (src/index/ivfquant.ts:33): k-means on the
    rotated reservoir sample, rows assigned by their codes."""

    kind = L.KIND_IVFQUANT

    def __init__(self, ctx, dim, bits=8, seed=0x9E3779B9, rounds=2, ivf: dict | None = None, chunk_rows=None,
                 metric="cosine"):
        NativeIndex.__init__(self, ctx, dim, metric, bits, seed=seed, rounds=rounds, chunk_rows=chunk_rows, ivf=ivf)
        st = self.stats()
        self.padded_dim = st["padded_dim"]
        self.words_per_row = st["words_per_row"]

    @property
    def ingest_mode(self) -> str:
        return "device" if self.size else "pending"


class GraphSearcher:
    """HNSWGpuSearcher (src/index/hnswGpu.ts:28-244): corpus rows and the
    layer-0 adjacency on the device, beam search of query batches
    (src/engine/wgsl/graphSearch.ts), one wave per query."""

    EF_CAP = 256
    EMPTY = 0xFFFFFFFF

    def __init__(self, ctx, dim, metric="cosine", degree=32):
        self.lib = ctx.lib
        self.dim = int(dim)
        self.degree = int(degree)
        h = ctypes.c_void_p()
        L.check(self.lib.bv_graph_create(ctx.handle, self.dim, L.METRICS[metric], self.degree, ctypes.byref(h)))
        self.handle = h

    def append(self, data, count: int) -> None:
        data = _f32(data).reshape(-1)
        L.check(self.lib.bv_graph_append(self.handle, _ptr(data), data.size, int(count)))

    def upload_graph(self, links, rows: int) -> None:
        links = np.ascontiguousarray(links, dtype=np.uint32).reshape(-1)
        if links.size < int(rows) * self.degree:
            raise ValueError(f"expected {int(rows) * self.degree} links, got {links.size}")
        L.check(self.lib.bv_graph_upload(self.handle, _ptr(links) if links.size else None, int(rows)))

    def search_arrays(self, queries, n: int, k: int, ef: int, entry: int):
        """search() as arrays: rows [n, k], scores [n, k], counts [n]."""
        qs = _f32(queries).reshape(-1)
        _check_len(qs, int(n) * self.dim)
        rows = np.empty((max(n, 1), max(k, 1)), np.uint32)
        scores = np.empty((max(n, 1), max(k, 1)), np.float32)
        cnt = np.zeros(max(n, 1), np.uint32)
        L.check(self.lib.bv_graph_search(self.handle, _ptr(qs), int(n), int(k), int(ef), int(entry) & 0xFFFFFFFF,
                                         _ptr(rows), _ptr(scores), _ptr(cnt)))
        return rows, scores, cnt

    def search(self, queries, n: int, k: int, ef: int, entry: int) -> list[list[FlatHit]]:
        rows, scores, cnt = self.search_arrays(queries, n, k, ef, entry)
        return [[FlatHit(int(rows[i, j]), float(scores[i, j])) for j in range(cnt[i])] for i in range(n)]

    def search_beams(self, queries, entries, ef: int, iter_cap: int):
        """Raw beams for parity: (dist [nq, 256], id [nq, 256])."""
        qs = _f32(queries).reshape(-1, self.dim)
        e = np.ascontiguousarray(entries, dtype=np.uint32).reshape(-1)
        nq = qs.shape[0]
        dist = np.empty((nq, self.EF_CAP), np.float32)
        ids = np.empty((nq, self.EF_CAP), np.uint32)
        L.check(self.lib.bv_graph_search_beams(self.handle, _ptr(qs), nq, _ptr(e), e.size, int(ef), int(iter_cap),
                                               _ptr(dist), _ptr(ids)))
        return dist, ids

    def destroy(self) -> None:
        if getattr(self, "handle", None):
            self.lib.bv_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass
