"""``BrowserVec``: the public API (src/index.ts:203-757) over the native indexes.

Only the search path is native; this module keeps the reference's host-side
orchestration (id/row bookkeeping, normalization, tombstones, filters,
kEff / fetch / re-rank arithmetic) so ``create / addBatch / query /
queryBatch`` behave as in the reference.  Persistence, encryption, embedders
and HNSW are outside this build.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass, field
from typing import Any, Callable

import numpy as np

from . import _lib as L
from .index import DeviceContext, FlatHit, FlatIndex, IVFIndex, IVFQuantIndex, NativeIndex, QuantIndex

DEFAULT_SEED = 0x9E3779B9  # src/index.ts:71
FILTER_CPU_SCAN_MAX = 4096  # src/index.ts:76


def default_rerank_factor(bits: int) -> int:
    """defaultRerankFactor (src/index.ts:99-103)."""
    if bits == 1:
        return 32
    return 16 if bits == 4 else 4


def normalize_in_place(v: np.ndarray) -> np.ndarray:
    """normalizeInPlace (src/store/store.ts:209-217) on the last axis:
    sequential f64 sum of squares (np.cumsum accumulates in order),
    inv = 1/sqrt, f32 store.  Works on one vector or a block of rows."""
    v64 = v.astype(np.float64)
    ss = np.cumsum(v64 * v64, axis=-1)[..., -1:] if v.shape[-1] else np.zeros(v.shape[:-1] + (1,))
    norm = np.sqrt(ss)
    with np.errstate(divide="ignore"):
        inv = np.where(norm > 0, 1.0 / np.where(norm > 0, norm, 1.0), 1.0)
    out = np.where(norm > 0, v64 * inv, v64).astype(np.float32)
    v[...] = out
    return v


@dataclass
class RowEntry:
    id: str
    row: int
    metadata: Any = None


class Store:
    """id <-> row bookkeeping, tombstones and the fp32 source rows
    (src/store/store.ts:25-217)."""

    def __init__(self, dimension: int, metric: str, normalize: bool):
        self.dimension = dimension
        self.metric = metric
        self.normalize = normalize
        self.by_id: dict[str, RowEntry] = {}
        self.by_row: list[RowEntry] = []
        self.deleted: set[int] = set()
        self.raw = np.zeros((0, dimension), np.float32)
        self.raw_rows = 0

    @property
    def count(self) -> int:
        return len(self.by_id)

    @property
    def row_count(self) -> int:
        return len(self.by_row)

    @property
    def deleted_count(self) -> int:
        return len(self.deleted)

    def prepare(self, vector) -> np.ndarray:
        v = np.array(vector, dtype=np.float32, copy=True).reshape(-1)
        if v.size != self.dimension:
            raise ValueError(f"vector dim {v.size} != store dim {self.dimension}")
        if self.normalize:
            normalize_in_place(v)
        return v

    def _ensure(self, rows: int) -> None:
        if rows <= self.raw.shape[0]:
            return
        nxt = max(rows, math.ceil(self.raw.shape[0] * 1.5), 1024)
        grown = np.zeros((nxt, self.dimension), np.float32)
        grown[: self.raw_rows] = self.raw[: self.raw_rows]
        self.raw = grown

    def insert(self, id: str, prepared: np.ndarray, metadata=None) -> int:
        if id in self.by_id:
            raise ValueError(f"duplicate id: {id}")
        row = len(self.by_row)
        e = RowEntry(id, row, metadata)
        self.by_id[id] = e
        self.by_row.append(e)
        self._ensure(row + 1)
        self.raw[row] = prepared
        self.raw_rows = row + 1
        return row

    def insert_block(self, ids: list[str], prepared: np.ndarray, metas: list) -> int:
        base = len(self.by_row)
        for i, id in enumerate(ids):
            if id in self.by_id:
                raise ValueError(f"duplicate id: {id}")
        self._ensure(base + len(ids))
        for i, id in enumerate(ids):
            e = RowEntry(id, base + i, metas[i])
            self.by_id[id] = e
            self.by_row.append(e)
        self.raw[base: base + len(ids)] = prepared
        self.raw_rows = base + len(ids)
        return base

    def delete(self, id: str) -> bool:
        e = self.by_id.pop(id, None)
        if e is None:
            return False
        self.deleted.add(e.row)
        return True

    def is_deleted(self, row: int) -> bool:
        return row in self.deleted

    def live_entries(self) -> list[RowEntry]:
        return [e for e in self.by_row if e.row not in self.deleted]

    def live_vectors(self) -> np.ndarray:
        keep = [e.row for e in self.by_row if e.row not in self.deleted]
        return self.raw[keep].copy()

    def clear(self) -> None:
        self.__init__(self.dimension, self.metric, self.normalize)


class BrowserVec:
    """Mirror of the reference class (src/index.ts:203-757) for the search
    path.  ``filter`` takes a predicate ``metadata -> bool`` (the reference's
    Mongo-style filter compiler, src/store/filter.ts, is outside this build;
    its output -- a row mask -- is what crosses into the index)."""

    def __init__(self, ctx, store: Store, index: NativeIndex, make_index: Callable[[], NativeIndex]):
        self.ctx = ctx
        self.store = store
        self.index = index
        self.make_index = make_index
        self.quant_bits = 0
        self.rerank_factor = 4
        self.last_query_ms: float | None = None
        self.last_query_gpu_ms: float | None = None

    # ------------------------------------------------------------- create
    @staticmethod
    def create(dimension: int, metric: str = "cosine", normalize: bool | None = None, quantBits: int = 0,
               quant: dict | None = None, ann: dict | None = None, chunkRows: int | None = None,
               device: int = 0, scorer: str = "asym") -> "BrowserVec":
        """BrowserVec.create (src/index.ts:232-263) + buildIndex (105-142)."""
        if not isinstance(dimension, int) or dimension <= 0:
            raise ValueError(f"dimension must be a positive integer, got {dimension}")
        norm = (metric == "cosine") if normalize is None else normalize
        quant = quant or {}
        seed = quant.get("seed", DEFAULT_SEED)
        rounds = quant.get("rounds", 2)
        if ann is not None:
            if ann.get("type") == "hnsw":
                raise L.BVError(L.BV_E_UNSUPPORTED, "HNSW is not part of this build")
            if metric == "l2":
                raise ValueError("IVF supports metric cosine/dot only (l2 is later work)")
        if quantBits not in (0, 1, 4, 8):
            raise ValueError(f"quantBits {quantBits} not supported (ships 0, 1, 4, 8)")
        if quantBits and metric == "l2" and ann is None:
            raise ValueError("quantized mode supports metric cosine/dot only (l2 quantization is later work)")
        ctx = DeviceContext(device)

        def make():
            if ann is not None:
                if quantBits:
                    return IVFQuantIndex(ctx, dimension, bits=quantBits, seed=seed, rounds=rounds, ivf=ann,
                                         chunk_rows=chunkRows, metric=metric)
                return IVFIndex(ctx, dimension, metric, ivf=ann, chunk_rows=chunkRows)
            if quantBits == 0:
                return FlatIndex(ctx, dimension, metric, chunkRows)
            return QuantIndex(ctx, dimension, seed, rounds, quantBits, chunkRows, scorer=scorer, metric=metric)

        db = BrowserVec(ctx, Store(dimension, metric, norm), make(), make)
        db.quant_bits = quantBits
        db.rerank_factor = quant.get("rerankFactor", default_rerank_factor(quantBits))
        return db

    @property
    def dimension(self) -> int:
        return self.store.dimension

    @property
    def count(self) -> int:
        return self.store.count

    @property
    def metric(self) -> str:
        return self.store.metric

    # -------------------------------------------------------------- ingest
    def add(self, record: dict) -> None:
        vec = self.store.prepare(record["vector"])
        row = self.store.insert(record["id"], vec, record.get("metadata"))
        if row != self.index.size:
            raise RuntimeError("internal: store/index row mismatch")
        self.index.append(vec, 1)

    def add_batch(self, records: list[dict]) -> None:
        """addBatch (src/index.ts:293-305): prepare each row, one upload."""
        if not records:
            return
        dim = self.store.dimension
        packed = np.empty((len(records), dim), np.float32)
        for i, r in enumerate(records):
            v = np.asarray(r["vector"], dtype=np.float32).reshape(-1)
            if v.size != dim:
                raise ValueError(f"vector dim {v.size} != store dim {dim}")
            packed[i] = v
        if self.store.normalize:
            normalize_in_place(packed)
        base = self.store.insert_block([r["id"] for r in records], packed, [r.get("metadata") for r in records])
        if base != self.index.size:
            raise RuntimeError("internal: row mismatch in batch")
        self.index.append(packed, len(records))

    def add_vectors(self, ids: list[str], vectors: np.ndarray) -> None:
        """Bulk variant of add_batch for arrays (same preparation)."""
        packed = np.array(vectors, dtype=np.float32, copy=True).reshape(len(ids), self.store.dimension)
        if self.store.normalize:
            normalize_in_place(packed)
        base = self.store.insert_block(list(ids), packed, [None] * len(ids))
        if base != self.index.size:
            raise RuntimeError("internal: row mismatch in batch")
        self.index.append(packed, len(ids))

    # --------------------------------------------------------------- query
    def _prep_query(self, query) -> np.ndarray:
        q = np.array(query, dtype=np.float32, copy=True).reshape(-1)
        if q.size != self.store.dimension:
            raise ValueError(f"query dim {q.size} != store dim {self.store.dimension}")
        if self.store.normalize:
            normalize_in_place(q)
        return q

    def query(self, query, k: int = 10, filter: Callable[[Any], bool] | None = None, rerank: bool | None = None,
              nprobe: int | None = None) -> list[dict]:
        """BrowserVec.query (src/index.ts:343-436)."""
        q = self._prep_query(query)
        if nprobe is not None and hasattr(self.index, "set_nprobe"):
            self.index.set_nprobe(nprobe)
        skip_rows = 0
        mask = None
        if filter is not None:
            rc = self.store.row_count
            words = np.zeros(max((rc + 31) // 32, 1), np.uint32)
            match = []
            for row in range(rc):
                if self.store.is_deleted(row):
                    continue
                if filter(self.store.by_row[row].metadata):
                    match.append(row)
                    words[row >> 5] |= np.uint32(1 << (row & 31))
            if not match:
                return []
            if len(match) <= FILTER_CPU_SCAN_MAX:
                return self._query_rows_exact(q, match, k)
            if hasattr(self.index, "query_masked") and not getattr(self.index, "is_ivf", False):
                mask = words
            else:
                skip_rows = self.store.count - len(match)
                if skip_rows > max(2 * k, 256):
                    return self._query_rows_exact(q, match, k)
        deleted = self.store.deleted_count
        total = self.index.size
        k_eff = min(total, k) if mask is not None else min(total, k + deleted + skip_rows)

        def search(kk):
            return self.index.query_masked(q, kk, mask) if mask is not None else self.index.query(q, kk)

        t0 = time.perf_counter()
        if self.quant_bits > 0:
            do_rerank = rerank if rerank is not None else self.rerank_factor > 1
            fetch = min(total, max(k_eff, k_eff * self.rerank_factor)) if do_rerank else k_eff
            if do_rerank and mask is None and fetch <= 1024 and k_eff > 0:
                rows, scores, cnt = self.index.search(q, fetch, k_eff)
                hits = [FlatHit(int(rows[0, j]), float(scores[0, j])) for j in range(cnt[0])]
            else:
                approx = search(fetch)
                hits = self.rerank_exact(q, approx, k_eff) if do_rerank else approx[:k_eff]
        else:
            hits = search(k_eff)
        self.last_query_ms = (time.perf_counter() - t0) * 1e3
        self.last_query_gpu_ms = self.index.stats()["last_query_gpu_ms"]
        out = []
        for h in hits:
            if deleted and self.store.is_deleted(h.row):
                continue
            e = self.store.by_row[h.row]
            if filter is not None and not filter(e.metadata):
                continue
            r = {"id": e.id, "score": h.score}
            if e.metadata is not None:
                r["metadata"] = e.metadata
            out.append(r)
            if len(out) == k:
                break
        return out

    def _query_rows_exact(self, q: np.ndarray, rows: list[int], k: int) -> list[dict]:
        """queryRowsExact (src/index.ts:445-464): the matching rows' exact
        Store.dotRow / Store.l2Row scores and their top k, computed on the
        device over the index's stored rows."""
        t0 = time.perf_counter()
        hits = self.index.query_rows(q, np.asarray(rows, dtype=np.uint32), k)
        self.last_query_ms = (time.perf_counter() - t0) * 1e3
        self.last_query_gpu_ms = self.index.stats()["last_query_gpu_ms"]
        out = []
        for h in hits:
            e = self.store.by_row[h.row]
            r = {"id": e.id, "score": h.score}
            if e.metadata is not None:
                r["metadata"] = e.metadata
            out.append(r)
        return out

    def rerank_exact(self, q: np.ndarray, candidates: list[FlatHit], k: int) -> list[FlatHit]:
        """rerankExact (src/index.ts:583-594) with Store.dotRow's f64
        arithmetic, evaluated on the device against the stored rows."""
        if not candidates:
            return []
        return self.index.rerank(q, [h.row for h in candidates], k)

    def query_batch(self, queries, k: int = 10, **opts) -> list[list[dict]]:
        """queryBatch (src/index.ts:473-517), with one more branch than the
        reference's.  A flat fp32 index answers with its own batch (the
        reference's `'queryBatch' in this.index` branch); a quantized or IVF
        index whose seam offers search() answers the whole batch in one
        device call with query()'s kEff / fetch / re-rank rules
        (src/index.ts:402-421) and a one-batch nprobe override, so each
        query's results equal query()'s; filtered batches, and fetches
        beyond the fused top-k, loop query() as the reference's fallback
        does."""
        if len(queries) == 0:
            return []
        rerank = opts.get("rerank")
        nprobe = opts.get("nprobe")
        flat = type(self.index) is FlatIndex
        quant = self.quant_bits > 0 and hasattr(self.index, "search")
        total = self.index.size
        deleted = self.store.deleted_count
        k_eff = min(total, k + deleted)
        do_rerank = rerank if rerank is not None else self.rerank_factor > 1
        fetch = min(total, max(k_eff, k_eff * self.rerank_factor)) if do_rerank else k_eff
        if opts.get("filter") is not None or not (flat or quant) or (quant and (fetch > 1024 or k_eff == 0)):
            return [self.query(q, k=k, **opts) for q in queries]
        packed = np.stack([self._prep_query(q) for q in queries])
        if nprobe is not None and hasattr(self.index, "set_nprobe"):
            self.index.set_nprobe(nprobe)  # consumed by the one batch call, as each query() consumes its own
        t0 = time.perf_counter()
        if flat:
            batch = self.index.query_batch(packed, len(queries), k_eff)
        else:
            rows, scores, cnt = self.index.search(packed, fetch if do_rerank else 0, k_eff)
            batch = [[FlatHit(int(rows[i, j]), float(scores[i, j])) for j in range(cnt[i])]
                     for i in range(len(queries))]
        self.last_query_ms = (time.perf_counter() - t0) * 1e3
        self.last_query_gpu_ms = self.index.stats()["last_query_gpu_ms"]
        out = []
        for hits in batch:
            res = []
            for h in hits:
                if deleted and self.store.is_deleted(h.row):
                    continue
                e = self.store.by_row[h.row]
                r = {"id": e.id, "score": h.score}
                if e.metadata is not None:
                    r["metadata"] = e.metadata
                res.append(r)
                if len(res) == k:
                    break
            out.append(res)
        return out

    # ----------------------------------------------------------- mutation
    def delete(self, id: str) -> bool:
        return self.store.delete(id)

    def update(self, record: dict) -> bool:
        existed = self.store.delete(record["id"])
        self.add(record)
        return existed

    def compact(self) -> int:
        """compact (src/index.ts:544-565): rebuild store and index dense."""
        removed = self.store.deleted_count
        if removed == 0:
            return 0
        entries = self.store.live_entries()
        vectors = self.store.live_vectors()
        self.store.clear()
        self.store.insert_block([e.id for e in entries], vectors, [e.metadata for e in entries])
        self.index.destroy()
        self.index = self.make_index()
        if entries:
            self.index.append(vectors, len(entries))
        return removed

    def get(self, id: str):
        e = self.store.by_id.get(id)
        if e is None:
            return None
        r = {"id": id, "vector": self.store.raw[e.row].copy()}
        if e.metadata is not None:
            r["metadata"] = e.metadata
        return r

    def stats(self) -> dict:
        """stats (src/index.ts:702-750)."""
        out = {"count": self.store.count, "dimension": self.store.dimension, "metric": self.store.metric,
               "device": "hip", "quantBits": self.quant_bits}
        if self.store.deleted_count:
            out["deleted"] = self.store.deleted_count
        if self.last_query_ms is not None:
            out["lastQueryMs"] = self.last_query_ms
            gpu = min(self.last_query_gpu_ms or 0.0, self.last_query_ms)
            out["lastQueryGpuMs"] = gpu
            out["lastQueryCpuMs"] = self.last_query_ms - gpu
        st = self.index.stats()
        if st["nlist"]:
            out["nlist"] = st["nlist"]
        if st["nprobe"]:
            out["nprobe"] = st["nprobe"]
        if st["tuned_recall"] >= 0:
            out["tunedRecall"] = st["tuned_recall"]
        if isinstance(self.index, QuantIndex):
            out["ingest"] = self.index.ingest_mode
        if st["chunk_count"] > 1:
            out["chunks"] = st["chunk_count"]
        return out

    def destroy(self) -> None:
        self.index.destroy()
        self.ctx.destroy()

