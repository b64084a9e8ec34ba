"""Benchmark of BrowserVec's search path on one MI355X.

Headline workload (`value`): 1,000,000 x 768 fp32 rows from a mixture of
1024 Gaussian clusters (unit-norm centres, sigma 0.1), L2-normalized;
rotated with the seeded randomized Hadamard transform to P=1024 and
int8-quantized on the device; 256 queries = corpus rows + N(0, 0.05^2)
noise, normalized.  One step = one query (batch 1): rotate, scan 1M codes
with fused top-100, exact f64 re-rank to top-10.  Inputs are resident in HBM
before timing starts.

Prints one JSON line.  `value` is batch-1 queries/s over the timed steps:
one query per call, two calls in flight on two streams (each call's final
selection overlaps the next one's scan); the one-stream figure and the
synchronous latency are carried beside it.
The line also carries, for the same workload, batch-256 throughput, recall@10
against the exact fp32 flat scan, the scan kernel's roofline position (HIP
events on the index's stream) and the CPU baseline (the kernel.wat
lane-order fp32 flat scan plus topK on one core, timed on this host); and
under "configs" the other workloads of the benchmark list, each with its own
throughput, roofline, recall and CPU baseline:
  c1  20,000 x 384 fp32 cosine, 100 queries: GPU top-10 ids vs the CPU scan
  c2  1,000,000 x 768 fp32 flat dot / cosine / l2, batch 1 and 256
  c4  4,000,000 x 1024 int4 and 1-bit (asym, Hamming), fetch 200 -> 10
  c5  4,000,000 x 768 IVF int8, 4096 lists, 20 iterations, nprobe 32,
      1024 queries, fetch 40 -> 10
  graph  HNSW layer-0 beam search, 200,000 x 768, degree 32, ef 64, 1024
      queries
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
INT8_PEAK_POPS = 5.0
METRIC = "queries/s at 1Mx768 int8 k=10 (batch 1 & 256); % HBM peak; recall@10"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def make_data(n, dim, nclusters, sigma, nq, qsigma, seed, with_source=False):
    """Gaussian mixture (unit-norm centres + sigma N(0,1), rows normalized)
    and noisy corpus rows as queries, generated on the device (with_source:
    also each query's source row)."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    centres = torch.randn(nclusters, dim, generator=g, device="cuda")
    centres /= centres.norm(dim=1, keepdim=True)
    x = torch.empty(n, dim, device="cuda")
    step = 1 << 18
    for s in range(0, n, step):
        e = min(n, s + step)
        lab = torch.randint(0, nclusters, (e - s,), generator=g, device="cuda")
        blk = centres[lab] + sigma * torch.randn(e - s, dim, generator=g, device="cuda")
        x[s:e] = blk / blk.norm(dim=1, keepdim=True)
    pick = torch.randint(0, n, (nq,), generator=g, device="cuda")
    q = x[pick] + qsigma * torch.randn(nq, dim, generator=g, device="cuda")
    q /= q.norm(dim=1, keepdim=True)
    torch.cuda.synchronize()
    if with_source:
        return x.contiguous(), q.contiguous(), pick.cpu().numpy()
    return x.contiguous(), q.contiguous()


def recall_at_1_source(rows_got, source):
    """The share of queries whose first result is the corpus row the query
    was drawn from (a control that needs no ground-truth scan)."""
    return float(np.mean(rows_got[:, 0].astype(np.int64) == source.astype(np.int64)))


def timed_search(idx, d_q, nq_total, batch, steps, warmup, fetch, k, torch, outs=1):
    """Runs `steps` timed search calls of `batch` queries each (cycling through
    the query set) after `warmup` untimed ones; returns seconds.  `outs`
    output sets are used in turn (two calls in flight need two)."""
    rows = torch.empty(outs, batch, k, dtype=torch.int32, device="cuda")
    scores = torch.empty(outs, batch, k, dtype=torch.float32, device="cuda")
    cnt = torch.empty(outs, batch, dtype=torch.int32, device="cuda")

    def one(i):
        s = (i * batch) % max(nq_total - batch + 1, 1)
        o = i % outs
        idx.search_device(d_q[s].data_ptr() if batch == 1 else d_q[s:s + batch].data_ptr(), batch, fetch, k,
                          rows[o].data_ptr(), scores[o].data_ptr(), cnt[o].data_ptr())

    for i in range(warmup):
        one(i)
    idx.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        one(i)
    idx.sync()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def qps(idx, q, nq_total, batch, steps, warmup, fetch, k, torch):
    return steps * batch / timed_search(idx, q, nq_total, batch, steps, warmup, fetch, k, torch)


def kernel_timed_b1(idx, q, nq_total, steps, fetch, k, torch):
    """Batch-1 q/s of `steps` timed steps and the scan kernel's mean duration
    (HIP events on the index's stream around each launch of a second pass
    of `steps` steps)."""
    timed_search(idx, q, nq_total, 1, max(steps // 10, 5), 0, fetch, k, torch)  # warmup, untimed
    el = timed_search(idx, q, nq_total, 1, steps, 0, fetch, k, torch)
    idx.kernel_timing(True)  # a second pass with events: they add a few us per step
    timed_search(idx, q, nq_total, 1, steps, 0, fetch, k, torch)
    ms, launches = idx.kernel_timing(False)
    return steps / el, ms / max(launches, 1) * 1e3


def cpu_baseline(x_host, q_host, metric="cosine", budget_s=12.0, min_q=3):
    """kernel.wat-order fp32 flat scan + topK (reference semantics) on one
    core, over as many queries as fit the time budget (at least min_q)."""
    from oracle import oracle as o

    cpus = None
    try:
        cpus = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {min(cpus)})
    except Exception:
        pass
    done = 0
    t0 = time.perf_counter()
    try:
        while done < q_host.shape[0]:
            s = o.wasm_scan(x_host, q_host[done], metric)
            o.topk_ref(s, 10)
            done += 1
            if done >= min_q and time.perf_counter() - t0 > budget_s:
                break
    finally:
        if cpus:
            os.sched_setaffinity(0, cpus)
    el = time.perf_counter() - t0
    return done / el, done, el


def cpu_entry(x_host, q_host, metric, budget_s, what):
    cqps, cn, cel = cpu_baseline(x_host, q_host, metric, budget_s)
    n, dim = x_host.shape
    return {"value": round(cqps, 3), "unit": "queries/s", "cores": 1, "kind": "port",
            "sample": f"{cn} queries x {n:,} x {dim} fp32 {metric} flat scan in kernel.wat lane order + topK "
                      f"k=10 ({what}), {cel:.1f} s on one core of {platform.processor() or 'host'} "
                      f"({os.cpu_count()} logical CPUs visible)"}


def hbm_roof(bytes_per_launch, kernel_us):
    a = bytes_per_launch / (kernel_us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(a, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(a / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": int(bytes_per_launch),
            "kernel_avg_us": round(kernel_us, 2)}


def recall_vs_flat(ctx, x, q, rows_got, k, torch):
    """recall@k of rows_got against the exact fp32 flat scan (whose batches
    equal single queries)."""
    from browservec_amd import FlatIndex

    flat = FlatIndex(ctx, x.shape[1], "cosine")
    flat.append_device(x.data_ptr(), x.shape[0])
    nq = q.shape[0]
    d_rows = torch.empty(nq, k, dtype=torch.int32, device="cuda")
    d_sc = torch.empty(nq, k, dtype=torch.float32, device="cuda")
    d_n = torch.empty(nq, dtype=torch.int32, device="cuda")
    for s0 in range(0, nq, 256):
        m = min(256, nq - s0)
        flat.search_device(q[s0:s0 + m].data_ptr(), m, 0, k, d_rows[s0:].data_ptr(), d_sc[s0:].data_ptr(),
                           d_n[s0:].data_ptr())
    flat.sync()
    truth = d_rows.cpu().numpy()
    flat.destroy()
    return float(np.mean([len(set(rows_got[i].tolist()) & set(truth[i].tolist())) / k for i in range(nq)]))


def device_rows(idx, q, fetch, k, torch, chunk=256):
    nq = q.shape[0]
    d_rows = torch.empty(nq, k, dtype=torch.int32, device="cuda")
    d_sc = torch.empty(nq, k, dtype=torch.float32, device="cuda")
    d_n = torch.empty(nq, dtype=torch.int32, device="cuda")
    for s0 in range(0, nq, chunk):
        m = min(chunk, nq - s0)
        idx.search_device(q[s0:s0 + m].data_ptr(), m, fetch, k, d_rows[s0:].data_ptr(), d_sc[s0:].data_ptr(),
                          d_n[s0:].data_ptr())
    idx.sync()
    return d_rows.cpu().numpy()


def free(torch):
    import gc

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


# ------------------------------------------------------------------ configs --
def bench_c1(ctx, torch):
    """20,000 x 384 fp32 cosine, 100 queries: the GPU's top-10 ids against the
    CPU baseline's (the kernel.wat lane-order scan + topK), all queries."""
    from browservec_amd import FlatIndex
    from oracle import oracle as o

    n, dim, nq = 20_000, 384, 100
    rng = np.random.default_rng(0xC1)
    x = rng.standard_normal((n, dim)).astype(np.float32)
    o.normalize_rows_store(x)
    q = rng.standard_normal((nq, dim)).astype(np.float32)
    o.normalize_rows_store(q)
    idx = FlatIndex(ctx, dim, "cosine")
    idx.append(x, n)
    dq = torch.from_numpy(q).cuda()
    b1 = qps(idx, dq, nq, 1, 200, 20, 0, 10, torch)
    gpu = idx.query_batch(q, nq, 10)
    t0 = time.perf_counter()
    same = near = 0
    for i in range(nq):
        s = o.wasm_scan(x, q[i])
        cpu_rows, _ = o.topk_ref(s, 10)
        g = [h.row for h in gpu[i]]
        if set(g) == set(cpu_rows.tolist()):
            same += 1
        else:  # a near-tie at the cut: the differing rows score within 1e-5 of the 10th
            kth = float(np.sort(s)[-10])
            if all(abs(float(s[r]) - kth) <= 1e-5 for r in set(g) ^ set(cpu_rows.tolist())):
                near += 1
    cpu_s = time.perf_counter() - t0
    idx.destroy()
    return {"workload": "20000x384 fp32 cosine flat, 100 queries, k=10",
            "batch1_qps": round(b1, 1), "queries": nq, "top10_ids_equal_cpu": same,
            "top10_ids_differ_only_at_near_ties": near,
            "cpu_baseline": {"value": round(nq / cpu_s, 1), "unit": "queries/s", "cores": 1, "kind": "port",
                             "sample": f"all {nq} queries, kernel.wat lane order + topK, {cpu_s:.2f} s"}}


def bench_c2(ctx, torch, budget_s):
    """1,000,000 x 768 fp32 flat scan, dot / cosine / l2, batch 1 and 256."""
    from browservec_amd import FlatIndex

    n, dim, nq, k = 1_000_000, 768, 256, 10
    g = torch.Generator(device="cuda").manual_seed(0xB5EC0002)
    x = torch.randn(n, dim, generator=g, device="cuda")
    q = torch.randn(nq, dim, generator=g, device="cuda")
    res = {}
    cpu = {}
    xh = None
    for metric in ("dot", "cosine", "l2"):
        if metric == "cosine":
            xm, qm = (x / x.norm(dim=1, keepdim=True)).contiguous(), (q / q.norm(dim=1, keepdim=True)).contiguous()
        else:
            xm, qm = x, q
        idx = FlatIndex(ctx, dim, metric)
        idx.append_device(xm.data_ptr(), n)
        b1, kus = kernel_timed_b1(idx, qm, nq, 200, 0, k, torch)
        t256 = timed_search(idx, qm, nq, nq, 4, 1, 0, k, torch) / 4
        flops = 2.0 * n * dim * nq
        a = flops / t256 / 1e12
        res[metric] = {"batch1_qps": round(b1, 1), "batch256_qps": round(nq / t256, 1),
                       "roofline_b1": hbm_roof(n * dim * 4, kus),
                       "roofline_b256": {"bound": "mfma", "achieved": round(a, 2), "peak": FP32_PEAK_TFLOPS,
                                         "unit": "TFLOP/s", "frac": round(a / FP32_PEAK_TFLOPS, 4),
                                         "algorithmic_flops_per_batch": flops,
                                         "note": "whole batch pipeline: matrix-core prefilter + exact re-score"}}
        idx.destroy()
        if budget_s > 0:
            xh = xm.cpu().numpy()
            cpu[metric] = cpu_entry(xh, qm.cpu().numpy(), metric, budget_s, "batch 256 = 256 serial queries")
            del xh
        if metric == "cosine":
            del xm, qm
        free(torch)
    del x, q
    free(torch)
    return {"workload": "1000000x768 fp32 N(0,1) flat scan (cosine: L2-normalized), 256 queries, k=10",
            "metrics": res, "recall_at_10": 1.0,
            "recall_note": "exact scan; batch rows and score bits equal single queries (tests)",
            "cpu_baseline": cpu or None}


def bench_c4(ctx, torch, budget_s):
    """4,000,000 x 1024 int4 and 1-bit (asym and Hamming), fetch 200 -> 10."""
    from browservec_amd import QuantIndex

    n, dim, nq, fetch, k = 4_000_000, 1024, 256, 200, 10
    x, q, src_rows = make_data(n, dim, 1024, 0.1, nq, 0.05, 0xB5EC0004, with_source=True)
    res = {}
    for name, bits, scorer in (("int4", 4, "asym"), ("1bit_asym", 1, "asym"), ("1bit_hamming", 1, "hamming")):
        idx = QuantIndex(ctx, dim, bits=bits, scorer=scorer)
        t0 = time.perf_counter()
        idx.append_device(x.data_ptr(), n)
        idx.sync()
        enc_s = time.perf_counter() - t0
        b1, kus = kernel_timed_b1(idx, q, nq, 300, fetch, k, torch)
        b256 = qps(idx, q, nq, nq, 3, 1, fetch, k, torch)
        rows_q = device_rows(idx, q, fetch, k, torch)
        # control: the same codes with the widest fetch the device serves; if
        # recall rises with the fetch, the loss at fetch 200 is the codec's
        # ranking, not the scan's
        rows_wide = device_rows(idx, q, 1024, k, torch) if bits == 1 else None
        rb = dim * bits // 8
        res[name] = {"batch1_qps": round(b1, 1), "batch256_qps": round(b256, 1),
                     "roofline_b1": hbm_roof(n * (rb + 4) + fetch * dim * 4, kus),
                     "encode_s": round(enc_s, 3), "rows_q": rows_q, "rows_wide": rows_wide,
                     "recall_at_1_source_row": round(recall_at_1_source(rows_q, src_rows), 4)}
        idx.destroy()
        free(torch)
    for key in res:
        res[key]["recall_at_10"] = round(recall_vs_flat(ctx, x, q, res[key].pop("rows_q"), k, torch), 4)
        wide = res[key].pop("rows_wide")
        if wide is not None:
            res[key]["recall_at_10_fetch_1024"] = round(recall_vs_flat(ctx, x, q, wide, k, torch), 4)
    cpu = None
    if budget_s > 0:
        cpu = cpu_entry(x.cpu().numpy(), q[:16].cpu().numpy(), "cosine", budget_s,
                        "the reference has no CPU quantized path")
    del x, q
    free(torch)
    return {"workload": "4000000x1024 from a 1024-cluster mixture (sigma 0.1); int4 (512 B/row) and 1-bit "
                        "(128 B/row) codes; fetch 200 -> exact f64 re-rank -> top-10; 256 noisy-row queries",
            "codecs": res, "cpu_baseline": cpu}


def bench_c5(ctx, torch, budget_s):
    """IVF int8, 4,000,000 x 768, 4096 lists, 20 iterations, nprobe 32, fetch 40 -> 10."""
    from browservec_amd import IVFQuantIndex

    n, dim, nq, fetch, k, nprobe = 4_000_000, 768, 1024, 40, 10, 32
    x, q, src_rows = make_data(n, dim, 4096, 0.15, nq, 0.05, 0xB5EC0005, with_source=True)
    idx = IVFQuantIndex(ctx, dim, bits=8, ivf={"nlist": 4096, "iters": 20, "nprobe": nprobe})
    t0 = time.perf_counter()
    idx.append_device(x.data_ptr(), n)
    idx.sync()
    enc_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    idx.build()
    build_s = time.perf_counter() - t0
    st = idx.stats()
    b1, kus = kernel_timed_b1(idx, q, nq, 500, fetch, k, torch)
    # single queries with two and three calls in flight (bv_index_set_query_streams)
    b1_multi = {}
    for ns in (2, 3):
        idx.set_query_streams(ns)
        timed_search(idx, q, nq, 1, 50, 0, fetch, k, torch, outs=ns)
        b1_multi[ns] = 1000 / timed_search(idx, q, nq, 1, 1000, 0, fetch, k, torch, outs=ns)
    idx.set_query_streams(1)
    bq = qps(idx, q, nq, nq, 3, 1, fetch, k, torch)
    # rows each query scans: the sizes of its 32 probed lists (pickProbes'
    # scores from the device, list offsets from the build), averaged
    _, off, _ = idx.export_ivf()
    sizes = np.diff(off.astype(np.int64))
    ps = idx.export_probe_scores(q.cpu().numpy())
    top = np.argpartition(-ps, nprobe - 1, axis=1)[:, :nprobe]
    scanned = float(sizes[top].sum(axis=1).mean())
    rows_q = device_rows(idx, q, fetch, k, torch, chunk=nq)
    recall = recall_vs_flat(ctx, x, q, rows_q, k, torch)
    # the same queries probing every list: the IVF scan then equals the
    # exhaustive quantized scan, so this recall isolates the loss of the lists
    qh = q[:64].cpu().numpy()
    rows_all = []
    for s0 in range(0, 64, 16):
        idx.set_nprobe(st["nlist"])
        r, _, _ = idx.search(qh[s0:s0 + 16], fetch, k)
        rows_all.append(r)
    recall_all = recall_vs_flat(ctx, x, q[:64].contiguous(), np.concatenate(rows_all), k, torch)
    idx.destroy()
    # control: the same lists trained on every row (sampleSize = trainSize =
    # N, the reservoir holding all rows): if recall stays low, the loss is the
    # workload's (noise norm ~4 per row against unit centres), not the
    # 16,384-row training sample's
    full = IVFQuantIndex(ctx, dim, bits=8, ivf={"nlist": 4096, "iters": 20, "nprobe": nprobe, "sampleSize": n,
                                                "trainSize": n})
    full.append_device(x.data_ptr(), n)
    full.sync()
    t0 = time.perf_counter()
    full.build()
    build_full_s = time.perf_counter() - t0
    rows_full = device_rows(full, q, fetch, k, torch, chunk=nq)
    recall_full = recall_vs_flat(ctx, x, q, rows_full, k, torch)
    full.destroy()
    free(torch)
    cpu = None
    if budget_s > 0:
        cpu = cpu_entry(x.cpu().numpy(), q[:16].cpu().numpy(), "cosine", budget_s,
                        "the reference has no CPU IVF path")
    del x, q
    free(torch)
    list_bytes = scanned * (1024 + 4 + 4)  # codes, scale and the candidate row id
    return {"workload": "4000000x768 from a 4096-cluster mixture (sigma 0.15), IVF int8: 4096 lists, 20 Lloyd "
                        "iterations on the 16384-row sample, nprobe 32, fetch 40 -> exact re-rank -> top-10, "
                        "1024 noisy-row queries",
            "batch1_qps": round(b1, 1), "batch1_two_stream_qps": round(b1_multi[2], 1),
            "batch1_three_stream_qps": round(b1_multi[3], 1), "batch1024_qps": round(bq, 1),
            "roofline_b1_list_scan": dict(hbm_roof(list_bytes + fetch * dim * 4, kus),
                                          avg_scanned_rows=round(scanned, 1)),
            "recall_at_10": round(recall, 4), "recall_at_10_all_lists_64q": round(recall_all, 4),
            "recall_at_1_source_row": round(recall_at_1_source(rows_q, src_rows), 4),
            "control_train_on_all_rows": {"sampleSize": n, "trainSize": n, "build_s": round(build_full_s, 3),
                                          "recall_at_10": round(recall_full, 4),
                                          "recall_at_1_source_row": round(recall_at_1_source(rows_full, src_rows),
                                                                          4)},
            "build_s": round(build_s, 3), "build_ms_device": round(st["build_ms"], 1),
            "build_final_assign_exact_rows": int(st["build_exact_rows"]), "encode_s": round(enc_s, 3),
            "nlist": st["nlist"], "nprobe": nprobe, "cpu_baseline": cpu}


def bench_graph(ctx, torch, budget_s):
    """HNSW layer-0 beam search (HNSWGpuSearcher, src/index/hnswGpu.ts; the
    shader of src/engine/wgsl/graphSearch.ts): 200,000 x 768 cosine rows, a
    degree-32 adjacency (each row's 16 nearest others by the exact flat scan
    and 16 random rows), 1024 queries, ef 128, k 10."""
    from browservec_amd import FlatIndex, GraphSearcher

    n, dim, K, nq, ef, k = 200_000, 768, 32, 1024, 128, 10
    near = 16  # nearest neighbours per row; the other slots are random long links
    # tight clusters (per-coordinate sigma 0.02: noise norm 0.55 against unit
    # centres), queries = rows + 0.01 noise: neighbourhoods a graph walk can
    # follow, unlike the near-isotropic mixtures of the scan workloads
    x, q = make_data(n, dim, 1024, 0.02, nq, 0.01, 0xB5EC0006)
    t0 = time.perf_counter()
    flat = FlatIndex(ctx, dim, "cosine")
    flat.append_device(x.data_ptr(), n)
    nb = torch.empty(n, K + 1, dtype=torch.int32, device="cuda")
    sc = torch.empty(n, K + 1, dtype=torch.float32, device="cuda")
    cn = torch.empty(n, dtype=torch.int32, device="cuda")
    for s0 in range(0, n, 1024):
        m = min(1024, n - s0)
        flat.search_device(x[s0:s0 + m].data_ptr(), m, 0, K + 1, nb[s0:].data_ptr(), sc[s0:].data_ptr(),
                           cn[s0:].data_ptr())
    flat.sync()
    nbh = nb.cpu().numpy().astype(np.int64)
    self_col = nbh == np.arange(n)[:, None]
    keep = ~self_col
    keep[self_col.sum(axis=1) == 0, K] = False  # no self hit: drop the last
    links = nbh[keep].reshape(n, K).astype(np.uint32)
    # a navigable small world: the nearest rows plus random long-range links
    # (a pure kNN graph of a clustered corpus splits into per-cluster islands)
    rng = np.random.default_rng(6)
    links[:, near:] = rng.integers(0, n, size=(n, K - near), dtype=np.uint32)
    adj_s = time.perf_counter() - t0
    xh = x.cpu().numpy()
    gs = GraphSearcher(ctx, dim, "cosine", K)
    gs.append(xh, n)
    gs.upload_graph(links, n)
    qh = q.cpu().numpy()
    gs.search_arrays(qh, nq, k, ef, 0)  # warmup
    reps = 5
    t0 = time.perf_counter()
    for _ in range(reps):
        rows_g, _, cnt_g = gs.search_arrays(qh, nq, k, ef, 0)
    bq = reps * nq / (time.perf_counter() - t0)
    lat = []
    for i in range(32):
        t0 = time.perf_counter()
        gs.search_arrays(qh[i:i + 1], 1, k, ef, 0)
        lat.append((time.perf_counter() - t0) * 1e3)
    rows_g = np.where(np.arange(k)[None, :] < cnt_g[:, None], rows_g.astype(np.int64), -1)
    recall = recall_vs_flat(ctx, x, q, rows_g, k, torch)
    flat.destroy()
    gs.destroy()
    cpu = None
    if budget_s > 0:
        from oracle import oracle as o

        e = o.graph_entries(0, n)
        t0 = time.perf_counter()
        done = 0
        while done < nq and (done < 4 or time.perf_counter() - t0 < budget_s):
            o.graph_search(xh, links, qh[done:done + 4], e, ef, ef)
            done += 4
        el = time.perf_counter() - t0
        cpu = {"value": round(done / el, 2), "unit": "queries/s", "cores": 1, "kind": "port",
               "sample": f"{done} queries through the oracle's single-thread restatement of the beam search "
                         f"(same graph, ef {ef}), {el:.1f} s"}
    del x, q, xh
    free(torch)
    return {"workload": f"{n}x{dim} cosine rows (1024 clusters, sigma 0.02), degree-{K} layer-0 adjacency ({near} exact nearest + "
                        f"{K - near} random links), "
                        f"{nq} queries, ef {ef}, k {k}, one wave per query",
            "batch1024_qps": round(bq, 1), "batch1_ms_p50": round(float(np.median(lat)), 3),
            "recall_at_10": round(recall, 4), "adjacency_build_s": round(adj_s, 2), "cpu_baseline": cpu}


def stream_ceiling(torch, nbytes=1 << 30, reps=20):
    """Read-only streaming kernel (libbv_bench.so) over nbytes: plain and
    nontemporal 16-byte loads, grid-stride or contiguous chunks per
    workgroup, GB/s from CUDA events on torch's stream.  Returns the best
    figure and the sweep."""
    lib = ctypes.CDLL(os.path.join(ROOT, "browservec_amd", "lib", "libbv_bench.so"))
    lib.bvb_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p,
                                    ctypes.c_uint32, ctypes.c_void_p]
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    sink = torch.empty(4096 * 256, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    sweep = {}
    for nt in (0, 1):
        for chunk, blocks in ((0, 2048), (16 << 10, 512), (64 << 10, 512), (64 << 10, 1024), (256 << 10, 512),
                              (64 << 10, 256)):
            lib.bvb_stream_read(buf.data_ptr(), nbytes, nt, chunk, sink.data_ptr(), blocks, stream)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                lib.bvb_stream_read(buf.data_ptr(), nbytes, nt, chunk, sink.data_ptr(), blocks, stream)
            e1.record()
            torch.cuda.synchronize()
            name = f"{'nontemporal' if nt else 'plain'} {'grid-stride' if not chunk else f'{chunk >> 10} KiB chunks'} x {blocks} wg"
            sweep[name] = round(nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    del buf, sink
    best = max(sweep, key=sweep.get)
    return {"best_gbs": sweep[best], "best": best, "sweep": sweep}


def copy_bandwidth(torch, nbytes=1 << 30, reps=10):
    """Device-to-device copy of nbytes (read + write), timed with CUDA events:
    the streaming ceiling of the card the run is on, in GB/s."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2 * nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    return gbs


# ------------------------------------------------------------------- main --
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--rows", type=int, default=1_000_000)
    ap.add_argument("--dim", type=int, default=768)
    ap.add_argument("--queries", type=int, default=256)
    ap.add_argument("--fetch", type=int, default=100)
    ap.add_argument("--k", type=int, default=10)
    ap.add_argument("--bits", type=int, default=8)
    ap.add_argument("--batch-steps", type=int, default=8, help="timed batch-256 steps")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--configs", default="c1,c2,c4,c5,graph",
                    help="extra workloads carried under 'configs' (comma list of c1,c2,c4,c5,graph; '' for none)")
    ap.add_argument("--profile-only", action="store_true", help="build + a short timed loop (for rocprofv3)")
    ap.add_argument("--profile-batch", action="store_true",
                    help="build + timed batch-256 searches on the matrix-core path (for rocprofv3)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 10 device copies of 1 GiB (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--stream-ceiling", action="store_true", help="only time the read-only streaming kernel")
    ap.add_argument("--config", default=None, choices=["c1", "c2", "c4", "c5", "graph"],
                    help="run one extra workload alone and print its object (for rocprofv3)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU; the search path shards by rows across GPUs "
                                   "with one top-k exchange (see DESIGN.md), which is not run here",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    if args.copy_calibration:
        src = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": src.numel() * 4, "launches": 10}))
        return
    if args.stream_ceiling:
        print(json.dumps({"stream_read_gbs": stream_ceiling(torch), "bytes_per_launch": 1 << 30}))
        return

    from browservec_amd import DeviceContext, FlatIndex, QuantIndex

    ctx = DeviceContext(0)
    info = ctx.info()
    budget = 0.0 if args.no_cpu_baseline else 6.0
    if args.config:
        fn = {"c1": lambda: bench_c1(ctx, torch), "c2": lambda: bench_c2(ctx, torch, budget),
              "c4": lambda: bench_c4(ctx, torch, budget), "c5": lambda: bench_c5(ctx, torch, budget),
              "graph": lambda: bench_graph(ctx, torch, budget)}[args.config]
        print(json.dumps({args.config: fn(), "device": info["name"]}))
        ctx.destroy()
        return

    seed = 0xB5EC0001
    log("generating data", args.rows, args.dim)
    x, q, src_rows = make_data(args.rows, args.dim, 1024, 0.1, args.queries, 0.05, seed, with_source=True)

    log("building int8 index")
    t0 = time.perf_counter()
    idx = QuantIndex(ctx, args.dim, bits=args.bits)
    idx.append_device(x.data_ptr(), args.rows)
    build_s = time.perf_counter() - t0
    P = idx.padded_dim
    row_bytes = P * args.bits // 8

    if args.profile_batch:
        nb = min(256, args.queries)
        el = timed_search(idx, q, args.queries, nb, args.batch_steps, 2, args.fetch, args.k, torch)
        print(json.dumps({"qps_b256": args.batch_steps * nb / el, "batch_ms_avg": el / args.batch_steps * 1e3,
                          "batches": args.batch_steps}))
        return

    # ---- batch 1 ------------------------------------------------------------
    log("timing batch 1")
    timed_search(idx, q, args.queries, 1, args.warmup, 0, args.fetch, args.k, torch)  # W untimed warmup steps
    el = timed_search(idx, q, args.queries, 1, args.steps, 0, args.fetch, args.k, torch)
    qps_b1_serial = args.steps / el
    # the kernel's duration: a second pass of K steps with HIP events around
    # each launch (the events add a few us per step, so no q/s is taken here)
    idx.kernel_timing(True)
    timed_search(idx, q, args.queries, 1, args.steps, 0, args.fetch, args.k, torch)
    scan_ms, launches = idx.kernel_timing(False)
    # two single-query calls in flight on two streams: each query is still
    # one call, but its final selection overlaps the next query's scan
    log("timing batch 1, two streams")
    idx.set_query_streams(2)
    timed_search(idx, q, args.queries, 1, args.warmup, 0, args.fetch, args.k, torch, outs=2)
    el2 = timed_search(idx, q, args.queries, 1, args.steps, 0, args.fetch, args.k, torch, outs=2)
    idx.set_query_streams(1)
    qps_b1 = args.steps / el2
    if args.profile_only:
        print(json.dumps({"qps_b1": qps_b1, "qps_b1_serial": qps_b1_serial, "scan_ms_avg": scan_ms / max(launches, 1)}))
        return
    scan_avg_ms = scan_ms / max(launches, 1)
    # algorithmic bytes of the one launch per query: codes + scales + the
    # fp32 rows of the re-ranked fetch
    scan_bytes = args.rows * (row_bytes + 4) + args.fetch * args.dim * 4
    achieved = scan_bytes / (scan_avg_ms * 1e-3) / 1e9
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "scan_topk_q8_1Mx768_traffic.json")
    if (args.rows, args.dim, args.bits, args.fetch) == (1_000_000, 768, 8, 100) and os.path.exists(tfile):
        with open(tfile) as f:
            traffic = json.load(f).get("traffic_bytes")

    # ---- batch 256 ------------------------------------------------------------
    nb = min(256, args.queries)
    log("timing batch", nb)
    el256 = timed_search(idx, q, args.queries, nb, args.batch_steps, 1, args.fetch, args.k, torch)
    qps_b256 = args.batch_steps * nb / el256

    # ---- synchronous latency (host API round trip per query) ------------------
    qh = q.cpu().numpy()
    lat = []
    for i in range(64):
        t = time.perf_counter()
        idx.search(qh[i % args.queries][None], args.fetch, args.k)
        lat.append((time.perf_counter() - t) * 1e3)
    lat_p50 = float(np.median(lat))

    # ---- recall@10 vs exact fp32 ------------------------------------------------
    log("exact fp32 ground truth")
    rows_q, _, _ = idx.search(qh, args.fetch, args.k)
    flat = FlatIndex(ctx, args.dim, "cosine")
    flat.append_device(x.data_ptr(), args.rows)
    d_rows = torch.empty(args.queries, args.k, dtype=torch.int32, device="cuda")
    d_sc = torch.empty(args.queries, args.k, dtype=torch.float32, device="cuda")
    d_n = torch.empty(args.queries, dtype=torch.int32, device="cuda")
    t = time.perf_counter()
    flat.search_device(q.data_ptr(), args.queries, 0, args.k, d_rows.data_ptr(), d_sc.data_ptr(), d_n.data_ptr())
    flat.sync()
    flat_qps = args.queries / (time.perf_counter() - t)
    truth = d_rows.cpu().numpy()
    recall = float(np.mean([len(set(rows_q[i].tolist()) & set(truth[i].tolist())) / args.k
                            for i in range(args.queries)]))
    flat.destroy()
    idx.destroy()

    # ---- host append: 262,144 rows from pageable host memory (staged through
    # pinned buffers, encode overlapped) and from a pinned source -----------------
    log("host append")
    nh = min(262_144, args.rows)
    xh_part = x[:nh].cpu().numpy()
    xh_pin = x[:nh].cpu().pin_memory()
    append_gbs = {}
    for label, src in (("pageable", xh_part), ("pinned", xh_pin.numpy())):
        best = 0.0
        for _ in range(3):
            ai = QuantIndex(ctx, args.dim, bits=args.bits)
            t = time.perf_counter()
            ai.append(src, nh)
            best = max(best, nh * args.dim * 4 / (time.perf_counter() - t) / 1e9)
            ai.destroy()
        append_gbs[label] = round(best, 1)
    del xh_part, xh_pin

    # ---- CPU baseline -------------------------------------------------------------
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        xh = x.cpu().numpy()
        cqps, cn, cel = cpu_baseline(xh, qh, "cosine", 12.0, 4)
        cpu = {"value": round(cqps, 3), "unit": "queries/s", "cores": 1, "kind": "port",
               "sample": f"{cn} queries x {args.rows:,} x {args.dim} fp32 cosine flat scan in kernel.wat lane "
                         f"order + topK k=10, {cel:.1f} s on one core of {platform.processor() or 'host'} "
                         f"({os.cpu_count()} logical CPUs visible)"}
        del xh
    del x, q
    free(torch)

    configs = {}
    for name in [c for c in args.configs.split(",") if c]:
        log("config", name)
        if name == "c1":
            configs["c1_fp32_cosine_20kx384"] = bench_c1(ctx, torch)
        elif name == "c2":
            configs["c2_fp32_flat_1Mx768"] = bench_c2(ctx, torch, budget)
        elif name == "c4":
            configs["c4_int4_1bit_4Mx1024"] = bench_c4(ctx, torch, budget)
        elif name == "c5":
            configs["c5_ivf_int8_4Mx768"] = bench_c5(ctx, torch, budget)
        elif name == "graph":
            configs["hnsw_layer0_beam_200kx768"] = bench_graph(ctx, torch, budget)
    log("streaming ceiling")
    ceiling = stream_ceiling(torch)

    algo_bytes_q = scan_bytes
    out = {
        "metric": METRIC,
        "value": round(qps_b1, 2),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(el2 / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: seeded Gaussian mixture (1024 unit-norm centres, sigma 0.1) generated on device",
        "config": {"workload": f"{args.rows}x{args.dim} int8 TurboQuant scan, fetch {args.fetch} -> exact f64 "
                               f"re-rank -> top-{args.k}, batch 1",
                   "batch1_mode": "one query per search_device call; two calls in flight on two streams "
                                  "(bv_index_set_query_streams(2)), so one query's final selection overlaps the "
                                  "next query's scan; two-stream calls run the register-lean build of the scan "
                                  "(scan_topk_lean), the roofline's kernel is the default build on one stream",
                   "rows": args.rows, "dim": args.dim, "padded_dim": P, "bits": args.bits, "fetch": args.fetch,
                   "k": args.k, "queries": args.queries, "rotation_seed": "0x9e3779b9", "data_seed": hex(seed)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "scan_topk<C_Q8,64,1> (query rotate+levels, scan, top-100, exact re-rank)",
                     "kernel_avg_us": round(scan_avg_ms * 1e3, 2),
                     "timed_over": "a second pass of the K one-stream steps with HIP events (no system-scope "
                                   "fence) around each launch on the index stream; the q/s figures come from "
                                   "passes without events, and with two streams launches overlap",
                     "algorithmic_bytes_per_launch": scan_bytes,
                     "traffic_source": "profiles/scan_topk_q8_1Mx768.md" if traffic else None},
        "cpu_baseline": cpu,
        "batch1_one_stream_qps": round(qps_b1_serial, 2),
        "batch1_one_stream_ms_per_step": round(el / args.steps * 1e3, 4),
        "batch256_qps": round(qps_b256, 1),
        # the batch's dense int8 work: one MFMA pass of every row against the
        # query's first int8 level (the other levels only for rows whose
        # bound can still reach the query's best fetch), over the whole batch
        # pipeline time (levels, sample pass, two threshold parts, joins,
        # selects, exact re-score, re-rank)
        "batch256_int8_mfma": {"pops": round(2.0 * args.rows * P * qps_b256 / 1e15, 3),
                               "peak": INT8_PEAK_POPS, "unit": "POP/s",
                               "frac": round(2.0 * args.rows * P * qps_b256 / 1e15 / INT8_PEAK_POPS, 4),
                               "dense_ops_per_batch": 2 * args.rows * nb * P,
                               "codes_read_gbs": round(args.rows * (row_bytes + 4) * qps_b256 / nb / 1e9, 1),
                               "trace_source": "profiles/mq1_scan_q8_1Mx768_b256.md"},
        "recall_at_10": round(recall, 4),
        "recall_at_1_source_row": round(recall_at_1_source(rows_q, src_rows), 4),
        "end_to_end_hbm_frac_b1": round(algo_bytes_q * qps_b1 / (HBM_PEAK_GBS * 1e9), 4),
        "end_to_end_hbm_frac_b1_one_stream": round(algo_bytes_q * qps_b1_serial / (HBM_PEAK_GBS * 1e9), 4),
        "latency_ms_sync_p50": round(lat_p50, 4),
        "fp32_flat_cosine_batch_qps": round(flat_qps, 1),
        "build_s": round(build_s, 3),
        "append_host_gbs": dict(append_gbs, rows=nh, what="QuantIndex.append of fp32 rows from host memory, "
                                                          "upload + rotate + quantize, best of 3"),
        "device": info["name"],
        "hbm_copy_gbs": round(copy_bandwidth(torch), 1),  # measured 1 GiB device copy, read + write
        "stream_read_gbs": ceiling,
        "configs": configs,
    }
    print(json.dumps(out))
    ctx.destroy()


if __name__ == "__main__":
    main()
