#!/usr/bin/env python3
"""Tree-sparse attention forward benchmark on one MI355X.

Workload (default): the Llama-3-8B verification step -- B=1, 32 query / 8 KV
heads, head_dim 128, bf16, 4096-token prefix, 64-node EAGLE tree (depth 6,
top-8), BLOCK_M=16, BLOCK_N=64.  Synthetic N(0,1) inputs (seed 42).

A step is one forward call (split-KV kernel + combine kernel) over the whole
batch with the metadata already on the device, as benchmark.py:228-237 times
the reference kernel.  The calls cycle through enough independent K/V copies
(>= 512 MiB) that every call reads its K/V from HBM rather than from the
256 MB Infinity Cache.

Timing: three regions, each K steps captured in one HIP graph (no host
launch gaps), replayed max(5, ceil(100/K)) times, each replay bracketed by a
synchronisation and HIP events on the stream the graph replays on, the median
replay reported (tsfa_fwd_set_kernel_mask selects the kernels a call
launches):
  * full calls (split-KV + combine)  -> value;
  * the combine alone                -> its duration; full - combine = the
                                        split-KV kernel's duration inside real
                                        calls (the roofline figure);
  * the split-KV kernel alone        -> reported beside it (back to back it
                                        runs faster than after a combine).

value        = K/V bytes per call * K / full-region seconds  (TB/s, whole call)
roofline     = K/V bytes / split-KV kernel duration in real calls, against
               8 TB/s HBM (algorithmic flops against 2.5 PFLOP/s dense MFMA for
               the shapes above the 312 flop/B ridge); traffic = HBM bytes per
               launch from the committed rocprofv3 PMC summary
cpu_baseline = the fp32 dense+mask oracle (benchmark.py:8-35 restated) on the
               host cores, over a bounded sample of calls
metadata     = the device metadata build (no host synchronisation), graph and
               eager, the library's host builder on a CPU mask, and the CPU
               oracle builder
eager        = the drop-in called eagerly as the reference's callers do:
               run_tree_sparse_kernel(q, k, v, tree_mask) (metadata built per
               call) and the forward with prebuilt metadata, host cost included
workloads    = the other forward workloads (16-sequence decode, 1024-token
               wide tree, 70B layout and its BLOCK_M x BLOCK_N sweep
               64x32 / 64x128 / 16x64), each timed like the headline: us per
               call, split-KV and combine, roofline fraction and bound, and
               its own cpu_baseline (the oracle over a bounded sample, query
               heads chunked to bound the fp32 score tensor; the sweep
               entries reuse their base workload's, the oracle having no
               block sizes)
cpu_baseline = also records the host CPU model, the oracle's dtype and the
               head chunking
backward     = tree_sparse_attention_bwd (dQ, dK, dV) over the same cycled
               K/V, against the MFMA and HBM peaks
paged        = the same forward reading FlashInfer's paged cache in place
               (page_size 16, scattered pages), its rate beside the
               contiguous call's
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

# this process times the split-KV kernel and the combine apart
# (tsfa_fwd_set_kernel_mask), a hook the library keeps locked otherwise
os.environ.setdefault("TSFA_BENCH_HOOKS", "1")

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "eagle3-tree-sparse-flashattn_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16 / fp16
MFMA_PEAK_TFLOPS_FP32 = 157.3  # dense fp32 MFMA
RIDGE_FLOP_PER_BYTE = MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBPS * 1e9)
METRIC = "tree-attn fwd µs + achieved HBM TB/s, 8B shape, 4k prefix, 64-node tree"


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


def _traffic(workload: str):
    """HBM bytes per split-kernel launch from the committed rocprofv3 PMC summary, if any."""
    path = os.path.join(ROOT, "profiles", "split_kernel_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(workload)
        return None if rec is None else float(rec["bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def algorithmic_flops(w, mask) -> float:
    """4*Hq*D*(B*T*P + visible tree pairs): Q K^T and P V over every visible key."""
    pairs = float(mask.to(bool).sum()) * (1 if w.per_sequence else w.batch)
    return 4.0 * w.q_heads * w.head_dim * (w.batch * w.tree_len * w.prefix_len + pairs)


def cpu_baseline(w, q, k, v, mask, seconds: float, head_chunk: int = 8):
    """The fp32 dense+mask oracle (benchmark.py:8-35 restated) on the host
    cores over a bounded sample: one warm-up call, then as many full calls as
    fit in `seconds` (at least one).  `head_chunk` query heads are processed
    at a time (the [B, chunk, T, KV] fp32 score tensor bounds memory; the
    result does not depend on it)."""
    import torch

    from oracle.attn_oracle import dense_mask_attention

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t0 = time.perf_counter()
    dense_mask_attention(q, k, v, mask, w.prefix_len, head_chunk=head_chunk)
    t1 = time.perf_counter() - t0
    n = max(1, min(1000, int(seconds / max(t1, 1e-6))))
    t0 = time.perf_counter()
    for _ in range(n):
        dense_mask_attention(q, k, v, mask, w.prefix_len, head_chunk=head_chunk)
    dt = (time.perf_counter() - t0) / n
    score_mib = w.batch * min(head_chunk, w.q_heads) * w.tree_len * w.kv_len * 4 / 2 ** 20
    return {
        "value": w.kv_bytes() / dt / 1e12,
        "unit": "TB/s",
        "us_per_call": dt * 1e6,
        "cores": cores,
        "cpu_model": _cpu_model(),
        "dtype": "fp32",
        "kind": "port",
        "head_chunk": head_chunk,
        "sample": f"{n} full calls of the fp32 dense+mask oracle on the same inputs after one warm-up call "
                  f"(torch CPU, {cores} threads; {head_chunk} query heads per chunk, "
                  f"{score_mib:.0f} MiB of fp32 scores per chunk)",
    }


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def metadata_timing(w, mask_dev, mask_cpu, reps: int = 200):
    """Device metadata build (tsfa_meta_build via prepare_tree_sparse_metadata_batched):
    graph-captured (device time) and eager (what a caller pays per call), beside
    the CPU oracle builder (numpy restatement of tree_sparse_flashattn.py:67-160)."""
    import torch

    import tree_sparse_flashattn as tsf
    from oracle import meta_oracle

    build = (lambda: tsf.prepare_tree_sparse_metadata_batched(mask_dev, w.prefix_len, w.block_m, w.block_n))
    for _ in range(5):
        build()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        build()
    b.record()
    torch.cuda.synchronize()
    eager_us = a.elapsed_time(b) * 1e3 / reps
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        build()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for _ in range(reps):
                build()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    graph_us = a.elapsed_time(b) * 1e3 / reps
    build_host = (lambda: tsf.prepare_tree_sparse_metadata_batched(mask_cpu, w.prefix_len, w.block_m, w.block_n))
    build_host()
    n_host = 0
    t0 = time.perf_counter()
    while n_host < 5 or time.perf_counter() - t0 < 0.5:
        build_host()
        n_host += 1
    host_us = (time.perf_counter() - t0) / n_host * 1e6
    masks = mask_cpu.numpy()
    build_cpu = ((lambda: [meta_oracle.build_metadata(m, w.prefix_len, w.block_m, w.block_n) for m in masks])
                 if masks.ndim == 3 else (lambda: meta_oracle.build_metadata(masks, w.prefix_len, w.block_m, w.block_n)))
    build_cpu()
    n = 0
    t0 = time.perf_counter()
    while n < 5 or time.perf_counter() - t0 < 1.0:
        build_cpu()
        n += 1
    cpu_us = (time.perf_counter() - t0) / n * 1e6
    return {"hip_graph_us_per_build": round(graph_us, 3), "hip_eager_us_per_build": round(eager_us, 3),
            "host_builder_us_per_build": round(host_us, 1), "cpu_oracle_us_per_build": round(cpu_us, 1),
            "sample": f"{reps} device builds per timing; {n_host} builds by the library's host builder "
                      f"(tsfa_meta_build_host, CPU mask); {n} CPU oracle builds (numpy, 1 thread)"}


def eager_call_timing(w, qd, ks, vs, mask_dev, meta, reps: int = 100, batches: int = 5):
    """The drop-in as the reference's callers use it, eagerly (no graph): the
    reference call form run_tree_sparse_kernel(q, k, v, tree_mask) -- metadata
    built on every call, eagle_tree_sparse_bridge.py:95-106 -- and the forward
    with metadata built once.  us_per_call: wall time per call over `reps`
    calls with one synchronisation at the end (host cost and device time
    overlap); host_us_per_call: time for the call to return (launch path).
    Each is the median of `batches` batches.  The slowest single call of each
    form is logged with its position, beside the Python garbage collector's
    pauses over the same batches (gc.callbacks): a rare stall of the host
    process moves one batch, and the log says whether it was a collection."""
    import gc

    import torch

    import eagle_tree_sparse_bridge as bridge
    import tree_sparse_flashattn as tsf

    out = torch.empty_like(qd)
    forms = {
        "reference_call_form": lambda i: bridge.run_tree_sparse_kernel(qd, ks[i % len(ks)], vs[i % len(vs)], mask_dev,
                                                                        block_m=w.block_m, block_n=w.block_n),
        "forward_with_metadata": lambda i: tsf.tree_sparse_attention_fwd(qd, ks[i % len(ks)], vs[i % len(vs)], meta,
                                                                         out=out),
    }
    gc_pauses = []
    gc_t0 = [0.0]

    def on_gc(phase, info):
        if phase == "start":
            gc_t0[0] = time.perf_counter()
        else:
            gc_pauses.append((info.get("generation", -1), (time.perf_counter() - gc_t0[0]) * 1e6))

    res = {}
    for name, fn in forms.items():
        for i in range(10):
            fn(i)
        torch.cuda.synchronize()
        walls, hosts = [], []
        slowest = (0.0, -1, -1)
        gc_pauses.clear()
        gc.callbacks.append(on_gc)
        try:
            for bi in range(batches):
                host = 0.0
                t0 = time.perf_counter()
                for i in range(reps):
                    h0 = time.perf_counter()
                    fn(i)
                    dh = time.perf_counter() - h0
                    host += dh
                    if dh > slowest[0]:
                        slowest = (dh, bi, i)
                torch.cuda.synchronize()
                walls.append((time.perf_counter() - t0) / reps * 1e6)
                hosts.append(host / reps * 1e6)
        finally:
            gc.callbacks.remove(on_gc)
        by_gen = {}
        for gen, us in gc_pauses:
            n, mx = by_gen.get(gen, (0, 0.0))
            by_gen[gen] = (n + 1, max(mx, us))
        res[name] = {"us_per_call": round(sorted(walls)[batches // 2], 2),
                     "host_us_per_call": round(sorted(hosts)[batches // 2], 2),
                     "batches_us_per_call": [round(x, 2) for x in walls],
                     "slowest_call": {"host_us": round(slowest[0] * 1e6, 1), "batch": slowest[1], "index": slowest[2]},
                     "gc_collections": {f"gen{g}": {"count": n, "max_pause_us": round(mx, 1)}
                                        for g, (n, mx) in sorted(by_gen.items())}}
    res["sample"] = (f"{batches} batches of {reps} eager calls each (median batch), cycling the cold K/V copies; "
                     "one synchronisation per batch")
    return res


def workload_by_name(name: str):
    """A named workload; `name@BMxBN`: the same workload at other block sizes;
    `name+d256` / `name+fp32`: at another head_dim / in fp32 (the generic
    kernel's shapes)."""
    import dataclasses

    import torch
    from tsfa import configs

    base, _, blocks = name.partition("@")
    base, *mods = base.split("+")
    w = configs.WORKLOADS[base]
    for m in mods:
        if m.startswith("d") and m[1:].isdigit():
            w = dataclasses.replace(w, head_dim=int(m[1:]), name=f"{w.name}+{m}")
        elif m == "fp32":
            w = dataclasses.replace(w, dtype=torch.float32, name=f"{w.name}+{m}")
        else:
            raise SystemExit(f"unknown workload modifier +{m} in {name}")
    if blocks:
        bm, bn = (int(x) for x in blocks.lower().split("x"))
        w = w.with_blocks(bm, bn)
    return w


def workload_timing(name: str, steps: int, cold_mib: int, cpu_seconds: float = 0.0, cpu_cache=None):
    """One forward workload timed as the headline is: graph of `steps` calls
    (median of 5 replays), the combine alone, cold K/V copies; plus its CPU
    baseline (the fp32 oracle over a bounded sample) when cpu_seconds > 0.
    One-slot plans launch no combine (the split kernel writes O): the combine
    region is then not captured, and the split kernel is the whole call."""
    import torch

    from tsfa import _lib, configs
    import tree_sparse_flashattn as tsf

    w = workload_by_name(name)
    base = name.partition("@")[0]
    dev = torch.device("cuda", 0)
    q, k, v = configs.make_qkv(w)
    mask = configs.make_tree_mask(w)
    kvb = w.kv_bytes()
    copies = max(1, min(64, math.ceil(cold_mib * 2 ** 20 / kvb)))
    qd = q.to(dev)
    ks = [k.to(dev) for _ in range(copies)]
    vs = [v.to(dev) for _ in range(copies)]
    build = tsf.prepare_tree_sparse_metadata_batched if w.per_sequence else tsf.prepare_tree_sparse_metadata
    meta = build(mask.to(dev), w.prefix_len, w.block_m, w.block_n)
    out = torch.empty_like(qd)
    lib = _lib.load()
    # head_dim above 128 and fp32 run the generic kernel (its own plan, one
    # region: the split-plan report and the combine-only hook are the split
    # kernel's)
    generic = w.head_dim > 128 or w.dtype == torch.float32
    plan = ({"kernel": "gen_kernel + combine_kernel"} if generic else
            _lib.fwd_plan(w.batch, w.q_heads, w.kv_heads, w.tree_len, w.kv_len, w.prefix_len, w.head_dim))

    def call(i):
        tsf.tree_sparse_attention_fwd(qd, ks[i % copies], vs[i % copies], meta, out=out)

    for i in range(3):
        call(i)
    torch.cuda.synchronize()
    secs = {"combine": 0.0}
    regions = (("full", 3), ("combine", 2)) if not generic and plan["slots"] > 1 else (("full", 3),)
    for region, kmask in regions:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        _lib.check("tsfa_fwd_set_kernel_mask", lib.tsfa_fwd_set_kernel_mask(kmask))
        try:
            with torch.cuda.stream(s):
                call(0)
                torch.cuda.synchronize()
                with torch.cuda.graph(g, stream=s):
                    for i in range(steps):
                        call(i)
        finally:
            _lib.check("tsfa_fwd_set_kernel_mask", lib.tsfa_fwd_set_kernel_mask(3))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        # the median of 5 replays: one replay can catch a stall of the host
        # process or the GPU (a combine once read 41 us against ~5)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = []
        for _ in range(5):
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                a.record()
                g.replay()
                b.record()
            torch.cuda.synchronize()
            reps.append(a.elapsed_time(b) / 1e3 / steps)
        secs[region] = sorted(reps)[len(reps) // 2]
        del g
    split_s = secs["full"] - secs["combine"]
    flops = algorithmic_flops(w, mask)
    peak_tflops = MFMA_PEAK_TFLOPS_FP32 if w.dtype == torch.float32 else MFMA_PEAK_TFLOPS
    mfma_bound = flops / kvb > peak_tflops * 1e12 / (HBM_PEAK_GBPS * 1e9)
    tflops, gbps = flops / split_s / 1e12, kvb / split_s / 1e9
    del ks, vs
    torch.cuda.empty_cache()
    res = {"us_per_call": round(secs["full"] * 1e6, 2), "split_kernel_us": round(split_s * 1e6, 2),
           "combine_kernel_us": round(secs["combine"] * 1e6, 2), "bound": "mfma" if mfma_bound else "hbm",
           "frac": round(tflops / peak_tflops if mfma_bound else gbps / HBM_PEAK_GBPS, 4),
           "achieved": round(tflops, 1) if mfma_bound else round(gbps, 1),
           "unit": "TFLOP/s" if mfma_bound else "GB/s", "algorithmic_flops": flops, "algorithmic_bytes": kvb,
           "block_m": w.block_m, "block_n": w.block_n, "steps": steps, "kv_copies_cycled": copies, "plan": plan,
           "tokens_per_s": round(w.batch * w.tree_len / secs["full"], 1), "cpu_baseline": None}
    if generic:
        res["note"] = "generic kernel: gen_kernel and its combine timed as one region (split_kernel_us is both)"
    if cpu_seconds > 0:
        cache = {} if cpu_cache is None else cpu_cache
        if base not in cache:
            # bound the fp32 score tensor to ~0.6 GB per head chunk
            per_head = w.batch * w.tree_len * w.kv_len * 4
            chunk = max(1, min(8, w.q_heads, int(0.6e9 // per_head)))
            _log(f"[bench] cpu baseline {base} (head chunk {chunk}) ...")
            cache[base] = cpu_baseline(w, q, k, v, mask, cpu_seconds, head_chunk=chunk)
        cb = dict(cache[base])
        if base != name:
            cb["sample"] += f"; measured on {base} (the oracle does not depend on BLOCK_M / BLOCK_N)"
        cb["vs_gpu"] = round(cb["us_per_call"] / res["us_per_call"], 1)
        res["cpu_baseline"] = cb
    return res


def paged_timing(w, qd, ks, vs, meta, steps: int, page_size: int, contiguous_us: float):
    """The same forward over FlashInfer's paged cache ([pages, 2, page_size, Hkv, D],
    benchmark.py:67-91) with each sequence's pages scattered in seeded random
    order, read in place by tree_sparse_attention_fwd_paged: graph of `steps`
    calls cycling the same number of cache copies as the contiguous timing."""
    import torch

    import tree_sparse_flashattn as tsf
    from tsfa import configs

    caches = [configs.make_paged_kv(k, v, page_size, seed=i) for i, (k, v) in enumerate(zip(ks, vs))]
    out = torch.empty_like(qd)

    def call(i):
        cache, indptr, indices = caches[i % len(caches)]
        tsf.tree_sparse_attention_fwd_paged(qd, cache, indices, meta, kv_len=w.kv_len, kv_indptr=indptr, out=out)

    for i in range(5):
        call(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call(0)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                call(i)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / steps
    del caches
    return {"page_size": page_size, "layout": "NHD", "pages": "scattered (seeded permutation), CSR page lists",
            "us_per_call": round(us, 3), "value": round(w.kv_bytes() / (us * 1e-6) / 1e12, 4), "unit": "TB/s",
            "vs_contiguous": round(contiguous_us / us, 4)}


def backward_timing(w, mask, qd, ks, vs, meta, steps: int, fwd_flops: float, cpu_seconds: float = 0.0):
    """tree_sparse_attention_bwd (dQ, dK, dV from O, the row LSE and dO) over the
    same cycled K/V copies: graph of `steps` calls, HIP events on the replay
    stream.  Algorithmic figures: five products per visible (row, key) pair --
    S recomputed, dP, dV, dK, dQ -- i.e. 2.5x the forward's flops; bytes = Q, O,
    dO, K, V read once and dQ, dK, dV written once."""
    import torch

    import tree_sparse_flashattn as tsf

    do = torch.randn(qd.shape, generator=torch.Generator().manual_seed(7)).to(w.dtype).to(qd.device)
    fwd = [tsf.tree_sparse_attention_fwd(qd, k, v, meta, return_lse=True) for k, v in zip(ks[:1], vs[:1])][0]
    o, lse = fwd
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(ks[0]), torch.empty_like(vs[0])

    def call(i):
        tsf.tree_sparse_attention_bwd(qd, ks[i % len(ks)], vs[i % len(vs)], o, lse, do, meta, dq=dq, dk=dk, dv=dv)

    for i in range(3):
        call(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call(0)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                call(i)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / steps
    flops = 2.5 * fwd_flops
    nbytes = 2 * w.kv_bytes() + 4 * qd.numel() * qd.element_size()
    tflops = flops / (us * 1e-6) / 1e12
    gbps = nbytes / (us * 1e-6) / 1e9
    res = {"us_per_call": round(us, 3), "algorithmic_flops": flops, "algorithmic_bytes": nbytes,
           "achieved_tflops": round(tflops, 1), "mfma_frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
           "achieved_gbps": round(gbps, 1), "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "cpu_baseline": None,
           "kernels": "prep and tree visibility (one launch) + key-parallel dK/dV beside row-parallel dQ on a side stream (+ dQ convert when the key range is split)"}
    if cpu_seconds > 0:
        # the fp32 gradient oracle (closed forms, oracle/attn_grad_oracle.py) on the host cores
        from oracle.attn_grad_oracle import attention_grads

        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        qc, kc, vc, dc = qd.cpu(), ks[0].cpu(), vs[0].cpu(), do.cpu()
        t0 = time.perf_counter()
        attention_grads(qc, kc, vc, mask, w.prefix_len, dc, head_chunk=8)
        t1 = time.perf_counter() - t0
        n = max(1, min(100, int(cpu_seconds / max(t1, 1e-6))))
        t0 = time.perf_counter()
        for _ in range(n):
            attention_grads(qc, kc, vc, mask, w.prefix_len, dc, head_chunk=8)
        dt = (time.perf_counter() - t0) / n
        res["cpu_baseline"] = {"us_per_call": round(dt * 1e6, 1), "cores": cores, "kind": "port",
                               "sample": f"{n} full backward calls of the fp32 gradient oracle (torch CPU, {cores} threads)"}
    return res


def calibrate_copy(mib: int, reps: int):
    """A plain device copy of known size, for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE."""
    import torch

    src = torch.ones(mib * 2 ** 18, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": mib * 2 ** 20, "reps": reps}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=None)
    ap.add_argument("--cold-mib", type=int, default=512, help="K/V bytes cycled through (defeats the MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-backward", action="store_true", help="skip the backward timing")
    ap.add_argument("--paged-page-size", type=int, default=16,
                    help="also time the paged-cache forward at this page size (0: skip)")
    ap.add_argument("--workloads", default="batched-decode-b16-p2048:100,wide-tree-1024-p16384:10,"
                    "llama3-70b-b4-p32768:5,llama3-70b-b4-p32768@64x32:5,llama3-70b-b4-p32768@64x128:5,"
                    "llama3-70b-b4-p32768@16x64:5,llama3-8b-eagle64-p4096+d256:100,tiny-random-tree-fp32:100",
                    help="other forward workloads timed into the `workloads` object, as "
                         "name[+d<head_dim>|+fp32][@BMxBN]:steps ('' skips)")
    ap.add_argument("--workload-cpu-seconds", type=float, default=6.0,
                    help="CPU baseline sample per other workload (0 skips)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain MIB-MiB device copy (rocprofv3 PMC calibration) and exit")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU: the library has no multi-GPU path (got --gpus {args.gpus}); "
              "the forward shards by (batch, kv head) with no exchange -- run one process per GPU.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.calibrate_copy > 0:
        calibrate_copy(args.calibrate_copy, max(1, args.steps))
        return

    from tsfa import _lib, configs
    import tree_sparse_flashattn as tsf

    w = configs.WORKLOADS[args.workload or configs.HEADLINE]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    q, k, v = configs.make_qkv(w)
    mask = configs.make_tree_mask(w)
    kvb = w.kv_bytes()
    copies = max(1, min(64, math.ceil(args.cold_mib * 2 ** 20 / kvb)))
    qd = q.to(dev)
    ks = [k.to(dev) for _ in range(copies)]
    vs = [v.to(dev) for _ in range(copies)]
    if w.per_sequence:
        meta = tsf.prepare_tree_sparse_metadata_batched(mask.to(dev), w.prefix_len, w.block_m, w.block_n)
    else:
        meta = tsf.prepare_tree_sparse_metadata(mask.to(dev), w.prefix_len, w.block_m, w.block_n)
    out = torch.empty_like(qd)
    plan = _lib.fwd_plan(w.batch, w.q_heads, w.kv_heads, w.tree_len, w.kv_len, w.prefix_len, w.head_dim)
    lib = _lib.load()

    def call(i):
        tsf.tree_sparse_attention_fwd(qd, ks[i % copies], vs[i % copies], meta, out=out)

    _log(f"[bench] {w.name}: warmup {args.warmup}, steps {args.steps}, K/V copies {copies}, plan {plan}")
    for i in range(max(1, args.warmup)):
        call(i)
    torch.cuda.synchronize()

    steps = args.steps
    # eager calls first: on this runtime, launches made after a graph is
    # instantiated and before it is first replayed measured ~5x slower
    _log("[bench] eager calls ...")
    eager = eager_call_timing(w, qd, ks, vs, mask.to(dev), meta)

    def capture(kernel_mask: int):
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        _lib.check("tsfa_fwd_set_kernel_mask", lib.tsfa_fwd_set_kernel_mask(kernel_mask))
        try:
            with torch.cuda.stream(s):
                call(0)  # allocator warm-up on the capture stream
                torch.cuda.synchronize()
                with torch.cuda.graph(g, stream=s):
                    for i in range(steps):
                        call(i)
        finally:
            _lib.check("tsfa_fwd_set_kernel_mask", lib.tsfa_fwd_set_kernel_mask(3))
        torch.cuda.synchronize()
        return g, s

    # each region: `reps` replays of its graph of exactly `steps` calls,
    # synchronised on both sides; the median replay is reported (at least
    # 100 calls over the replays)
    reps = max(5, math.ceil(100 / steps))

    def timed(g, s):
        g.replay()  # upload / warm
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        out_s = []
        for _ in range(reps):
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                a.record()
                g.replay()
                b.record()
            torch.cuda.synchronize()
            out_s.append(a.elapsed_time(b) / 1e3)
        return sorted(out_s)

    # one-slot plans launch no combine (the split kernel writes O): nothing to
    # capture for it, and the split kernel is the whole call
    kinds = (("full", 3), ("combine", 2), ("split", 1)) if plan["slots"] > 1 else (("full", 3), ("split", 1))
    regions = {name: capture(mask) for name, mask in kinds}
    samples = {name: timed(*gs) for name, gs in regions.items()}
    secs = {name: v[len(v) // 2] / steps for name, v in samples.items()}
    secs.setdefault("combine", 0.0)
    per_call_s = secs["full"]
    split_avg_s = secs["full"] - secs["combine"]
    _log(f"[bench] {steps} calls: {per_call_s * 1e6:.2f} us/call = split-KV {split_avg_s * 1e6:.2f} + combine "
         f"{secs['combine'] * 1e6:.2f} us; split-KV back to back {secs['split'] * 1e6:.2f} us/launch")

    achieved_gbps = kvb / split_avg_s / 1e9
    traffic = _traffic(w.name)
    flops = algorithmic_flops(w, mask)
    mfma_bound = flops / kvb > RIDGE_FLOP_PER_BYTE
    achieved_tflops = flops / split_avg_s / 1e12
    result = {
        "metric": METRIC,
        "value": round(kvb / per_call_s / 1e12, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(per_call_s * 1e3, 6),
        "us_per_call": round(per_call_s * 1e6, 3),
        "tokens_per_s": round(w.batch * w.tree_len / per_call_s, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16"}[w.dtype],
        "data": "synthetic N(0,1) q/k/v, seeded EAGLE draft tree; metadata built on the device beforehand",
        "config": {
            "workload": w.name,
            "batch": w.batch, "q_heads": w.q_heads, "kv_heads": w.kv_heads, "head_dim": w.head_dim,
            "prefix_len": w.prefix_len, "tree_len": w.tree_len, "block_m": w.block_m, "block_n": w.block_n,
            "kv_bytes_per_call": kvb, "kv_copies_cycled": copies, "plan": plan,
            "timing": f"hip graph of all steps, replayed {reps} times (median replay); HIP events on the replay "
                      "stream",
        },
        "samples": {"replays": reps, "calls_per_replay": steps,
                    "us_per_call": [round(x / steps * 1e6, 3) for x in samples["full"]],
                    "median_us_per_call": round(per_call_s * 1e6, 3),
                    "min_us_per_call": round(samples["full"][0] / steps * 1e6, 3),
                    "max_us_per_call": round(samples["full"][-1] / steps * 1e6, 3)},
        "roofline": {
            "bound": "mfma" if mfma_bound else "hbm",
            "kernel": "tsfa::fwd::split_kernel",
            "achieved": round(achieved_tflops, 1) if mfma_bound else round(achieved_gbps, 1),
            "peak": MFMA_PEAK_TFLOPS if mfma_bound else HBM_PEAK_GBPS,
            "unit": "TFLOP/s" if mfma_bound else "GB/s",
            "frac": round(achieved_tflops / MFMA_PEAK_TFLOPS if mfma_bound else achieved_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "algorithmic_bytes": kvb,
            "algorithmic_flops": flops,
            "hbm_frac": round(achieved_gbps / HBM_PEAK_GBPS, 4),
            "mfma_frac": round(achieved_tflops / MFMA_PEAK_TFLOPS, 4),
            "split_kernel_us": round(split_avg_s * 1e6, 3),
            "split_kernel_back_to_back_us": round(secs["split"] * 1e6, 3),
            "combine_kernel_us": round(secs["combine"] * 1e6, 3),
        },
        "cpu_baseline": None,
        "metadata": None,
        "eager": None,
        "workloads": None,
        "paged": None,
        "backward": None,
    }
    result["eager"] = eager
    _log("[bench] metadata build ...")
    result["metadata"] = metadata_timing(w, mask.to(dev), mask)
    if not args.no_backward:
        _log("[bench] backward ...")
        result["backward"] = backward_timing(w, mask, qd, ks, vs, meta, steps, flops,
                                             0.0 if args.no_cpu_baseline else min(5.0, args.cpu_seconds))
    if args.paged_page_size > 0:
        _log(f"[bench] paged cache, page_size {args.paged_page_size} ...")
        regions = None
        result["paged"] = paged_timing(w, qd, ks, vs, meta, steps, args.paged_page_size, per_call_s * 1e6)
    others = [x for x in args.workloads.split(",") if x and x.split(":")[0] != w.name]
    if others:
        regions = None
        torch.cuda.empty_cache()
        result["workloads"] = {}
        cpu_cache = {}
        for item in others:
            name, _, n = item.partition(":")
            _log(f"[bench] workload {name} ...")
            result["workloads"][name] = workload_timing(
                name, int(n or 10), args.cold_mib,
                0.0 if args.no_cpu_baseline else args.workload_cpu_seconds, cpu_cache)
    if not args.no_cpu_baseline:
        _log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(w, q, k, v, mask, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
