"""Benchmark of the paged-attention hot path on one MI355X.

A step is one pass of the path over one batch: append the new tokens' K/V
into their pages, then paged attention (decode: one query per sequence;
prefill: ragged causal chunks).  The plan is built once per batch (the engine
builds it once per forward and reuses it across layers).

Default workload: TinyLlama-1.1B paged decode at scale (32q/4kv heads, D=64,
page 16, B=256, kv_len U[256,2048], bf16).  `value` is whole-step
throughput in algorithmic HBM GB/s; `roofline` is the decode attention
launch (algorithmic bytes / average launch time from HIP events);
`cpu_baseline` is the fp32 CPU oracle on a bounded sample of the same batch.
Pools are rotated across replicas totalling > 1 GB so the 256 MB Infinity
Cache cannot hold the KV between steps.

Prints ONE JSON line.  `--gpus N` with N > 1 exits: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "llm-inference-runtime_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
WS_BYTES = 128 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _replicas(bytes_per_instance: int, min_total: int = 1 << 30, cap: int = 8) -> int:
    r = 1
    while r * bytes_per_instance < min_total and r < cap:
        r += 1
    return r


def bench_decode(w, args, dev, dtype, label, cpu_sample: int = 0):
    import numpy as np
    import torch

    import pagedattn
    from pagedattn import workloads as W

    kv_elem = 1 if w.fp8 else 2
    alg_attn = W.decode_bytes(w, kv_elem)
    alg_step = W.decode_bytes(w, kv_elem, with_append=True)
    pool_bytes = w.num_pages * 2 * w.hkv * 16 * w.d * kv_elem
    reps = _replicas(pool_bytes)
    log(f"{label}: B={w.meta.batch_size} pages={w.num_pages} kv={alg_attn / 1e9:.3f} GB "
        f"replicas={reps}")
    inst = []
    for r in range(reps):
        t = W.materialize(w, dev, dtype, seed=w.seed * 100 + r)
        if w.fp8:
            t.pool, t.scales = pagedattn.quantize_pages_e4m3(t.pool)
        inst.append(t)
    torch.cuda.synchronize()
    ws = torch.zeros(WS_BYTES, dtype=torch.uint8, device=dev)
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    t0 = inst[0]
    tp = time.perf_counter()
    dw.plan(t0.kv_indptr, t0.kv_indices, t0.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=dtype, split_pages=w.split_pages)
    torch.cuda.synchronize()
    plan_ms = (time.perf_counter() - tp) * 1e3
    outs = [torch.empty((w.meta.batch_size, w.hq, w.d), dtype=dtype, device=dev)
            for _ in range(reps)]

    def step(i):
        # the decode step: new token's K/V appended at kv_len - 1, then
        # attention, in one launch (pagedattn_decode_run_append) plus the
        # split-KV merge launch when the plan cut sequences
        t = inst[i % reps]
        dw.run(t.q, t.pool, kv_scales=t.scales, out=outs[i % reps], append_key=t.k_new,
               append_value=t.v_new)

    for i in range(args.warmup):
        step(i)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        step(args.warmup + i)
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    attn_avg = total_ms / args.steps
    res = {
        "workload": label,
        "ms_per_step": total_ms / args.steps,
        "step_GBps": alg_step / (total_ms / args.steps * 1e-3) / 1e9,
        "attn_ms_avg": attn_avg,
        "attn_GBps": alg_attn / (attn_avg * 1e-3) / 1e9,
        "alg_bytes_attn": alg_attn,
        "alg_bytes_step": alg_step,
        "plan_ms_host": plan_ms,
        "replicas": reps,
        "batch": w.meta.batch_size,
        "kv_tokens": int(w.meta.seq_lens.sum()),
        "split_pages": w.split_pages,
    }
    res["attn_frac"] = res["attn_GBps"] / HBM_PEAK_GBS
    if cpu_sample:
        res["cpu"] = cpu_decode_baseline(w, inst[0], cpu_sample, kv_elem)
    del inst, outs
    torch.cuda.empty_cache()
    return res


def bench_prefill(w, args, dev, dtype, label):
    import numpy as np
    import torch

    import pagedattn
    from pagedattn import workloads as W

    flops = W.prefill_flops(w)
    t = W.materialize(w, dev, dtype)
    if w.fp8:
        t.pool, t.scales = pagedattn.quantize_pages_e4m3(t.pool)
    ws = torch.zeros(WS_BYTES, dtype=torch.uint8, device=dev)
    pw = pagedattn.BatchPrefillWithPagedKVCacheWrapper(ws, "HND")
    pw.plan(t.qo_indptr, t.kv_indptr, t.kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=dtype, causal=True)
    out = torch.empty_like(t.q)

    def step():
        pagedattn.append_paged_kv_cache(t.k_new, t.v_new, t.batch_indices, t.positions, t.pool,
                                        t.kv_indices, t.kv_indptr, t.kv_last_page_len,
                                        kv_layout="HND", kv_scales=t.scales)
        pw.run(t.q, t.pool, kv_scales=t.scales, out=out)

    for _ in range(args.warmup):
        step()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    # attention launches back to back: HIP events around the loop
    start.record()
    for _ in range(args.steps):
        pw.run(t.q, t.pool, kv_scales=t.scales, out=out)
    end.record()
    torch.cuda.synchronize()
    avg = start.elapsed_time(end) / args.steps
    res = {
        "workload": label,
        "ms_per_step": total_ms / args.steps,
        "attn_ms_avg": avg,
        "attn_TFLOPs": flops / (avg * 1e-3) / 1e12,
        "alg_flops_attn": flops,
        "rows": int(w.meta.nnz),
        "kv_tokens": int(w.meta.seq_lens.sum()),
    }
    res["attn_frac"] = res["attn_TFLOPs"] / BF16_PEAK_TFLOPS
    del t, out
    torch.cuda.empty_cache()
    return res


def _time_ms(fn, steps: int, warmup: int) -> float:
    import torch
    for i in range(warmup):
        fn(i)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        fn(warmup + i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _time_graph_ms(fn, steps: int, warmup: int) -> float:
    """Device time per call of fn: `steps` calls captured in one HIP graph,
    replayed and timed, so the host's per-call argument checks (tens of us
    for a small launch) stay out of the figure."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(warmup):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def bench_device_plan(w, dev, dtype, steps: int = 30, warmup: int = 5) -> dict:
    """The same fused decode step with the device-side partition
    (pagedattn_decode_plan_device), eagerly and replayed from a HIP graph,
    and the device metadata builder for the batch."""
    import numpy as np
    import torch

    import pagedattn
    from pagedattn import workloads as W

    alg_step = W.decode_bytes(w, 2, with_append=True)
    reps = _replicas(w.num_pages * 2 * w.hkv * 16 * w.d * 2)
    inst = [W.materialize(w, dev, dtype, seed=w.seed * 100 + r) for r in range(reps)]
    ws = torch.zeros(WS_BYTES, dtype=torch.uint8, device=dev)
    out = torch.empty((w.meta.batch_size, w.hq, w.d), dtype=dtype, device=dev)
    t0 = inst[0]
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    dw.plan(t0.kv_indptr, t0.kv_indices, t0.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=dtype, device_plan=True)

    def step(t):
        dw.run(t.q, t.pool, out=out, append_key=t.k_new, append_value=t.v_new)

    eager_ms = _time_ms(lambda i: step(inst[i % reps]), steps, warmup)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for t in inst:
            step(t)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphs = []
    for t in inst:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(t)
        graphs.append(g)
    graph1_ms = _time_ms(lambda i: graphs[i % reps].replay(), steps, warmup)
    # an engine captures a whole forward (every layer's call) in one graph:
    # `steps` calls in one graph spread the graph launch over them
    graph_ms = _time_graph_ms(lambda i: step(inst[i % reps]), steps, warmup)
    # metadata of the batch from a block table on the device
    m = w.meta
    npg = np.diff(m.kv_indptr)
    tables = np.full((m.batch_size, int(npg.max())), -1, dtype=np.int32)
    for b in range(m.batch_size):
        tables[b, :npg[b]] = m.kv_indices[m.kv_indptr[b]:m.kv_indptr[b + 1]]
    bt = torch.from_numpy(tables).to(dev)
    lens = torch.from_numpy(m.seq_lens.astype(np.int32)).to(dev)
    buf = pagedattn.ops.new_paged_buffers(m.batch_size, tables.size, m.batch_size, dev)
    meta_ms = _time_graph_ms(lambda i: pagedattn.build_paged_metadata(bt, lens, out=buf),
                             steps, warmup)
    del graphs, inst
    torch.cuda.empty_cache()
    return {"eager_ms_per_step": eager_ms, "eager_GBps": alg_step / (eager_ms * 1e-3) / 1e9,
            "graph_ms_per_step": graph_ms, "graph_GBps": alg_step / (graph_ms * 1e-3) / 1e9,
            "graph_steps_per_graph": steps,
            "graph_one_step_ms": graph1_ms,
            "metadata_build_ms": meta_ms}


def bench_kv_write(dev, steps: int = 20, warmup: int = 3) -> dict:
    """The engine's KV write path: e4m3 append that keeps running-amax page
    scales (a 4096-token prefill chunk of a Llama-3-70B layer, 8 KV heads,
    D=128; and a 128-sequence decode step of that layer, timed for its
    latency), and a copy-on-write fork of 256 pages across every layer of a
    Llama-3-8B pool (32 layers, 8 KV heads, D=128, bf16).  Both move bytes
    only: GB/s of algorithmic bytes (read + written)."""
    import numpy as np
    import torch

    import pagedattn
    from pagedattn.metadata import prefill_metadata

    rng = np.random.default_rng(7)
    hkv, d = 8, 128
    # 4 sequences x 1024 new tokens after prefixes of 0..8191 tokens
    computed = [int(x) // 16 * 16 for x in rng.integers(0, 8192, 4)]
    chunks = [1024] * 4
    need = [(c + n + 15) // 16 for c, n in zip(computed, chunks)]
    perm = rng.permutation(sum(need) + 16)
    tables, at = [], 0
    for k in need:
        tables.append(perm[at:at + k].tolist())
        at += k
    meta = prefill_metadata(tables, computed, chunks)
    num_pages = len(perm)
    q8 = torch.zeros((num_pages, 2, hkv, 16, d), dtype=torch.uint8,
                     device=dev).view(torch.float8_e4m3fn)
    scales = torch.zeros((num_pages, 2, hkv), dtype=torch.float32, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    k = torch.randn((meta.nnz, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((meta.nnz, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)
    bi, pos, ind, indptr, last = (i32(meta.batch_indices), i32(meta.positions),
                                  i32(meta.kv_indices), i32(meta.kv_indptr),
                                  i32(meta.kv_last_page_len))
    app_ms = _time_graph_ms(lambda i: pagedattn.append_paged_kv_cache_e4m3_amax(
        k, v, bi, pos, q8, ind, indptr, last, scales, kv_layout="HND"), steps, warmup)
    app_bytes = meta.nnz * hkv * d * 2 * (2 + 1)  # bf16 rows in, e4m3 rows out
    # a decode step of the same layer: 128 sequences, one token each
    from pagedattn.metadata import decode_metadata
    lens = [int(x) for x in rng.integers(1, 8192, 128)]
    need = [(n + 15) // 16 for n in lens]
    perm = rng.permutation(sum(need))
    tables, at = [], 0
    for n_p in need:
        tables.append(perm[at:at + n_p].tolist())
        at += n_p
    dm = decode_metadata(tables, lens)
    q8d = torch.zeros((len(perm), 2, hkv, 16, d), dtype=torch.uint8,
                      device=dev).view(torch.float8_e4m3fn)
    sd = torch.zeros((len(perm), 2, hkv), dtype=torch.float32, device=dev)
    kd = torch.randn((dm.nnz, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    vd = torch.randn((dm.nnz, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    dargs = (i32(dm.batch_indices), i32(dm.positions), q8d, i32(dm.kv_indices),
             i32(dm.kv_indptr), i32(dm.kv_last_page_len), sd)
    dec_ms = _time_graph_ms(lambda i: pagedattn.append_paged_kv_cache_e4m3_amax(
        kd, vd, *dargs, kv_layout="HND"), steps, warmup)
    layers, pages, n_fork = 32, 1024, 256
    pool = torch.zeros((layers, pages, 2, hkv, 16, d), dtype=torch.bfloat16, device=dev)
    src = rng.choice(pages // 2, n_fork, replace=False)
    dst = pages // 2 + rng.choice(pages // 2, n_fork, replace=False)
    src_d, dst_d = i32(src), i32(dst)
    fork_ms = _time_graph_ms(lambda i: pagedattn.fork_pages(pool, src_d, dst_d), steps, warmup)
    fork_bytes = n_fork * layers * 2 * hkv * 16 * d * 2 * 2  # read + write
    del pool
    torch.cuda.empty_cache()
    return {"append_e4m3_amax": {"tokens": meta.nnz, "ms": app_ms,
                                 "GBps": app_bytes / (app_ms * 1e-3) / 1e9},
            "append_e4m3_amax.decode": {"tokens": dm.nnz, "ms": dec_ms},
            "fork_pages": {"forks": n_fork, "layers": layers, "ms": fork_ms,
                           "GBps": fork_bytes / (fork_ms * 1e-3) / 1e9}}


def cpu_decode_baseline(w, t, n_seq: int, kv_elem: int):
    """fp32 oracle decode over the first n_seq sequences, timed on the host."""
    import numpy as np
    import torch

    import oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rows = list(range(min(n_seq, w.meta.batch_size)))
    m = w.meta
    # compact pool of the sampled sequences, copied to host once (untimed)
    parts = [m.kv_indices[m.kv_indptr[b]:m.kv_indptr[b + 1]] for b in rows]
    pages = np.concatenate(parts)
    indptr = np.concatenate([[0], np.cumsum([len(p) for p in parts])]).astype(np.int32)
    idx = torch.from_numpy(pages.astype(np.int64)).to(t.pool.device)
    sub = t.pool.index_select(0, idx).cpu()
    scales = None if t.scales is None else t.scales.index_select(0, idx).cpu()
    q = t.q[rows].float().cpu()
    ind = np.arange(len(pages), dtype=np.int32)
    last = m.kv_last_page_len[rows]
    # repeat the sample until about 10 s of CPU work has been timed
    reps, elapsed = 0, 0.0
    while elapsed < 10.0 or reps < 3:
        t0 = time.perf_counter()
        O.decode(q, sub, indptr, ind, last, scales=scales)
        elapsed += time.perf_counter() - t0
        reps += 1
    sec = elapsed / reps
    kv_bytes = int(m.seq_lens[rows].astype(np.int64).sum()) * w.hkv * w.d * 2 * kv_elem
    byts = kv_bytes + len(rows) * w.hq * w.d * 4
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")),
                         "unknown")
    except OSError:
        model = "unknown"
    return {
        "value": byts / sec / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{len(rows)} of {w.meta.batch_size} sequences of {w.name} "
                   f"({int(m.seq_lens[rows].sum())} kv tokens), fp32 torch oracle, "
                   f"{reps} passes in {elapsed:.1f} s ({sec:.3f} s each) on {model}"),
    }


def copy_calibration(dev, nbytes: int = 1 << 30, reps: int = 3) -> dict:
    """A plain copy of known size: the reference point for HBM byte counters."""
    import torch

    import pagedattn

    src = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        pagedattn.copy_bytes(dst, src)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    pagedattn.copy_bytes(dst, src)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b)
    return {"bytes_read": nbytes, "bytes_written": nbytes, "ms": ms,
            "GBps": 2 * nbytes / (ms * 1e-3) / 1e9}


def load_traffic() -> dict | None:
    """HBM bytes per decode step measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    runs of this bench (scaled by the plain-copy calibration), as committed in
    profiles/; None when absent."""
    path = os.path.join(ROOT, "profiles", "decode_tinyllama_b256_hbm_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None
    d["source"] = os.path.relpath(path, ROOT)
    return d


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the other workloads (long-context decode, ...)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported",
              file=sys.stderr)
        return 2
    import torch

    from pagedattn import workloads as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    dtype = torch.bfloat16

    main_w = W.tinyllama_decode(seed=args.seed)
    r = bench_decode(main_w, args, dev, dtype, "tinyllama_decode",
                     cpu_sample=0 if args.no_cpu else 256)
    log(f"tinyllama_decode: step {r['ms_per_step']:.4f} ms, attention {r['attn_ms_avg']:.4f} ms "
        f"= {r['attn_GBps']:.0f} GB/s ({100 * r['attn_frac']:.1f}% of 8 TB/s)")
    extra = {}
    if not args.no_extra:
        lw = W.llama3_8b_long_decode(seed=args.seed)
        lr = bench_decode(lw, argparse.Namespace(steps=max(5, args.steps // 3),
                                                 warmup=2), dev, dtype,
                          "llama3_8b_long_decode")
        log(f"llama3_8b_long_decode: attention {lr['attn_ms_avg']:.3f} ms = "
            f"{lr['attn_GBps']:.0f} GB/s ({100 * lr['attn_frac']:.1f}%)")
        extra["llama3_8b_long_decode"] = {k: lr[k] for k in (
            "ms_per_step", "attn_ms_avg", "attn_GBps", "attn_frac", "alg_bytes_attn",
            "split_pages", "batch", "kv_tokens")}
        # the planner's own balanced partition of the same batch
        lb = bench_decode(dataclasses.replace(lw, split_pages=0),
                          argparse.Namespace(steps=max(5, args.steps // 3), warmup=2), dev,
                          dtype, "llama3_8b_long_decode.balanced")
        log(f"llama3_8b_long_decode (balanced split): {lb['attn_GBps']:.0f} GB/s "
            f"({100 * lb['attn_frac']:.1f}%)")
        extra["llama3_8b_long_decode.balanced"] = {k: lb[k] for k in (
            "ms_per_step", "attn_GBps", "attn_frac", "split_pages")}
        pa_ = argparse.Namespace(steps=max(5, args.steps // 2), warmup=2)
        pr = bench_prefill(W.llama3_8b_prefill(seed=args.seed), pa_, dev, dtype,
                           "llama3_8b_prefill")
        log(f"llama3_8b_prefill: attention {pr['attn_ms_avg']:.4f} ms = "
            f"{pr['attn_TFLOPs']:.1f} TFLOP/s ({100 * pr['attn_frac']:.1f}% of bf16 peak)")
        extra["llama3_8b_prefill"] = pr
        dec5, pre5 = W.llama3_70b_mixed_fp8(seed=args.seed)
        d5 = bench_decode(dec5, pa_, dev, dtype, "llama3_70b_mixed_fp8.decode")
        p5 = bench_prefill(pre5, pa_, dev, dtype, "llama3_70b_mixed_fp8.prefill")
        log(f"llama3_70b_mixed_fp8: decode {d5['attn_GBps']:.0f} GB/s "
            f"({100 * d5['attn_frac']:.1f}%), prefill {p5['attn_TFLOPs']:.1f} TFLOP/s "
            f"({100 * p5['attn_frac']:.1f}% of bf16 peak)")
        extra["llama3_70b_mixed_fp8"] = {
            "decode": {k: d5[k] for k in ("attn_ms_avg", "attn_GBps", "attn_frac",
                                          "alg_bytes_attn", "batch", "kv_tokens")},
            "prefill": p5,
        }
        dp = bench_device_plan(main_w, dev, dtype)
        log(f"tinyllama_decode (device plan): eager {dp['eager_ms_per_step']:.4f} ms, "
            f"HIP graph {dp['graph_ms_per_step']:.4f} ms per step "
            f"({dp['graph_steps_per_graph']} steps per graph; "
            f"{dp['graph_one_step_ms']:.4f} ms with one step per graph); metadata build "
            f"{1e3 * dp['metadata_build_ms']:.1f} us")
        extra["tinyllama_decode.device_plan"] = dp
        kw = bench_kv_write(dev)
        log(f"kv write path: e4m3 running-amax append {kw['append_e4m3_amax']['GBps']:.0f} GB/s "
            f"(4096-token chunk), {1e3 * kw['append_e4m3_amax.decode']['ms']:.1f} us per "
            f"128-token decode step; CoW fork {kw['fork_pages']['GBps']:.0f} GB/s")
        extra["kv_write"] = kw
    cal = copy_calibration(dev)
    traffic = load_traffic()
    log(f"copy calibration: {cal['GBps']:.0f} GB/s (read+write)")

    line = {
        "metric": "paged decode attn HBM GB/s (% of 8 TB/s); prefill attn TFLOP/s (% MFMA peak)",
        "value": round(r["step_GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) pool/q/k/v, random block tables)",
        "config": {
            "workload": "tinyllama_decode: TinyLlama-1.1B paged decode at scale, 32q/4kv heads, "
                        "head_dim 64, page 16, batch 256, kv_len U[256,2048], fused append",
            "batch": r["batch"],
            "kv_tokens": r["kv_tokens"],
            "page_size": 16,
            "parallelism": "single GPU",
            "seed": args.seed,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode step launch: decode_kernel<64, bf16, append> (new token's K/V "
                      "written, then attention) plus its split-KV merge launch",
            "achieved": round(r["step_GBps"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r["step_GBps"] / HBM_PEAK_GBS, 4),
            "traffic": traffic.get("traffic_bytes_per_step") if traffic else None,
            "traffic_source": traffic.get("source") if traffic else None,
            "alg_bytes_per_launch": r["alg_bytes_step"],
            "avg_launch_ms": round(r["ms_per_step"], 5),
        },
        "cpu_baseline": r.get("cpu"),
        "extra": extra,
        "copy_calibration": cal,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
