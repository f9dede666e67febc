"""Benchmark of the paged-attention hot path on one MI355X.

A step is one pass of the path over one batch: append the new tokens' K/V
into their pages, then paged attention (decode: one query per sequence;
prefill: ragged causal chunks).  The plan is built once per batch (the engine
builds it once per forward and reuses it across layers).

Headline (`value`): TinyLlama-1.1B paged decode at scale (32q/4kv heads,
D=64, page 16, B=256, kv_len U[256,2048], bf16), whole-step throughput in
algorithmic HBM GB/s.  Every configuration is timed step by step with HIP
events on the launch stream (median of >= 20 steps) over pools rotated
across replicas totalling > 512 MB, so the 256 MB Infinity Cache cannot hold
the KV between steps.  Each configuration carries a `roofline` block (HBM
GB/s against 8 TB/s for decode, TFLOP/s against the 2.5 PFLOP/s bf16 dense
MFMA peak for prefill; `traffic` from the committed rocprofv3 FETCH_SIZE /
WRITE_SIZE summaries when they match the built sources) and a
`cpu_baseline` (the fp32 CPU oracle on a bounded, stated sample).

Prints ONE JSON line.  `--gpus N` with N > 1 exits: this build runs on one GPU.
`--config` runs a subset (for profiling runs), e.g. `--config c4 --no-cpu`.
"""

from __future__ import annotations

import argparse
import dataclasses
import hashlib
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "llm-inference-runtime_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
WS_BYTES = 128 << 20
CONFIGS = ("c2", "c3", "c4", "c4b", "c5d", "c5p", "devplan", "kvwrite")
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "hbm_traffic.json")
# device time the prefill launches run untimed before they are timed
PREFILL_SETTLE_MS = 150.0
DECODE_TIMING = ("K back-to-back steps between one HIP event pair on the launch stream "
                 "(queued behind a few ms of copies), divided by K")
PREFILL_TIMING = ("K back-to-back launches between one HIP event pair on the launch stream "
                  "(queued behind two untimed launches), divided by K")
CSRC = os.path.join(ROOT, "llm-inference-runtime_amd", "csrc")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def sources_sha() -> str:
    """Hash of the kernel sources; a committed traffic figure applies only
    to the sources it was measured with."""
    h = hashlib.sha256()
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".h", ".cpp")):
            with open(os.path.join(CSRC, name), "rb") as f:
                h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def _replicas(bytes_per_instance: int, min_total: int = 1 << 30, cap: int = 8) -> int:
    r = 1
    while r * bytes_per_instance < min_total and r < cap:
        r += 1
    return r


_busy = None


def _fill_queue(ms: float = 3.0) -> None:
    """Puts a few ms of streaming copies on the stream, so that the host has
    queued every timed step before the GPU reaches them: the event pairs
    then time the device, not the Python launch path."""
    import torch

    import pagedattn
    global _busy
    if _busy is None:
        n = 256 << 20
        _busy = (torch.empty(n, dtype=torch.uint8, device="cuda"),
                 torch.empty(n, dtype=torch.uint8, device="cuda"))
    for _ in range(max(1, int(ms / 0.11))):  # ~0.11 ms per 256 MiB copy
        pagedattn.copy_bytes(_busy[1], _busy[0])


def settle(fn, min_ms: float, max_calls: int = 2000) -> int:
    """Untimed calls of fn until min_ms of device time have passed (at most
    max_calls); returns the number of calls.  The MFMA-bound prefill needs
    this: its launch time falls by about 10 % over the first ~100 ms of
    back-to-back launches and then holds (Llama-3-8B prefill on MI355X:
    228 -> 205 us), while the HBM-bound decode steps are flat from the
    first call."""
    import torch
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    n, chunk, spent = 0, 8, 0.0
    while spent < min_ms and n < max_calls:
        a.record()
        for i in range(chunk):
            fn(n + i)
        b.record()
        b.synchronize()
        spent += a.elapsed_time(b)
        n += chunk
    return n


def time_steps(fn, steps: int, warmup: int, fill: bool = True) -> list[float]:
    """Per-step device time (ms): a HIP event pair around every call, on the
    stream the library launches on (torch's current stream).  With `fill`
    the steps are queued behind a few ms of other work (_fill_queue), so
    that short steps run back to back; launches of hundreds of us keep the
    queue ahead by themselves and are timed without it (the fill's copy
    kernels slow the MFMA-bound launches after them by 2-3 %)."""
    import torch
    for i in range(warmup):
        fn(i)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    torch.cuda.synchronize()
    if fill:
        _fill_queue(0.15 * steps + 1.0)
    for i, (a, b) in enumerate(evs):
        a.record()
        fn(warmup + i)
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in evs]


def time_block(fn, steps: int, warmup: int, fill: bool = True) -> float:
    """Device time per call (ms) of `steps` back-to-back calls of fn between
    one HIP event pair, after `warmup` untimed calls: the whole-job rate of
    a stream of steps.  The calls are queued behind other work so that the
    GPU never waits for the host between the events: a few ms of copies
    (_fill_queue), or with fill=False two untimed calls of fn itself (for
    launches of hundreds of us, which keep ahead of the host on their own
    and which the copy kernels slow by 2-3 %)."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    if fill:
        _fill_queue(0.15 * steps + 1.0)
    else:
        fn(warmup)
        fn(warmup + 1)
        warmup += 2
    a.record()
    for i in range(steps):
        fn(warmup + i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def _stats(ms: list[float]) -> dict:
    return {"ms_median": statistics.median(ms), "ms_mean": statistics.fmean(ms),
            "ms_min": min(ms), "ms_max": max(ms), "iterations": len(ms)}


def _time_graph_ms(fn, steps: int, warmup: int, settle_ms: float = 0.0) -> float:
    """Device time per call of fn: `steps` calls captured in one HIP graph,
    replayed and timed, so the host's per-call argument checks (tens of us
    for a small launch) stay out of the figure.  With settle_ms the graph is
    first replayed untimed for that much device time and the median of three
    timed replays is taken (see settle)."""
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
    if settle_ms > 0:
        settle(lambda i: g.replay(), settle_ms)
    times = []
    for _ in range(3 if settle_ms > 0 else 1):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        g.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / steps)
    return statistics.median(times)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            return next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")),
                        "unknown")
    except OSError:
        return "unknown"


def _cpu_time(fn, min_reps: int = 3, budget_s: float = 8.0) -> tuple[float, int, float]:
    """Median seconds of fn over at least min_reps passes (more while the
    budget lasts)."""
    import torch
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    times = []
    while len(times) < min_reps or (sum(times) < budget_s and len(times) < 200):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times), sum(times)


def load_traffic(workload: str) -> dict:
    """HBM bytes per step measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    (scaled by the plain-copy calibration), as committed in
    profiles/hbm_traffic.json; null when absent or measured on other sources."""
    try:
        with open(TRAFFIC_JSON) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return {"traffic": None, "traffic_note": "no committed counter profile"}
    e = d.get("workloads", {}).get(workload)
    if e is None:
        return {"traffic": None, "traffic_note": "no committed counter profile"}
    if d.get("sources_sha") != sources_sha():
        return {"traffic": None,
                "traffic_note": "committed counter profile was measured on other kernel sources"}
    return {"traffic": e["traffic_bytes_per_step"],
            "traffic_source": os.path.relpath(TRAFFIC_JSON, ROOT)}


def roofline(bound: str, kernel: str, achieved: float, work: int, ms: float,
             workload: str, timing: str) -> dict:
    peak = HBM_PEAK_GBS if bound == "hbm" else BF16_PEAK_TFLOPS
    r = {"bound": bound, "kernel": kernel, "achieved": round(achieved, 2), "peak": peak,
         "unit": "GB/s" if bound == "hbm" else "TFLOP/s", "frac": round(achieved / peak, 4)}
    r.update(load_traffic(workload))
    r["alg_bytes_per_launch" if bound == "hbm" else "alg_flops_per_launch"] = work
    r["launch_ms"] = round(ms, 5)
    r["launch_timing"] = timing
    return r


# -----------------------------------------------------------------------------
# decode

def bench_decode(w, args, dev, dtype, label: str, cpu_seqs: list[int] | None,
                 kernel: str) -> dict:
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
    kind = dw.plan_kind
    if isinstance(kernel, dict):
        kernel = kernel.get(kind, kernel["split"])
    outs = [torch.empty((w.meta.batch_size, w.hq, w.d), dtype=dtype, device=dev)
            for _ in range(reps)]

    def step(i):
        # the decode step: each sequence's new K/V appended at kv_len - 1,
        # then attention, in one launch (pagedattn_decode_run_append), plus
        # the split-KV merge launch when a split plan cut sequences
        t = inst[i % reps]
        dw.run(t.q, t.pool, kv_scales=t.scales, out=outs[i % reps], append_key=t.k_new,
               append_value=t.v_new)

    # the steps as a stream (the rate reported), then each step between
    # its own event pair (spread statistics; each pair adds ~2-3 us)
    ms = time_block(step, args.steps, args.warmup)
    st = _stats(time_steps(step, args.steps, 1))
    res = {
        "workload": label,
        "ms_per_step": round(ms, 5),
        "per_step_events_ms": {k: round(v, 5) if isinstance(v, float) else v
                               for k, v in st.items()},
        "step_GBps": alg_step / (ms * 1e-3) / 1e9,
        "alg_bytes_step": alg_step,
        "alg_bytes_attn": alg_attn,
        "plan_ms_host": plan_ms,
        "replicas": reps,
        "batch": w.meta.batch_size,
        "kv_tokens": int(w.meta.seq_lens.sum()),
        "split_pages": w.split_pages,
        "plan_kind": kind,
    }
    res["frac"] = res["step_GBps"] / HBM_PEAK_GBS
    res["roofline"] = roofline("hbm", kernel, res["step_GBps"], alg_step, ms, label,
                               DECODE_TIMING)
    if cpu_seqs is not None:
        res["cpu_baseline"] = cpu_decode_baseline(w, inst[0], cpu_seqs, kv_elem)
    del inst, outs
    torch.cuda.empty_cache()
    return res


def cpu_decode_baseline(w, t, rows: list[int], kv_elem: int) -> dict:
    """fp32 oracle decode over the sequences `rows` of the batch (the pool
    pages they use copied to the host beforehand, untimed)."""
    import numpy as np
    import torch

    import oracle as O

    m = w.meta
    parts = [m.kv_indices[m.kv_indptr[b]:m.kv_indptr[b + 1]] for b in rows]
    pages = np.concatenate(parts)
    indptr = np.concatenate([[0], np.cumsum([len(p) for p in parts])]).astype(np.int32)
    idx = torch.from_numpy(pages.astype(np.int64)).to(t.pool.device)
    sub = t.pool.index_select(0, idx).cpu()
    scales = None if t.scales is None else t.scales.index_select(0, idx).cpu()
    q = t.q[rows].float().cpu()
    ind = np.arange(len(pages), dtype=np.int32)
    last = m.kv_last_page_len[rows]
    sec, n, total = _cpu_time(lambda: O.decode(q, sub, indptr, ind, last, scales=scales))
    kv_tok = int(m.seq_lens[rows].astype(np.int64).sum())
    byts = kv_tok * w.hkv * w.d * 2 * kv_elem + len(rows) * w.hq * w.d * 4
    cores = len(os.sched_getaffinity(0))
    subset = "all" if len(rows) == m.batch_size else "a seeded subset of"
    return {
        "value": round(byts / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
        "seconds_median": round(sec, 4),
        "sample": (f"{subset} {len(rows)} of {m.batch_size} sequences of {w.name} "
                   f"({kv_tok} kv tokens), fp32 torch oracle decode, median of {n} passes "
                   f"({total:.1f} s) on {cores} threads of {cpu_model()}"),
    }


# -----------------------------------------------------------------------------
# prefill

def bench_prefill(w, args, dev, dtype, label: str, cpu_seqs: list[int] | None,
                  kernel: str) -> dict:
    import torch

    import pagedattn
    from pagedattn import workloads as W

    flops = W.prefill_flops(w)
    kv_elem = 1 if w.fp8 else 2
    inst_bytes = (w.num_pages * 2 * w.hkv * 16 * w.d * kv_elem
                  + w.meta.nnz * w.hq * w.d * 2 * 2)
    reps = _replicas(inst_bytes, min_total=512 << 20)
    log(f"{label}: {w.meta.nnz} rows, {flops / 1e9:.1f} GFLOP, replicas={reps}")
    inst = []
    for r in range(reps):
        t = W.materialize(w, dev, dtype, seed=w.seed * 100 + r)
        if w.fp8:
            t.pool, t.scales = pagedattn.quantize_pages_e4m3(t.pool)
        inst.append(t)
    ws = torch.zeros(WS_BYTES, dtype=torch.uint8, device=dev)
    pw = pagedattn.BatchPrefillWithPagedKVCacheWrapper(ws, "HND")
    t0 = inst[0]
    torch.cuda.synchronize()
    tp = time.perf_counter()
    pw.plan(t0.qo_indptr, t0.kv_indptr, t0.kv_indices, t0.kv_last_page_len, w.hq, w.hkv, w.d,
            16, q_data_type=dtype, causal=True)
    torch.cuda.synchronize()
    plan_ms = (time.perf_counter() - tp) * 1e3
    outs = [torch.empty_like(t.q) for t in inst]

    def step(i):
        t = inst[i % reps]
        pagedattn.append_paged_kv_cache(t.k_new, t.v_new, t.batch_indices, t.positions, t.pool,
                                        t.kv_indices, t.kv_indptr, t.kv_last_page_len,
                                        kv_layout="HND", kv_scales=t.scales)
        pw.run(t.q, t.pool, kv_scales=t.scales, out=outs[i % reps])

    def attn(i):
        t = inst[i % reps]
        pw.run(t.q, t.pool, kv_scales=t.scales, out=outs[i % reps])

    # steady state: launch times settle after ~100 ms of back-to-back launches
    settle_calls = settle(attn, PREFILL_SETTLE_MS)
    # the launches as a stream (the rate reported), then each launch between
    # its own event pair (spread statistics)
    ms = time_block(attn, args.steps, args.warmup, fill=False)
    step_ms = time_block(step, args.steps, args.warmup, fill=False)
    st = _stats(time_steps(attn, args.steps, 1, fill=False))
    # the same attention with the q-tile list cut on the device by every run
    # (pagedattn_prefill_plan_device: a one-workgroup plan launch ahead of
    # the attention), eagerly and `steps` runs replayed from one HIP graph
    ws_dev = torch.zeros(WS_BYTES, dtype=torch.uint8, device=dev)
    pd = pagedattn.BatchPrefillWithPagedKVCacheWrapper(ws_dev, "HND")
    pd.plan(t0.qo_indptr, t0.kv_indptr, t0.kv_indices, t0.kv_last_page_len, w.hq, w.hkv, w.d,
            16, q_data_type=dtype, causal=True, device_plan=True, max_qo_tokens=int(w.meta.nnz))

    def attn_dev(i):
        t = inst[i % reps]
        pd.run(t.q, t.pool, kv_scales=t.scales, out=outs[i % reps])

    dev_ms = time_block(attn_dev, args.steps, args.warmup, fill=False)
    dev_graph_ms = _time_graph_ms(attn_dev, args.steps, args.warmup, settle_ms=PREFILL_SETTLE_MS)
    # a captured engine step: the list cut once for the step (update_plan,
    # as plan_prefill once per step) and every layer's run reading it
    layers = 32  # Llama-3-8B decoder layers

    def engine_step(i):
        pd.update_plan()
        for layer in range(layers):
            attn_dev(i * layers + layer)

    step_graph_ms = _time_graph_ms(engine_step, 2, 1, settle_ms=PREFILL_SETTLE_MS) / layers
    dropped = int(ws_dev[12:16].view(torch.int32).item())
    res = {
        "workload": label,
        "ms_per_launch": round(ms, 5),
        "per_launch_events_ms": {k: round(v, 5) if isinstance(v, float) else v
                                 for k, v in st.items()},
        "step_ms_per_step": round(step_ms, 5),
        "attn_TFLOPs": flops / (ms * 1e-3) / 1e12,
        "alg_flops_attn": flops,
        "rows": int(w.meta.nnz),
        "kv_tokens": int(w.meta.seq_lens.sum()),
        "plan_ms_host": plan_ms,
        "replicas": reps,
        "timing": f"after {settle_calls} untimed launches ({PREFILL_SETTLE_MS:.0f} ms of device "
                  f"time, where launch times have settled): {PREFILL_TIMING}",
        "device_plan": {"attn_ms_per_launch": round(dev_ms, 5),
                        "attn_TFLOPs": flops / (dev_ms * 1e-3) / 1e12,
                        "graph_ms_per_run": round(dev_graph_ms, 5),
                        "graph_TFLOPs": flops / (dev_graph_ms * 1e-3) / 1e12,
                        "step_graph_ms_per_run": round(step_graph_ms, 5),
                        "step_graph_TFLOPs": flops / (step_graph_ms * 1e-3) / 1e12,
                        "step_graph_layers_per_update": layers,
                        "dropped_tiles": dropped,
                        "note": "attn_*: runs that each cut their q-tile list (a plan launch "
                                "ahead of each); graph_*: such runs, `steps` per graph; "
                                "step_graph_*: one captured engine step = update_plan + 32 "
                                "runs reading its list, per run"},
    }
    res["frac"] = res["attn_TFLOPs"] / BF16_PEAK_TFLOPS
    res["roofline"] = roofline("mfma", kernel, res["attn_TFLOPs"], flops, ms, label,
                               PREFILL_TIMING)
    if cpu_seqs is not None:
        res["cpu_baseline"] = cpu_prefill_baseline(w, inst[0], cpu_seqs)
    del inst, outs, ws_dev
    torch.cuda.empty_cache()
    return res


def cpu_prefill_baseline(w, t, rows: list[int]) -> dict:
    """fp32 oracle prefill of the sequences `rows` (their chunks over their
    whole cached prefixes)."""
    import numpy as np
    import torch

    import oracle as O
    from pagedattn import workloads as W

    m = w.meta
    parts = [m.kv_indices[m.kv_indptr[b]:m.kv_indptr[b + 1]] for b in rows]
    pages = np.concatenate(parts)
    kv_indptr = np.concatenate([[0], np.cumsum([len(p) for p in parts])]).astype(np.int32)
    idx = torch.from_numpy(pages.astype(np.int64)).to(t.pool.device)
    sub = t.pool.index_select(0, idx).cpu()
    scales = None if t.scales is None else t.scales.index_select(0, idx).cpu()
    qo = np.diff(m.qo_indptr)
    q = torch.cat([t.q[int(m.qo_indptr[b]):int(m.qo_indptr[b + 1])] for b in rows]).float().cpu()
    qo_indptr = np.concatenate([[0], np.cumsum(qo[rows])]).astype(np.int32)
    ind = np.arange(len(pages), dtype=np.int32)
    last = m.kv_last_page_len[rows]
    sec, n, total = _cpu_time(
        lambda: O.prefill(q, qo_indptr, sub, kv_indptr, ind, last, causal=True, scales=scales),
        budget_s=4.0)
    sw = dataclasses.replace(w, meta=dataclasses.replace(
        m, qo_indptr=qo_indptr, kv_indptr=kv_indptr, kv_indices=ind, kv_last_page_len=last,
        seq_lens=m.seq_lens[rows]))
    flops = W.prefill_flops(sw)
    cores = len(os.sched_getaffinity(0))
    subset = "all" if len(rows) == m.batch_size else "a seeded subset of"
    return {
        "value": round(flops / sec / 1e9, 2), "unit": "GFLOP/s", "cores": cores, "kind": "port",
        "seconds_median": round(sec, 4),
        "sample": (f"{subset} {len(rows)} of {m.batch_size} sequences of {w.name} "
                   f"({int(qo[rows].sum())} query rows, {flops / 1e9:.1f} GFLOP), fp32 torch "
                   f"oracle prefill, median of {n} passes ({total:.1f} s) on {cores} threads "
                   f"of {cpu_model()}"),
    }


# -----------------------------------------------------------------------------
# device plan, KV write path, calibration

def bench_device_plan(w, dev, dtype, steps: int = 30, warmup: int = 5) -> dict:
    """The same fused decode step with the device-side partition
    (pagedattn_decode_plan_device), eagerly and replayed from a HIP graph,
    and the device metadata builder for the batch."""
    import numpy as np
    import torch

    import pagedattn
    from pagedattn import workloads as W

    alg_step = W.decode_bytes(w, 2, with_append=True)
    reps = _replicas(w.num_pages * 2 * w.hkv * 16 * w.d * 2)  # as the headline step
    inst = [W.materialize(w, dev, dtype, seed=w.seed * 100 + r) for r in range(reps)]
    ws = torch.zeros(WS_BYTES, dtype=torch.uint8, device=dev)
    out = torch.empty((w.meta.batch_size, w.hq, w.d), dtype=dtype, device=dev)
    t0 = inst[0]
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    dw.plan(t0.kv_indptr, t0.kv_indices, t0.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=dtype, device_plan=True)

    def step(t):
        dw.run(t.q, t.pool, out=out, append_key=t.k_new, append_value=t.v_new)

    eager_ms = statistics.median(time_steps(lambda i: step(inst[i % reps]), steps, warmup))
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
    graph1_ms = statistics.median(time_steps(lambda i: graphs[i % reps].replay(), steps, warmup))
    # an engine captures a whole forward (every layer's call) in one graph:
    # `steps` calls in one graph spread the graph launch over them
    deal_graph_ms = _time_graph_ms(lambda i: step(inst[i % reps]), steps, warmup)
    # the engine step as a graph captures it: the step's items dealt once
    # (update_plan, as plan_decode once per step) and then every layer's run
    # reading that deal; per-layer time = the step's time / layers
    layers = 22  # TinyLlama-1.1B decoder layers

    def engine_step(i):
        dw.update_plan()
        for layer in range(layers):
            step(inst[(i * layers + layer) % reps])

    update_ms = _time_graph_ms(lambda i: dw.update_plan(), steps, warmup)
    graph_ms = _time_graph_ms(engine_step, 3, 1) / layers
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
    return {"plan_kind": dw.plan_kind,
            "eager_ms_per_step": eager_ms, "eager_GBps": alg_step / (eager_ms * 1e-3) / 1e9,
            "graph_ms_per_step": graph_ms, "graph_GBps": alg_step / (graph_ms * 1e-3) / 1e9,
            "graph_layers_per_update": layers,
            "update_plan_ms": update_ms,
            "dealing_graph_ms_per_step": deal_graph_ms,
            "dealing_graph_GBps": alg_step / (deal_graph_ms * 1e-3) / 1e9,
            "dealing_graph_steps_per_graph": steps,
            "graph_one_step_ms": graph1_ms,
            "metadata_build_ms": meta_ms,
            "note": "graph_*: one captured engine step = update_plan (the step's items dealt "
                    "once on the device) + 22 layer runs reading that deal, per layer; "
                    "dealing_graph_*: runs that each deal in their prologue, `steps` per graph; "
                    "eager_*: dealing runs launched one by one"}


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
    from pagedattn.metadata import decode_metadata, prefill_metadata

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


def calibration(dev, nbytes: int = 1 << 30, reps: int = 3) -> dict:
    """A plain copy and a plain read of known size: the reference points for
    the HBM byte counters (FETCH_SIZE / WRITE_SIZE)."""
    import torch

    import pagedattn

    src = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    copy_ms = statistics.median(time_steps(lambda i: pagedattn.copy_bytes(dst, src), reps + 2, 1))
    read_ms = statistics.median(time_steps(lambda i: pagedattn.read_bytes(src), reps + 2, 1))
    del src, dst
    torch.cuda.empty_cache()
    return {"copy": {"bytes_read": nbytes, "bytes_written": nbytes, "ms": copy_ms,
                     "GBps": 2 * nbytes / (copy_ms * 1e-3) / 1e9},
            "read": {"bytes_read": nbytes, "ms": read_ms,
                     "GBps": nbytes / (read_ms * 1e-3) / 1e9}}


# -----------------------------------------------------------------------------

# decode kernels per plan kind ("split": head-group work list + merge launch;
# "shared": whole (sequence, KV head) items per CU workgroup, one launch)
DECODE_KERNEL = {
    "c2": "decode step: decode_kernel<64, bf16, append> (each sequence's new K/V written, "
          "then attention) + decode_merge_kernel (split-KV merge)",
    "c2.shared": "decode step: decode_shared_kernel<64, bf16, append> (each sequence's new "
                 "K/V written, then attention; whole (sequence, KV head) items shared by the "
                 "four waves of one workgroup per CU, one launch)",
    "c4": "decode step: decode_kernel<128, bf16, append>, fixed 4096-token split-KV chunks "
          "+ decode_merge_kernel",
    "c4b": "decode step: decode_kernel<128, bf16, append>, planner's balanced split "
           "+ decode_merge_kernel",
    "c5d": "decode step: decode_kernel<128, e4m3 pool, append> + decode_merge_kernel",
    "c5d.shared": "decode step: decode_shared_kernel<128, e4m3 pool, append> (each "
                  "sequence's new K/V written, then attention; whole (sequence, KV head) "
                  "items shared by the four waves of one workgroup per CU, one launch)",
}
PREFILL_KERNEL = {
    "c3": "prefill_kernel<128, bf16> (causal, ragged, paged; bf16 MFMA)",
    "c5p": "prefill_kernel<128, e4m3 pool> (K/V converted to bf16 in LDS; bf16 MFMA, priced "
           "against the bf16 peak)",
}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--config", default="all",
                    help="comma-separated subset of " + ",".join(CONFIGS) + " (default all)")
    ap.add_argument("--no-extra", action="store_true", help="only the headline (c2)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported",
              file=sys.stderr)
        return 2
    args.steps = max(args.steps, 1)
    import torch

    from pagedattn import workloads as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    dtype = torch.bfloat16
    want = set(CONFIGS) if args.config == "all" else set(args.config.split(","))
    if args.no_extra:
        want = {"c2"}
    unknown = want - set(CONFIGS)
    if unknown:
        print(f"bench.py: unknown config(s) {sorted(unknown)}", file=sys.stderr)
        return 2
    cpu = not args.no_cpu
    extra: dict = {}
    steps_n = max(20, args.steps)  # >= 20 timed iterations per configuration

    r = None
    main_w = W.tinyllama_decode(seed=args.seed)
    if "c2" in want:
        r = bench_decode(main_w, args, dev, dtype, "tinyllama_decode",
                         list(range(main_w.meta.batch_size)) if cpu else None,
                         {"split": DECODE_KERNEL["c2"], "shared": DECODE_KERNEL["c2.shared"]})
        log(f"tinyllama_decode: step {r['ms_per_step'] * 1e3:.1f} us = "
            f"{r['step_GBps']:.0f} GB/s ({100 * r['frac']:.1f}% of 8 TB/s); "
            f"{r['per_step_events_ms']['ms_median'] * 1e3:.1f} us median with an event "
            f"pair per step")
    sub = argparse.Namespace(steps=steps_n, warmup=3)
    if "c3" in want:
        pw = W.llama3_8b_prefill(seed=args.seed)
        pr = bench_prefill(pw, sub, dev, dtype, "llama3_8b_prefill",
                           list(range(pw.meta.batch_size)) if cpu else None, PREFILL_KERNEL["c3"])
        log(f"llama3_8b_prefill: {pr['ms_per_launch'] * 1e3:.1f} us = {pr['attn_TFLOPs']:.1f} "
            f"TFLOP/s ({100 * pr['frac']:.1f}% of bf16 peak); device plan "
            f"{pr['device_plan']['attn_ms_per_launch'] * 1e3:.1f} us eager, "
            f"{pr['device_plan']['graph_ms_per_run'] * 1e3:.1f} us from a graph")
        extra["llama3_8b_prefill"] = pr
    if "c4" in want or "c4b" in want:
        lw = W.llama3_8b_long_decode(seed=args.seed)
        if "c4" in want:
            lr = bench_decode(lw, sub, dev, dtype, "llama3_8b_long_decode",
                              [0] if cpu else None, DECODE_KERNEL["c4"])
            log(f"llama3_8b_long_decode: {lr['ms_per_step'] * 1e3:.0f} us = {lr['step_GBps']:.0f} "
                f"GB/s ({100 * lr['frac']:.1f}%)")
            extra["llama3_8b_long_decode"] = lr
        if "c4b" in want:
            lb = bench_decode(dataclasses.replace(lw, split_pages=0), sub, dev, dtype,
                              "llama3_8b_long_decode.balanced", None, DECODE_KERNEL["c4b"])
            log(f"llama3_8b_long_decode (balanced split): {lb['step_GBps']:.0f} GB/s "
                f"({100 * lb['frac']:.1f}%)")
            extra["llama3_8b_long_decode.balanced"] = lb
    if "c5d" in want or "c5p" in want:
        dec5, pre5 = W.llama3_70b_mixed_fp8(seed=args.seed)
        c5 = {}
        if "c5d" in want:
            rng = __import__("numpy").random.default_rng(5)
            rows = sorted(rng.choice(dec5.meta.batch_size, 8, replace=False).tolist())
            d5 = bench_decode(dec5, sub, dev, dtype, "llama3_70b_mixed_fp8.decode",
                              rows if cpu else None,
                              {"split": DECODE_KERNEL["c5d"], "shared": DECODE_KERNEL["c5d.shared"]})
            log(f"llama3_70b_mixed_fp8 decode: {d5['step_GBps']:.0f} GB/s "
                f"({100 * d5['frac']:.1f}%)")
            c5["decode"] = d5
        if "c5p" in want:
            p5 = bench_prefill(pre5, sub, dev, dtype, "llama3_70b_mixed_fp8.prefill",
                               [0] if cpu else None, PREFILL_KERNEL["c5p"])
            log(f"llama3_70b_mixed_fp8 prefill: {p5['attn_TFLOPs']:.1f} TFLOP/s "
                f"({100 * p5['frac']:.1f}% of bf16 peak)")
            c5["prefill"] = p5
        extra["llama3_70b_mixed_fp8"] = c5
    if "devplan" in want:
        dp = bench_device_plan(main_w, dev, dtype)
        log(f"tinyllama_decode (device plan, {dp['plan_kind']}): eager "
            f"{dp['eager_ms_per_step'] * 1e3:.1f} us, "
            f"HIP graph {dp['graph_ms_per_step'] * 1e3:.1f} us per step")
        extra["tinyllama_decode.device_plan"] = dp
    if "kvwrite" in want:
        kw = bench_kv_write(dev)
        log(f"kv write path: e4m3 running-amax append {kw['append_e4m3_amax']['GBps']:.0f} GB/s "
            f"(4096-token chunk); CoW fork {kw['fork_pages']['GBps']:.0f} GB/s")
        extra["kv_write"] = kw
    cal = calibration(dev)
    log(f"calibration: copy {cal['copy']['GBps']:.0f} GB/s, read {cal['read']['GBps']:.0f} GB/s")

    if r is None:  # a profiling subset without the headline
        print(json.dumps({"config_subset": sorted(want), "extra": extra, "calibration": cal}),
              flush=True)
        return 0
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
            "timing": DECODE_TIMING + "; step_stats_ms: an event pair around each step",
        },
        "roofline": r["roofline"],
        "cpu_baseline": r.get("cpu_baseline"),
        "step_stats_ms": r["per_step_events_ms"],
        "extra": extra,
        "calibration": cal,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
