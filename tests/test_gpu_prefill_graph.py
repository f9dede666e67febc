"""Device-planned prefill (pagedattn_prefill_plan_device): the q-tile list is
cut on the device by every run, so a chunked-prefill step needs no host copy
of its metadata.  Outputs and LSE must equal the host plan's bit for bit (the
tiles are the same, only their scheduling differs), tiles past the plan's
capacity are counted, and one whole step -- metadata from the block table,
RoPE + page append, prefill attention -- captured in a HIP graph replays
bit-identical to the same step run eagerly, while the chunk lengths change
between replays, and follows the fp32 oracle."""

import numpy as np
import pytest
import torch

import pagedattn
from pagedattn import ops
from pagedattn import workloads as W
from pagedattn.metadata import prefill_metadata

from paged_cases import (i32, lse_err, max_err, oracle_prefill_rows, prefill_case,
                         random_tables, workspace)

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_FP8 = 3e-2
TOL_LSE = 2e-3

# (cached prefix, new chunk): empty and one-token chunks, partial and exact
# pages, chunks longer than a q-tile, and sequences with no new tokens
EDGE = [(0, 1), (0, 15), (0, 16), (16, 1), (5, 33), (100, 64), (0, 130), (1000, 129),
        (31, 200), (64, 0), (300, 300), (7, 0), (2000, 45)]


def _dropped(ws):
    """q-tiles device-planned runs dropped for capacity (int32 at byte 12)."""
    return int(ws[12:16].view(torch.int32).item())


def _prefill(gpu, meta, pool, q, hq, hkv, d, *, device_plan, causal=True, scales=None,
             ws=None, max_qo_tokens=None, out=None, update=False):
    ws = workspace(gpu) if ws is None else ws
    w = pagedattn.BatchPrefillWithPagedKVCacheWrapper(ws, "HND")
    kw = {}
    if device_plan:
        kw = dict(device_plan=True,
                  max_qo_tokens=meta.nnz if max_qo_tokens is None else max_qo_tokens)
    w.plan(i32(meta.qo_indptr, gpu), i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu),
           i32(meta.kv_last_page_len, gpu), hq, hkv, d, 16, q_data_type=q.dtype, **kw)
    assert w.plan_kind == ("device" if device_plan else "host")
    if update:
        w.update_plan()  # the q-tile list cut once; the run launches none
    if out is None:
        out = torch.full((q.shape[0], hq, d), float("nan"), dtype=q.dtype, device=gpu)
    lse = torch.full((q.shape[0], hq), float("nan"), device=gpu)
    w.run(q, pool, kv_scales=scales, out=out, lse=lse, causal=causal)
    torch.cuda.synchronize()
    return out, lse, ws


def _case(gpu, name):
    if name == "llama3_8b":
        w = W.llama3_8b_prefill(seed=3)
        t = W.materialize(w, gpu)
        return w.meta, t.pool, t.q, w.hq, w.hkv, w.d, None
    if name == "e4m3_70b":
        w = W.llama3_70b_mixed_fp8(seed=3)[1]
        t = W.materialize(w, gpu)
        pool, scales = pagedattn.quantize_pages_e4m3(t.pool)
        return w.meta, pool, t.q, w.hq, w.hkv, w.d, scales
    hq, hkv, d = {"edges_d128": (32, 8, 128), "edges_d64": (32, 4, 64),
                  "edges_odd_heads": (12, 3, 128)}[name]
    computed = [c for c, _ in EDGE]
    chunks = [n for _, n in EDGE]
    meta, pool, q = prefill_case(gpu, computed, chunks, hq, hkv, d, seed=hq + hkv + d)
    return meta, pool, q, hq, hkv, d, None


@pytest.mark.parametrize("name", ["edges_d128", "edges_d64", "edges_odd_heads", "llama3_8b",
                                  "e4m3_70b"])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_device_plan_equals_host_plan(gpu, name, causal):
    meta, pool, q, hq, hkv, d, scales = _case(gpu, name)
    o_h, l_h, _ = _prefill(gpu, meta, pool, q, hq, hkv, d, device_plan=False, causal=causal,
                           scales=scales)
    o_d, l_d, ws = _prefill(gpu, meta, pool, q, hq, hkv, d, device_plan=True, causal=causal,
                            scales=scales)
    assert torch.equal(o_d, o_h)
    assert torch.equal(l_d, l_h)
    assert _dropped(ws) == 0
    # a second run of the same plan (a fresh tile list, the same bits)
    o_d2, l_d2, _ = _prefill(gpu, meta, pool, q, hq, hkv, d, device_plan=True, causal=causal,
                             scales=scales, ws=ws)
    assert torch.equal(o_d2, o_h) and torch.equal(l_d2, l_h)
    # and a run that reads the list update_plan cut ahead of it
    o_u, l_u, ws_u = _prefill(gpu, meta, pool, q, hq, hkv, d, device_plan=True, causal=causal,
                              scales=scales, update=True)
    assert torch.equal(o_u, o_h) and torch.equal(l_u, l_h)
    assert _dropped(ws_u) == 0
    if name in ("edges_d64", "e4m3_70b"):
        # and the oracle, on some rows (the bit equality covers the rest)
        b = len(meta.kv_last_page_len) - 1 if name == "edges_d64" else 0
        q0 = int(meta.qo_indptr[b])
        qo = int(meta.qo_indptr[b + 1]) - q0
        lo, hi = max(0, qo - 40), qo
        ref_o, ref_l = oracle_prefill_rows(meta, pool, q, b, lo, hi, causal, scales)
        rows = list(range(q0 + lo, q0 + hi))
        tol = TOL_FP8 if scales is not None else TOL_BF16
        assert max_err(o_d[rows], ref_o) <= tol
        assert lse_err(l_d[rows], ref_l) <= TOL_LSE


def test_prefill_device_plan_sequence_order_past_1024_tiles(gpu):
    # 1056 q-tiles: more than the device plan orders longest first, so they
    # keep sequence order; the outputs are still the host plan's bits
    n_seq, chunk = 48, 1400  # 22 tiles of 64 tokens each
    computed = [int(x) for x in np.random.default_rng(4).integers(0, 600, n_seq)]
    meta, pool, q = prefill_case(gpu, computed, [chunk] * n_seq, 32, 8, 128, seed=4)
    o_h, l_h, _ = _prefill(gpu, meta, pool, q, 32, 8, 128, device_plan=False)
    o_d, l_d, ws = _prefill(gpu, meta, pool, q, 32, 8, 128, device_plan=True)
    assert torch.equal(o_d, o_h) and torch.equal(l_d, l_h)
    assert _dropped(ws) == 0


def test_prefill_device_plan_capacity_is_counted(gpu):
    # a run with more query tokens than the plan's bound: the tiles past the
    # capacity are skipped (their rows left as they were) and counted; the
    # planned ones are exact
    hq, hkv, d = 32, 8, 128
    computed = [0, 100, 7, 0]
    chunks = [300, 200, 500, 64]
    meta, pool, q = prefill_case(gpu, computed, chunks, hq, hkv, d, seed=9)
    q_tile = 256 // (hq // hkv)
    tiles = sum(-(-n // q_tile) for n in chunks)
    bound = 320  # capacity ceil(320 / 64) + 4 = 9 tiles
    cap = -(-bound // q_tile) + len(chunks)
    assert tiles > cap
    o_h, l_h, _ = _prefill(gpu, meta, pool, q, hq, hkv, d, device_plan=False)
    o_d, l_d, ws = _prefill(gpu, meta, pool, q, hq, hkv, d, device_plan=True,
                            max_qo_tokens=bound)
    assert _dropped(ws) == tiles - cap
    # the first `cap` tiles in sequence order were planned
    planned = []
    for b, n in enumerate(chunks):
        q0 = int(meta.qo_indptr[b])
        for lo in range(0, n, q_tile):
            planned.append((q0 + lo, q0 + min(n, lo + q_tile)))
    done = [r for lo, hi in planned[:cap] for r in range(lo, hi)]
    skipped = [r for lo, hi in planned[cap:] for r in range(lo, hi)]
    assert torch.equal(o_d[done], o_h[done]) and torch.equal(l_d[done], l_h[done])
    assert torch.isnan(o_d[skipped].float()).all()


def _tables_tensor(tables, max_pages, device, fill=-7):
    t = np.full((len(tables), max_pages), fill, dtype=np.int32)
    for b, row in enumerate(tables):
        t[b, :len(row)] = row
    return i32(t, device)


class _PrefillStep:
    """One chunked-prefill step of the engine on fixed buffers: metadata from
    the block table, kv lengths and chunk lengths (device), RoPE of q and the
    new K rows with the page append (one launch), then prefill attention with
    a device plan.  Nothing is read on the host."""

    def __init__(self, gpu, tables, maxp, tokens, hq, hkv, d, table=False):
        self.table = table  # the q-tile list cut once per step (update_plan) for the run
        bsz = len(tables)
        self.bt = _tables_tensor(tables, maxp, gpu)
        self.lens = torch.zeros(bsz, dtype=torch.int32, device=gpu)
        self.new = torch.zeros(bsz, dtype=torch.int32, device=gpu)
        self.buf = ops.new_paged_buffers(bsz, bsz * maxp, tokens, gpu)
        self.q = torch.zeros((tokens, hq, d), dtype=torch.bfloat16, device=gpu)
        self.k = torch.zeros((tokens, hkv, d), dtype=torch.bfloat16, device=gpu)
        self.v = torch.zeros_like(self.k)
        self.out = torch.zeros_like(self.q)
        self.lse = torch.zeros((tokens, hq), dtype=torch.float32, device=gpu)
        self.w = pagedattn.BatchPrefillWithPagedKVCacheWrapper(workspace(gpu), "HND")
        self.w.plan(self.buf.qo_indptr, self.buf.kv_indptr, self.buf.kv_indices,
                    self.buf.kv_last_page_len, hq, hkv, d, 16, causal=True,
                    q_data_type=torch.bfloat16, device_plan=True, max_qo_tokens=tokens)

    def __call__(self, pool):
        pagedattn.build_paged_metadata(self.bt, self.lens, self.new, out=self.buf)
        ops.rope_append_paged_kv_cache(self.q, self.k, self.v, self.buf.batch_indices,
                                       self.buf.positions, pool, self.buf.kv_indices,
                                       self.buf.kv_indptr, self.buf.kv_last_page_len,
                                       kv_layout="HND", rope_scale=1.0, rope_theta=5e5)
        if self.table:
            self.w.update_plan()
        self.w.run(self.q, pool, out=self.out, lse=self.lse)


@pytest.mark.parametrize("table", [False, True])
def test_chunked_prefill_step_graph_replay(gpu, table):
    """The graphed step (with `table`: its q-tile list cut by update_plan
    inside the graph) equals the eager step whose run cuts its own list."""
    hq, hkv, d = 32, 8, 128
    rng = np.random.default_rng(31)
    bsz = 8
    chunk_set = [1, 17, 64, 100, 130, 150, 200, 106]  # 768 tokens per step
    tokens = sum(chunk_set)
    steps = 4
    start = [0, 5, 16, 300, 0, 1000, 31, 64]
    plans = [list(rng.permutation(chunk_set)) for _ in range(steps)]
    final = [s + sum(p[b] for p in plans) for b, s in enumerate(start)]
    tables, num_pages = random_tables(rng, final, extra_pages=2)
    maxp = max(len(t) for t in tables)
    g = torch.Generator(device=gpu)
    g.manual_seed(31)
    pool_g = torch.randn((num_pages, 2, hkv, 16, d), generator=g, device=gpu).to(torch.bfloat16)
    pool_e = pool_g.clone()
    eager = _PrefillStep(gpu, tables, maxp, tokens, hq, hkv, d)
    graphed = _PrefillStep(gpu, tables, maxp, tokens, hq, hkv, d, table=table)
    lens = torch.tensor(start, dtype=torch.int32, device=gpu)
    first = torch.tensor(plans[0], dtype=torch.int32, device=gpu)
    graphed.lens.copy_(lens + first)
    graphed.new.copy_(first)
    # warm up on a side stream, as torch asks before a capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    scratch = pool_g.clone()
    with torch.cuda.stream(s):
        graphed(scratch)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    del scratch
    cg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(cg):
        graphed(pool_g)
    for step in range(steps):
        new = torch.tensor(plans[step], dtype=torch.int32, device=gpu)
        lens += new  # the chunk's tokens are in the cache once appended
        q = torch.randn((tokens, hq, d), generator=g, device=gpu).to(torch.bfloat16)
        k = torch.randn((tokens, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
        v = torch.randn((tokens, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
        for st in (eager, graphed):
            st.lens.copy_(lens)
            st.new.copy_(new)
            st.q.copy_(q)
            st.k.copy_(k)
            st.v.copy_(v)
        cg.replay()
        eager(pool_e)
        torch.cuda.synchronize()
        assert torch.equal(graphed.out, eager.out), step
        assert torch.equal(graphed.lse, eager.lse), step
        assert torch.equal(pool_g, pool_e), step
        assert torch.equal(graphed.buf.qo_indptr.cpu(),
                           torch.tensor(np.concatenate([[0], np.cumsum(plans[step])]),
                                        dtype=torch.int32)), step
    assert _dropped(graphed.w._ws) == 0 and _dropped(eager.w._ws) == 0
    # the last step against the oracle: q as rotated in place, the pool after
    # every append
    lens_h = lens.cpu().tolist()
    chunks = [int(x) for x in plans[-1]]
    meta = prefill_metadata(tables, [n - c for n, c in zip(lens_h, chunks)], chunks)
    for b in (0, 3, 5, 6):
        q0 = int(meta.qo_indptr[b])
        n = chunks[b]
        lo = max(0, n - 24)
        ref_o, ref_l = oracle_prefill_rows(meta, pool_e, eager.q, b, lo, n)
        rows = list(range(q0 + lo, q0 + n))
        assert max_err(eager.out[rows], ref_o) <= TOL_BF16, b
        assert lse_err(eager.lse[rows], ref_l) <= TOL_LSE, b
