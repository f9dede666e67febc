"""Device-side metadata and planner, and a decode step replayed from a HIP
graph.

* build_paged_metadata on the GPU equals the step executor's metadata rules
  (pagedattn.metadata, bit-exact), for decode and chunked-prefill steps;
* a device-planned decode equals the host-planned balanced split bit for bit
  (same partition, same merge order) and the oracle within tolerance, for
  empty, short, long and mixed batches;
* a decode step (metadata build + RoPE + append + attention + merge)
  captured once and replayed over several steps, with the lengths, the
  inputs and the pool changing in place between replays, matches the same
  step run eagerly, every replay."""

import numpy as np
import pytest
import torch

import pagedattn
from pagedattn.metadata import decode_metadata, prefill_metadata

from paged_cases import (decode_case, i32, lse_err, max_err, oracle_decode, random_tables,
                         require_fixed_chunks, require_shared_plans, run_decode, workspace)

pytestmark = pytest.mark.gpu


def _tables_tensor(tables, max_pages, device, fill=-7):
    t = np.full((len(tables), max_pages), fill, dtype=np.int32)
    for b, row in enumerate(tables):
        t[b, :len(row)] = row
    return i32(t, device)


@pytest.mark.parametrize("seed", [0, 1])
def test_build_paged_metadata_decode(gpu, seed):
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, 700, size=57).tolist()
    lens[3] = 16
    lens[4] = 32  # page-aligned lengths: the table is cut, not passed whole
    tables, _ = random_tables(rng, [n + 40 for n in lens])  # rows longer than needed
    maxp = max(len(t) for t in tables)
    bt = _tables_tensor(tables, maxp, gpu)
    got = pagedattn.build_paged_metadata(bt, i32(lens, gpu))
    want = decode_metadata(tables, lens)
    assert np.array_equal(got.kv_indptr.cpu().numpy(), want.kv_indptr)
    n = int(want.kv_indptr[-1])
    assert np.array_equal(got.kv_indices[:n].cpu().numpy(), want.kv_indices)
    assert np.array_equal(got.kv_last_page_len.cpu().numpy(), want.kv_last_page_len)
    assert np.array_equal(got.qo_indptr.cpu().numpy(), want.qo_indptr)
    assert np.array_equal(got.batch_indices.cpu().numpy(), want.batch_indices)
    assert np.array_equal(got.positions.cpu().numpy(), want.positions)


def test_build_paged_metadata_prefill(gpu):
    rng = np.random.default_rng(2)
    computed = [0, 16, 35, 100, 0, 7]
    chunks = [17, 1, 64, 29, 0, 512]
    lens = [c + n for c, n in zip(computed, chunks)]
    tables, _ = random_tables(rng, [n + 20 for n in lens])
    maxp = max(len(t) for t in tables)
    bt = _tables_tensor(tables, maxp, gpu)
    got = pagedattn.build_paged_metadata(bt, i32(lens, gpu), i32(chunks, gpu))
    want = prefill_metadata(tables, computed, chunks)
    for name in ("kv_indptr", "kv_last_page_len", "qo_indptr", "batch_indices", "positions"):
        assert np.array_equal(getattr(got, name).cpu().numpy(), getattr(want, name)), name
    n = int(want.kv_indptr[-1])
    assert np.array_equal(got.kv_indices[:n].cpu().numpy(), want.kv_indices)


def test_build_paged_metadata_overflow_is_counted(gpu):
    tables = [[1, 2], [3, 4, 5]]
    bt = _tables_tensor(tables, 3, gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    # sequence 0 needs 4 pages but its row has 3 columns; indices capacity 4 < 3 + 2
    out = pagedattn.ops.new_paged_buffers(2, 4, 2, gpu)
    pagedattn.build_paged_metadata(bt, i32([60, 20], gpu), out=out, error_flag=err)
    assert out.kv_indptr.cpu().tolist() == [0, 3, 5]
    assert out.kv_indices.cpu().tolist() == [1, 2, -7, 3]
    assert int(err.item()) == 2


def _meta_closed_form(tables, max_pages, lens, new_lens, idx_cap, tok_cap):
    """The outputs and the error count of build_paged_metadata written out:
    rows cut to max_pages pages, outputs past a capacity dropped, one count
    per cut row and one per sequence with dropped outputs."""
    pages = [min(-(-L // 16), max_pages) for L in lens]
    nt = [1] * len(lens) if new_lens is None else [min(max(n, 0), max(L, 0))
                                                   for n, L in zip(new_lens, lens)]
    indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int64)
    qo = np.concatenate([[0], np.cumsum(nt)]).astype(np.int64)
    idx = np.concatenate([np.asarray(t[:p], np.int64) for t, p in zip(tables, pages)] +
                         [np.zeros(0, np.int64)])
    bi = np.repeat(np.arange(len(lens)), nt)
    pos = np.concatenate([np.arange(L - n, L) for L, n in zip(lens, nt)] + [np.zeros(0, np.int64)])
    cut = sum(-(-L // 16) > p for L, p in zip(lens, pages))
    dropped = sum((p > 0 and indptr[b] + p > idx_cap) or
                  (new_lens is not None and n > 0 and qo[b] + n > tok_cap)
                  for b, (p, n) in enumerate(zip(pages, nt)))
    last = [(L - 1) % 16 + 1 if L > 0 else 16 for L in lens]
    return indptr, idx, last, qo, bi, pos, cut + dropped


@pytest.mark.parametrize("bsz", [1000, 1100])  # one launch up to 1024 sequences, two above
@pytest.mark.parametrize("prefill", [False, True])
def test_build_paged_metadata_large_batch(gpu, bsz, prefill):
    """Batches on both launch shapes: equal to the host metadata rules
    (pagedattn.metadata) when nothing is cut, and with rows cut to max_pages
    and capacities too small, equal to the closed form with one error count
    per cut row and per sequence with dropped outputs."""
    rng = np.random.default_rng(bsz + prefill)
    lens = rng.integers(1, 300, size=bsz).tolist()
    new = rng.integers(1, 40, size=bsz).tolist() if prefill else None
    if prefill:
        new = [min(n, L) for n, L in zip(new, lens)]
    tables, _ = random_tables(rng, [L + 16 for L in lens])
    maxp = max(len(t) for t in tables)
    bt = _tables_tensor(tables, maxp, gpu)
    new_t = i32(new, gpu) if prefill else None
    got = pagedattn.build_paged_metadata(bt, i32(lens, gpu), new_t)
    want = (prefill_metadata(tables, [L - n for L, n in zip(lens, new)], new) if prefill
            else decode_metadata(tables, lens))
    for name in ("kv_indptr", "kv_last_page_len", "qo_indptr", "batch_indices", "positions"):
        assert np.array_equal(getattr(got, name).cpu().numpy(), getattr(want, name)), name
    n = int(want.kv_indptr[-1])
    assert np.array_equal(got.kv_indices[:n].cpu().numpy(), want.kv_indices)

    # cut rows (lengths past max_pages pages) and capacities below the need
    lens2 = list(lens)
    for b in (3, 500, bsz - 1):
        lens2[b] = 16 * maxp + 37
    new2 = None
    if prefill:
        new2 = [min(n, L) for n, L in zip(new, lens2)]
    pages = [min(-(-L // 16), maxp) for L in lens2]
    idx_cap = int(sum(pages) * 0.9)
    tok_cap = int(sum(new2) * 0.8) if prefill else bsz
    out = pagedattn.ops.new_paged_buffers(bsz, idx_cap, tok_cap, gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    pagedattn.build_paged_metadata(bt, i32(lens2, gpu), i32(new2, gpu) if prefill else None,
                                   out=out, error_flag=err)
    padded = [list(t) + [-7] * (maxp - len(t)) for t in tables]  # the table tensor's rows
    indptr, idx, last, qo, bi, pos, count = _meta_closed_form(padded, maxp, lens2, new2,
                                                               idx_cap, tok_cap)
    assert np.array_equal(out.kv_indptr.cpu().numpy(), indptr)
    assert np.array_equal(out.kv_indices.cpu().numpy(), idx[:idx_cap])
    assert np.array_equal(out.kv_last_page_len.cpu().numpy(), last)
    if prefill:
        assert np.array_equal(out.qo_indptr.cpu().numpy(), qo)
    ntok = min(tok_cap, len(bi))
    assert np.array_equal(out.batch_indices[:ntok].cpu().numpy(), bi[:ntok])
    assert np.array_equal(out.positions[:ntok].cpu().numpy(), pos[:ntok])
    assert int(err.item()) == count and count > 3


def _device_plan_run(gpu, meta, pool, q, hq, hkv, d, kv_scales=None):
    w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(workspace(gpu), "HND")
    w.plan(i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu), i32(meta.kv_last_page_len, gpu),
           hq, hkv, d, 16, q_data_type=q.dtype, device_plan=True)
    out, lse = w.run(q, pool, kv_scales=kv_scales, return_lse=True)
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.parametrize("name,lens,hq,hkv,d", [
    ("tinyllama", list(np.random.default_rng(5).integers(256, 2049, 256)), 32, 4, 64),
    ("long", [40000, 3, 70000, 16, 123457, 9000, 1, 17], 32, 8, 128),
    ("empties", [0, 5, 0, 0, 300, 0], 32, 8, 128),
    ("single", [1], 8, 8, 128),
    ("mixed_g8", list(np.random.default_rng(6).integers(1, 9000, 40)), 64, 8, 128),
])
def test_device_plan_equals_host_plan(gpu, name, lens, hq, hkv, d, monkeypatch):
    # the device partition cuts equal page shares; the host planner's
    # balanced split does the same with no per-item charge (a split plan:
    # shared-item plans are another partition)
    monkeypatch.setenv("PAGEDATTN_DECODE_ITEM_COST", "0")
    monkeypatch.setenv("PAGEDATTN_DECODE_SHARED", "0")
    lens = [int(x) for x in lens]
    meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=len(lens))
    got, got_lse = _device_plan_run(gpu, meta, pool, q, hq, hkv, d)
    want, want_lse = run_decode(gpu, meta, pool, q, hq, hkv, d, split_pages=0)
    assert torch.equal(got, want)
    assert torch.equal(got_lse, want_lse)
    rows = [b for b in range(len(lens)) if lens[b] <= 20000][:24]
    ref, ref_lse = oracle_decode(meta, pool, q, batch=rows)
    assert max_err(got, ref, rows) < 2e-2
    assert lse_err(got_lse, ref_lse, rows) < 2e-2


@pytest.mark.parametrize("cost", ["6", "40"])
@pytest.mark.parametrize("name,lens,hq,hkv,d", [
    ("tinyllama", list(np.random.default_rng(5).integers(256, 2049, 256)), 32, 4, 64),
    ("empties", [0, 5, 0, 0, 300, 0, 17, 0], 32, 8, 128),
    ("mixed_g8", list(np.random.default_rng(6).integers(1, 9000, 40)), 64, 8, 128),
])
def test_device_plan_item_cost(gpu, monkeypatch, cost, name, lens, hq, hkv, d):
    # the device split with a per-segment charge (header units before each
    # (sequence, head group) segment) is still a partition: oracle answer,
    # and the host plan's answer to the rounding of the merges
    monkeypatch.setenv("PAGEDATTN_DECODE_ITEM_COST", cost)
    monkeypatch.setenv("PAGEDATTN_DECODE_SHARED", "0")
    lens = [int(x) for x in lens]
    meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=len(lens) + 1)
    got, got_lse = _device_plan_run(gpu, meta, pool, q, hq, hkv, d)
    want, want_lse = run_decode(gpu, meta, pool, q, hq, hkv, d, split_pages=0)
    assert float((got.float() - want.float()).abs().max()) <= 1e-2
    rows = [b for b in range(len(lens)) if lens[b] <= 20000][:24]
    ref, ref_lse = oracle_decode(meta, pool, q, batch=rows)
    assert max_err(got, ref, rows) < 2e-2
    assert lse_err(got_lse, ref_lse, rows) < 2e-2


def test_device_plan_e4m3(gpu, monkeypatch):
    monkeypatch.setenv("PAGEDATTN_DECODE_ITEM_COST", "0")
    monkeypatch.setenv("PAGEDATTN_DECODE_SHARED", "0")
    lens = [int(x) for x in np.random.default_rng(7).integers(1, 8192, 32)]
    meta, pool, q = decode_case(gpu, lens, 64, 8, 128, seed=7)
    q8, scales = pagedattn.quantize_pages_e4m3(pool)
    got, got_lse = _device_plan_run(gpu, meta, q8, q, 64, 8, 128, kv_scales=scales)
    want, want_lse = run_decode(gpu, meta, q8, q, 64, 8, 128, split_pages=0, kv_scales=scales)
    assert torch.equal(got, want) and torch.equal(got_lse, want_lse)


class _Step:
    """One engine decode step on fixed buffers: metadata from the block table
    and lengths, then RoPE + append + attention (+ merge) in the fused
    launch."""

    def __init__(self, gpu, tables, maxp, hq, hkv, d, graph, table=False):
        self.table = table  # deal the items once per step (update_plan) for the runs
        self.bsz = len(tables)
        self.bt = _tables_tensor(tables, maxp, gpu)
        self.lens = torch.zeros(self.bsz, dtype=torch.int32, device=gpu)
        self.buf = pagedattn.ops.new_paged_buffers(self.bsz, self.bsz * maxp, self.bsz, gpu)
        self.q = torch.zeros((self.bsz, hq, d), dtype=torch.bfloat16, device=gpu)
        self.k = torch.zeros((self.bsz, hkv, d), dtype=torch.bfloat16, device=gpu)
        self.v = torch.zeros_like(self.k)
        self.out = torch.zeros_like(self.q)
        kw = {}
        if graph:
            kw = dict(use_cuda_graph=True, paged_kv_indptr_buffer=self.buf.kv_indptr,
                      paged_kv_indices_buffer=self.buf.kv_indices,
                      paged_kv_last_page_len_buffer=self.buf.kv_last_page_len)
        self.w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(workspace(gpu), "HND", **kw)
        self.w.plan(self.buf.kv_indptr, self.buf.kv_indices, self.buf.kv_last_page_len, hq, hkv,
                    d, 16, q_data_type=torch.bfloat16, device_plan=True)

    def __call__(self, pool):
        pagedattn.build_paged_metadata(self.bt, self.lens, out=self.buf)
        if self.table:
            self.w.update_plan()
        self.w.run(self.q, pool, out=self.out, append_key=self.k, append_value=self.v,
                   rope=(1.0, 5e5), positions=self.buf.positions)


@pytest.mark.parametrize("bsz,hq,hkv,d,kind,table", [
    (48, 32, 8, 128, "device", False),           # 384 items: the split device partition
    (48, 32, 8, 128, "device", True),            # (update_plan is a no-op there)
    (128, 32, 8, 128, "device_shared", False),   # 1024 items: whole items dealt on the device
    (256, 32, 4, 64, "device_shared", False),    # the TinyLlama batch shape
    (128, 32, 8, 128, "device_shared", True),    # dealt once per step by update_plan
    (256, 32, 4, 64, "device_shared", True),
])
def test_decode_step_graph_replay(gpu, bsz, hq, hkv, d, kind, table):
    """The graphed step (with `table`: metadata, update_plan and the run
    captured together) equals the eager step that deals in every run, bit
    for bit, every replay."""
    if kind == "device_shared":
        require_shared_plans()
        require_fixed_chunks()
    rng = np.random.default_rng(11)
    start = [int(x) for x in rng.integers(1, 3000, bsz)]
    start[0], start[1] = 15, 16  # crosses a page boundary in the first replays
    steps = 6
    tables, num_pages = random_tables(rng, [n + steps for n in start], extra_pages=2)
    maxp = max(len(t) for t in tables)
    g = torch.Generator(device=gpu)
    g.manual_seed(11)
    pool_g = torch.randn((num_pages, 2, hkv, 16, d), generator=g, device=gpu).to(torch.bfloat16)
    pool_e = pool_g.clone()
    eager = _Step(gpu, tables, maxp, hq, hkv, d, graph=False)
    graphed = _Step(gpu, tables, maxp, hq, hkv, d, graph=True, table=table)
    assert eager.w.plan_kind == graphed.w.plan_kind == kind
    lens0 = torch.tensor(start, dtype=torch.int32, device=gpu)
    graphed.lens.copy_(lens0)
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
    lens = lens0.clone()
    for step in range(steps):
        lens += 1  # each step appends one token per sequence
        for st in (eager, graphed):
            st.lens.copy_(lens)
        q = torch.randn((len(start), hq, d), generator=g, device=gpu).to(torch.bfloat16)
        k = torch.randn((len(start), hkv, d), generator=g, device=gpu).to(torch.bfloat16)
        v = torch.randn((len(start), hkv, d), generator=g, device=gpu).to(torch.bfloat16)
        for st in (eager, graphed):
            st.q.copy_(q)
            st.k.copy_(k)
            st.v.copy_(v)
        cg.replay()
        eager(pool_e)
        torch.cuda.synchronize()
        assert torch.equal(graphed.out, eager.out), step
        assert torch.equal(pool_g, pool_e), step
        assert torch.equal(graphed.buf.positions, lens - 1)
    # and the eager step itself follows the oracle on the final state
    meta = decode_metadata(tables, lens.cpu().tolist())
    rows = list(range(0, len(start), 4))
    qr = eager.q.clone()
    # the fused launch rotated q in registers only: rotate a copy for the oracle
    from pagedattn import ops
    ops.apply_rope_pos_ids_inplace(qr, torch.zeros_like(eager.k), i32(meta.positions, gpu),
                                   rope_scale=1.0, rope_theta=5e5)
    ref, _ = oracle_decode(meta, pool_e, qr, batch=rows)
    assert max_err(eager.out, ref, rows) < 2e-2


@pytest.mark.parametrize("name,lens,hq,hkv,d,fp8", [
    ("tinyllama", list(np.random.default_rng(21).integers(1, 2049, 300)), 32, 4, 64, False),
    ("empties", [0, 0, 3] + list(np.random.default_rng(22).integers(1, 700, 260)) + [0],
     32, 4, 64, False),
    ("skewed", [60000] + list(np.random.default_rng(23).integers(1, 300, 300)), 16, 4, 64, False),
    ("e4m3_d128", list(np.random.default_rng(24).integers(1, 8193, 128)), 64, 8, 128, True),
    ("bf16_d128", list(np.random.default_rng(25).integers(1, 3000, 160)), 32, 8, 128, False),
])
def test_device_shared_plan(gpu, name, lens, hq, hkv, d, fp8):
    """The device-dealt shared-item partition: one launch, repeated runs
    bit-identical, outputs and lse against the oracle, faults counter zero."""
    require_shared_plans()
    require_fixed_chunks()
    lens = [int(x) for x in lens]
    meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=len(lens) + 3)
    scales = None
    if fp8:
        pool, scales = pagedattn.quantize_pages_e4m3(pool)
    ws = workspace(gpu)
    w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    w.plan(i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu), i32(meta.kv_last_page_len, gpu),
           hq, hkv, d, 16, q_data_type=q.dtype, device_plan=True)
    assert w.plan_kind == "device_shared"
    out, lse = w.run(q, pool, kv_scales=scales, return_lse=True)
    out2, lse2 = w.run(q, pool, kv_scales=scales, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    assert int(ws[8:12].view(torch.int32).item()) == 0
    rows = sorted({0, len(lens) - 1, int(np.argmax(lens)), int(np.argmin(lens))} |
                  set(range(1, len(lens), max(1, len(lens) // 12))))
    rows = [b for b in rows if 0 < lens[b] <= 20000] + ([int(np.argmax(lens))]
                                                         if name == "skewed" else [])
    ref, ref_lse = oracle_decode(meta, pool, q, batch=rows, scales=scales)
    tol = 3e-2 if fp8 else 2e-2
    assert max_err(out, ref, rows) <= tol
    assert lse_err(lse, ref_lse, rows) <= 2e-3
    for b in range(len(lens)):
        if lens[b] == 0:
            assert torch.all(out[b] == 0) and torch.all(torch.isinf(lse[b]))


@pytest.mark.parametrize("name,lens,hq,hkv,d,fp8", [
    ("tinyllama", list(np.random.default_rng(21).integers(1, 2049, 300)), 32, 4, 64, False),
    ("empties", [0, 0, 3] + list(np.random.default_rng(22).integers(1, 700, 260)) + [0],
     32, 4, 64, False),
    ("e4m3_d128", list(np.random.default_rng(24).integers(1, 8193, 128)), 64, 8, 128, True),
    ("max_batch", list(np.random.default_rng(26).integers(1, 400, 512)), 32, 4, 64, False),
])
def test_device_shared_table_equals_dealing(gpu, name, lens, hq, hkv, d, fp8):
    """update_plan deals the items once into the workspace; the runs that
    read that table give the bits of runs that deal in their prologue, and
    the table follows the metadata of each update."""
    require_shared_plans()
    require_fixed_chunks()
    lens = [int(x) for x in lens]
    meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=len(lens) + 5)
    scales = None
    if fp8:
        pool, scales = pagedattn.quantize_pages_e4m3(pool)
    ws = workspace(gpu)
    w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    indptr, last = i32(meta.kv_indptr, gpu), i32(meta.kv_last_page_len, gpu)
    w.plan(indptr, i32(meta.kv_indices, gpu), last, hq, hkv, d, 16, q_data_type=q.dtype,
           device_plan=True)
    assert w.plan_kind == "device_shared"
    want, want_lse = w.run(q, pool, kv_scales=scales, return_lse=True)
    w.update_plan()
    got, got_lse = w.run(q, pool, kv_scales=scales, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(got_lse, want_lse)
    assert int(ws[8:12].view(torch.int32).item()) == 0
    # the same plan on other metadata of the batch: a fresh deal per update,
    # and the new plan() drops the table (runs deal on their own again)
    lens2 = [max(0, n - 17) for n in lens]
    meta2, pool2, q2 = decode_case(gpu, lens2, hq, hkv, d, seed=len(lens) + 6)
    if fp8:
        pool2, scales = pagedattn.quantize_pages_e4m3(pool2)
    indptr.copy_(i32(meta2.kv_indptr, gpu))
    last.copy_(i32(meta2.kv_last_page_len, gpu))
    ind2 = i32(meta2.kv_indices, gpu)
    w2 = pagedattn.BatchDecodeWithPagedKVCacheWrapper(workspace(gpu), "HND")
    w2.plan(indptr, ind2, last, hq, hkv, d, 16, q_data_type=q.dtype, device_plan=True)
    want2, want2_lse = w2.run(q2, pool2, kv_scales=scales, return_lse=True)
    w.plan(indptr, ind2, last, hq, hkv, d, 16, q_data_type=q.dtype, device_plan=True)
    w.update_plan()
    got2, got2_lse = w.run(q2, pool2, kv_scales=scales, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(got2, want2) and torch.equal(got2_lse, want2_lse)
    rows = sorted({0, len(lens2) - 1, int(np.argmax(lens2))} |
                  set(range(1, len(lens2), max(1, len(lens2) // 10))))
    rows = [b for b in rows if lens2[b] > 0]
    ref, ref_lse = oracle_decode(meta2, pool2, q2, batch=rows, scales=scales)
    tol = 3e-2 if fp8 else 2e-2
    assert max_err(got2, ref, rows) < tol
