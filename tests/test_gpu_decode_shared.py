"""GPU parity of the shared-item decode partition (whole (sequence, KV head)
items per CU-sized workgroup, the four waves of the workgroup claiming the
items' page pairs, states merged in LDS, one launch) against the fp32 CPU
oracle, at the bounds of the bf16 and e4m3 decode tests.  The partition is
forced with PAGEDATTN_DECODE_SHARED=1 wherever the default would not take
it, and every test checks that the plan holds it.  By default wave w takes
the pairs w, w + 4, ... of its workgroup, so repeated runs are bit-identical
(FlashInfer's decode, which this replaces, is deterministic);
PAGEDATTN_DECODE_DETERMINISTIC=0 lets the waves claim pairs in arrival
order, and those runs agree to the last bits."""

import numpy as np
import pytest
import torch

import oracle as O
import pagedattn
from pagedattn import workloads as W

from paged_cases import (decode_case, i32, log2_max_jumps, lse_err, max_err, oracle_decode,
                         rel_err, require_fixed_chunks, require_shared_plans,
                         scale_keys_by_page, workspace)

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_FP8 = 3e-2
TOL_LSE = 2e-3
TOL_REL_BF16 = 2e-2

EDGE_LENS = [1, 2, 15, 16, 17, 31, 32, 33, 47, 48, 64, 100, 255, 256, 257, 700]


@pytest.fixture
def shared(monkeypatch):
    monkeypatch.setenv("PAGEDATTN_DECODE_SHARED", "1")


@pytest.fixture
def deterministic(monkeypatch):
    # fixed chunk assignment (the default, set explicitly): the states merged
    # per item, and so the output bits, do not depend on timing
    monkeypatch.setenv("PAGEDATTN_DECODE_DETERMINISTIC", "1")


@pytest.fixture
def arrival(monkeypatch):
    # chunks claimed in arrival order through the workgroup's LDS counter
    monkeypatch.setenv("PAGEDATTN_DECODE_DETERMINISTIC", "0")


def _faults(ws):
    """Merge-slot waits of shared-item runs that gave up (int32 2 of the
    workspace header): zero in every consistent run."""
    return int(ws[8:12].view(torch.int32).item())


def _plan(gpu, meta, hq, hkv, d, dtype, ws=None, kind="shared"):
    ws = workspace(gpu) if ws is None else ws
    w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    w.plan(i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu), i32(meta.kv_last_page_len, gpu),
           hq, hkv, d, 16, q_data_type=dtype, split_pages=0)
    assert w.plan_kind == kind
    return w


@pytest.mark.parametrize("hq,hkv,d", [(32, 4, 64), (32, 8, 64), (8, 8, 64), (16, 2, 64),
                                       (64, 8, 64), (16, 1, 64), (32, 8, 128), (64, 8, 128),
                                       (8, 1, 128)])
def test_shared_edge_lengths(gpu, shared, hq, hkv, d):
    meta, pool, q = decode_case(gpu, EDGE_LENS, hq, hkv, d, seed=hq + hkv + d)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    w = _plan(gpu, meta, hq, hkv, d, q.dtype)
    out, lse = w.run(q, pool, return_lse=True)
    torch.cuda.synchronize()
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE


@pytest.mark.parametrize("hq,hkv", [(64, 8), (32, 4)])
def test_shared_e4m3_head_dim_128(gpu, shared, hq, hkv):
    # the 70B-shaped decode's partition: e4m3 pool at head_dim 128
    lens = EDGE_LENS + [int(x) for x in np.random.default_rng(hq).integers(1, 3000, 40)]
    meta, pool16, q = decode_case(gpu, lens, hq, hkv, 128, seed=hq + 1)
    pool8, scales = pagedattn.quantize_pages_e4m3(pool16)
    ref_o, ref_l = oracle_decode(meta, pool8, q, scales=scales)
    ws = workspace(gpu)
    out, lse = _plan(gpu, meta, hq, hkv, 128, q.dtype, ws=ws).run(q, pool8, kv_scales=scales,
                                                                   return_lse=True)
    torch.cuda.synchronize()
    assert max_err(out, ref_o) <= TOL_FP8
    assert lse_err(lse, ref_l) <= TOL_LSE
    assert _faults(ws) == 0


def test_shared_eight_items_per_workgroup(gpu, shared):
    # 2048 one-chunk items over 256 workgroups: eight items per workgroup,
    # more than the LDS slots (four at head_dim 64), so every slot is reused
    lens = [64] * 512
    meta, pool, q = decode_case(gpu, lens, 32, 4, 64, seed=7)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    w = _plan(gpu, meta, 32, 4, 64, q.dtype)
    out, lse = w.run(q, pool, return_lse=True)
    torch.cuda.synchronize()
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_shared_ragged_batch(gpu, shared):
    require_fixed_chunks()
    # several items of different lengths per workgroup, including items of a
    # single chunk next to items that all four waves share; the default
    # assignment is fixed, so repeated runs are bit-identical
    lens = [int(x) for x in np.random.default_rng(9).integers(1, 900, 400)]
    meta, pool, q = decode_case(gpu, lens, 32, 4, 64, seed=9)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    ws = workspace(gpu)
    w = _plan(gpu, meta, 32, 4, 64, q.dtype, ws=ws)
    out, lse = w.run(q, pool, return_lse=True)
    torch.cuda.synchronize()
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE
    for _ in range(3):
        out2, lse2 = w.run(q, pool, return_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(out2, out)
        assert torch.equal(lse2, lse)
    assert _faults(ws) == 0


def test_shared_arrival_order_runs_agree(gpu, shared, arrival):
    # chunks claimed in arrival order: runs may differ in the last bits only
    lens = [int(x) for x in np.random.default_rng(9).integers(1, 900, 400)]
    meta, pool, q = decode_case(gpu, lens, 32, 4, 64, seed=9)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    w = _plan(gpu, meta, 32, 4, 64, q.dtype)
    out, lse = w.run(q, pool, return_lse=True)
    out2, lse2 = w.run(q, pool, return_lse=True)
    torch.cuda.synchronize()
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE
    assert float((out2.float() - out.float()).abs().max()) <= 1e-2
    assert float((lse2 - lse).abs().max()) <= 1e-4


def test_shared_deterministic_runs_are_bit_identical(gpu, shared, deterministic):
    lens = [int(x) for x in np.random.default_rng(9).integers(1, 900, 400)]
    meta, pool, q = decode_case(gpu, lens, 32, 4, 64, seed=9)
    w = _plan(gpu, meta, 32, 4, 64, q.dtype)
    out, lse = w.run(q, pool, return_lse=True)
    out2, lse2 = w.run(q, pool, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    assert torch.equal(lse, lse2)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_shared_fp16_and_e4m3(gpu, shared):
    meta, pool, q = decode_case(gpu, EDGE_LENS, 32, 4, 64, dtype=torch.float16, seed=11)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    out, lse = _plan(gpu, meta, 32, 4, 64, q.dtype).run(q, pool, return_lse=True)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE
    meta, pool16, q = decode_case(gpu, EDGE_LENS, 32, 4, 64, seed=21)
    pool8, scales = pagedattn.quantize_pages_e4m3(pool16)
    ref_o, ref_l = oracle_decode(meta, pool8, q, scales=scales)
    out, lse = _plan(gpu, meta, 32, 4, 64, q.dtype).run(q, pool8, kv_scales=scales,
                                                        return_lse=True)
    torch.cuda.synchronize()
    assert max_err(out, ref_o) <= TOL_FP8
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_shared_empty_sequence_and_bad_page(gpu, shared):
    # a sequence with no pages gets zeros and lse = -inf; an out-of-range
    # page id reads as an empty page and the other rows stay exact
    from types import SimpleNamespace
    d, hq, hkv = 64, 32, 4
    meta = SimpleNamespace(kv_indptr=np.array([0, 3, 3, 4], np.int32),
                           kv_indices=np.array([6, 2, 0, 4], np.int32),
                           kv_last_page_len=np.array([8, 1, 5], np.int32))
    g = torch.Generator(device=gpu)
    g.manual_seed(1)
    pool = torch.randn((8, 2, hkv, 16, d), generator=g, device=gpu).to(torch.bfloat16)
    q = torch.randn((3, hq, d), generator=g, device=gpu).to(torch.bfloat16)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    out, lse = _plan(gpu, meta, hq, hkv, d, q.dtype).run(q, pool, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out[1].float().cpu(), torch.zeros(hq, d))
    assert bool(torch.isinf(lse[1]).all())
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE
    meta, pool, q = decode_case(gpu, [40, 40, 40], 32, 4, 64, seed=4)
    bad = meta.kv_indices.copy()
    bad[meta.kv_indptr[1]] = pool.shape[0] + 1000
    ws = workspace(gpu)
    w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    w.plan(i32(meta.kv_indptr, gpu), i32(bad, gpu), i32(meta.kv_last_page_len, gpu), 32, 4, 64,
           16, q_data_type=torch.bfloat16)
    assert w.plan_kind == "shared"
    out = w.run(q, pool)
    ref_o, _ = oracle_decode(meta, pool, q)
    assert torch.isfinite(out.float()).all()
    assert max_err(out, ref_o, rows=[0, 2]) <= TOL_BF16


@pytest.mark.parametrize("fp8", [False, True])
def test_shared_fused_append_equals_separate(gpu, shared, deterministic, fp8):
    # one launch (append at kv_len - 1 + attention) == append kernel + decode
    d, hq, hkv = 64, 32, 4
    lens = EDGE_LENS + [int(x) for x in np.random.default_rng(35).integers(1, 900, 300)]
    meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=33)
    g = torch.Generator(device=gpu)
    g.manual_seed(34)
    kn = torch.randn((len(lens), hkv, d), generator=g, device=gpu).to(torch.bfloat16) * 3
    vn = torch.randn((len(lens), hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    scales = None
    if fp8:
        pool, scales = pagedattn.quantize_pages_e4m3(pool)
    pa_, pb_ = pool.clone(), pool.clone()
    pagedattn.append_paged_kv_cache(kn, vn, i32(meta.batch_indices, gpu),
                                    i32(meta.positions, gpu), pa_, i32(meta.kv_indices, gpu),
                                    i32(meta.kv_indptr, gpu), i32(meta.kv_last_page_len, gpu),
                                    kv_layout="HND", kv_scales=scales)
    w = _plan(gpu, meta, hq, hkv, d, torch.bfloat16)
    o_sep, l_sep = w.run(q, pa_, kv_scales=scales, return_lse=True)
    o_fus, l_fus = w.run(q, pb_, kv_scales=scales, return_lse=True, append_key=kn,
                         append_value=vn)
    torch.cuda.synchronize()
    assert np.array_equal(O.to_bits(pa_), O.to_bits(pb_))
    assert torch.equal(o_sep, o_fus)
    assert torch.equal(l_sep, l_fus)
    ref_o, _ = oracle_decode(meta, pb_, q, scales=scales)
    assert max_err(o_fus, ref_o) <= (TOL_FP8 if fp8 else TOL_BF16)


def test_shared_rope_append_equals_separate(gpu, shared, deterministic):
    # RoPE of q and the new K row + append + attention in one launch ==
    # apply_rope_pos_ids_inplace, append_paged_kv_cache, decode: bit for bit
    d, hq, hkv = 64, 32, 4
    meta, pool, q = decode_case(gpu, EDGE_LENS, hq, hkv, d, seed=41)
    bsz = len(EDGE_LENS)
    g = torch.Generator(device=gpu)
    g.manual_seed(42)
    kn = torch.randn((bsz, hkv, d), generator=g, device=gpu).to(torch.bfloat16) * 3
    vn = torch.randn((bsz, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    lens = np.asarray(EDGE_LENS, dtype=np.int64)
    pos = np.random.default_rng(43).integers(0, lens)
    w = _plan(gpu, meta, hq, hkv, d, torch.bfloat16)
    pa_, qa, ka = pool.clone(), q.clone(), kn.clone()
    pagedattn.apply_rope_pos_ids_inplace(qa, ka, i32(pos, gpu), rope_theta=10000.0,
                                         rope_scale=1.0)
    pagedattn.append_paged_kv_cache(ka, vn, i32(np.arange(bsz), gpu), i32(pos, gpu), pa_,
                                    i32(meta.kv_indices, gpu), i32(meta.kv_indptr, gpu),
                                    i32(meta.kv_last_page_len, gpu), kv_layout="HND")
    o_sep, l_sep = w.run(qa, pa_, return_lse=True)
    pb_ = pool.clone()
    o_fus, l_fus = w.run(q, pb_, return_lse=True, append_key=kn, append_value=vn,
                         rope=(1.0, 10000.0), positions=i32(pos, gpu))
    torch.cuda.synchronize()
    assert np.array_equal(O.to_bits(pa_), O.to_bits(pb_))
    assert torch.equal(o_sep, o_fus)
    assert torch.equal(l_sep, l_fus)


@pytest.mark.parametrize("fp8", [False, True])
def test_shared_rescale_branch(gpu, shared, fp8):
    # scores that keep growing page after page: the running max moves past
    # the lazy-rescale slack inside every wave's chunks, and the merged
    # states carry different maxima
    d, hq, hkv = 64, 32, 4
    lens = [1, 17, 300, 700, 1500, 2500]
    meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=61 + d)
    pool = scale_keys_by_page(pool, meta, 0.25)
    q = (q.float() * 2.0).to(q.dtype)
    scales = None
    if fp8:
        pool, scales = pagedattn.quantize_pages_e4m3(pool)
    assert log2_max_jumps(meta, pool, q, len(lens) - 1, scales=scales) >= 3 * hq
    ref_o, ref_l = oracle_decode(meta, pool, q, scales=scales)
    lse_tol = TOL_LSE + 2e-5 * float(ref_l[torch.isfinite(ref_l)].abs().max())
    out, lse = _plan(gpu, meta, hq, hkv, d, q.dtype).run(q, pool, kv_scales=scales,
                                                         return_lse=True)
    torch.cuda.synchronize()
    assert rel_err(out, ref_o) <= (3e-2 if fp8 else TOL_REL_BF16)
    assert lse_err(lse, ref_l) <= lse_tol


def test_shared_is_the_default_for_tinyllama(gpu, monkeypatch):
    require_shared_plans()
    # the TinyLlama B=256 batch balances over the CUs as whole items, so the
    # default plan is the shared one; it agrees with the split plan and the
    # oracle (which the at-scale decode tests also check)
    w = W.tinyllama_decode(seed=0)
    t = W.materialize(w, gpu)
    ws = workspace(gpu)
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    dw.plan(t.kv_indptr, t.kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=t.q.dtype)
    assert dw.plan_kind == "shared"
    out, lse = dw.run(t.q, t.pool, return_lse=True)
    monkeypatch.setenv("PAGEDATTN_DECODE_SHARED", "0")
    d2 = pagedattn.BatchDecodeWithPagedKVCacheWrapper(workspace(gpu), "HND")
    d2.plan(t.kv_indptr, t.kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=t.q.dtype)
    assert d2.plan_kind == "split"
    o2, l2 = d2.run(t.q, t.pool, return_lse=True)
    torch.cuda.synchronize()
    assert float((o2.float() - out.float()).abs().max()) <= 1e-2
    assert float((l2 - lse).abs().max()) <= 1e-3
    subset = [0, 5, 77, 128, 255]
    ref_o, ref_l = oracle_decode(w.meta, t.pool, t.q, batch=subset)
    assert max_err(out, ref_o, rows=subset) <= TOL_BF16
    assert lse_err(lse, ref_l, rows=subset) <= TOL_LSE


@pytest.mark.parametrize("order", ["arrival", "fixed"])
def test_shared_fused_append_claim_orders(gpu, shared, order, monkeypatch):
    # both claim orders: the fused append writes the pool bit for bit as the
    # stand-alone append does (with the fixed order each row is written by
    # the wave that loads its page, with no barrier), and the attention
    # agrees with the oracle
    monkeypatch.setenv("PAGEDATTN_DECODE_DETERMINISTIC", "0" if order == "arrival" else "1")
    d, hq, hkv = 64, 32, 4
    lens = EDGE_LENS + [int(x) for x in np.random.default_rng(36).integers(1, 900, 300)]
    meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=37)
    g = torch.Generator(device=gpu)
    g.manual_seed(38)
    kn = torch.randn((len(lens), hkv, d), generator=g, device=gpu).to(torch.bfloat16) * 3
    vn = torch.randn((len(lens), hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    pa_, pb_ = pool.clone(), pool.clone()
    pagedattn.append_paged_kv_cache(kn, vn, i32(meta.batch_indices, gpu),
                                    i32(meta.positions, gpu), pa_, i32(meta.kv_indices, gpu),
                                    i32(meta.kv_indptr, gpu), i32(meta.kv_last_page_len, gpu),
                                    kv_layout="HND")
    w = _plan(gpu, meta, hq, hkv, d, torch.bfloat16)
    o_fus, l_fus = w.run(q, pb_, return_lse=True, append_key=kn, append_value=vn)
    torch.cuda.synchronize()
    assert np.array_equal(O.to_bits(pa_), O.to_bits(pb_))
    ref_o, ref_l = oracle_decode(meta, pb_, q)
    assert max_err(o_fus, ref_o) <= TOL_BF16
    assert lse_err(l_fus, ref_l) <= TOL_LSE
