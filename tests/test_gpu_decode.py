"""GPU parity of paged decode attention (bf16/fp16 and e4m3 pools) against the
fp32 CPU oracle: max-abs 2e-2 for bf16/fp16 outputs, 3e-2 for e4m3 pools,
log-sum-exp within 2e-3.  Full-size workloads add size-independent checks:
every split-KV partition must give the same output."""

import math

import numpy as np
import pytest
import torch

import oracle as O
import pagedattn
from pagedattn import workloads as W
from pagedattn.metadata import decode_metadata

from paged_cases import (decode_case, i32, log2_max_jumps, lse_err, max_err, oracle_decode,
                         random_tables, rel_err, run_decode, scale_keys_by_page, workspace)

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_FP8 = 3e-2
TOL_LSE = 2e-3
# error relative to the row's largest reference value (paged_cases.rel_err)
TOL_REL_BF16 = 2e-2
TOL_REL_FP8 = 3e-2

EDGE_LENS = [1, 2, 15, 16, 17, 31, 32, 33, 47, 48, 64, 100, 255, 256, 257, 700]


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(32, 4), (32, 8), (8, 8), (16, 8), (32, 2), (64, 8)])
def test_decode_edge_lengths(gpu, d, hq, hkv):
    meta, pool, q = decode_case(gpu, EDGE_LENS, hq, hkv, d, seed=hq + hkv + d)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    for split in (-1, 0, 8):
        out, lse = run_decode(gpu, meta, pool, q, hq, hkv, d, split_pages=split)
        assert max_err(out, ref_o) <= TOL_BF16, (split, max_err(out, ref_o))
        assert lse_err(lse, ref_l) <= TOL_LSE, split


@pytest.mark.parametrize("head_group", ["1", "2", "4"])
@pytest.mark.parametrize("hq,hkv", [(32, 8), (16, 2)])
def test_decode_head_groups(gpu, monkeypatch, head_group, hq, hkv):
    # every head-group width (waves walking the same pages, one per KV head)
    # gives the oracle's answer, whole-sequence, balanced and fixed splits
    monkeypatch.setenv("PAGEDATTN_DECODE_HEAD_GROUP", head_group)
    meta, pool, q = decode_case(gpu, EDGE_LENS, hq, hkv, 64, seed=5 + hkv)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    for split in (-1, 0, 8):
        out, lse = run_decode(gpu, meta, pool, q, hq, hkv, 64, split_pages=split)
        assert max_err(out, ref_o) <= TOL_BF16, (split, max_err(out, ref_o))
        assert lse_err(lse, ref_l) <= TOL_LSE, split


@pytest.mark.parametrize("cost", ["0", "6", "40"])
def test_decode_balanced_item_cost(gpu, monkeypatch, cost):
    # the balanced split charges page-equivalents per item (shares of many
    # short pieces get fewer pages); any charge is still a partition of the
    # (sequence, head group, page) stream and gives the oracle's answer
    monkeypatch.setenv("PAGEDATTN_DECODE_ITEM_COST", cost)
    lens = EDGE_LENS + [int(x) for x in np.random.default_rng(3).integers(1, 3000, 60)]
    meta, pool, q = decode_case(gpu, lens, 32, 8, 128, seed=13)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    out, lse = run_decode(gpu, meta, pool, q, 32, 8, 128, split_pages=0)
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_decode_fp16(gpu):
    meta, pool, q = decode_case(gpu, EDGE_LENS, 32, 4, 64, dtype=torch.float16, seed=11)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    out, lse = run_decode(gpu, meta, pool, q, 32, 4, 64)
    assert out.dtype == torch.float16
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_decode_empty_and_single_sequences(gpu):
    # a sequence with no pages gets zeros and lse = -inf; B = 1 works
    d, hq, hkv = 64, 32, 4
    from types import SimpleNamespace
    meta = SimpleNamespace(kv_indptr=np.array([0, 3, 3, 4], np.int32),
                           kv_indices=np.array([6, 2, 0, 4], np.int32),
                           kv_last_page_len=np.array([8, 1, 5], np.int32))
    num_pages = 8
    g = torch.Generator(device=gpu)
    g.manual_seed(1)
    pool = torch.randn((num_pages, 2, hkv, 16, d), generator=g, device=gpu).to(torch.bfloat16)
    q = torch.randn((3, hq, d), generator=g, device=gpu).to(torch.bfloat16)
    ref_o, ref_l = oracle_decode(meta, pool, q)
    out, lse = run_decode(gpu, meta, pool, q, hq, hkv, d)
    assert torch.equal(out[1].float().cpu(), torch.zeros(hq, d))
    assert bool(torch.isinf(lse[1]).all())
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE
    meta1, pool1, q1 = decode_case(gpu, [333], hq, hkv, d, seed=3)
    o1, _ = run_decode(gpu, meta1, pool1, q1, hq, hkv, d)
    assert max_err(o1, oracle_decode(meta1, pool1, q1)[0]) <= TOL_BF16


def test_decode_bad_page_ids_do_not_fault(gpu):
    # out-of-range page ids read as empty pages (no fault); other rows stay exact
    meta, pool, q = decode_case(gpu, [40, 40, 40], 32, 4, 64, seed=4)
    bad = meta.kv_indices.copy()
    bad[meta.kv_indptr[1]] = pool.shape[0] + 1000
    ws = workspace(gpu)
    w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    w.plan(i32(meta.kv_indptr, gpu), i32(bad, gpu), i32(meta.kv_last_page_len, gpu), 32, 4, 64,
           16, q_data_type=torch.bfloat16)
    out = w.run(q, pool)
    ref_o, _ = oracle_decode(meta, pool, q)
    assert torch.isfinite(out.float()).all()
    assert max_err(out, ref_o, rows=[0, 2]) <= TOL_BF16


def _fused_append_then_decode(gpu, w, t, split_pages=None, ws=None):
    m = w.meta
    pagedattn.append_paged_kv_cache(t.k_new, t.v_new, t.batch_indices, t.positions, t.pool,
                                    t.kv_indices, t.kv_indptr, t.kv_last_page_len,
                                    kv_layout="HND", kv_scales=t.scales)
    ws = workspace(gpu) if ws is None else ws
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    dw.plan(t.kv_indptr, t.kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=t.q.dtype,
            split_pages=w.split_pages if split_pages is None else split_pages)
    out, lse = dw.run(t.q, t.pool, kv_scales=t.scales, return_lse=True)
    torch.cuda.synchronize()
    return out, lse


def test_decode_tinyllama_small(gpu):
    w = W.tinyllama_decode_small(seed=0)
    t = W.materialize(w, gpu)
    before = O.to_bits(t.pool)
    out, lse = _fused_append_then_decode(gpu, w, t)
    m = w.meta
    want, _ = O.append_pages(before, O.to_bits(t.k_new), O.to_bits(t.v_new), m.batch_indices,
                             m.positions, m.kv_indices, m.kv_indptr)
    assert np.array_equal(O.to_bits(t.pool), want)
    ref_o, ref_l = oracle_decode(m, t.pool, t.q)
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_decode_tinyllama_at_scale(gpu):
    w = W.tinyllama_decode(seed=0)
    t = W.materialize(w, gpu)
    out, lse = _fused_append_then_decode(gpu, w, t)
    ref_o, ref_l = oracle_decode(w.meta, t.pool, t.q)
    assert max_err(out, ref_o) <= TOL_BF16
    assert rel_err(out, ref_o) <= TOL_REL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE
    # size-independent: every split-KV partition gives the same answer
    ws = workspace(gpu)
    for split in (-1, 8, 40):
        dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
        dw.plan(t.kv_indptr, t.kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
                q_data_type=t.q.dtype, split_pages=split)
        o2 = dw.run(t.q, t.pool)
        assert float((o2.float() - out.float()).abs().max()) <= 1e-2, split
        assert rel_err(o2, out.float().cpu()) <= TOL_REL_BF16, split


def test_decode_long_context_split(gpu):
    # full-size long-context batch; oracle on a seeded subset of sequences,
    # all sequences through the split-invariance property
    w = W.llama3_8b_long_decode(seed=0)
    t = W.materialize(w, gpu)
    out, lse = _fused_append_then_decode(gpu, w, t)  # 4096-token chunks
    lens = w.meta.seq_lens
    subset = sorted({0, 7, 19, int(np.argmax(lens))})
    ref_o, ref_l = oracle_decode(w.meta, t.pool, t.q, batch=subset)
    assert max_err(out, ref_o, rows=subset) <= TOL_BF16
    # |o| is ~0.02 at these lengths: the relative bound is the one that bites
    assert rel_err(out, ref_o, rows=subset) <= TOL_REL_BF16
    assert lse_err(lse, ref_l, rows=subset) <= TOL_LSE
    ws = workspace(gpu)
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    dw.plan(t.kv_indptr, t.kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=t.q.dtype, split_pages=0)
    o_auto, l_auto = dw.run(t.q, t.pool, return_lse=True)
    assert float((o_auto.float() - out.float()).abs().max()) <= 1e-2
    assert rel_err(o_auto, out.float().cpu()) <= TOL_REL_BF16
    assert float((l_auto - lse).abs().max()) <= 1e-3


@pytest.mark.parametrize("d,hq,hkv", [(128, 64, 8), (64, 32, 4)])
def test_decode_e4m3(gpu, d, hq, hkv):
    meta, pool16, q = decode_case(gpu, EDGE_LENS, hq, hkv, d, seed=21)
    pool8, scales = pagedattn.quantize_pages_e4m3(pool16)
    ref_o, ref_l = oracle_decode(meta, pool8, q, scales=scales)
    for split in (-1, 0, 8):
        out, lse = run_decode(gpu, meta, pool8, q, hq, hkv, d, split_pages=split,
                              kv_scales=scales)
        assert max_err(out, ref_o) <= TOL_FP8, split
        assert lse_err(lse, ref_l) <= TOL_LSE


@pytest.mark.parametrize("d,hq,hkv,fp8", [(64, 32, 4, False), (128, 32, 8, False),
                                          (128, 64, 8, True), (64, 32, 4, True)])
def test_decode_fused_append_equals_separate(gpu, d, hq, hkv, fp8):
    # one launch (append at kv_len - 1 + attention) == append kernel + decode
    meta, pool, q = decode_case(gpu, EDGE_LENS, hq, hkv, d, seed=33)
    g = torch.Generator(device=gpu)
    g.manual_seed(34)
    kn = torch.randn((len(EDGE_LENS), hkv, d), generator=g, device=gpu).to(torch.bfloat16) * 3
    vn = torch.randn((len(EDGE_LENS), hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    scales = None
    if fp8:
        pool, scales = pagedattn.quantize_pages_e4m3(pool)
    pool_a, pool_b = pool.clone(), pool.clone()
    ws = workspace(gpu)
    for split in (-1, 0, 8):
        pa_, pb_ = pool_a.clone(), pool_b.clone()
        pagedattn.append_paged_kv_cache(kn, vn, i32(meta.batch_indices, gpu),
                                        i32(meta.positions, gpu), pa_,
                                        i32(meta.kv_indices, gpu), i32(meta.kv_indptr, gpu),
                                        i32(meta.kv_last_page_len, gpu), kv_layout="HND",
                                        kv_scales=scales)
        w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
        w.plan(i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu),
               i32(meta.kv_last_page_len, gpu), hq, hkv, d, 16, q_data_type=torch.bfloat16,
               split_pages=split)
        o_sep, l_sep = w.run(q, pa_, kv_scales=scales, return_lse=True)
        o_fus, l_fus = w.run(q, pb_, kv_scales=scales, return_lse=True, append_key=kn,
                             append_value=vn)
        torch.cuda.synchronize()
        assert np.array_equal(O.to_bits(pa_), O.to_bits(pb_)), split
        assert torch.equal(o_sep, o_fus), split
        assert torch.equal(l_sep, l_fus), split
    ref_o, _ = oracle_decode(meta, pb_, q, scales=scales)
    assert max_err(o_fus, ref_o) <= (TOL_FP8 if fp8 else TOL_BF16)


def test_decode_fused_append_tinyllama_at_scale(gpu):
    w = W.tinyllama_decode(seed=2)
    t = W.materialize(w, gpu)
    before = O.to_bits(t.pool)
    ws = workspace(gpu)
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    dw.plan(t.kv_indptr, t.kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=t.q.dtype)
    out = dw.run(t.q, t.pool, append_key=t.k_new, append_value=t.v_new)
    torch.cuda.synchronize()
    m = w.meta
    want, _ = O.append_pages(before, O.to_bits(t.k_new), O.to_bits(t.v_new), m.batch_indices,
                             m.positions, m.kv_indices, m.kv_indptr)
    assert np.array_equal(O.to_bits(t.pool), want)
    ref_o, _ = oracle_decode(m, t.pool, t.q)
    assert max_err(out, ref_o) <= TOL_BF16


@pytest.mark.parametrize("d,hq,hkv,fp8", [(64, 32, 4, False), (128, 32, 8, False),
                                          (128, 64, 8, True)])
def test_decode_rope_append_equals_separate(gpu, d, hq, hkv, fp8):
    # one launch (RoPE of q and the new K row + append + attention) ==
    # apply_rope_pos_ids_inplace, append_paged_kv_cache, decode: bit for bit
    meta, pool, q = decode_case(gpu, EDGE_LENS, hq, hkv, d, seed=41)
    bsz = len(EDGE_LENS)
    g = torch.Generator(device=gpu)
    g.manual_seed(42)
    kn = torch.randn((bsz, hkv, d), generator=g, device=gpu).to(torch.bfloat16) * 3
    vn = torch.randn((bsz, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    scales = None
    if fp8:
        pool, scales = pagedattn.quantize_pages_e4m3(pool)
    lens = np.asarray(EDGE_LENS, dtype=np.int64)
    rng = np.random.default_rng(43)
    # the engine's positions (kv_len - 1) and arbitrary earlier positions
    for pos in (lens - 1, rng.integers(0, lens)):
        ws = workspace(gpu)
        for split in (0, 8):
            w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
            w.plan(i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu),
                   i32(meta.kv_last_page_len, gpu), hq, hkv, d, 16,
                   q_data_type=torch.bfloat16, split_pages=split)
            pa_, qa, ka = pool.clone(), q.clone(), kn.clone()
            pagedattn.apply_rope_pos_ids_inplace(qa, ka, i32(pos, gpu), rope_theta=10000.0,
                                                 rope_scale=1.0)
            pagedattn.append_paged_kv_cache(ka, vn, i32(np.arange(bsz), gpu), i32(pos, gpu),
                                            pa_, i32(meta.kv_indices, gpu),
                                            i32(meta.kv_indptr, gpu),
                                            i32(meta.kv_last_page_len, gpu), kv_layout="HND",
                                            kv_scales=scales)
            o_sep, l_sep = w.run(qa, pa_, kv_scales=scales, return_lse=True)
            pb_ = pool.clone()
            o_fus, l_fus = w.run(q, pb_, kv_scales=scales, return_lse=True, append_key=kn,
                                 append_value=vn, rope=(1.0, 10000.0),
                                 positions=i32(pos, gpu))
            torch.cuda.synchronize()
            assert np.array_equal(O.to_bits(pa_), O.to_bits(pb_)), split
            assert torch.equal(o_sep, o_fus), split
            assert torch.equal(l_sep, l_fus), split
    # positions omitted means kv_len - 1
    pc_ = pool.clone()
    o_def = w.run(q, pc_, kv_scales=scales, append_key=kn, append_value=vn,
                  rope=(1.0, 10000.0))
    pd_ = pool.clone()
    o_exp = w.run(q, pd_, kv_scales=scales, append_key=kn, append_value=vn,
                  rope=(1.0, 10000.0), positions=i32(lens - 1, gpu))
    torch.cuda.synchronize()
    assert torch.equal(o_def, o_exp)
    assert np.array_equal(O.to_bits(pc_), O.to_bits(pd_))


def test_decode_llama3_70b_e4m3_workload(gpu):
    # the 70B-shaped e4m3 decode batch exactly as the benchmark times it:
    # fused e4m3 append at kv_len - 1 with the page's fixed scale, then
    # attention under the planner's balanced split; oracle on a seeded subset
    # that includes the longest sequences, every split over all 128
    dec, _ = W.llama3_70b_mixed_fp8(seed=0)
    t = W.materialize(dec, gpu)
    t.pool, t.scales = pagedattn.quantize_pages_e4m3(t.pool)
    before = O.to_bits(t.pool)
    ws = workspace(gpu)
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    dw.plan(t.kv_indptr, t.kv_indices, t.kv_last_page_len, dec.hq, dec.hkv, dec.d, 16,
            q_data_type=t.q.dtype, split_pages=dec.split_pages)
    out, lse = dw.run(t.q, t.pool, kv_scales=t.scales, return_lse=True, append_key=t.k_new,
                      append_value=t.v_new)
    torch.cuda.synchronize()
    m = dec.meta
    want, skipped = O.append_pages_e4m3(before, t.scales.cpu(), t.k_new.cpu().float(),
                                        t.v_new.cpu().float(), m.batch_indices, m.positions,
                                        m.kv_indices, m.kv_indptr)
    assert skipped == 0
    assert np.array_equal(O.to_bits(t.pool), want)
    # the counter at byte 4 of the workspace holds the clamped pieces, the
    # one at byte 0 the skipped tokens (none)
    clamped = O.e4m3_clamped_pieces(t.k_new.cpu().float(), t.v_new.cpu().float(),
                                    t.scales.cpu(), m.batch_indices, m.positions,
                                    m.kv_indices, m.kv_indptr, dec.num_pages)
    assert ws[:8].view(torch.int32).tolist() == [0, clamped]
    lens = m.seq_lens
    rng = np.random.default_rng(70)
    subset = sorted(set(np.argsort(lens)[-3:].tolist()) |
                    set(rng.choice(len(lens), 4, replace=False).tolist()))
    ref_o, ref_l = oracle_decode(m, t.pool, t.q, scales=t.scales, batch=subset)
    assert max_err(out, ref_o, rows=subset) <= TOL_FP8
    assert rel_err(out, ref_o, rows=subset) <= TOL_REL_FP8
    assert lse_err(lse, ref_l, rows=subset) <= TOL_LSE
    # (8-page chunks would need more than the engine's 128 MiB workspace here)
    for split in (-1, 0, 32, 256):
        w2 = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
        w2.plan(t.kv_indptr, t.kv_indices, t.kv_last_page_len, dec.hq, dec.hkv, dec.d, 16,
                q_data_type=t.q.dtype, split_pages=split)
        o2, l2 = w2.run(t.q, t.pool, kv_scales=t.scales, return_lse=True)
        assert float((o2.float() - out.float()).abs().max()) <= 1e-2, split
        assert rel_err(o2, out.float().cpu()) <= TOL_REL_FP8, split
        assert float((l2 - lse).abs().max()) <= 1e-3, split


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("d,hq,hkv", [(64, 32, 4), (128, 64, 8)])
def test_decode_rescale_branch(gpu, fp8, d, hq, hkv):
    # scores that keep growing page after page (K of page i scaled by
    # 1 + i/4): the running max moves by more than the lazy-rescale slack
    # (8 in log2 units) many times per sequence, so O and l are rescaled
    # from a finite max and split pieces merge with different maxima
    lens = [1, 17, 300, 700, 1500, 2500]
    meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=61 + d)
    pool = scale_keys_by_page(pool, meta, 0.25)
    q = (q.float() * 2.0).to(q.dtype)
    scales = None
    if fp8:
        pool, scales = pagedattn.quantize_pages_e4m3(pool)
    assert log2_max_jumps(meta, pool, q, len(lens) - 1, scales=scales) >= 3 * hq
    tol, tol_rel = (TOL_FP8, TOL_REL_FP8) if fp8 else (TOL_BF16, TOL_REL_BF16)
    ref_o, ref_l = oracle_decode(meta, pool, q, scales=scales)
    lse_tol = TOL_LSE + 2e-5 * float(ref_l[torch.isfinite(ref_l)].abs().max())
    ws = workspace(gpu)
    for split in (-1, 0, 8):
        out, lse = run_decode(gpu, meta, pool, q, hq, hkv, d, split_pages=split,
                              kv_scales=scales, ws=ws)
        assert max_err(out, ref_o) <= tol, split
        assert rel_err(out, ref_o) <= tol_rel, split
        assert lse_err(lse, ref_l) <= lse_tol, split
    # device-side partition
    w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    w.plan(i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu), i32(meta.kv_last_page_len, gpu),
           hq, hkv, d, 16, q_data_type=q.dtype, device_plan=True)
    out, lse = w.run(q, pool, kv_scales=scales, return_lse=True)
    torch.cuda.synchronize()
    assert rel_err(out, ref_o) <= tol_rel
    assert lse_err(lse, ref_l) <= lse_tol
    # fused append of a new token whose K row is larger still
    g = torch.Generator(device=gpu)
    g.manual_seed(62)
    kn = (torch.randn((len(lens), hkv, d), generator=g, device=gpu) * 30).to(torch.bfloat16)
    vn = torch.randn((len(lens), hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    pa = pool.clone()
    w8 = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    w8.plan(i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu),
            i32(meta.kv_last_page_len, gpu), hq, hkv, d, 16, q_data_type=q.dtype,
            split_pages=8)
    o_f = w8.run(q, pa, kv_scales=scales, append_key=kn, append_value=vn)
    torch.cuda.synchronize()
    ref_f, _ = oracle_decode(meta, pa, q, scales=scales)
    assert rel_err(o_f, ref_f) <= tol_rel


def test_decode_fused_append_counts(gpu):
    # the fused e4m3 append counts what the stand-alone append counts:
    # clamped pieces (rows past +-448 x scale, a zero or infinite page
    # scale) at byte 4 of the workspace and new tokens outside their
    # sequence's pages at byte 0, apart; the pool bytes equal the oracle's
    d, hq, hkv = 128, 64, 8
    lens = [5, 16, 17, 40, 100, 333]
    meta, pool16, q = decode_case(gpu, lens, hq, hkv, d, seed=71)
    pool, scales = pagedattn.quantize_pages_e4m3(pool16)
    bsz = len(lens)
    g = torch.Generator(device=gpu)
    g.manual_seed(72)
    kn = (torch.randn((bsz, hkv, d), generator=g, device=gpu) * 8).to(torch.bfloat16)
    vn = torch.randn((bsz, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    last_pages = [int(meta.kv_indices[meta.kv_indptr[b + 1] - 1]) for b in range(bsz)]
    scales[last_pages[1], 0, 3] = 0.0
    scales[last_pages[4], 1, 0] = float("inf")
    pos = np.asarray(lens, np.int64) - 1
    pos[2] = lens[2] + 40  # past the sequence's pages: skipped and counted
    before = O.to_bits(pool)
    ka = kn.clone()
    qa = q.clone()
    pagedattn.apply_rope_pos_ids_inplace(qa, ka, i32(pos, gpu), rope_theta=1e4, rope_scale=1.0)
    bi = np.arange(bsz)
    want, skipped = O.append_pages_e4m3(before, scales.cpu(), ka.cpu().float(),
                                        vn.cpu().float(), bi, pos, meta.kv_indices,
                                        meta.kv_indptr)
    clamped = O.e4m3_clamped_pieces(ka.cpu().float(), vn.cpu().float(), scales.cpu(), bi, pos,
                                    meta.kv_indices, meta.kv_indptr, pool.shape[0])
    assert skipped == 1 and clamped > 2 * (d // 8)
    for split in (-1, 0, 8):
        ws = workspace(gpu)
        w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
        w.plan(i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu),
               i32(meta.kv_last_page_len, gpu), hq, hkv, d, 16, q_data_type=q.dtype,
               split_pages=split)
        pb = pool.clone()
        w.run(q, pb, kv_scales=scales, append_key=kn, append_value=vn, rope=(1.0, 1e4),
              positions=i32(pos, gpu))
        torch.cuda.synchronize()
        assert np.array_equal(O.to_bits(pb), want), split
        assert ws[:8].view(torch.int32).tolist() == [skipped, clamped], split
