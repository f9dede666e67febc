"""GPU parity of ragged paged prefill attention (bottom-right causal and
full) against the fp32 CPU oracle: max-abs 2e-2 for bf16/fp16 outputs,
3e-2 for e4m3 pools, log-sum-exp within 2e-3."""

import numpy as np
import pytest
import torch

import oracle as O
import pagedattn
from pagedattn import workloads as W

from paged_cases import (i32, lse_err, max_err, oracle_prefill, oracle_prefill_rows,
                         prefill_case, rel_err, run_decode, run_prefill, scale_keys_by_page,
                         workspace)

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_FP8 = 3e-2
TOL_LSE = 2e-3
# error relative to the row's largest reference value (paged_cases.rel_err)
TOL_REL_BF16 = 2e-2
TOL_REL_FP8 = 3e-2

# (cached prefix, new chunk) pairs: empty prefix, partial pages, exact pages,
# single-token chunks, chunks longer than a row tile
EDGE = [(0, 1), (0, 15), (0, 16), (0, 17), (16, 1), (5, 33), (100, 64), (0, 130), (1000, 129),
        (31, 200), (64, 7), (300, 300)]


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(32, 8), (32, 4), (8, 8), (64, 8), (32, 2), (12, 3)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_edges(gpu, d, hq, hkv, causal):
    computed = [c for c, _ in EDGE]
    chunks = [n for _, n in EDGE]
    meta, pool, q = prefill_case(gpu, computed, chunks, hq, hkv, d, seed=hq * 3 + hkv + d)
    ref_o, ref_l = oracle_prefill(meta, pool, q, causal=causal)
    out, lse = run_prefill(gpu, meta, pool, q, hq, hkv, d, causal=causal)
    assert max_err(out, ref_o) <= TOL_BF16, max_err(out, ref_o)
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_prefill_fp16(gpu):
    meta, pool, q = prefill_case(gpu, [0, 70, 333], [200, 65, 17], 32, 8, 128,
                                 dtype=torch.float16, seed=9)
    ref_o, ref_l = oracle_prefill(meta, pool, q)
    out, lse = run_prefill(gpu, meta, pool, q, 32, 8, 128)
    assert out.dtype == torch.float16
    assert max_err(out, ref_o) <= TOL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_prefill_single_row_equals_decode(gpu):
    # a one-token chunk is a decode step: both kernels must agree
    lens_prev = [0, 15, 16, 100, 777]
    meta, pool, q = prefill_case(gpu, lens_prev, [1] * 5, 32, 4, 64, seed=3)
    out_p, lse_p = run_prefill(gpu, meta, pool, q, 32, 4, 64)
    out_d, lse_d = run_decode(gpu, meta, pool, q, 32, 4, 64)
    assert float((out_p.float() - out_d.float()).abs().max()) <= 1e-2
    assert float((lse_p - lse_d).abs().max()) <= 1e-3


def _append_chunk(t):
    pagedattn.append_paged_kv_cache(t.k_new, t.v_new, t.batch_indices, t.positions, t.pool,
                                    t.kv_indices, t.kv_indptr, t.kv_last_page_len,
                                    kv_layout="HND", kv_scales=t.scales)


def test_prefill_llama3_8b_chunked(gpu):
    w = W.llama3_8b_prefill(seed=0)
    t = W.materialize(w, gpu)
    _append_chunk(t)
    m = w.meta
    out, lse = run_prefill(gpu, m, t.pool, t.q, w.hq, w.hkv, w.d)
    ref_o, ref_l = oracle_prefill(m, t.pool, t.q)
    assert max_err(out, ref_o) <= TOL_BF16
    assert rel_err(out, ref_o) <= TOL_REL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_prefill_tinyllama_shape(gpu):
    # the reference engine's default model (TinyLlama: 32 query heads, 4 KV
    # heads, head_dim 64) on chunked prefills over long and short prefixes,
    # partial pages included; oracle on every row
    computed = [0, 16, 256, 1000, 2048, 37, 512, 3000]
    chunks = [512, 300, 129, 64, 256, 400, 33, 128]
    meta, pool, q = prefill_case(gpu, computed, chunks, 32, 4, 64, seed=64)
    out, lse = run_prefill(gpu, meta, pool, q, 32, 4, 64)
    ref_o, ref_l = oracle_prefill(meta, pool, q)
    assert max_err(out, ref_o) <= TOL_BF16
    assert rel_err(out, ref_o) <= TOL_REL_BF16
    assert lse_err(lse, ref_l) <= TOL_LSE


def test_prefill_split_chunk_equivalence(gpu):
    # size-independent: prefilling a chunk at once equals prefilling its two
    # halves one after the other (the second half attends to the first)
    w = W.llama3_8b_prefill(seed=1)
    t = W.materialize(w, gpu)
    _append_chunk(t)
    m = w.meta
    full, _ = run_prefill(gpu, m, t.pool, t.q, w.hq, w.hkv, w.d)
    qo = np.diff(m.qo_indptr)
    half = qo // 2
    # second halves only: qo' = qo - half rows, same kv
    qo2 = np.concatenate([[0], np.cumsum(qo - half)]).astype(np.int32)
    rows = np.concatenate([np.arange(m.qo_indptr[b] + half[b], m.qo_indptr[b + 1])
                           for b in range(len(qo))])
    q2 = t.q[torch.from_numpy(rows).to(gpu)].contiguous()
    from types import SimpleNamespace
    m2 = SimpleNamespace(qo_indptr=qo2, kv_indptr=m.kv_indptr, kv_indices=m.kv_indices,
                         kv_last_page_len=m.kv_last_page_len)
    out2, _ = run_prefill(gpu, m2, t.pool, q2, w.hq, w.hkv, w.d)
    assert float((out2.float() - full[torch.from_numpy(rows).to(gpu)].float()).abs().max()) <= 1e-2


def test_prefill_e4m3_mixed(gpu):
    dec, pre = W.llama3_70b_mixed_fp8(seed=0)
    t = W.materialize(pre, gpu)
    t.pool, t.scales = pagedattn.quantize_pages_e4m3(t.pool)
    _append_chunk(t)
    m = pre.meta
    out, lse = run_prefill(gpu, m, t.pool, t.q, pre.hq, pre.hkv, pre.d, kv_scales=t.scales)
    # oracle on a seeded sample of 128-row slices of every sequence
    rng = np.random.default_rng(0)
    for b in range(m.batch_size):
        for lo in sorted(rng.choice(8, size=2, replace=False) * 128):
            o, l = oracle_prefill_rows(m, t.pool, t.q, b, int(lo), int(lo) + 128,
                                       scales=t.scales)
            r0 = int(m.qo_indptr[b]) + int(lo)
            assert max_err(out[r0:r0 + 128], o) <= TOL_FP8
            assert rel_err(out[r0:r0 + 128], o) <= TOL_REL_FP8
            assert lse_err(lse[r0:r0 + 128], l) <= TOL_LSE


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("d,hq,hkv", [(128, 32, 8), (64, 32, 4)])
def test_prefill_rescale_branch(gpu, fp8, d, hq, hkv):
    # K of page i scaled by 1 + i/4: every query row's running max moves by
    # more than the lazy-rescale slack (8 in log2 units) across KV tiles, so
    # O and l are rescaled from a finite max in the causal multi-tile loop
    computed = [1000, 0, 512, 2048]
    chunks = [300, 257, 64, 129]
    meta, pool, q = prefill_case(gpu, computed, chunks, hq, hkv, d, seed=81 + d)
    pool = scale_keys_by_page(pool, meta, 0.25)
    q = (q.float() * 2.0).to(q.dtype)
    scales = None
    if fp8:
        pool, scales = pagedattn.quantize_pages_e4m3(pool)
    ref_o, ref_l = oracle_prefill(meta, pool, q, scales=scales)
    lse_tol = TOL_LSE + 2e-5 * float(ref_l[torch.isfinite(ref_l)].abs().max())
    tol, tol_rel = (TOL_FP8, TOL_REL_FP8) if fp8 else (TOL_BF16, TOL_REL_BF16)
    out, lse = run_prefill(gpu, meta, pool, q, hq, hkv, d, kv_scales=scales)
    assert max_err(out, ref_o) <= tol
    assert rel_err(out, ref_o) <= tol_rel
    assert lse_err(lse, ref_l) <= lse_tol


@pytest.mark.parametrize("case", ["edges", "llama3_8b"])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_paired_tiles_bit_identical(gpu, monkeypatch, case, causal):
    # q-tiles with at most half a workgroup's rows run two KV heads in one
    # workgroup (D = 128, 16-bit pools); each row's arithmetic is unchanged,
    # so output and LSE bits equal the unpaired plan's
    if case == "edges":
        computed = [c for c, _ in EDGE] + [2000, 37]
        chunks = [n for _, n in EDGE] + [20, 45]
        hq, hkv, d = 32, 8, 128
        meta, pool, q = prefill_case(gpu, computed, chunks, hq, hkv, d, seed=77)
    else:
        w = W.llama3_8b_prefill(seed=5)
        t = W.materialize(w, gpu)
        meta, pool, q, hq, hkv, d = w.meta, t.pool, t.q, w.hq, w.hkv, w.d
    out1, lse1 = run_prefill(gpu, meta, pool, q, hq, hkv, d, causal=causal)
    monkeypatch.setenv("PAGEDATTN_PREFILL_PAIR", "0")
    out0, lse0 = run_prefill(gpu, meta, pool, q, hq, hkv, d, causal=causal)
    assert torch.equal(out0, out1)
    assert torch.equal(lse0, lse1)
