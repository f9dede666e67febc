"""Size-independent properties of the attention kernels at the full benchmark
sizes, where the fp32 oracle covers only subsets:

* relabelling the physical pages (moving page i to slot perm[i] and renaming
  the block tables) leaves decode and prefill outputs bit-identical;
* when every V row that a sequence can see is one vector c, the output is c
  whatever the scores (softmax weights sum to one): a wrong page, a row of
  another sequence or a wrong head shows as a different vector;
* with q = 0 every visible score is 0, so the output is the mean of the
  visible V rows: the causal limit, last_page_len and every page of the
  table are checked against a closed form.

Page relabelling and the softmax identities are the reference's own
invariants of block-table indexing (src/models/llama.py:70-83, 230-245;
allocator.py:25-36).  Tolerances: the constant-V and mean outputs carry
only the bf16 rounding of P (exact for q = 0) and of the output, so they
are bounded relative to the expected value."""

import numpy as np
import pytest
import torch

import pagedattn
from pagedattn import workloads as W

from paged_cases import require_fixed_chunks, workspace

pytestmark = pytest.mark.gpu

# |out - c| <= REL |c| + ABS: bf16 rounding of P and of the output (2^-9
# each), with margin
REL = 2.0 ** -7
ABS = 1e-4


def _decode(gpu, w, pool, t, kv_indices, q, scales=None, split_pages=0):
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(workspace(gpu), "HND")
    dw.plan(t.kv_indptr, kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=q.dtype, split_pages=split_pages)
    out, lse = dw.run(q, pool, kv_scales=scales, return_lse=True)
    torch.cuda.synchronize()
    return out, lse, dw.plan_kind


def _prefill(gpu, w, pool, t, kv_indices, q):
    pw = pagedattn.BatchPrefillWithPagedKVCacheWrapper(workspace(gpu), "HND")
    pw.plan(t.qo_indptr, t.kv_indptr, kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=q.dtype)
    out, lse = pw.run(q, pool, return_lse=True, causal=True)
    torch.cuda.synchronize()
    return out, lse


def _relabel(pool, kv_indices, seed, scales=None):
    n = pool.shape[0]
    perm = torch.from_numpy(np.random.default_rng(seed).permutation(n)).to(pool.device)
    pool2 = torch.empty_like(pool)
    pool2[perm] = pool
    s2 = None
    if scales is not None:
        s2 = torch.empty_like(scales)
        s2[perm] = scales
    return pool2, perm[kv_indices.long()].to(torch.int32), s2


def _seq_lens(m):
    npg = np.diff(m.kv_indptr).astype(np.int64)
    return np.where(npg > 0, (npg - 1) * 16 + m.kv_last_page_len, 0)


def _token_rows(m, b):
    """(page, slot) of every kv token of sequence b, in order."""
    pages = m.kv_indices[m.kv_indptr[b]:m.kv_indptr[b + 1]].astype(np.int64)
    n = int(_seq_lens(m)[b])
    tok = np.arange(n)
    return pages[tok // 16], tok % 16


def _v_rows(pool, m, b, scales=None):
    """V rows [kv_len, Hkv, D] of sequence b in fp32 (dequantised for e4m3)."""
    pg, sl = _token_rows(m, b)
    pg_t = torch.from_numpy(pg).to(pool.device)
    sl_t = torch.from_numpy(sl).to(pool.device)
    v = pool[pg_t, 1, :, sl_t, :].float()
    if scales is not None:
        v = v * scales[pg_t, 1, :].float()[:, :, None]
    return v


def _components(m):
    """Sequences that share a page belong to one component."""
    parent = list(range(m.batch_size))

    def find(x):
        while parent[x] != x:
            parent[x] = parent[parent[x]]
            x = parent[x]
        return x
    owner = {}
    for b in range(m.batch_size):
        for p in m.kv_indices[m.kv_indptr[b]:m.kv_indptr[b + 1]].tolist():
            if p in owner:
                parent[find(b)] = find(owner[p])
            else:
                owner[p] = b
    return [find(b) for b in range(m.batch_size)]


def _fill_v(pool, m, comp, c):
    """Every V row of every page of sequence b := c[comp[b]] (per KV head)."""
    for b in range(m.batch_size):
        pages = torch.from_numpy(
            m.kv_indices[m.kv_indptr[b]:m.kv_indptr[b + 1]].astype(np.int64)).to(pool.device)
        pool[pages, 1] = c[comp[b]][None, :, None, :].to(pool.dtype)


def _check_close(out, want):
    err = (out.float() - want).abs()
    bound = REL * want.abs() + ABS
    assert bool((err <= bound).all()), float((err - bound).max())


@pytest.mark.parametrize("plan", ["shared", "split"])
def test_decode_page_relabel_bit_exact(gpu, monkeypatch, plan):
    # TinyLlama at scale; the shared plan with its fixed chunk assignment so
    # that output bits do not depend on timing
    monkeypatch.setenv("PAGEDATTN_DECODE_SHARED", "1" if plan == "shared" else "0")
    monkeypatch.setenv("PAGEDATTN_DECODE_DETERMINISTIC", "1")
    w = W.tinyllama_decode(seed=3)
    t = W.materialize(w, gpu)
    out1, lse1, kind = _decode(gpu, w, t.pool, t, t.kv_indices, t.q)
    assert kind == plan
    pool2, idx2, _ = _relabel(t.pool, t.kv_indices, seed=4)
    out2, lse2, _ = _decode(gpu, w, pool2, t, idx2, t.q)
    assert torch.equal(out1, out2)
    assert torch.equal(lse1, lse2)


def test_decode_e4m3_page_relabel_bit_exact(gpu):
    require_fixed_chunks()
    # the 70B-shaped e4m3 batch: page scales move with their pages
    dec, _ = W.llama3_70b_mixed_fp8(seed=1)
    t = W.materialize(dec, gpu)
    pool, scales = pagedattn.quantize_pages_e4m3(t.pool)
    out1, lse1, _ = _decode(gpu, dec, pool, t, t.kv_indices, t.q, scales=scales)
    pool2, idx2, s2 = _relabel(pool, t.kv_indices, seed=5, scales=scales)
    out2, lse2, _ = _decode(gpu, dec, pool2, t, idx2, t.q, scales=s2)
    assert torch.equal(out1, out2)
    assert torch.equal(lse1, lse2)


def test_prefill_page_relabel_bit_exact(gpu):
    # Llama-3-8B chunked prefill over shared prefixes, full size
    w = W.llama3_8b_prefill(seed=2)
    t = W.materialize(w, gpu)
    out1, lse1 = _prefill(gpu, w, t.pool, t, t.kv_indices, t.q)
    pool2, idx2, _ = _relabel(t.pool, t.kv_indices, seed=6)
    out2, lse2 = _prefill(gpu, w, pool2, t, idx2, t.q)
    assert torch.equal(out1, out2)
    assert torch.equal(lse1, lse2)


@pytest.mark.parametrize("plan", ["shared", "split"])
def test_decode_constant_v_per_sequence(gpu, monkeypatch, plan):
    monkeypatch.setenv("PAGEDATTN_DECODE_SHARED", "1" if plan == "shared" else "0")
    w = W.tinyllama_decode(seed=7)
    t = W.materialize(w, gpu)
    m = w.meta
    g = torch.Generator(device=gpu)
    g.manual_seed(7)
    c = torch.randn((m.batch_size, w.hkv, w.d), generator=g, device=gpu).to(torch.bfloat16)
    _fill_v(t.pool, m, list(range(m.batch_size)), c)
    out, _, kind = _decode(gpu, w, t.pool, t, t.kv_indices, t.q)
    assert kind == plan
    want = c.float().repeat_interleave(w.hq // w.hkv, dim=1)
    _check_close(out, want)


def test_decode_fused_append_zero_q(gpu):
    # the benchmark's decode step, fused append then attention: with q = 0
    # and every earlier V row 0, the output is the appended row over the
    # sequence's token count, so a row written to the wrong slot, page or
    # sequence shows up
    w = W.tinyllama_decode(seed=8)
    t = W.materialize(w, gpu)
    m = w.meta
    _fill_v(t.pool, m, list(range(m.batch_size)),
            torch.zeros((m.batch_size, w.hkv, w.d), device=gpu))
    n = torch.from_numpy(_seq_lens(m).astype(np.float32)).to(gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(8)
    c = torch.randn((m.batch_size, w.hkv, w.d), generator=g, device=gpu)
    v_new = (c * n[:, None, None]).to(torch.bfloat16)
    dw = pagedattn.BatchDecodeWithPagedKVCacheWrapper(workspace(gpu), "HND")
    dw.plan(t.kv_indptr, t.kv_indices, t.kv_last_page_len, w.hq, w.hkv, w.d, 16,
            q_data_type=t.q.dtype)
    out = dw.run(torch.zeros_like(t.q), t.pool, append_key=t.k_new, append_value=v_new)
    torch.cuda.synchronize()
    want = (v_new.float() / n[:, None, None]).repeat_interleave(w.hq // w.hkv, dim=1)
    _check_close(out, want)


def test_prefill_constant_v_per_component(gpu):
    # sequences that share prefix pages get one constant; all others their own
    w = W.llama3_8b_prefill(seed=9)
    t = W.materialize(w, gpu)
    m = w.meta
    comp = _components(m)
    assert len(set(comp)) < m.batch_size  # the workload does share prefixes
    g = torch.Generator(device=gpu)
    g.manual_seed(9)
    c = torch.randn((m.batch_size, w.hkv, w.d), generator=g, device=gpu).to(torch.bfloat16)
    _fill_v(t.pool, m, comp, c)
    out, _ = _prefill(gpu, w, t.pool, t, t.kv_indices, t.q)
    gq = w.hq // w.hkv
    for b in range(m.batch_size):
        rows = out[m.qo_indptr[b]:m.qo_indptr[b + 1]]
        want = c[comp[b]].float().repeat_interleave(gq, dim=0)[None].expand_as(rows)
        _check_close(rows, want)


@pytest.mark.parametrize("plan", ["shared", "split"])
def test_decode_zero_q_is_mean_of_v(gpu, monkeypatch, plan):
    monkeypatch.setenv("PAGEDATTN_DECODE_SHARED", "1" if plan == "shared" else "0")
    w = W.tinyllama_decode(seed=10)
    t = W.materialize(w, gpu)
    m = w.meta
    q = torch.zeros_like(t.q)
    out, _, _ = _decode(gpu, w, t.pool, t, t.kv_indices, q)
    gq = w.hq // w.hkv
    for b in range(m.batch_size):
        want = _v_rows(t.pool, m, b).mean(dim=0).repeat_interleave(gq, dim=0)
        _check_close(out[b], want)


def test_decode_e4m3_zero_q_is_mean_of_v(gpu):
    # e4m3 pages: each page's V scale enters through P and is rounded to
    # bf16 there (relative 2^-9), so the bound adds 2^-8 of the sum of the
    # pages' |partial sums| over the token count
    dec, _ = W.llama3_70b_mixed_fp8(seed=11)
    t = W.materialize(dec, gpu)
    pool, scales = pagedattn.quantize_pages_e4m3(t.pool)
    m = dec.meta
    q = torch.zeros_like(t.q)
    out, _, _ = _decode(gpu, dec, pool, t, t.kv_indices, q, scales=scales)
    gq = dec.hq // dec.hkv
    for b in range(m.batch_size):
        v = _v_rows(pool, m, b, scales=scales)
        n = v.shape[0]
        pad = torch.zeros(((-n) % 16,) + tuple(v.shape[1:]), device=gpu)
        pages = torch.cat([v, pad]).view(-1, 16, *v.shape[1:]).sum(dim=1)
        slack = (2.0 ** -8) * pages.abs().sum(dim=0) / n
        want = v.mean(dim=0)
        err = (out[b].float() - want.repeat_interleave(gq, dim=0)).abs()
        bound = (REL * want.abs() + ABS + slack).repeat_interleave(gq, dim=0)
        assert bool((err <= bound).all()), (b, float((err - bound).max()))


def test_prefill_zero_q_is_causal_mean_of_v(gpu):
    # row i of a chunk of qo tokens over kv_len tokens sees kv_len - qo + i + 1
    w = W.llama3_8b_prefill(seed=12)
    t = W.materialize(w, gpu)
    m = w.meta
    q = torch.zeros_like(t.q)
    out, _ = _prefill(gpu, w, t.pool, t, t.kv_indices, q)
    gq = w.hq // w.hkv
    for b in range(m.batch_size):
        v = _v_rows(t.pool, m, b).double()
        n = v.shape[0]
        qo = int(m.qo_indptr[b + 1] - m.qo_indptr[b])
        csum = torch.cumsum(v, dim=0)
        seen = torch.arange(n - qo + 1, n + 1, device=gpu, dtype=torch.float64)
        want = (csum[n - qo:] / seen[:, None, None]).float().repeat_interleave(gq, dim=1)
        _check_close(out[m.qo_indptr[b]:m.qo_indptr[b + 1]], want)


@pytest.mark.parametrize("kind", ["decode", "prefill"])
def test_fp16_pools_zero_q_is_mean_of_v(gpu, kind):
    # the fp16 kernels at full size: TinyLlama decode and the Llama-3-8B
    # prefill with fp16 pool and q
    w = W.tinyllama_decode(seed=13) if kind == "decode" else W.llama3_8b_prefill(seed=13)
    t = W.materialize(w, gpu, dtype=torch.float16)
    m = w.meta
    q = torch.zeros_like(t.q)
    gq = w.hq // w.hkv
    if kind == "decode":
        out, _, _ = _decode(gpu, w, t.pool, t, t.kv_indices, q)
        for b in range(m.batch_size):
            want = _v_rows(t.pool, m, b).mean(dim=0).repeat_interleave(gq, dim=0)
            _check_close(out[b], want)
    else:
        out, _ = _prefill(gpu, w, t.pool, t, t.kv_indices, q)
        for b in range(m.batch_size):
            v = _v_rows(t.pool, m, b).double()
            n = v.shape[0]
            qo = int(m.qo_indptr[b + 1] - m.qo_indptr[b])
            csum = torch.cumsum(v, dim=0)
            seen = torch.arange(n - qo + 1, n + 1, device=gpu, dtype=torch.float64)
            want = (csum[n - qo:] / seen[:, None, None]).float().repeat_interleave(gq, dim=1)
            _check_close(out[m.qo_indptr[b]:m.qo_indptr[b + 1]], want)
