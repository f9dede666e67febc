"""Shared builders for the GPU parity tests: random paged batches with given
lengths, run helpers for the HIP path, and the oracle comparisons."""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

import oracle as O
import pagedattn
from pagedattn.metadata import decode_metadata, prefill_metadata

WS_BYTES = 128 * 1024 * 1024


def require_shared_plans():
    """Skip a test of the shared-item decode plans when the environment
    switches them off (the planner knob PAGEDATTN_DECODE_SHARED=0)."""
    if os.environ.get("PAGEDATTN_DECODE_SHARED") == "0":
        pytest.skip("PAGEDATTN_DECODE_SHARED=0 switches shared-item decode plans off")


def require_fixed_chunks():
    """Skip a bit-equality test of shared-item decode when the environment
    selects arrival-order chunk claims (PAGEDATTN_DECODE_DETERMINISTIC=0),
    under which repeated runs may differ in the last bits."""
    if os.environ.get("PAGEDATTN_DECODE_DETERMINISTIC") == "0":
        pytest.skip("PAGEDATTN_DECODE_DETERMINISTIC=0 claims chunks in arrival order")


def workspace(device) -> torch.Tensor:
    return torch.zeros(WS_BYTES, dtype=torch.uint8, device=device)


def random_tables(rng, lens, extra_pages=3):
    need = [math.ceil(n / 16) for n in lens]
    pool = sum(need) + extra_pages
    perm = rng.permutation(pool)
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n].tolist())
        at += n
    return tables, pool


def strided_rows(n, heads, d, dtype, device, gen, lead=0, tail=0):
    """[n, heads, d] view inside a wider row (like q/k/v views of a fused qkv)."""
    width = (lead + heads + tail) * d
    base = torch.randn((n, width), generator=gen, device=device, dtype=torch.float32).to(dtype)
    return base[:, lead * d:(lead + heads) * d].view(n, heads, d)


def i32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(device)


def decode_case(device, lens, hq, hkv, d, dtype=torch.bfloat16, seed=0, strided_q=True):
    rng = np.random.default_rng(seed)
    tables, num_pages = random_tables(rng, lens)
    meta = decode_metadata(tables, lens)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    pool = torch.randn((num_pages, 2, hkv, 16, d), generator=g, device=device,
                       dtype=torch.float32).to(dtype)
    bsz = len(lens)
    if strided_q:
        q = strided_rows(bsz, hq, d, dtype, device, g, lead=0, tail=2 * hkv)
    else:
        q = torch.randn((bsz, hq, d), generator=g, device=device, dtype=torch.float32).to(dtype)
    return meta, pool, q


def run_decode(device, meta, pool, q, hq, hkv, d, split_pages=0, kv_scales=None, ws=None):
    ws = workspace(device) if ws is None else ws
    w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    w.plan(i32(meta.kv_indptr, device), i32(meta.kv_indices, device),
           i32(meta.kv_last_page_len, device), hq, hkv, d, 16, q_data_type=q.dtype,
           split_pages=split_pages)
    out, lse = w.run(q, pool, kv_scales=kv_scales, return_lse=True)
    torch.cuda.synchronize()
    return out, lse


def compact(meta, pool, batch, scales=None):
    """Pages of the sequences in `batch` copied to a compact CPU pool with
    remapped tables (keeps oracle checks of huge pools cheap)."""
    indptr = [0]
    parts = []
    for b in batch:
        parts.append(meta.kv_indices[meta.kv_indptr[b]:meta.kv_indptr[b + 1]])
        indptr.append(indptr[-1] + len(parts[-1]))
    pages = np.concatenate(parts) if parts else np.zeros(0, np.int64)
    idx = torch.from_numpy(pages.astype(np.int64)).to(pool.device)
    sub = pool.index_select(0, idx).cpu()
    sub_scales = None if scales is None else scales.index_select(0, idx).cpu()
    return (np.asarray(indptr, np.int32), np.arange(len(pages), dtype=np.int32),
            np.asarray(meta.kv_last_page_len)[batch], sub, sub_scales)


def oracle_decode(meta, pool, q, scales=None, batch=None):
    """fp32 oracle rows for all sequences (or `batch`), NaN elsewhere."""
    bsz = len(meta.kv_last_page_len)
    rows = list(range(bsz)) if batch is None else list(batch)
    indptr, ind, last, sub, sub_scales = compact(meta, pool, rows, scales)
    o, l = O.decode(q[rows].float().cpu(), sub, indptr, ind, last, scales=sub_scales)
    out = torch.full((bsz,) + tuple(q.shape[1:]), float("nan"))
    lse = torch.full((bsz, q.shape[1]), float("nan"))
    out[rows] = o
    lse[rows] = l
    return out, lse


def max_err(out, ref, rows=None):
    o = out.float().cpu()
    if rows is not None:
        o, ref = o[rows], ref[rows]
    return float((o - ref).abs().max()) if o.numel() else 0.0


def rel_err(out, ref, rows=None):
    """Largest error of a (row, head) output relative to that row's largest
    reference value: max|out - ref| / max|ref|.  Attention outputs shrink
    like sqrt(1 / kv_len) for N(0, 1) data, so an absolute bound alone would
    accept a near-zero output at long contexts; this one does not."""
    o = out.float().cpu()
    r = ref
    if rows is not None:
        o, r = o[rows], r[rows]
    if not o.numel():
        return 0.0
    num = (o - r).abs().amax(-1)
    den = r.abs().amax(-1)
    keep = torch.isfinite(den) & (den > 0)
    if not bool(keep.any()):
        return 0.0
    return float((num[keep] / den[keep]).max())


def scale_keys_by_page(pool, meta, per_page, seqs=None):
    """Multiplies the K rows of page i of every sequence (i counted within the
    sequence's table) by 1 + per_page * i: scores then grow from page to
    page, so the kernels' online softmax must move its running max (and
    rescale O and l) many times within a sequence, and split pieces carry
    different maxima into the merge."""
    factor = torch.ones(pool.shape[0], dtype=torch.float32)
    for b in (range(len(meta.kv_last_page_len)) if seqs is None else seqs):
        pages = meta.kv_indices[meta.kv_indptr[b]:meta.kv_indptr[b + 1]]
        for i, pg in enumerate(pages.tolist()):
            factor[pg] = 1.0 + per_page * i
    f = factor.to(pool.device)[:, None, None, None]
    pool[:, 0] = (pool[:, 0].float() * f).to(pool.dtype)
    return pool


def log2_max_jumps(meta, pool, q, b, slack=8.0, scales=None, sm_scale=None):
    """How often, over sequence b's pages in order, the running max of the
    scores (log2 units, per query head) rises by more than `slack` past its
    previous value: a lower bound on the rescales a kernel with that slack
    performs."""
    indptr, ind, last, sub, sub_scales = compact(meta, pool, [b], scales)
    k, _ = O.gather_pages(sub, indptr, ind, last, 0, sub_scales)
    hq, d = q.shape[1], q.shape[2]
    g = hq // k.shape[1]
    sc = (1.0 / math.sqrt(d)) if sm_scale is None else sm_scale
    qq = q[b].float().cpu()
    s = torch.einsum("hd,lhd->hl", qq, k.repeat_interleave(g, 1)) * sc / math.log(2.0)
    jumps = 0
    for h in range(hq):
        m = -math.inf
        for lo in range(0, s.shape[1], 16):
            pm = float(s[h, lo:lo + 16].max())
            if pm > m + slack:
                if m != -math.inf:
                    jumps += 1
                m = pm
    return jumps


def lse_err(lse, ref, rows=None):
    a = lse.float().cpu()
    if rows is not None:
        a, ref = a[rows], ref[rows]
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(a), fin), "lse -inf pattern differs"
    return float((a[fin] - ref[fin]).abs().max()) if fin.any() else 0.0


def prefill_case(device, computed, chunks, hq, hkv, d, dtype=torch.bfloat16, seed=0):
    rng = np.random.default_rng(seed)
    lens = [c + n for c, n in zip(computed, chunks)]
    tables, num_pages = random_tables(rng, lens)
    meta = prefill_metadata(tables, computed, chunks)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    pool = torch.randn((num_pages, 2, hkv, 16, d), generator=g, device=device,
                       dtype=torch.float32).to(dtype)
    q = strided_rows(meta.nnz, hq, d, dtype, device, g, lead=0, tail=2 * hkv)
    return meta, pool, q


def run_prefill(device, meta, pool, q, hq, hkv, d, causal=True, kv_scales=None, ws=None):
    ws = workspace(device) if ws is None else ws
    w = pagedattn.BatchPrefillWithPagedKVCacheWrapper(ws, "HND")
    w.plan(i32(meta.qo_indptr, device), i32(meta.kv_indptr, device),
           i32(meta.kv_indices, device), i32(meta.kv_last_page_len, device), hq, hkv, d, 16,
           q_data_type=q.dtype)
    out, lse = w.run(q, pool, kv_scales=kv_scales, return_lse=True, causal=causal)
    torch.cuda.synchronize()
    return out, lse


def oracle_prefill_rows(meta, pool, q, b, lo, hi, causal=True, scales=None):
    """Oracle rows [lo, hi) of sequence b's chunk: a causal row slice is a
    bottom-right aligned chunk over the first kv - qo + hi keys."""
    indptr, ind, last, sub, sub_scales = compact(meta, pool, [b], scales)
    k, v = O.gather_pages(sub, indptr, ind, last, 0, sub_scales)
    qo = int(meta.qo_indptr[b + 1] - meta.qo_indptr[b])
    kv = k.shape[0]
    q0 = int(meta.qo_indptr[b])
    if causal:
        n_keys = max(0, kv - qo + hi)
        return O.attention(q[q0 + lo:q0 + hi].float().cpu(), k[:n_keys], v[:n_keys], causal=True)
    return O.attention(q[q0 + lo:q0 + hi].float().cpu(), k, v, causal=False)


def oracle_prefill(meta, pool, q, causal=True, scales=None, row_block=256):
    n = meta.nnz
    out = torch.full((n,) + tuple(q.shape[1:]), float("nan"))
    lse = torch.full((n, q.shape[1]), float("nan"))
    for b in range(len(meta.kv_last_page_len)):
        qo = int(meta.qo_indptr[b + 1] - meta.qo_indptr[b])
        q0 = int(meta.qo_indptr[b])
        for lo in range(0, qo, row_block):
            hi = min(qo, lo + row_block)
            o, l = oracle_prefill_rows(meta, pool, q, b, lo, hi, causal, scales)
            out[q0 + lo:q0 + hi] = o
            lse[q0 + lo:q0 + hi] = l
    return out, lse
