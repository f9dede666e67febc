"""Shared builders for the GPU parity tests: random paged batches with given
lengths, run helpers for the HIP path, and the oracle comparisons."""

from __future__ import annotations

import math

import numpy as np
import torch

import oracle as O
import pagedattn
from pagedattn.metadata import decode_metadata, prefill_metadata

WS_BYTES = 128 * 1024 * 1024


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


def lse_err(lse, ref, rows=None):
    a = lse.float().cpu()
    if rows is not None:
        a, ref = a[rows], ref[rows]
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(a), fin), "lse -inf pattern differs"
    return float((a[fin] - ref[fin]).abs().max()) if fin.any() else 0.0
