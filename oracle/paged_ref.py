"""CPU restatement of the paged-attention path (TEST INFRASTRUCTURE ONLY).

Integer/byte work (batch positions, page append, page gather, fp8 encoding)
is numpy over raw bit patterns, so it is bit-exact by construction.
Attention is fp32 torch (fp64 on request): gather the pages of a sequence
into dense K/V, then softmax(scale * q k^T) v with an explicit GQA head map
and a bottom-right aligned causal mask.
"""

from __future__ import annotations

import math

import numpy as np
import torch

PAGE = 16
E4M3_MAX = 448.0

__all__ = [
    "PAGE", "E4M3_MAX", "kv_lengths", "batch_indices_positions", "append_pages",
    "e4m3_encode", "e4m3_decode", "quantize_pages", "append_pages_e4m3",
    "e4m3_clamped_pieces", "pow2_scale",
    "append_pages_e4m3_running", "fork_pages", "gather_pages",
    "attention", "decode", "prefill", "split_attention", "merge_states", "rope",
    "to_bits", "from_bits",
]


# -----------------------------------------------------------------------------
# metadata

def kv_lengths(kv_indptr, last_page_len, page: int = PAGE) -> np.ndarray:
    """kv_len_b = (npages_b - 1) * page + last_page_len_b, 0 for an empty table.
    Follows src/engine/runtime/step_executor.py:116-126, :209-214 (the
    metadata the caller builds) and the kv_last_page_len contract of
    src/models/llama.py:106-116, :138-147.
    Pinned by: tests/test_oracle.py::test_kv_lengths_closed_form."""
    indptr = np.asarray(kv_indptr, dtype=np.int64)
    last = np.asarray(last_page_len, dtype=np.int64)
    npages = indptr[1:] - indptr[:-1]
    return np.where(npages > 0, (npages - 1) * page + last, 0)


def batch_indices_positions(append_indptr, seq_lens, nnz: int):
    """flashinfer.get_batch_indices_positions as called at src/models/llama.py:79-83:
    for j in [append_indptr[b], append_indptr[b+1]):
      batch_indices[j] = b, positions[j] = seq_lens[b] - append_len_b + (j - append_indptr[b]).
    Pinned by: test_batch_positions_loop (pure-Python loop) and
    test_batch_positions_match_caller (the caller's own position_ids,
    step_executor.py:149-152)."""
    indptr = np.asarray(append_indptr, dtype=np.int64)
    lens = np.asarray(seq_lens, dtype=np.int64)
    counts = indptr[1:] - indptr[:-1]
    b = np.repeat(np.arange(len(counts), dtype=np.int64), counts)
    j = np.arange(int(indptr[-1] - indptr[0]), dtype=np.int64) + indptr[0]
    pos = lens[b] - counts[b] + (j - indptr[b])
    bi = np.zeros(nnz, dtype=np.int32)
    po = np.zeros(nnz, dtype=np.int32)
    bi[j] = b
    po[j] = pos
    return bi, po


# -----------------------------------------------------------------------------
# bit views

def to_bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit pattern of a 16- or 8-bit tensor as a numpy uint array."""
    t = t.detach().cpu().contiguous()
    if t.element_size() == 2:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.element_size() == 1:
        return t.view(torch.uint8).numpy()
    raise TypeError(f"unsupported element size {t.element_size()}")


def from_bits(bits: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    """Inverse of to_bits."""
    if dtype in (torch.float16, torch.bfloat16):
        return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dtype)
    if dtype == torch.float8_e4m3fn:
        return torch.from_numpy(np.ascontiguousarray(bits).astype(np.uint8)).view(dtype)
    raise TypeError(dtype)


# -----------------------------------------------------------------------------
# page append (bit-exact scatter)

def _append_targets(batch_indices, positions, kv_indices, kv_indptr, num_pages, page=PAGE):
    bi = np.asarray(batch_indices, dtype=np.int64)
    pos = np.asarray(positions, dtype=np.int64)
    indptr = np.asarray(kv_indptr, dtype=np.int64)
    ind = np.asarray(kv_indices, dtype=np.int64)
    bsz = len(indptr) - 1
    ok = (bi >= 0) & (bi < bsz) & (pos >= 0)
    bic = np.clip(bi, 0, max(bsz - 1, 0))
    it = indptr[bic] + pos // page
    ok &= (it >= indptr[bic]) & (it < indptr[np.minimum(bic + 1, bsz)]) & (it < len(ind))
    page_id = np.where(ok, ind[np.clip(it, 0, max(len(ind) - 1, 0))], -1)
    ok &= (page_id >= 0) & (page_id < num_pages)
    return ok, page_id, pos % page


def append_pages(pool_bits: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray,
                 batch_indices, positions, kv_indices, kv_indptr):
    """flashinfer.append_paged_kv_cache(kv_layout="HND") as called at
    src/models/llama.py:188-210 on the pool of allocator.py:25-36:
      page = kv_indices[kv_indptr[b] + pos // 16], slot = pos % 16,
      pool[page, 0, :, slot, :] = k[j], pool[page, 1, :, slot, :] = v[j].
    Works on raw bits (any element type).  Tokens whose metadata points
    outside the tables are skipped and counted.  Returns (new_pool, skipped).
    Pinned by: test_append_loop (pure-Python loop), test_append_untouched
    (sentinel slots unchanged), test_append_gather_roundtrip."""
    out = pool_bits.copy()
    ok, page_id, slot = _append_targets(batch_indices, positions, kv_indices, kv_indptr,
                                        pool_bits.shape[0])
    js = np.nonzero(ok)[0]
    out[page_id[js], 0, :, slot[js], :] = k_bits[js]
    out[page_id[js], 1, :, slot[js], :] = v_bits[js]
    return out, int((~ok).sum())


# -----------------------------------------------------------------------------
# fp8 e4m3fn (no reference counterpart: the reference pool dtype is the model
# dtype, allocator.py:34)

def e4m3_encode(x: torch.Tensor, scale) -> np.ndarray:
    """round_to_nearest_even(clamp(x / scale, -448, 448)) as e4m3fn bits; x and
    scale are fp32 (scale broadcastable).  Pinned by: test_e4m3_roundtrip_exact
    (every finite e4m3 value maps to itself) and test_e4m3_rounding_ties."""
    y = (x.float() / torch.as_tensor(scale, dtype=torch.float32)).clamp(-E4M3_MAX, E4M3_MAX)
    return y.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def e4m3_decode(bits: np.ndarray, scale) -> torch.Tensor:
    """bits * scale in fp32 (exact: e4m3 values have 4 significant bits)."""
    v = torch.from_numpy(np.ascontiguousarray(bits)).view(torch.float8_e4m3fn).float()
    return v * torch.as_tensor(scale, dtype=torch.float32)


def quantize_pages(pool: torch.Tensor):
    """pool [P, 2, H, 16, D] (bf16/fp16) -> (e4m3 bits, scales [P, 2, H]) with
    scale = amax / 448 of each (page, K|V, head) block, 1.0 for an all-zero
    block.  Pinned by: test_quantize_pages_scale (amax maps to +-448 exactly)."""
    f = pool.float()
    amax = f.abs().amax(dim=(3, 4))
    scale = amax / E4M3_MAX
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    bits = e4m3_encode(f, scale[..., None, None])
    return bits, scale


def _scale_ok(scale: torch.Tensor) -> torch.Tensor:
    return (scale > 0) & torch.isfinite(scale)


def _encode_fixed(x: torch.Tensor, scale: torch.Tensor) -> np.ndarray:
    """e4m3_encode of rows x [n, H, D] with per-(row, head) scales [n, H, 1];
    rows whose scale is not positive and finite become zero codes."""
    bits = e4m3_encode(x, scale)
    bad = (~_scale_ok(scale)).expand_as(x).numpy()
    bits[bad] = 0
    return bits


def append_pages_e4m3(pool_bits: np.ndarray, scales: torch.Tensor, k: torch.Tensor,
                      v: torch.Tensor, batch_indices, positions, kv_indices, kv_indptr):
    """append_pages (the scatter of src/models/llama.py:188-210 onto the
    allocator.py:25-36 layout) into an e4m3 pool with fixed scales: row
    (token j, K|V, head h) landing in page p is stored as
    e4m3(round(clamp(x / scales[p, K|V, h], +-448))), or as zero codes when
    that scale is not positive and finite.  Returns (new_pool_bits, skipped).
    Pinned by: test_append_e4m3_loop (pure-Python per-element loop with a
    brute-force e4m3 rounding) and test_e4m3_pins_catch_planted_mistakes."""
    out = pool_bits.copy()
    ok, page_id, slot = _append_targets(batch_indices, positions, kv_indices, kv_indptr,
                                        pool_bits.shape[0])
    js = np.nonzero(ok)[0]
    if len(js):
        pj = torch.from_numpy(page_id[js])
        ks = scales[pj, 0][:, :, None].float()  # [n, H, 1]
        vs = scales[pj, 1][:, :, None].float()
        out[page_id[js], 0, :, slot[js], :] = _encode_fixed(k[js].float(), ks)
        out[page_id[js], 1, :, slot[js], :] = _encode_fixed(v[js].float(), vs)
    return out, int((~ok).sum())


def e4m3_clamped_pieces(k: torch.Tensor, v: torch.Tensor, scales: torch.Tensor,
                        batch_indices, positions, kv_indices, kv_indptr,
                        num_pages: int) -> int:
    """What a fixed-scale e4m3 append counts besides skipped tokens: over the
    rows it writes (token, K|V, head), the 8-element pieces [8i, 8i + 8) in
    which some |x / scale| > 448 (the clamp changes a value) or whose scale is
    not positive and finite.
    Pinned by: test_e4m3_clamped_pieces_loop (pure-Python loop)."""
    ok, page_id, _ = _append_targets(batch_indices, positions, kv_indices, kv_indptr,
                                     num_pages)
    js = np.nonzero(ok)[0]
    if not len(js):
        return 0
    pj = torch.from_numpy(page_id[js])
    n = 0
    for kind, src in ((0, k), (1, v)):
        x = src[js].float()  # [n, H, D]
        s = scales[pj, kind][:, :, None].float()
        over = ~((x / s).abs() <= E4M3_MAX)  # NaN counts as over
        over = over | ~_scale_ok(s)
        d = x.shape[-1]
        n += int(over.reshape(x.shape[0], x.shape[1], d // 8, 8).any(-1).sum())
    return n


def pow2_scale(amax) -> np.ndarray:
    """Smallest power of two s with 448 * s >= amax, per element; 0 where
    amax == 0; never below 2**-126.  With amax = m * 2**e (m in [0.5, 1)),
    448 = 0.875 * 2**9 gives s = 2**(e - 9 + [m > 0.875]).
    Pinned by: test_pow2_scale_brute (ldexp search over every exponent) and
    test_running_amax_scale_bounds."""
    a = np.asarray(amax, dtype=np.float32)
    m, e = np.frexp(a)
    ex = np.maximum(e.astype(np.int64) - 9 + (m > np.float32(0.875)), -126)
    s = np.ldexp(np.float32(1.0), ex).astype(np.float32)
    return np.where(a > 0, s, np.float32(0.0)).astype(np.float32)


def _runs(bi: np.ndarray, pos: np.ndarray):
    """Maximal runs of tokens that continue one another inside one page: token
    t continues t - 1 iff same batch index, position + 1 and not a page start."""
    n = len(bi)
    t = 0
    while t < n:
        e = t + 1
        while e < n and bi[e] == bi[e - 1] and pos[e] == pos[e - 1] + 1 and pos[e] % PAGE != 0:
            e += 1
        yield t, e
        t = e


def append_pages_e4m3_running(pool_bits: np.ndarray, scales: torch.Tensor, k: torch.Tensor,
                              v: torch.Tensor, batch_indices, positions, kv_indices,
                              kv_indptr):
    """e4m3 page append that keeps each (page, K|V, head) scale a running
    amax (no reference counterpart; the engine's fp8 write path).  Runs of
    consecutive tokens landing in one page are applied in token order:
      s_old = scale if the run starts past slot 0 else 0
      s_new = max(s_old, pow2_scale(amax of the run's rows))
      if s_new > s_old: rows [0, slot0) <- encode(decode(rows) * (s_old / s_new))
      run rows <- encode(x / s_new)   (all zero codes when s_new == 0)
    With power-of-two scales the re-encode is exact for values that stay in
    e4m3's normal range.  Returns (new_pool_bits, new_scales, skipped).
    Pinned by: test_running_append_one_shot_equals_incremental,
    test_running_append_fresh_page_equals_direct and
    test_running_amax_scale_bounds."""
    out = pool_bits.copy()
    sc = scales.clone().float()
    bi = np.asarray(batch_indices, dtype=np.int64)
    pos = np.asarray(positions, dtype=np.int64)
    ok, page_id, slot = _append_targets(bi, pos, kv_indices, kv_indptr, pool_bits.shape[0])
    skipped = 0
    for t0, t1 in _runs(bi, pos):
        if not ok[t0]:
            skipped += t1 - t0
            continue
        pg = int(page_id[t0])
        s0 = int(slot[t0])
        for kind, src in ((0, k), (1, v)):
            rows = src[t0:t1].float()  # [n, H, D]
            amax = rows.abs().amax(dim=(0, 2)).numpy()  # [H]
            s_old = sc[pg, kind].numpy() if s0 > 0 else np.zeros_like(amax)
            s_new = np.maximum(s_old, pow2_scale(amax)).astype(np.float32)
            for h in range(rows.shape[1]):
                if s0 > 0 and s_new[h] > s_old[h]:
                    r = np.float32(s_old[h]) / np.float32(s_new[h])
                    old = e4m3_decode(out[pg, kind, h, :s0], 1.0) * torch.tensor(r)
                    out[pg, kind, h, :s0] = (
                        old.clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
                        .view(torch.uint8).numpy())
                if s_new[h] > 0:
                    out[pg, kind, h, s0:s0 + (t1 - t0)] = e4m3_encode(rows[:, h], s_new[h])
                else:
                    out[pg, kind, h, s0:s0 + (t1 - t0)] = 0
                sc[pg, kind, h] = float(s_new[h])
    return out, sc, skipped


def fork_pages(pool_bits: np.ndarray, src_pages, dst_pages, valid_tokens=None,
               scales: torch.Tensor | None = None):
    """Copy-on-write page fork over a whole pool [L, P, 2, H, 16, D]
    (allocator.py:25-36 layout; the fork itself is the CoW step the
    reference's todo.md:17-19 asks for): for every fork f and layer l,
    rows [0, n_f) of every (K|V, head) block of page src_f are copied to
    page dst_f (n_f = valid_tokens[f], 16 when absent); scales [L, P, 2, H]
    follow.  Forks with a page or count out of range are skipped and counted.
    Returns (new_pool_bits, new_scales, skipped).
    Pinned by: test_fork_pages_loop (pure-Python loop) and
    test_fork_then_gather."""
    out = pool_bits.copy()
    sc = scales.clone() if scales is not None else None
    num_pages = pool_bits.shape[1]
    skipped = 0
    for f, (s, d) in enumerate(zip(src_pages, dst_pages)):
        n = PAGE if valid_tokens is None else int(valid_tokens[f])
        if not (0 <= s < num_pages and 0 <= d < num_pages and 0 <= n <= PAGE):
            skipped += 1
            continue
        out[:, d, :, :, :n, :] = pool_bits[:, s, :, :, :n, :]
        if sc is not None:
            sc[:, d] = scales[:, s]
    return out, sc, skipped


# -----------------------------------------------------------------------------
# gather

def gather_pages(pool: torch.Tensor, kv_indptr, kv_indices, last_page_len, b: int,
                 scales: torch.Tensor | None = None, dtype=torch.float32):
    """Dense K, V [kv_len, H, D] of sequence b from the HND pool
    (allocator.py:25-36 layout; kv_indices[kv_indptr[b]:kv_indptr[b+1]] is the
    block table, step_executor.py:137-144).  e4m3 pools are dequantised with
    their per-(page, K|V, head) scales: code_value(bits) * scales[page, K|V, h].
    Pinned by: test_append_gather_roundtrip, test_gather_permutation (permuting
    physical pages permutes nothing), test_gather_e4m3_loop (pure-Python
    per-element decode loop) and test_e4m3_pins_catch_planted_mistakes."""
    indptr = np.asarray(kv_indptr, dtype=np.int64)
    ind = np.asarray(kv_indices, dtype=np.int64)
    pages = ind[indptr[b]:indptr[b + 1]]
    kv_len = int(kv_lengths(indptr[b:b + 2], [np.asarray(last_page_len)[b]])[0])
    if len(pages) == 0:
        h, d = pool.shape[2], pool.shape[4]
        z = torch.zeros((0, h, d), dtype=dtype)
        return z, z.clone()
    pt = torch.from_numpy(pages)
    blk = pool[pt]  # [n, 2, H, 16, D]
    if pool.dtype == torch.float8_e4m3fn:
        blk = blk.float() * scales[pt][..., None, None].float()
    blk = blk.to(dtype)
    k = blk[:, 0].permute(0, 2, 1, 3).reshape(-1, pool.shape[2], pool.shape[4])[:kv_len]
    v = blk[:, 1].permute(0, 2, 1, 3).reshape(-1, pool.shape[2], pool.shape[4])[:kv_len]
    return k, v


# -----------------------------------------------------------------------------
# attention

def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
              sm_scale: float | None = None):
    """One sequence: q [n, Hq, D], k/v [L, Hkv, D] -> (out [n, Hq, D], lse [n, Hq]).
    Query head h reads kv head h // (Hq / Hkv).  With causal, row i sees key j
    iff j <= L - n + i (bottom-right aligned, the mask FlashInfer applies for
    causal=True at src/models/llama.py:218-222).  lse is the natural-log
    softmax denominator of the scaled scores; rows that see no key give 0 and
    -inf.  Computed in the dtype of q (fp32 or fp64).
    Pinned by: test_attention_* known answers (kv_len 1, equal V rows, q = 0,
    MHA vs torch SDPA, square causal vs SDPA is_causal, page permutation) and
    the fp64 brute-force golden vectors in tests/golden/."""
    n, hq, d = q.shape
    L, hkv, _ = k.shape
    g = hq // hkv
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    # query head h = kv_head * g + r reads kv head h // g
    qg = q.reshape(n, hkv, g, d)
    s = torch.einsum("nkrd,lkd->krnl", qg, k.to(q.dtype)) * sm_scale  # [Hkv, g, n, L]
    if causal:
        i = torch.arange(n)[:, None]
        j = torch.arange(L)[None, :]
        s = s.masked_fill(j > (L - n + i), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)  # [Hkv, g, n]
    finite = torch.isfinite(lse)
    p = torch.exp(s - torch.where(finite, lse, torch.zeros_like(lse))[..., None])
    p = torch.where(finite[..., None], p, torch.zeros_like(p))
    out = torch.einsum("krnl,lkd->nkrd", p, v.to(q.dtype)).reshape(n, hq, d)
    lse = lse.reshape(hq, n)
    return out, lse.transpose(0, 1).contiguous()


def decode(q: torch.Tensor, pool: torch.Tensor, kv_indptr, kv_indices, last_page_len,
           sm_scale: float | None = None, scales: torch.Tensor | None = None,
           batch: list[int] | None = None):
    """BatchDecodeWithPagedKVCacheWrapper.forward (src/models/llama.py:230-245):
    one query row per sequence, no mask.  q [B, Hq, D]; returns fp32
    (out [B, Hq, D], lse [B, Hq]); `batch` restricts to a subset (rows of the
    others are left NaN)."""
    bsz, hq, d = q.shape
    out = torch.full((bsz, hq, d), float("nan"))
    lse = torch.full((bsz, hq), float("nan"))
    for b in (range(bsz) if batch is None else batch):
        k, v = gather_pages(pool, kv_indptr, kv_indices, last_page_len, b, scales)
        o, l = attention(q[b:b + 1].float(), k, v, causal=False, sm_scale=sm_scale)
        out[b] = o[0]
        lse[b] = l[0]
    return out, lse


def prefill(q: torch.Tensor, qo_indptr, pool: torch.Tensor, kv_indptr, kv_indices,
            last_page_len, causal: bool = True, sm_scale: float | None = None,
            scales: torch.Tensor | None = None, batch: list[int] | None = None):
    """BatchPrefillWithPagedKVCacheWrapper.forward (src/models/llama.py:212-228):
    ragged rows q[qo_indptr[b]:qo_indptr[b+1]] against sequence b's pages."""
    qo = np.asarray(qo_indptr, dtype=np.int64)
    n, hq, d = q.shape
    out = torch.full((n, hq, d), float("nan"))
    lse = torch.full((n, hq), float("nan"))
    for b in (range(len(qo) - 1) if batch is None else batch):
        lo, hi = int(qo[b]), int(qo[b + 1])
        if hi == lo:
            continue
        k, v = gather_pages(pool, kv_indptr, kv_indices, last_page_len, b, scales)
        o, l = attention(q[lo:hi].float(), k, v, causal=causal, sm_scale=sm_scale)
        out[lo:hi] = o
        lse[lo:hi] = l
    return out, lse


def split_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, chunk: int,
                    sm_scale: float | None = None):
    """Decode attention of one sequence over kv chunks [c*chunk, (c+1)*chunk):
    list of (o_c, lse_c) partials (FlashInfer's internal split-KV, explicit in
    the long-context decode workload)."""
    parts = []
    for lo in range(0, k.shape[0], chunk):
        parts.append(attention(q, k[lo:lo + chunk], v[lo:lo + chunk], causal=False,
                               sm_scale=sm_scale))
    return parts


def merge_states(outs, lses):
    """Log-sum-exp merge: lse = log sum_c e^{lse_c}, o = sum_c e^{lse_c - lse} o_c.
    Pinned by: test_merge_identity (split at any chunk equals the unsplit
    result; merging one state is the identity)."""
    l = torch.stack(lses)  # [C, n, H]
    o = torch.stack(outs)  # [C, n, H, D]
    lse = torch.logsumexp(l, dim=0)
    finite = torch.isfinite(lse)
    w = torch.exp(l - torch.where(finite, lse, torch.zeros_like(lse)))
    w = torch.where(finite, w, torch.zeros_like(w))
    return (w[..., None] * o).sum(0), lse


# -----------------------------------------------------------------------------
# RoPE

def rope(x: torch.Tensor, pos, theta: float, scale: float = 1.0, rotary_dim: int | None = None,
         interleave: bool = False) -> torch.Tensor:
    """flashinfer.apply_rope_pos_ids_inplace (src/models/llama.py:175-182) on
    x [N, H, D] (fp32 result): angle_i = (pos / scale) * theta^(-2i/rotary_dim),
    rotate-half pairs (i, i + rotary_dim/2) or interleaved pairs (2i, 2i+1).
    Angles are formed in fp64.  Pinned by: test_rope_matches_transformers
    (transformers' rotate_half / apply_rotary_pos_emb, modeling_llama.py),
    test_rope_is_rotation (norm preserved, pos 0 is the identity) and, for the
    interleaved pairs, test_rope_interleave_closed_form (rotate-half RoPE of
    the de-interleaved vector, re-interleaved; a planted -angle rotation and
    planted rotate-half pairs fail it)."""
    n, h, d = x.shape
    rd = rotary_dim or d
    half = rd // 2
    i = torch.arange(half, dtype=torch.float64)
    inv_freq = theta ** (-(2.0 * i) / rd)
    p = torch.as_tensor(np.asarray(pos), dtype=torch.float64)
    ang = (p[:, None] / scale) * inv_freq[None, :]  # [N, half]
    c = torch.cos(ang).float()[:, None, :]
    s = torch.sin(ang).float()[:, None, :]
    y = x.float().clone()
    if interleave:
        a, b = x[..., 0:rd:2].float(), x[..., 1:rd:2].float()
        y[..., 0:rd:2] = a * c - b * s
        y[..., 1:rd:2] = b * c + a * s
    else:
        a, b = x[..., :half].float(), x[..., half:rd].float()
        y[..., :half] = a * c - b * s
        y[..., half:rd] = b * c + a * s
    return y
