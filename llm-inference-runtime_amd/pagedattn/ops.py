"""FlashInfer-compatible Python surface over libpagedattn.

These are the FlashInfer entry points the serving engine calls on its
attention path (src/models/llama.py:3, :49-67, :79-83, :106-116, :138-147,
:175-182, :188-210, :218-222, :236-239), with the same names, argument
meaning and error behaviour (Python exceptions, never a device fault):

* ``get_batch_indices_positions``
* ``apply_rope_pos_ids_inplace``
* ``append_paged_kv_cache``
* ``BatchDecodeWithPagedKVCacheWrapper`` (``plan``/``begin_forward``,
  ``run``/``forward``)
* ``BatchPrefillWithPagedKVCacheWrapper`` (same)

Only the "HND" pool layout the engine uses is implemented
([num_pages, 2, num_kv_heads, page_size, head_dim] per layer).  Options the
engine never passes (positional encoding inside attention, sliding windows,
logit soft-capping, custom masks) raise NotImplementedError.

Additions with no FlashInfer counterpart: ``build_paged_metadata`` (the
step metadata built on the device), ``quantize_pages_e4m3``, the
``kv_scales`` argument for e4m3 pools with per-(page, K|V, kv-head) scales,
``append_paged_kv_cache_e4m3_amax`` (e4m3 append that maintains those
scales as pages fill) and ``fork_pages`` (copy-on-write page fork).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call, dtype_code, ptr

PAGE_SIZE = 16


def _dtype_of(x) -> torch.dtype:
    if isinstance(x, torch.dtype):
        return x
    if isinstance(x, str):
        return getattr(torch, x)
    raise TypeError(f"not a dtype: {x!r}")


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device (cuda/hip) tensor, got {t.device}")


def _i32(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    return t.to(device=device, dtype=torch.int32).contiguous()


def _host_i32(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to("cpu", torch.int32).contiguous()


def _stream(device: torch.device) -> int:
    return _lib.stream_of(device)


def _check_pool(paged_kv_cache, num_kv_heads: int | None, head_dim: int | None,
                kv_layout: str) -> tuple[int, int, int]:
    if kv_layout != "HND":
        raise NotImplementedError(
            f"kv_layout {kv_layout!r}: only the HND page layout is implemented")
    if isinstance(paged_kv_cache, (tuple, list)):
        raise NotImplementedError(
            "separate (k_cache, v_cache) tensors are not supported; pass the "
            "[num_pages, 2, num_kv_heads, page_size, head_dim] layer pool")
    _require_cuda(paged_kv_cache, "paged_kv_cache")
    if paged_kv_cache.dim() != 5 or paged_kv_cache.shape[1] != 2:
        raise ValueError(
            "paged_kv_cache must be [num_pages, 2, num_kv_heads, page_size, "
            f"head_dim], got {tuple(paged_kv_cache.shape)}")
    p, _, hkv, page, d = paged_kv_cache.shape
    if page != PAGE_SIZE:
        raise NotImplementedError(f"page_size {page} (only 16 is implemented)")
    if num_kv_heads is not None and hkv != num_kv_heads:
        raise ValueError(f"pool has {hkv} kv heads, plan says {num_kv_heads}")
    if head_dim is not None and d != head_dim:
        raise ValueError(f"pool head_dim {d}, plan says {head_dim}")
    if not paged_kv_cache.is_contiguous():
        raise ValueError("paged_kv_cache (one layer of the pool) must be contiguous")
    return p, hkv, d


def _check_scales(kv_scales, paged_kv_cache) -> torch.Tensor | None:
    if paged_kv_cache.dtype != torch.float8_e4m3fn:
        return None
    if kv_scales is None:
        raise ValueError("an e4m3 pool needs kv_scales [num_pages, 2, num_kv_heads]")
    p, _, hkv, _, _ = paged_kv_cache.shape
    if kv_scales.dtype != torch.float32 or tuple(kv_scales.shape) != (p, 2, hkv):
        raise ValueError(
            f"kv_scales must be float32 [{p}, 2, {hkv}], got "
            f"{kv_scales.dtype} {tuple(kv_scales.shape)}")
    _require_cuda(kv_scales, "kv_scales")
    return kv_scales.contiguous()


def _check_rows(x: torch.Tensor, name: str, heads: int | None, d: int | None):
    _require_cuda(x, name)
    if x.dim() != 3:
        raise ValueError(f"{name} must be [tokens, heads, head_dim], got {tuple(x.shape)}")
    if heads is not None and x.shape[1] != heads:
        raise ValueError(f"{name} has {x.shape[1]} heads, expected {heads}")
    if d is not None and x.shape[2] != d:
        raise ValueError(f"{name} head_dim {x.shape[2]}, expected {d}")
    if x.shape[0] > 0 and x.stride(2) != 1:
        raise ValueError(f"{name}: the head_dim axis must be contiguous")


# -----------------------------------------------------------------------------
def get_batch_indices_positions(append_indptr: torch.Tensor, seq_lens: torch.Tensor,
                                nnz: int) -> tuple[torch.Tensor, torch.Tensor]:
    """batch_indices[j] = b and positions[j] = seq_lens[b] - append_len_b + (j - append_indptr[b])
    for j in [append_indptr[b], append_indptr[b+1]) (src/models/llama.py:70-83)."""
    _require_cuda(append_indptr, "append_indptr")
    device = append_indptr.device
    indptr = _i32(append_indptr, device)
    lens = _i32(seq_lens, device)
    bsz = lens.numel()
    if indptr.numel() != bsz + 1:
        raise ValueError(f"append_indptr has {indptr.numel()} entries for {bsz} sequences")
    nnz = int(nnz)
    bi = torch.empty(nnz, dtype=torch.int32, device=device)
    pos = torch.empty(nnz, dtype=torch.int32, device=device)
    call("pagedattn_get_batch_indices_positions", ptr(indptr), ptr(lens), bsz, nnz,
         ptr(bi), ptr(pos), _stream(device))
    return bi, pos


def apply_rope_pos_ids_inplace(q: torch.Tensor, k: torch.Tensor, pos_ids: torch.Tensor,
                               rotary_dim: int | None = None, interleave: bool = False,
                               rope_scale: float = 1.0, rope_theta: float = 1e4) -> None:
    """RoPE in place on q [nnz, Hq, D] and k [nnz, Hkv, D] (src/models/llama.py:175-182)."""
    _check_rows(q, "q", None, None)
    _check_rows(k, "k", None, q.shape[2])
    if q.dtype != k.dtype:
        raise ValueError("q and k must share a dtype")
    if k.shape[0] != q.shape[0] or pos_ids.numel() != q.shape[0]:
        raise ValueError("q, k and pos_ids must have the same number of tokens")
    nnz, hq, d = q.shape
    hkv = k.shape[1]
    pos = _i32(pos_ids, q.device)
    call("pagedattn_apply_rope_pos_ids_inplace", ptr(q), ptr(k), ptr(pos), nnz, hq, hkv, d,
         int(rotary_dim or d), q.stride(0), q.stride(1), k.stride(0), k.stride(1),
         int(bool(interleave)), float(rope_scale), float(rope_theta), dtype_code(q.dtype),
         _stream(q.device))


def _check_error_flag(error_flag: torch.Tensor | None, n: int) -> None:
    if error_flag is None:
        return
    if (error_flag.dtype != torch.int32 or error_flag.numel() < n
            or not error_flag.is_contiguous() or error_flag.device.type != "cuda"):
        raise ValueError(f"error_flag must be a contiguous int32 device tensor of at least {n} "
                         "entries")


def append_paged_kv_cache(append_key: torch.Tensor, append_value: torch.Tensor,
                          batch_indices: torch.Tensor, positions: torch.Tensor,
                          paged_kv_cache: torch.Tensor, kv_indices: torch.Tensor,
                          kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor,
                          kv_layout: str = "NHD", kv_scales: torch.Tensor | None = None,
                          error_flag: torch.Tensor | None = None) -> None:
    """Scatter k/v rows into their pages (src/models/llama.py:188-210).

    Bit-exact for a pool of the source dtype; an e4m3 pool stores
    round(clamp(x / scale, +-448)) with kv_scales [num_pages, 2, Hkv] (zero
    codes where a scale is not positive and finite).
    `error_flag` (int32 device tensor, optional): error_flag[0] is
    incremented once per token whose metadata pointed outside the page table
    (the token is skipped); for an e4m3 pool it holds two int32 and
    error_flag[1] is incremented once per 8-element piece of a written row
    that was clamped or had a bad scale.  Zeros mean every token landed
    intact."""
    num_pages, hkv, d = _check_pool(paged_kv_cache, None, None, kv_layout)
    _check_rows(append_key, "append_key", hkv, d)
    _check_rows(append_value, "append_value", hkv, d)
    if append_key.dtype != append_value.dtype:
        raise ValueError("append_key and append_value must share a dtype")
    nnz = append_key.shape[0]
    if append_value.shape[0] != nnz or batch_indices.numel() != nnz or positions.numel() != nnz:
        raise ValueError("append_key/value, batch_indices and positions disagree on nnz")
    scales = _check_scales(kv_scales, paged_kv_cache)
    if paged_kv_cache.dtype not in (append_key.dtype, torch.float8_e4m3fn):
        raise ValueError(f"pool dtype {paged_kv_cache.dtype} cannot take {append_key.dtype} rows")
    device = paged_kv_cache.device
    bi = _i32(batch_indices, device)
    pos = _i32(positions, device)
    ind = _i32(kv_indices, device)
    indptr = _i32(kv_indptr, device)
    bsz = indptr.numel() - 1
    _check_error_flag(error_flag, 2 if paged_kv_cache.dtype == torch.float8_e4m3fn else 1)
    call("pagedattn_append_paged_kv_cache", ptr(append_key), ptr(append_value),
         append_key.stride(0), append_key.stride(1), append_value.stride(0),
         append_value.stride(1), dtype_code(append_key.dtype), ptr(bi), ptr(pos), nnz,
         ptr(paged_kv_cache), dtype_code(paged_kv_cache.dtype), ptr(scales), num_pages,
         ptr(ind), ind.numel(), ptr(indptr), ptr(kv_last_page_len), bsz, hkv, d, PAGE_SIZE,
         ptr(error_flag), _stream(device))


def rope_append_paged_kv_cache(q: torch.Tensor, append_key: torch.Tensor,
                               append_value: torch.Tensor, batch_indices: torch.Tensor,
                               positions: torch.Tensor, paged_kv_cache: torch.Tensor,
                               kv_indices: torch.Tensor, kv_indptr: torch.Tensor,
                               kv_last_page_len: torch.Tensor, kv_layout: str = "NHD",
                               rope_scale: float = 1.0, rope_theta: float = 1e4,
                               kv_scales: torch.Tensor | None = None,
                               error_flag: torch.Tensor | None = None) -> None:
    """apply_rope_pos_ids_inplace(q, append_key, positions, interleave=False)
    followed by append_paged_kv_cache(...) in one launch
    (src/models/llama.py:175-210): q and append_key are rotated in place, the
    rotated K rows and the V rows land in their pages.  Same results as the
    two calls."""
    num_pages, hkv, d = _check_pool(paged_kv_cache, None, None, kv_layout)
    _check_rows(q, "q", None, d)
    _check_rows(append_key, "append_key", hkv, d)
    _check_rows(append_value, "append_value", hkv, d)
    if not (q.dtype == append_key.dtype == append_value.dtype):
        raise ValueError("q, append_key and append_value must share a dtype")
    nnz = append_key.shape[0]
    if (q.shape[0] != nnz or append_value.shape[0] != nnz or batch_indices.numel() != nnz
            or positions.numel() != nnz):
        raise ValueError("q, append_key/value, batch_indices and positions disagree on nnz")
    scales = _check_scales(kv_scales, paged_kv_cache)
    if paged_kv_cache.dtype not in (append_key.dtype, torch.float8_e4m3fn):
        raise ValueError(f"pool dtype {paged_kv_cache.dtype} cannot take {append_key.dtype} rows")
    device = paged_kv_cache.device
    bi = _i32(batch_indices, device)
    pos = _i32(positions, device)
    ind = _i32(kv_indices, device)
    indptr = _i32(kv_indptr, device)
    bsz = indptr.numel() - 1
    _check_error_flag(error_flag, 2 if paged_kv_cache.dtype == torch.float8_e4m3fn else 1)
    call("pagedattn_rope_append_paged_kv_cache", ptr(q), q.stride(0), q.stride(1), q.shape[1],
         ptr(append_key), ptr(append_value), append_key.stride(0), append_key.stride(1),
         append_value.stride(0), append_value.stride(1), dtype_code(append_key.dtype), ptr(bi),
         ptr(pos), nnz, float(rope_scale), float(rope_theta), ptr(paged_kv_cache),
         dtype_code(paged_kv_cache.dtype), ptr(scales), num_pages, ptr(ind), ind.numel(),
         ptr(indptr), bsz, hkv, d, PAGE_SIZE, ptr(error_flag), _stream(device))


def append_paged_kv_cache_e4m3_amax(append_key: torch.Tensor, append_value: torch.Tensor,
                                    batch_indices: torch.Tensor, positions: torch.Tensor,
                                    paged_kv_cache: torch.Tensor, kv_indices: torch.Tensor,
                                    kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor,
                                    kv_scales: torch.Tensor, kv_layout: str = "HND",
                                    error_flag: torch.Tensor | None = None) -> None:
    """append_paged_kv_cache into an e4m3 pool that keeps every (page, K|V,
    kv-head) scale a running amax as the page fills (no FlashInfer
    counterpart: the engine's fp8 write path).

    Tokens of one sequence that land in one page must be consecutive and in
    position order (what get_batch_indices_positions produces); the scale of
    that page becomes max(old scale, smallest power of two s with 448 s >=
    amax of the new rows) -- the old scale only counts when the page already
    holds rows.  When the scale grows, the rows already in the page are
    re-encoded with it (an exact exponent shift for values that stay in
    e4m3's normal range).  kv_scales [num_pages, 2, Hkv] is updated in place.
    Two sequences writing one page in the same call race: fork shared pages
    first (fork_pages)."""
    num_pages, hkv, d = _check_pool(paged_kv_cache, None, None, kv_layout)
    if paged_kv_cache.dtype != torch.float8_e4m3fn:
        raise ValueError("append_paged_kv_cache_e4m3_amax needs an e4m3 pool")
    _check_rows(append_key, "append_key", hkv, d)
    _check_rows(append_value, "append_value", hkv, d)
    if append_key.dtype != append_value.dtype:
        raise ValueError("append_key and append_value must share a dtype")
    nnz = append_key.shape[0]
    if append_value.shape[0] != nnz or batch_indices.numel() != nnz or positions.numel() != nnz:
        raise ValueError("append_key/value, batch_indices and positions disagree on nnz")
    scales = _check_scales(kv_scales, paged_kv_cache)
    if scales is None or scales.data_ptr() != kv_scales.data_ptr():
        raise ValueError("kv_scales must be contiguous: it is updated in place")
    device = paged_kv_cache.device
    bi = _i32(batch_indices, device)
    pos = _i32(positions, device)
    ind = _i32(kv_indices, device)
    indptr = _i32(kv_indptr, device)
    bsz = indptr.numel() - 1
    if error_flag is not None and (error_flag.dtype != torch.int32 or error_flag.numel() < 1):
        raise ValueError("error_flag must be an int32 device tensor")
    call("pagedattn_append_paged_kv_cache_e4m3_amax", ptr(append_key), ptr(append_value),
         append_key.stride(0), append_key.stride(1), append_value.stride(0),
         append_value.stride(1), dtype_code(append_key.dtype), ptr(bi), ptr(pos), nnz,
         ptr(paged_kv_cache), ptr(scales), num_pages, ptr(ind), ind.numel(), ptr(indptr), bsz,
         hkv, d, PAGE_SIZE, ptr(error_flag), _stream(device))


def fork_pages(kv_pool: torch.Tensor, src_pages, dst_pages, valid_tokens=None,
               kv_scales: torch.Tensor | None = None,
               error_flag: torch.Tensor | None = None) -> None:
    """Copy-on-write fork of pages across every layer of the engine's pool
    [L, num_pages, 2, Hkv, 16, D] (allocator.py:25-36 layout): for fork f,
    rows [0, valid_tokens[f]) (all 16 when valid_tokens is None) of every
    (K|V, kv-head) block of page src_pages[f] are copied to page
    dst_pages[f] in every layer; e4m3 pools copy kv_scales [L, P, 2, Hkv]
    entries too.  No FlashInfer counterpart: the reference's todo.md:17-19
    asks for this before a sequence appends to a shared partial block.

    Page lists given on the host are checked here (in range, destinations
    distinct and not among the sources); device tensors are checked in the
    kernel, which skips a bad fork and counts it in `error_flag`."""
    _require_cuda(kv_pool, "kv_pool")
    if kv_pool.dim() != 6 or kv_pool.shape[2] != 2 or kv_pool.shape[4] != PAGE_SIZE:
        raise ValueError("kv_pool must be [L, num_pages, 2, num_kv_heads, 16, head_dim], "
                         f"got {tuple(kv_pool.shape)}")
    if not kv_pool.is_contiguous():
        raise ValueError("kv_pool must be contiguous")
    n_layers, num_pages, _, hkv, _, d = kv_pool.shape
    device = kv_pool.device
    scales = None
    if kv_pool.dtype == torch.float8_e4m3fn:
        if kv_scales is None:
            raise ValueError("an e4m3 pool needs kv_scales [L, num_pages, 2, num_kv_heads]")
        if (kv_scales.dtype != torch.float32 or not kv_scales.is_contiguous()
                or tuple(kv_scales.shape) != (n_layers, num_pages, 2, hkv)):
            raise ValueError(f"kv_scales must be contiguous float32 [{n_layers}, {num_pages}, "
                             f"2, {hkv}], got {kv_scales.dtype} {tuple(kv_scales.shape)}")
        _require_cuda(kv_scales, "kv_scales")
        scales = kv_scales

    def as_dev(x, name):
        if isinstance(x, torch.Tensor) and x.device.type == "cuda":
            return _i32(x, device), None
        host = torch.as_tensor(x, dtype=torch.int64).reshape(-1)
        return host.to(device=device, dtype=torch.int32), host

    src, src_h = as_dev(src_pages, "src_pages")
    dst, dst_h = as_dev(dst_pages, "dst_pages")
    if src.numel() != dst.numel():
        raise ValueError("src_pages and dst_pages differ in length")
    valid = None
    valid_h = None
    if valid_tokens is not None:
        valid, valid_h = as_dev(valid_tokens, "valid_tokens")
        if valid.numel() != src.numel():
            raise ValueError("valid_tokens must have one entry per fork")
    if src_h is not None and dst_h is not None:
        for name, h in (("src_pages", src_h), ("dst_pages", dst_h)):
            if h.numel() and (int(h.min()) < 0 or int(h.max()) >= num_pages):
                raise ValueError(f"{name} outside [0, {num_pages})")
        moved = dst_h[dst_h != src_h]
        if moved.unique().numel() != moved.numel():
            raise ValueError("dst_pages must be distinct")
        if bool(torch.isin(moved, src_h).any()):
            raise ValueError("a destination page is also a source page")
    if valid_h is not None and valid_h.numel() and (
            int(valid_h.min()) < 0 or int(valid_h.max()) > PAGE_SIZE):
        raise ValueError(f"valid_tokens outside [0, {PAGE_SIZE}]")
    if error_flag is not None and (error_flag.dtype != torch.int32 or error_flag.numel() < 1):
        raise ValueError("error_flag must be an int32 device tensor")
    call("pagedattn_fork_pages", ptr(kv_pool), dtype_code(kv_pool.dtype), n_layers, num_pages,
         hkv, d, PAGE_SIZE, ptr(scales), ptr(src), ptr(dst), ptr(valid), src.numel(),
         ptr(error_flag), _stream(device))


@dataclass
class PagedBuffers:
    """Device metadata of one step, in the layout the attention calls take."""
    qo_indptr: torch.Tensor        # [B + 1]
    kv_indptr: torch.Tensor        # [B + 1]
    kv_indices: torch.Tensor       # [capacity]
    kv_last_page_len: torch.Tensor  # [B]
    batch_indices: torch.Tensor    # [token capacity]
    positions: torch.Tensor        # [token capacity]


def new_paged_buffers(batch_size: int, indices_capacity: int, tokens_capacity: int,
                      device) -> PagedBuffers:
    """Fixed-capacity buffers for build_paged_metadata (a captured step keeps
    reusing the same ones)."""
    def z(n):
        return torch.zeros(max(int(n), 1), dtype=torch.int32, device=device)[:int(n)]
    return PagedBuffers(z(batch_size + 1), z(batch_size + 1), z(indices_capacity),
                        z(batch_size), z(tokens_capacity), z(tokens_capacity))


def build_paged_metadata(block_tables: torch.Tensor, kv_lens: torch.Tensor,
                         new_lens: torch.Tensor | None = None, *,
                         out: PagedBuffers | None = None,
                         indices_capacity: int | None = None,
                         tokens_capacity: int | None = None,
                         error_flag: torch.Tensor | None = None) -> PagedBuffers:
    """Step metadata built on the device from a block table [B, max_pages]
    (int32, row b = sequence b's pages) and kv lengths [B] (tokens in the
    cache once this step's tokens are appended).  The engine builds the same
    lists in Python and uploads them every step
    (src/engine/runtime/step_executor.py:98-165 prefill, :204-234 decode);
    here nothing leaves the device:
      kv_indptr / kv_indices: the first ceil(L/16) pages of every row
        (decode too: the reference passes the whole row, which overstates
        kv_len by a page when L % 16 == 0),
      kv_last_page_len = L % 16 or 16,
      qo_indptr: prefix sum of new_lens (decode: arange(B + 1)),
      batch_indices / positions: each new token's sequence and position
        (decode: row b = sequence b at L - 1; prefill: L - n .. L - 1).
    With `out`, the results land in those buffers (fixed addresses for HIP
    graph capture); otherwise new tensors sized for this call are returned.
    Pages past a row's max_pages or outputs past a capacity are dropped and
    counted in `error_flag`."""
    _require_cuda(block_tables, "block_tables")
    device = block_tables.device
    if block_tables.dim() != 2 or block_tables.dtype != torch.int32 or \
            block_tables.stride(1) != 1:
        raise ValueError("block_tables must be an int32 [batch, max_pages] tensor with "
                         "contiguous rows")
    bsz, max_pages = block_tables.shape
    for name, t in (("kv_lens", kv_lens), ("new_lens", new_lens)):
        if t is None:
            continue
        _require_cuda(t, name)
        if t.dtype != torch.int32 or t.numel() != bsz or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32 device tensor of {bsz} entries")
    if out is None:
        if indices_capacity is None:
            indices_capacity = bsz * max_pages
        if tokens_capacity is None:
            tokens_capacity = bsz if new_lens is None else int(new_lens.sum().item())
        out = new_paged_buffers(bsz, indices_capacity, tokens_capacity, device)
    for name in ("qo_indptr", "kv_indptr"):
        if getattr(out, name).numel() < bsz + 1:
            raise ValueError(f"out.{name} holds fewer than {bsz + 1} entries")
    if out.kv_last_page_len.numel() < bsz:
        raise ValueError(f"out.kv_last_page_len holds fewer than {bsz} entries")
    n_tok = min(out.batch_indices.numel(), out.positions.numel())
    if error_flag is not None and (error_flag.dtype != torch.int32 or error_flag.numel() < 1):
        raise ValueError("error_flag must be an int32 device tensor")
    call("pagedattn_build_paged_metadata", ptr(block_tables), block_tables.stride(0), max_pages,
         ptr(kv_lens), ptr(new_lens), bsz, ptr(out.qo_indptr), ptr(out.kv_indptr),
         ptr(out.kv_indices), out.kv_indices.numel(), ptr(out.kv_last_page_len),
         ptr(out.batch_indices), ptr(out.positions), n_tok, ptr(error_flag), _stream(device))
    return out


def quantize_pages_e4m3(pool: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16/fp16 layer pool -> (e4m3 pool, fp32 scales [P, 2, Hkv]) with
    scale = amax / 448 per (page, K|V, kv-head) block (1.0 for an all-zero block)."""
    num_pages, hkv, d = _check_pool(pool, None, None, "HND")
    out = torch.empty(pool.shape, dtype=torch.float8_e4m3fn, device=pool.device)
    scales = torch.empty((num_pages, 2, hkv), dtype=torch.float32, device=pool.device)
    call("pagedattn_quantize_pages_e4m3", ptr(pool), dtype_code(pool.dtype), ptr(out),
         ptr(scales), num_pages, hkv, d, PAGE_SIZE, _stream(pool.device))
    return out, scales


def copy_bytes(dst: torch.Tensor, src: torch.Tensor) -> None:
    """Plain 16-byte streaming copy (HBM counter calibration)."""
    n = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() < n:
        raise ValueError("dst smaller than src")
    call("pagedattn_copy_bytes", ptr(dst), ptr(src), n, _stream(src.device))


def read_bytes(src: torch.Tensor) -> torch.Tensor:
    """Plain streaming read of src (HBM counter calibration, read-only point);
    returns the per-workgroup XOR of what was read."""
    n = src.numel() * src.element_size()
    sink = torch.empty(8 * max(1, _lib.lib().pagedattn_device_cu_count()), dtype=torch.int32,
                       device=src.device)
    call("pagedattn_read_bytes", ptr(src), n, ptr(sink), sink.numel(), _stream(src.device))
    return sink


# -----------------------------------------------------------------------------
class _Plan:
    """Owns one host plan object of the library."""

    def __init__(self):
        self.handle = _lib.lib().pagedattn_plan_create()
        if not self.handle:
            raise MemoryError("pagedattn_plan_create failed")

    def __del__(self):
        h = getattr(self, "handle", None)
        if h and _lib._lib is not None:
            _lib._lib.pagedattn_plan_destroy(h)
            self.handle = None


def _unsupported_options(pos_encoding_mode="NONE", window_left=-1, logits_soft_cap=None,
                         custom_mask=None, packed_custom_mask=None) -> None:
    if pos_encoding_mode not in ("NONE", None):
        raise NotImplementedError(
            f"pos_encoding_mode={pos_encoding_mode!r}: RoPE is applied by "
            "apply_rope_pos_ids_inplace before attention")
    if window_left not in (-1, None):
        raise NotImplementedError("sliding-window attention is not implemented")
    if logits_soft_cap not in (None, 0, 0.0):
        raise NotImplementedError("logits_soft_cap is not implemented")
    if custom_mask is not None or packed_custom_mask is not None:
        raise NotImplementedError("custom masks are not implemented")


class _WrapperBase:
    _graph_capable = False

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, **_unused):
        if kv_layout != "HND":
            raise NotImplementedError(
                f"kv_layout {kv_layout!r}: only the HND page layout is implemented")
        if use_cuda_graph and not self._graph_capable:
            raise NotImplementedError(
                f"use_cuda_graph is not implemented for {type(self).__name__}")
        self._use_graph = bool(use_cuda_graph)
        _require_cuda(float_workspace_buffer, "float_workspace_buffer")
        if not float_workspace_buffer.is_contiguous():
            raise ValueError("the workspace must be contiguous")
        self._ws = float_workspace_buffer
        self._kv_layout = kv_layout
        self._plan = _Plan()
        self._planned = False

    @property
    def _ws_bytes(self) -> int:
        return self._ws.numel() * self._ws.element_size()

    def reset_workspace_buffer(self, float_workspace_buffer: torch.Tensor, *_a) -> None:
        self._ws = float_workspace_buffer
        self._planned = False

    def end_forward(self) -> None:
        """Kept for interface parity; the plan needs no teardown."""


class BatchDecodeWithPagedKVCacheWrapper(_WrapperBase):
    """Paged decode attention: one query token per sequence over its whole
    paged KV, GQA, no mask (src/models/llama.py:62-67, :119-147, :230-245).

    Long sequences are split into KV chunks whose partials are merged by
    log-sum-exp; `plan(..., split_pages=n)` fixes the chunk size (pages),
    0 lets the planner balance the work over the GPU, -1 disables splitting.

    `plan(..., device_plan=True)` -- and every plan of a wrapper made with
    use_cuda_graph=True -- reads nothing on the host: the attention launch
    partitions the work itself from kv_indptr at run time (the same balanced
    split), so a step can be replayed from a HIP graph while the metadata
    changes in place.  With use_cuda_graph=True the run reads the metadata
    from paged_kv_indptr_buffer / paged_kv_indices_buffer /
    paged_kv_last_page_len_buffer (int32, fixed addresses); plan() copies
    the tensors it is given into them unless they are those buffers."""

    _graph_capable = True

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, use_tensor_cores: bool = False,
                 paged_kv_indptr_buffer: torch.Tensor | None = None,
                 paged_kv_indices_buffer: torch.Tensor | None = None,
                 paged_kv_last_page_len_buffer: torch.Tensor | None = None, **kw):
        super().__init__(float_workspace_buffer, kv_layout, use_cuda_graph, **kw)
        self._graph_bufs = None
        if use_cuda_graph:
            bufs = (paged_kv_indptr_buffer, paged_kv_indices_buffer,
                    paged_kv_last_page_len_buffer)
            if any(b is None for b in bufs):
                raise ValueError("use_cuda_graph needs paged_kv_indptr_buffer, "
                                 "paged_kv_indices_buffer and paged_kv_last_page_len_buffer")
            for b in bufs:
                _require_cuda(b, "paged_kv buffer")
                if b.dtype != torch.int32 or not b.is_contiguous():
                    raise ValueError("the paged_kv buffers must be contiguous int32")
            if paged_kv_indptr_buffer.numel() != paged_kv_last_page_len_buffer.numel() + 1:
                raise ValueError("paged_kv_indptr_buffer must hold batch + 1 entries")
            self._graph_bufs = bufs

    def plan(self, indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
             pos_encoding_mode: str = "NONE", window_left: int = -1,
             logits_soft_cap: float | None = None, q_data_type="float16",
             kv_data_type=None, data_type=None, sm_scale: float | None = None,
             rope_scale=None, rope_theta=None, non_blocking: bool = True,
             split_pages: int = 0, device_plan: bool = False,
             indptr_host: torch.Tensor | None = None,
             last_page_len_host: torch.Tensor | None = None, **_unused) -> None:
        """indptr_host / last_page_len_host: CPU copies of indptr and
        last_page_len that the caller already holds; the plan then makes no
        device-to-host copy of its own."""
        _unsupported_options(pos_encoding_mode, window_left, logits_soft_cap)
        if page_size != PAGE_SIZE:
            raise NotImplementedError(f"page_size {page_size} (only 16 is implemented)")
        if self._use_graph or device_plan:
            self._plan_device(indptr, indices, last_page_len, num_qo_heads, num_kv_heads,
                              head_dim, page_size, q_data_type, kv_data_type, data_type,
                              sm_scale)
            return
        device = self._ws.device
        indptr_h = _host_i32(indptr if indptr_host is None else indptr_host)
        last_h = _host_i32(last_page_len if last_page_len_host is None else last_page_len_host)
        if indptr_host is not None and indptr_h.shape != indptr.shape:
            raise ValueError("indptr_host must have indptr's shape")
        if last_page_len_host is not None and last_h.shape != last_page_len.shape:
            raise ValueError("last_page_len_host must have last_page_len's shape")
        bsz = last_h.numel()
        if indptr_h.numel() != bsz + 1:
            raise ValueError(f"indptr has {indptr_h.numel()} entries for {bsz} sequences")
        n_ind = int(indptr_h[-1]) if bsz else 0
        if indices.numel() < n_ind:
            raise ValueError(f"indices has {indices.numel()} entries, indptr needs {n_ind}")
        self._q_dtype = _dtype_of(data_type if data_type is not None else q_data_type)
        self._kv_dtype = _dtype_of(kv_data_type) if kv_data_type is not None else None
        call("pagedattn_decode_plan", self._plan.handle, ptr(indptr_h), ptr(last_h), bsz,
             int(num_qo_heads), int(num_kv_heads), int(head_dim), int(page_size),
             int(split_pages), ptr(self._ws), self._ws_bytes, _stream(device))
        self._indptr = _i32(indptr, device)
        self._indices = _i32(indices, device)
        self._last = _i32(last_page_len, device)
        self._bsz, self._hq, self._hkv, self._d = bsz, int(num_qo_heads), int(num_kv_heads), int(head_dim)
        self._sm_scale = sm_scale
        self._planned = True

    def _plan_device(self, indptr, indices, last_page_len, num_qo_heads, num_kv_heads,
                     head_dim, page_size, q_data_type, kv_data_type, data_type, sm_scale):
        device = self._ws.device
        bsz = last_page_len.numel()
        if indptr.numel() != bsz + 1:
            raise ValueError(f"indptr has {indptr.numel()} entries for {bsz} sequences")
        if self._graph_bufs is not None:
            b_indptr, b_indices, b_last = self._graph_bufs
            if b_last.numel() != bsz:
                raise ValueError(f"the graph buffers hold {b_last.numel()} sequences, "
                                 f"the plan has {bsz}")
            if indices.numel() > b_indices.numel():
                raise ValueError("indices do not fit paged_kv_indices_buffer")
            for src, dst in ((indptr, b_indptr), (last_page_len, b_last),
                             (indices, b_indices[:indices.numel()])):
                if src.data_ptr() != dst.data_ptr():
                    dst.copy_(src, non_blocking=True)
            self._indptr, self._indices, self._last = b_indptr, b_indices, b_last
        else:
            self._indptr = _i32(indptr, device)
            self._indices = _i32(indices, device)
            self._last = _i32(last_page_len, device)
        self._q_dtype = _dtype_of(data_type if data_type is not None else q_data_type)
        self._kv_dtype = _dtype_of(kv_data_type) if kv_data_type is not None else None
        call("pagedattn_decode_plan_device", self._plan.handle, bsz, int(num_qo_heads),
             int(num_kv_heads), int(head_dim), int(page_size), ptr(self._ws), self._ws_bytes)
        self._bsz, self._hq, self._hkv, self._d = bsz, int(num_qo_heads), int(num_kv_heads), int(head_dim)
        self._sm_scale = sm_scale
        self._planned = True

    begin_forward = plan

    def update_plan(self) -> None:
        """For a device plan: deal the (sequence, KV head) items of the
        metadata now in the plan's indptr / last_page_len tensors to the
        workgroups, on the device and the current stream (one small launch,
        no host synchronisation, captured with the runs in a HIP graph).
        Until the next plan(), every run reads that deal instead of making
        its own in its prologue, so the metadata must not change between
        this call and the runs it serves: an engine step calls it once after
        writing the step's metadata, before the layers' runs.  A no-op for
        host plans and for device plans of the split kind."""
        if not self._planned:
            raise RuntimeError("plan() must be called before update_plan()")
        if self.plan_kind != "device_shared":
            return
        call("pagedattn_decode_plan_device_update", self._plan.handle, ptr(self._indptr),
             ptr(self._last), _stream(self._indptr.device))

    @property
    def plan_kind(self) -> str | None:
        """The partition the current plan holds: "split" (head-group work
        list, cut sequences merged by a second launch), "shared" (whole
        (sequence, KV head) items per CU workgroup, one launch), "device"
        (split partition made on the device at run time), "device_shared"
        (whole items dealt to the CUs on the device at run time, one launch),
        or None before plan()."""
        k = _lib.lib().pagedattn_decode_plan_kind(self._plan.handle)
        return {1: "split", 2: "shared", 3: "device", 4: "device_shared"}.get(int(k))

    def run(self, q: torch.Tensor, paged_kv_cache: torch.Tensor, *,
            kv_scales: torch.Tensor | None = None, out: torch.Tensor | None = None,
            lse: torch.Tensor | None = None, return_lse: bool = False,
            sm_scale: float | None = None, append_key: torch.Tensor | None = None,
            append_value: torch.Tensor | None = None, rope: tuple[float, float] | None = None,
            positions: torch.Tensor | None = None):
        """Decode attention.  With append_key/append_value ([B, Hkv, D], the
        newest token of every sequence, position kv_len - 1) the page append
        of the decode step runs inside the same launch (the engine's decode
        step: batch_indices = arange(B), positions = kv_len - 1).  With
        rope=(rope_scale, rope_theta) as well, q and append_key are rotated
        (non-interleaved RoPE at `positions`, default kv_len - 1) inside that
        launch too: apply_rope_pos_ids_inplace + append + attention in one
        kernel (q and append_key themselves are left unrotated)."""
        if not self._planned:
            raise RuntimeError("plan()/begin_forward() must be called before run()/forward()")
        num_pages, _, _ = _check_pool(paged_kv_cache, self._hkv, self._d, self._kv_layout)
        _check_rows(q, "q", self._hq, self._d)
        if q.shape[0] != self._bsz:
            raise ValueError(f"q has {q.shape[0]} rows, the plan has {self._bsz} sequences")
        if q.dtype not in (torch.float16, torch.bfloat16):
            raise NotImplementedError(f"q dtype {q.dtype}")
        scales = _check_scales(kv_scales, paged_kv_cache)
        if out is None:
            out = torch.empty((self._bsz, self._hq, self._d), dtype=q.dtype, device=q.device)
        elif not out.is_contiguous() or tuple(out.shape) != (self._bsz, self._hq, self._d):
            raise ValueError("out must be a contiguous [batch, num_qo_heads, head_dim] tensor")
        if return_lse and lse is None:
            lse = torch.empty((self._bsz, self._hq), dtype=torch.float32, device=q.device)
        scale = sm_scale if sm_scale is not None else self._sm_scale
        if scale is None:
            scale = 1.0 / math.sqrt(self._d)
        common = (ptr(paged_kv_cache), dtype_code(paged_kv_cache.dtype), ptr(scales),
                  num_pages, ptr(self._indices), self._indices.numel(), ptr(self._indptr),
                  ptr(self._last), ptr(out), ptr(lse), float(scale), _stream(q.device))
        if append_key is None and append_value is None:
            call("pagedattn_decode_run", self._plan.handle, ptr(q), q.stride(0), q.stride(1),
                 dtype_code(q.dtype), *common)
        else:
            if append_key is None or append_value is None:
                raise ValueError("append_key and append_value go together")
            for name, t in (("append_key", append_key), ("append_value", append_value)):
                _check_rows(t, name, self._hkv, self._d)
                if t.shape[0] != self._bsz or t.dtype != q.dtype:
                    raise ValueError(f"{name} must be [batch, num_kv_heads, head_dim] in q's dtype")
            if rope is None:
                if positions is not None:
                    raise ValueError("positions only applies together with rope")
                call("pagedattn_decode_run_append", self._plan.handle, ptr(q), q.stride(0),
                     q.stride(1), dtype_code(q.dtype), ptr(append_key), ptr(append_value),
                     append_key.stride(0), append_key.stride(1), append_value.stride(0),
                     append_value.stride(1), *common)
            else:
                rope_scale, rope_theta = rope
                pos = None
                if positions is not None:
                    if positions.numel() != self._bsz:
                        raise ValueError("positions must hold one entry per sequence")
                    pos = _i32(positions, q.device)
                call("pagedattn_decode_run_rope_append", self._plan.handle, ptr(q),
                     q.stride(0), q.stride(1), dtype_code(q.dtype), ptr(append_key),
                     ptr(append_value), append_key.stride(0), append_key.stride(1),
                     append_value.stride(0), append_value.stride(1), ptr(pos),
                     float(rope_scale), float(rope_theta), *common)
        return (out, lse) if return_lse else out

    def forward(self, q: torch.Tensor, paged_kv_cache: torch.Tensor,
                pos_encoding_mode: str = "NONE", q_scale=None, k_scale=None, v_scale=None,
                window_left: int = -1, logits_soft_cap: float | None = None,
                sm_scale: float | None = None, rope_scale=None, rope_theta=None,
                return_lse: bool = False, kv_scales: torch.Tensor | None = None):
        _unsupported_options(pos_encoding_mode, window_left, logits_soft_cap)
        if q_scale is not None or k_scale is not None or v_scale is not None:
            raise NotImplementedError("scalar q/k/v scales; pass per-page kv_scales")
        return self.run(q, paged_kv_cache, kv_scales=kv_scales, return_lse=return_lse,
                        sm_scale=sm_scale)


class BatchPrefillWithPagedKVCacheWrapper(_WrapperBase):
    """Ragged-query, paged-KV attention with GQA and a bottom-right aligned
    causal mask (src/models/llama.py:55-60, :86-116, :212-228): row i of
    sequence b sees kv token j iff j <= kv_len_b - qo_len_b + i.

    `plan(..., device_plan=True, max_qo_tokens=n)` reads nothing on the
    host: every run cuts the q-tiles of the qo_indptr / paged_kv_indptr it
    was planned with, in their current contents, on the device, for up to n
    query tokens per run, so a chunked-prefill step can be captured in a HIP
    graph and replayed while the metadata changes in place.  The outputs are
    those of a host plan, bit for bit."""

    def plan(self, qo_indptr: torch.Tensor, paged_kv_indptr: torch.Tensor,
             paged_kv_indices: torch.Tensor, paged_kv_last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim_qk: int, page_size: int,
             head_dim_vo: int | None = None, custom_mask=None, packed_custom_mask=None,
             causal: bool = False, pos_encoding_mode: str = "NONE",
             window_left: int = -1, logits_soft_cap: float | None = None,
             q_data_type="float16", kv_data_type=None, sm_scale: float | None = None,
             rope_scale=None, rope_theta=None, non_blocking: bool = True,
             device_plan: bool = False, max_qo_tokens: int | None = None,
             **_unused) -> None:
        _unsupported_options(pos_encoding_mode, window_left, logits_soft_cap, custom_mask,
                             packed_custom_mask)
        if head_dim_vo is not None and head_dim_vo != head_dim_qk:
            raise NotImplementedError("head_dim_vo != head_dim_qk")
        if page_size != PAGE_SIZE:
            raise NotImplementedError(f"page_size {page_size} (only 16 is implemented)")
        device = self._ws.device
        if device_plan:
            for name, t in (("qo_indptr", qo_indptr), ("paged_kv_indptr", paged_kv_indptr),
                            ("paged_kv_indices", paged_kv_indices),
                            ("paged_kv_last_page_len", paged_kv_last_page_len)):
                _require_cuda(t, name)
                if t.dtype != torch.int32 or not t.is_contiguous():
                    raise ValueError(f"{name} must be a contiguous int32 device tensor "
                                     "for a device plan (the runs read it in place)")
            if max_qo_tokens is None:
                raise ValueError("device_plan needs max_qo_tokens (query tokens per run)")
            bsz = paged_kv_last_page_len.numel()
            if qo_indptr.numel() != bsz + 1 or paged_kv_indptr.numel() != bsz + 1:
                raise ValueError("qo_indptr and paged_kv_indptr need batch_size + 1 entries")
            self._q_dtype = _dtype_of(q_data_type)
            call("pagedattn_prefill_plan_device", self._plan.handle, bsz, int(num_qo_heads),
                 int(num_kv_heads), int(head_dim_qk), int(page_size), int(max_qo_tokens),
                 ptr(self._ws), self._ws_bytes)
            self._qo_rows = None  # known on the device only
            self._device_plan = True
        else:
            self._plan_host(qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len,
                            num_qo_heads, num_kv_heads, head_dim_qk, page_size, q_data_type)
            self._device_plan = False
        self._qo_indptr = _i32(qo_indptr, device)
        self._indptr = _i32(paged_kv_indptr, device)
        self._indices = _i32(paged_kv_indices, device)
        self._last = _i32(paged_kv_last_page_len, device)
        self._bsz = paged_kv_last_page_len.numel()
        self._hq, self._hkv, self._d = int(num_qo_heads), int(num_kv_heads), int(head_dim_qk)
        self._causal = bool(causal)
        self._sm_scale = sm_scale
        self._planned = True

    def _plan_host(self, qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len,
                   num_qo_heads, num_kv_heads, head_dim_qk, page_size, q_data_type) -> None:
        device = self._ws.device
        qo_h = _host_i32(qo_indptr)
        indptr_h = _host_i32(paged_kv_indptr)
        last_h = _host_i32(paged_kv_last_page_len)
        bsz = last_h.numel()
        if qo_h.numel() != bsz + 1 or indptr_h.numel() != bsz + 1:
            raise ValueError("qo_indptr and paged_kv_indptr need batch_size + 1 entries")
        n_ind = int(indptr_h[-1]) if bsz else 0
        if paged_kv_indices.numel() < n_ind:
            raise ValueError(
                f"paged_kv_indices has {paged_kv_indices.numel()} entries, indptr needs {n_ind}")
        self._q_dtype = _dtype_of(q_data_type)
        call("pagedattn_prefill_plan", self._plan.handle, ptr(qo_h), ptr(indptr_h),
             ptr(last_h), bsz, int(num_qo_heads), int(num_kv_heads), int(head_dim_qk),
             int(page_size), ptr(self._ws), self._ws_bytes, _stream(device))
        self._qo_rows = int(qo_h[-1]) if bsz else 0

    begin_forward = plan

    def update_plan(self) -> None:
        """For a device plan: cut the q-tile list of the metadata now in the
        plan's qo_indptr / paged_kv_indptr / paged_kv_last_page_len tensors,
        on the device and the current stream (one small launch, captured
        with the runs in a HIP graph).  Until the next plan(), the runs read
        that list instead of cutting their own, so the metadata must not
        change between this call and the runs it serves: an engine step
        calls it once after writing the step's metadata, before the layers'
        runs.  A no-op for host plans."""
        if not self._planned:
            raise RuntimeError("plan() must be called before update_plan()")
        if not self._device_plan:
            return
        call("pagedattn_prefill_plan_device_update", self._plan.handle, ptr(self._qo_indptr),
             ptr(self._indptr), ptr(self._last), _stream(self._qo_indptr.device))

    @property
    def plan_kind(self) -> str | None:
        """"host" (q-tile list built by plan()), "device" (built on the
        device by every run, or once per update_plan()), or None before
        plan()."""
        if not self._planned:
            return None
        return "device" if self._device_plan else "host"

    def run(self, q: torch.Tensor, paged_kv_cache: torch.Tensor, *,
            kv_scales: torch.Tensor | None = None, out: torch.Tensor | None = None,
            lse: torch.Tensor | None = None, return_lse: bool = False,
            causal: bool | None = None, sm_scale: float | None = None):
        if not self._planned:
            raise RuntimeError("plan()/begin_forward() must be called before run()/forward()")
        num_pages, _, _ = _check_pool(paged_kv_cache, self._hkv, self._d, self._kv_layout)
        _check_rows(q, "q", self._hq, self._d)
        if self._qo_rows is not None and q.shape[0] < self._qo_rows:
            raise ValueError(f"q has {q.shape[0]} rows, qo_indptr needs {self._qo_rows}")
        if q.dtype not in (torch.float16, torch.bfloat16):
            raise NotImplementedError(f"q dtype {q.dtype}")
        scales = _check_scales(kv_scales, paged_kv_cache)
        n = q.shape[0]
        if out is None:
            out = torch.empty((n, self._hq, self._d), dtype=q.dtype, device=q.device)
        elif not out.is_contiguous() or tuple(out.shape) != (n, self._hq, self._d):
            raise ValueError("out must be a contiguous [nnz, num_qo_heads, head_dim] tensor")
        if return_lse and lse is None:
            lse = torch.empty((n, self._hq), dtype=torch.float32, device=q.device)
        scale = sm_scale if sm_scale is not None else self._sm_scale
        if scale is None:
            scale = 1.0 / math.sqrt(self._d)
        is_causal = self._causal if causal is None else bool(causal)
        call("pagedattn_prefill_run", self._plan.handle, ptr(q), q.stride(0), q.stride(1),
             dtype_code(q.dtype), ptr(self._qo_indptr), ptr(paged_kv_cache),
             dtype_code(paged_kv_cache.dtype), ptr(scales), num_pages, ptr(self._indices),
             self._indices.numel(), ptr(self._indptr), ptr(self._last), ptr(out), ptr(lse),
             int(is_causal), float(scale), _stream(q.device))
        return (out, lse) if return_lse else out

    def forward(self, q: torch.Tensor, paged_kv_cache: torch.Tensor, causal: bool = False,
                pos_encoding_mode: str = "NONE", window_left: int = -1,
                logits_soft_cap: float | None = None, sm_scale: float | None = None,
                rope_scale=None, rope_theta=None, return_lse: bool = False,
                kv_scales: torch.Tensor | None = None, **_unused):
        _unsupported_options(pos_encoding_mode, window_left, logits_soft_cap)
        return self.run(q, paged_kv_cache, kv_scales=kv_scales, return_lse=return_lse,
                        causal=causal, sm_scale=sm_scale)
