"""Paging metadata built the way the engine's step executor builds it
(src/engine/runtime/step_executor.py:98-165 prefill, :204-243 decode).

Inputs are the scheduler's per-sequence block tables (lists of physical page
ids, src/engine/memory/allocator.py:56) and token counts; outputs are the
int32 arrays the plan and run calls take: qo_indptr, kv_indptr, kv_indices,
kv_last_page_len, plus the positions the caller derives.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

PAGE = 16


@dataclass
class PagedMetadata:
    kv_indptr: np.ndarray  # [B+1] int32
    kv_indices: np.ndarray  # [sum pages] int32
    kv_last_page_len: np.ndarray  # [B] int32
    qo_indptr: np.ndarray  # [B+1] int32 (decode: arange(B+1))
    seq_lens: np.ndarray  # [B] kv length after this step's tokens
    positions: np.ndarray  # [nnz] position of every new token
    batch_indices: np.ndarray  # [nnz] sequence of every new token

    @property
    def batch_size(self) -> int:
        return len(self.kv_last_page_len)

    @property
    def nnz(self) -> int:
        return int(self.qo_indptr[-1])


def _pack(tables: list[list[int]], counts: list[int]):
    indptr = np.zeros(len(tables) + 1, dtype=np.int32)
    flat: list[int] = []
    for b, (t, n) in enumerate(zip(tables, counts)):
        flat.extend(t[:n])
        indptr[b + 1] = len(flat)
    return indptr, np.asarray(flat, dtype=np.int32)


def _last_len(total: int, page: int) -> int:
    r = total % page
    return r if r > 0 else page


def prefill_metadata(block_tables: list[list[int]], computed_lens: list[int],
                     chunk_lens: list[int], page: int = PAGE) -> PagedMetadata:
    """Chunked prefill of `chunk_lens[b]` new tokens after `computed_lens[b]`
    cached ones (step_executor.py:98-165): the table is cut to
    ceil(new_len / page) pages and last_page_len = new_len % page or page."""
    new_lens = [c + n for c, n in zip(computed_lens, chunk_lens)]
    need = [math.ceil(n / page) for n in new_lens]
    for b, (t, k) in enumerate(zip(block_tables, need)):
        if len(t) < k:
            raise ValueError(f"sequence {b}: block table has {len(t)} pages, needs {k}")
    kv_indptr, kv_indices = _pack(block_tables, need)
    qo = np.zeros(len(chunk_lens) + 1, dtype=np.int32)
    qo[1:] = np.cumsum(chunk_lens)
    pos = np.concatenate([np.arange(c, c + n, dtype=np.int32)
                          for c, n in zip(computed_lens, chunk_lens)]) if chunk_lens else \
        np.zeros(0, np.int32)
    bi = np.repeat(np.arange(len(chunk_lens), dtype=np.int32), chunk_lens)
    return PagedMetadata(kv_indptr, kv_indices,
                         np.asarray([_last_len(n, page) for n in new_lens], dtype=np.int32),
                         qo, np.asarray(new_lens, dtype=np.int32), pos, bi)


def decode_metadata(block_tables: list[list[int]], seq_lens: list[int], page: int = PAGE,
                    trim_tables: bool = True) -> PagedMetadata:
    """One new token per sequence whose length (including it) is seq_lens[b]
    (step_executor.py:204-243: last_page_len = len % page or page,
    positions = len - 1, batch_indices = arange(B)).

    trim_tables=True passes block_table[:ceil(len / page)], as prefill does.
    The reference passes the whole table (step_executor.py:209), which
    overstates kv_len by a page whenever len % 16 == 0 because the scheduler
    reserves ceil((len + 1) / 16) pages (admission_controller.py:275);
    trim_tables=False reproduces that behaviour."""
    need = [math.ceil(n / page) for n in seq_lens]
    counts = [len(t) for t in block_tables] if not trim_tables else need
    for b, (t, k) in enumerate(zip(block_tables, need)):
        if len(t) < k:
            raise ValueError(f"sequence {b}: block table has {len(t)} pages, needs {k}")
    kv_indptr, kv_indices = _pack(block_tables, counts)
    bsz = len(seq_lens)
    return PagedMetadata(kv_indptr, kv_indices,
                         np.asarray([_last_len(n, page) for n in seq_lens], dtype=np.int32),
                         np.arange(bsz + 1, dtype=np.int32),
                         np.asarray(seq_lens, dtype=np.int32),
                         np.asarray([n - 1 for n in seq_lens], dtype=np.int32),
                         np.arange(bsz, dtype=np.int32))
