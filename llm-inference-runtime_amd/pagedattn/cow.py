"""Copy-on-write of shared partial pages before an append.

The reference's todo.md:17-19 plans to share half-filled decode blocks
through the radix cache (src/engine/memory/radix_cache.py:60-88) and
requires that "if a sequence attempts to append a token to a shared
partial block (ref_count > 1), the allocator must fork the block to a new
memory address".  ``fork_for_append`` is that step for a whole batch: the
decisions are made on the host against the engine's ``BlockAllocator``
(allocate / decref / ref_counts, src/engine/memory/allocator.py:52-87) and
all copies run in one ``fork_pages`` launch on the current stream, ahead of
the append that follows on the same stream.
"""

from __future__ import annotations

import torch

from . import ops

PAGE = ops.PAGE_SIZE


def fork_for_append(allocator, block_tables: list[list[int]], seq_lens: list[int],
                    kv_pool: torch.Tensor, kv_scales: torch.Tensor | None = None
                    ) -> list[tuple[int, int, int]]:
    """For each sequence whose next token (position seq_lens[i]) lands in a
    page that already holds rows (seq_lens[i] % 16 != 0) and is shared
    (ref count > 1): allocate a fresh page, copy the page's seq_lens[i] % 16
    valid rows into it in every layer, put it in the block table in place of
    the shared page and drop this sequence's reference to the shared one.
    Block tables are updated in place.  Returns the (sequence, old page, new
    page) forks made.  Raises whatever ``allocator.allocate`` raises when
    the pool is exhausted, before anything is changed."""
    if len(block_tables) != len(seq_lens):
        raise ValueError("one seq_len per block table")
    want: list[tuple[int, int, int]] = []  # (sequence, table slot, shared page)
    refs = allocator.ref_counts
    pending: dict[int, int] = {}  # references this batch already dropped
    for i, (table, n) in enumerate(zip(block_tables, seq_lens)):
        if n % PAGE == 0:
            continue  # the next token opens a fresh page
        slot = n // PAGE
        if slot >= len(table):
            raise ValueError(f"sequence {i}: {n} tokens but {len(table)} pages")
        page = table[slot]
        if refs[page] - pending.get(page, 0) > 1:
            want.append((i, slot, page))
            pending[page] = pending.get(page, 0) + 1
    if not want:
        return []
    fresh = allocator.allocate(len(want))
    src = [p for _, _, p in want]
    valid = [seq_lens[i] % PAGE for i, _, _ in want]
    ops.fork_pages(kv_pool, src, fresh, valid_tokens=valid, kv_scales=kv_scales)
    forks = []
    for (i, slot, page), new in zip(want, fresh):
        block_tables[i][slot] = new
        forks.append((i, page, new))
    allocator.decref(src)
    return forks
