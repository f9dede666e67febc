"""KV pool sizing for the engine (src/engine/memory/capacity.py:16-82), with
the e4m3 pool's per-(layer, page, K|V, kv-head) fp32 scales counted.

``bytes_per_block`` and ``estimate_num_blocks`` keep the reference's names,
arguments and rules (85 % of free memory, at least 2 GiB held back, a
RuntimeError below ``min_blocks``); ``dtype`` may also be
``torch.float8_e4m3fn``.  ``new_kv_scales`` allocates the scale tensor that
goes with an e4m3 pool.
"""

from __future__ import annotations

import logging

import torch

logger = logging.getLogger(__name__)

KV_CACHE_MEMORY_FRACTION = 0.85          # capacity.py:12
MIN_RESERVED_BYTES = 2 * 1024 ** 3       # capacity.py:13
SCALE_BYTES = 4                          # one fp32 scale per (layer, K|V, kv-head) of a page


def bytes_per_block(block_size: int, num_layers: int, num_kv_heads: int, head_dim: int,
                    dtype: torch.dtype) -> int:
    """Bytes one KV block takes in the pool (layers, K|V, kv-heads, block_size
    rows of head_dim elements), plus its scales for an e4m3 pool
    (capacity.py:16-32)."""
    elem = torch.tensor([], dtype=dtype).element_size()
    n = num_layers * 2 * num_kv_heads * block_size * head_dim * elem
    if dtype == torch.float8_e4m3fn:
        n += num_layers * 2 * num_kv_heads * SCALE_BYTES
    return n


def estimate_num_blocks(device: torch.device, block_size: int, num_layers: int,
                        num_kv_heads: int, head_dim: int, dtype: torch.dtype,
                        min_blocks: int = 256) -> int:
    """How many KV blocks fit in the device's free memory (capacity.py:35-82):
    -1 on a non-GPU device, RuntimeError below `min_blocks`."""
    device = torch.device(device)
    if device.type != "cuda":
        logger.warning("estimate_num_blocks: non-GPU device (%s), cannot query free memory",
                       device)
        return -1
    free_bytes, _total = torch.cuda.mem_get_info(device)
    return blocks_for_free_bytes(free_bytes, block_size, num_layers, num_kv_heads, head_dim,
                                 dtype, min_blocks)


def blocks_for_free_bytes(free_bytes: int, block_size: int, num_layers: int,
                          num_kv_heads: int, head_dim: int, dtype: torch.dtype,
                          min_blocks: int = 256) -> int:
    """The sizing rule of estimate_num_blocks for a given free byte count."""
    reserved = max(MIN_RESERVED_BYTES, int(free_bytes * (1 - KV_CACHE_MEMORY_FRACTION)))
    usable = max(0, free_bytes - reserved)
    per_block = bytes_per_block(block_size, num_layers, num_kv_heads, head_dim, dtype)
    num_blocks = usable // per_block
    logger.info("KV cache sizing: free=%.2fGiB reserved=%.2fGiB bytes/block=%d -> %d blocks",
                free_bytes / 1024 ** 3, reserved / 1024 ** 3, per_block, num_blocks)
    if num_blocks < min_blocks:
        raise RuntimeError(
            f"Only {num_blocks} KV cache blocks fit in {free_bytes / 1024 ** 3:.2f}GiB of free "
            f"memory - need at least {min_blocks}.")
    return int(num_blocks)


def new_kv_scales(kv_pool: torch.Tensor) -> torch.Tensor:
    """Zeroed fp32 scales [L, num_pages, 2, num_kv_heads] for an e4m3 pool
    [L, num_pages, 2, num_kv_heads, 16, head_dim] (a zero scale marks a page
    with no rows yet)."""
    if kv_pool.dim() != 6:
        raise ValueError(f"kv_pool must be [L, P, 2, Hkv, 16, D], got {tuple(kv_pool.shape)}")
    n_layers, num_pages, _, hkv = kv_pool.shape[:4]
    return torch.zeros((n_layers, num_pages, 2, hkv), dtype=torch.float32,
                       device=kv_pool.device)
