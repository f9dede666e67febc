"""Seeded synthetic paged-attention workloads at the engine's shapes.

Each generator draws sequence lengths and block tables on the host (numpy,
seeded), builds the metadata with the step executor's rules
(pagedattn.metadata), and fills the pool / queries / new K,V rows with
N(0, 1) values from a seeded torch generator on the target device.

Workloads (page 16 everywhere, pool layout [P, 2, Hkv, 16, D]):
* tinyllama_decode_small  - 32q/4kv, D=64, B=8, kv_len U[64,512], 256-page pool,
                            tables = slices of one random permutation.
* tinyllama_decode        - same heads, B=256, kv_len U[256,2048], pages drawn
                            without replacement from a shuffled pool of
                            ceil(1.2 x need) pages; one appended token per sequence.
* llama3_8b_prefill       - 32q/8kv, D=128, 16 sequences in 4 groups sharing a
                            cached prefix (U[0,4096], whole pages) and a new chunk
                            U[64,512] on fresh pages; causal.
* llama3_8b_long_decode   - 32q/8kv, D=128, B=32, kv_len U[32768,131072], random
                            non-contiguous tables, split-KV chunks of 4096 tokens.
* llama3_70b_mixed_fp8    - 64q/8kv, D=128, 128 decode sequences (kv U[1024,8192])
                            plus 4 prefill chunks of 1024 on prefixes U[0,8192];
                            pool stored e4m3 with per-(page, K|V, head) scales.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from .metadata import PAGE, PagedMetadata, decode_metadata, prefill_metadata


@dataclass
class Workload:
    name: str
    hq: int
    hkv: int
    d: int
    num_pages: int
    meta: PagedMetadata
    kind: str  # "decode" | "prefill"
    split_pages: int = 0  # decode plan: 0 auto, >0 fixed chunk (pages), -1 none
    seed: int = 0
    fp8: bool = False
    extra: dict = field(default_factory=dict)

    @property
    def kv_len(self) -> np.ndarray:
        return self.meta.seq_lens

    def kv_bytes_per_token(self, dtype_bytes: int) -> int:
        return self.hkv * self.d * 2 * dtype_bytes


@dataclass
class Tensors:
    """Device (or CPU) tensors of one workload instance."""
    pool: torch.Tensor  # [P, 2, Hkv, 16, D] (bf16/fp16 or e4m3)
    scales: torch.Tensor | None  # [P, 2, Hkv] fp32 for e4m3
    q: torch.Tensor  # [nnz, Hq, D]
    k_new: torch.Tensor  # [nnz, Hkv, D]
    v_new: torch.Tensor
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    kv_last_page_len: torch.Tensor
    qo_indptr: torch.Tensor
    batch_indices: torch.Tensor
    positions: torch.Tensor


def _tables_from_pool(rng: np.random.Generator, pages_needed: list[int], pool_pages: int):
    perm = rng.permutation(pool_pages)
    tables, at = [], 0
    for n in pages_needed:
        tables.append(perm[at:at + n].tolist())
        at += n
    return tables


def tinyllama_decode_small(seed: int = 0) -> Workload:
    rng = np.random.default_rng(seed)
    lens = rng.integers(64, 512, size=8, endpoint=True).tolist()
    need = [math.ceil(n / PAGE) for n in lens]
    tables = _tables_from_pool(rng, need, 256)
    return Workload("tinyllama_decode_small", 32, 4, 64, 256, decode_metadata(tables, lens),
                    "decode", seed=seed)


def tinyllama_decode(seed: int = 0, batch: int = 256, lo: int = 256, hi: int = 2048) -> Workload:
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi, size=batch, endpoint=True).tolist()
    need = [math.ceil(n / PAGE) for n in lens]
    pool = math.ceil(1.2 * sum(need))
    tables = _tables_from_pool(rng, need, pool)
    return Workload("tinyllama_decode", 32, 4, 64, pool, decode_metadata(tables, lens),
                    "decode", seed=seed)


def llama3_8b_long_decode(seed: int = 0, batch: int = 32, lo: int = 32768,
                          hi: int = 131072, split_tokens: int = 4096) -> Workload:
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi, size=batch, endpoint=True).tolist()
    need = [math.ceil(n / PAGE) for n in lens]
    pool = math.ceil(1.02 * sum(need))
    tables = _tables_from_pool(rng, need, pool)
    return Workload("llama3_8b_long_decode", 32, 8, 128, pool, decode_metadata(tables, lens),
                    "decode", split_pages=split_tokens // PAGE, seed=seed)


def _prefix_groups(rng, groups: int, per_group: int, prefix_hi: int, chunk_lo: int,
                   chunk_hi: int, fixed_chunk: int | None = None):
    prefixes = [(int(rng.integers(0, prefix_hi, endpoint=True)) // PAGE) * PAGE
                for _ in range(groups)]
    computed, chunks = [], []
    for gi in range(groups):
        for _ in range(per_group):
            computed.append(prefixes[gi])
            chunks.append(fixed_chunk if fixed_chunk is not None
                          else int(rng.integers(chunk_lo, chunk_hi, endpoint=True)))
    return prefixes, computed, chunks


def _prefill_tables(rng, prefixes, per_group, computed, chunks, extra_pages: int = 0):
    """Prefix pages shared inside a group; every sequence's chunk on fresh pages."""
    prefix_pages = [p // PAGE for p in prefixes]
    chunk_pages = [math.ceil((c + n) / PAGE) - c // PAGE for c, n in zip(computed, chunks)]
    total = sum(prefix_pages) + sum(chunk_pages) + extra_pages
    perm = rng.permutation(total).tolist()
    at = 0
    group_tab = []
    for npg in prefix_pages:
        group_tab.append(perm[at:at + npg])
        at += npg
    tables = []
    for b, cp in enumerate(chunk_pages):
        tables.append(group_tab[b // per_group] + perm[at:at + cp])
        at += cp
    return tables, total, perm[at:]


def llama3_8b_prefill(seed: int = 0) -> Workload:
    rng = np.random.default_rng(seed)
    prefixes, computed, chunks = _prefix_groups(rng, 4, 4, 4096, 64, 512)
    tables, total, _ = _prefill_tables(rng, prefixes, 4, computed, chunks)
    return Workload("llama3_8b_prefill", 32, 8, 128, total,
                    prefill_metadata(tables, computed, chunks), "prefill", seed=seed,
                    extra={"prefixes": prefixes})


def llama3_70b_mixed_fp8(seed: int = 0, n_decode: int = 128, n_prefill: int = 4):
    """(decode workload, prefill workload) sharing one e4m3 pool."""
    rng = np.random.default_rng(seed)
    dec_lens = rng.integers(1024, 8192, size=n_decode, endpoint=True).tolist()
    dec_need = [math.ceil(n / PAGE) for n in dec_lens]
    prefixes, computed, chunks = _prefix_groups(rng, n_prefill, 1, 8192, 0, 0, fixed_chunk=1024)
    tables_p, _, rest = _prefill_tables(rng, prefixes, 1, computed, chunks,
                                        extra_pages=sum(dec_need))
    total = sum(p // PAGE for p in prefixes) + sum(
        math.ceil((c + n) / PAGE) - c // PAGE for c, n in zip(computed, chunks)) + sum(dec_need)
    tables_d, at = [], 0
    for n in dec_need:
        tables_d.append(rest[at:at + n])
        at += n
    dec = Workload("llama3_70b_mixed_fp8.decode", 64, 8, 128, total,
                   decode_metadata(tables_d, dec_lens), "decode", seed=seed, fp8=True)
    pre = Workload("llama3_70b_mixed_fp8.prefill", 64, 8, 128, total,
                   prefill_metadata(tables_p, computed, chunks), "prefill", seed=seed, fp8=True,
                   extra={"prefixes": prefixes})
    return dec, pre


WORKLOADS = {
    "tinyllama_decode_small": tinyllama_decode_small,
    "tinyllama_decode": tinyllama_decode,
    "llama3_8b_prefill": llama3_8b_prefill,
    "llama3_8b_long_decode": llama3_8b_long_decode,
}


def _i32(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(device)


def materialize(w: Workload, device, dtype=torch.bfloat16, seed: int | None = None,
                pool: torch.Tensor | None = None) -> Tensors:
    """Random N(0,1) pool / q / new rows for workload `w` on `device`.
    For fp8 workloads the pool is drawn in `dtype` and quantised with
    per-(page, K|V, head) scales = amax / 448 (`quantize` must be given the
    device quantiser; the oracle's is used on CPU)."""
    s = w.seed if seed is None else seed
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(10007 * s + 17)
    nnz = w.meta.nnz
    if pool is None:
        pool = torch.randn((w.num_pages, 2, w.hkv, PAGE, w.d), generator=g, device=dev,
                           dtype=torch.float32).to(dtype) if dev.type == "cpu" else \
            torch.randn((w.num_pages, 2, w.hkv, PAGE, w.d), generator=g, device=dev, dtype=dtype)
    q = torch.randn((nnz, w.hq, w.d), generator=g, device=dev, dtype=torch.float32).to(dtype)
    kn = torch.randn((nnz, w.hkv, w.d), generator=g, device=dev, dtype=torch.float32).to(dtype)
    vn = torch.randn((nnz, w.hkv, w.d), generator=g, device=dev, dtype=torch.float32).to(dtype)
    m = w.meta
    return Tensors(pool, None, q, kn, vn, _i32(m.kv_indptr, dev), _i32(m.kv_indices, dev),
                   _i32(m.kv_last_page_len, dev), _i32(m.qo_indptr, dev),
                   _i32(m.batch_indices, dev), _i32(m.positions, dev))


# -----------------------------------------------------------------------------
# algorithmic work (the roofline numerators)

def decode_bytes(w: Workload, kv_elem_bytes: int, q_elem_bytes: int = 2,
                 with_append: bool = False) -> int:
    """Algorithmic HBM bytes of one decode attention launch: every K/V element
    of every sequence once, q in and out once, the page table, and for e4m3
    the per-page scales; with_append adds the appended rows (read + write)."""
    m = w.meta
    kv = int(np.sum(m.seq_lens.astype(np.int64))) * w.hkv * w.d * 2 * kv_elem_bytes
    qo = m.batch_size * w.hq * w.d * 2 * q_elem_bytes
    meta = 4 * (len(m.kv_indices) + 2 * m.batch_size + 1)
    scales = len(m.kv_indices) * w.hkv * 2 * 4 if kv_elem_bytes == 1 else 0
    app = m.batch_size * w.hkv * w.d * 2 * (kv_elem_bytes + q_elem_bytes) if with_append else 0
    return kv + qo + meta + scales + app


def prefill_flops(w: Workload, causal: bool = True) -> int:
    """4 * Hq * D * (number of (query row, visible key) pairs)."""
    m = w.meta
    qo = (m.qo_indptr[1:] - m.qo_indptr[:-1]).astype(np.int64)
    kv = m.seq_lens.astype(np.int64)
    if causal:
        # sum_{i<qo} (kv - qo + i + 1), clipped at 0 and kv
        pairs = 0
        for q_b, k_b in zip(qo.tolist(), kv.tolist()):
            first = k_b - q_b + 1
            if first >= 1:
                pairs += q_b * first + q_b * (q_b - 1) // 2
            else:
                i = np.arange(q_b)
                pairs += int(np.clip(k_b - q_b + i + 1, 0, k_b).sum())
    else:
        pairs = int(np.sum(qo * kv))
    return 4 * w.hq * w.d * pairs
