"""GPU parity of the KV write path against the oracle, bit-exact: the e4m3
running-amax append (prefill chunks, decode steps, partial pages, scale
growth, bad metadata) and the copy-on-write page fork (bf16 and e4m3 pools,
partial rows, bad forks), plus the CoW helper against a block allocator."""

import numpy as np
import pytest
import torch

import oracle as O
import pagedattn
from pagedattn import cow
from pagedattn.metadata import decode_metadata, prefill_metadata

from paged_cases import i32, random_tables

pytestmark = pytest.mark.gpu


def _rows(gen, n, hkv, d, dtype, device, lead=3):
    """[n, hkv, d] strided view, magnitudes spread over a few binades per row."""
    base = torch.randn((n, (lead + hkv) * d), generator=gen, device=device)
    spread = torch.exp(torch.randn((n, 1), generator=gen, device=device))
    return (base * spread).to(dtype)[:, lead * d:].view(n, hkv, d)


def _amax_append(gpu, meta, q8, scales, k, v, err=None, bi=None, pos=None):
    pagedattn.append_paged_kv_cache_e4m3_amax(
        k, v, i32(meta.batch_indices if bi is None else bi, gpu),
        i32(meta.positions if pos is None else pos, gpu), q8, i32(meta.kv_indices, gpu),
        i32(meta.kv_indptr, gpu), i32(meta.kv_last_page_len, gpu), scales, kv_layout="HND",
        error_flag=err)


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_amax_append_prefill_then_decode(gpu, src, d):
    rng = np.random.default_rng(10 + d)
    hkv = 4
    computed = [0, 0, 0, 0, 0]
    chunks = [17, 1, 64, 29, 5]
    steps = 21
    final = [c + steps for c in chunks]
    tables, num_pages = random_tables(rng, final, extra_pages=4)
    g = torch.Generator(device=gpu)
    g.manual_seed(d)
    q8 = torch.full((num_pages, 2, hkv, 16, d), 0x5A, dtype=torch.uint8,
                    device=gpu).view(torch.float8_e4m3fn)
    scales = torch.full((num_pages, 2, hkv), 7.0, device=gpu)  # stale values of a reused pool
    want_bits = O.to_bits(q8)
    want_sc = scales.cpu()
    # chunked prefill of every sequence, then single-token decode steps
    meta = prefill_metadata(tables, computed, chunks)
    k = _rows(g, meta.nnz, hkv, d, src, gpu)
    v = _rows(g, meta.nnz, hkv, d, src, gpu)
    _amax_append(gpu, meta, q8, scales, k, v)
    want_bits, want_sc, sk = O.append_pages_e4m3_running(
        want_bits, want_sc, k.cpu(), v.cpu(), meta.batch_indices, meta.positions,
        meta.kv_indices, meta.kv_indptr)
    assert sk == 0
    assert torch.equal(scales.cpu(), want_sc)
    assert np.array_equal(O.to_bits(q8), want_bits)
    lens = list(chunks)
    for step in range(steps):
        lens = [n + 1 for n in lens]
        meta = decode_metadata(tables, lens)
        grow = 1.0 + 3.0 * (step % 5 == 0)  # some steps raise the page amax
        k = _rows(g, meta.nnz, hkv, d, src, gpu) * grow
        v = _rows(g, meta.nnz, hkv, d, src, gpu)
        _amax_append(gpu, meta, q8, scales, k, v)
        want_bits, want_sc, sk = O.append_pages_e4m3_running(
            want_bits, want_sc, k.cpu(), v.cpu(), meta.batch_indices, meta.positions,
            meta.kv_indices, meta.kv_indptr)
        assert sk == 0
    assert torch.equal(scales.cpu(), want_sc)
    assert np.array_equal(O.to_bits(q8), want_bits)


def test_amax_append_continues_partial_pages_and_zero_rows(gpu):
    rng = np.random.default_rng(3)
    hkv, d = 8, 128
    computed = [5, 16, 31, 0, 40]
    chunks = [40, 3, 1, 16, 9]
    tables, num_pages = random_tables(rng, [c + n for c, n in zip(computed, chunks)])
    meta0 = prefill_metadata(tables, [0] * 5, computed)
    meta = prefill_metadata(tables, computed, chunks)
    g = torch.Generator(device=gpu)
    g.manual_seed(3)
    q8 = torch.zeros((num_pages, 2, hkv, 16, d), dtype=torch.uint8,
                     device=gpu).view(torch.float8_e4m3fn)
    scales = torch.zeros((num_pages, 2, hkv), device=gpu)
    bits, sc = O.to_bits(q8), scales.cpu()
    for m, mult in ((meta0, 1.0), (meta, 50.0)):
        k = _rows(g, m.nnz, hkv, d, torch.bfloat16, gpu) * mult
        v = _rows(g, m.nnz, hkv, d, torch.bfloat16, gpu) * 0.01
        if m is meta0:
            # head 2 of sequence 0's first 5 rows and of sequence 1's page are
            # all zero: zero scales, later grown from zero by the second call
            k[0:21, 2] = 0
        _amax_append(gpu, m, q8, scales, k, v)
        bits, sc, sk = O.append_pages_e4m3_running(bits, sc, k.cpu(), v.cpu(), m.batch_indices,
                                                   m.positions, m.kv_indices, m.kv_indptr)
        assert sk == 0
    assert float(sc[tables[1][0], 0, 2]) == 0.0
    assert torch.equal(scales.cpu(), sc)
    assert np.array_equal(O.to_bits(q8), bits)


def test_amax_append_bad_metadata_is_skipped_and_counted(gpu):
    rng = np.random.default_rng(4)
    hkv, d = 4, 64
    lens = [30, 17, 2, 50]
    tables, num_pages = random_tables(rng, lens)
    meta = prefill_metadata(tables, [0] * 4, lens)
    bi = meta.batch_indices.copy()
    pos = meta.positions.copy()
    bi[0] = 1000        # sequence 0's first token: a run of one
    pos[81:97] += 16 * 9  # sequence 3's third page: 16 tokens past its table
    pos[98] = -3        # sequence 3's last token
    g = torch.Generator(device=gpu)
    g.manual_seed(4)
    k = _rows(g, meta.nnz, hkv, d, torch.bfloat16, gpu)
    v = _rows(g, meta.nnz, hkv, d, torch.bfloat16, gpu)
    q8 = torch.zeros((num_pages, 2, hkv, 16, d), dtype=torch.uint8,
                     device=gpu).view(torch.float8_e4m3fn)
    scales = torch.zeros((num_pages, 2, hkv), device=gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    want, want_sc, skipped = O.append_pages_e4m3_running(
        O.to_bits(q8), scales.cpu(), k.cpu(), v.cpu(), bi, pos, meta.kv_indices, meta.kv_indptr)
    _amax_append(gpu, meta, q8, scales, k, v, err=err, bi=bi, pos=pos)
    assert skipped == 18 and int(err.item()) == 18
    assert torch.equal(scales.cpu(), want_sc)
    assert np.array_equal(O.to_bits(q8), want)


def _pool6(gpu, dtype, L, P, hkv, d, seed):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    x = torch.randn((L, P, 2, hkv, 16, d), generator=g, device=gpu)
    if dtype == torch.float8_e4m3fn:
        return (x * 40).clamp(-448, 448).to(dtype)
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_fork_pages_bit_exact(gpu, dtype):
    L, P, hkv, d = 4, 40, 8, 128
    pool = _pool6(gpu, dtype, L, P, hkv, d, 7)
    scales = None
    if dtype == torch.float8_e4m3fn:
        scales = torch.rand((L, P, 2, hkv), device=gpu)
    src = [3, 3, 17, 0, 22, 9]
    dst = [30, 31, 5, 39, 22, 12]
    valid = [7, 16, 1, 0, 4, 15]
    before = O.to_bits(pool)
    want, want_sc, sk = O.fork_pages(before, src, dst, valid,
                                     scales.cpu() if scales is not None else None)
    pagedattn.fork_pages(pool, src, dst, valid_tokens=valid, kv_scales=scales)
    assert sk == 0
    assert np.array_equal(O.to_bits(pool), want)
    if scales is not None:
        assert torch.equal(scales.cpu(), want_sc)
    # whole pages
    before = O.to_bits(pool)
    want, _, _ = O.fork_pages(before, [1, 2], [33, 34], None, None)
    pagedattn.fork_pages(pool, [1, 2], [33, 34], kv_scales=scales)
    assert np.array_equal(O.to_bits(pool), want)


def test_fork_pages_bad_forks_are_skipped_and_counted(gpu):
    L, P, hkv, d = 2, 10, 2, 64
    pool = _pool6(gpu, torch.float16, L, P, hkv, d, 8)
    src = [1, 11, 2, -1, 4]
    dst = [5, 6, 10, 7, 8]
    valid = [16, 3, 2, 2, 17]
    before = O.to_bits(pool)
    want, _, sk = O.fork_pages(before, src, dst, valid)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    # device tensors skip the host checks: the kernel checks and counts
    pagedattn.fork_pages(pool, i32(src, gpu), i32(dst, gpu), valid_tokens=i32(valid, gpu),
                         error_flag=err)
    assert sk == 4 and int(err.item()) == 4
    assert np.array_equal(O.to_bits(pool), want)
    with pytest.raises(ValueError, match="outside"):
        pagedattn.fork_pages(pool, src, dst, valid_tokens=valid)


class _Allocator:
    """The block allocator's interface (src/engine/memory/allocator.py:52-87)."""

    def __init__(self, n):
        self.free_blocks = list(range(n))
        self.ref_counts = [0] * n

    def allocate(self, n):
        if len(self.free_blocks) < n:
            raise RuntimeError("out of blocks")
        out, self.free_blocks = self.free_blocks[:n], self.free_blocks[n:]
        for b in out:
            self.ref_counts[b] = 1
        return out

    def incref(self, blocks):
        for b in blocks:
            self.ref_counts[b] += 1

    def decref(self, blocks):
        for b in blocks:
            assert self.ref_counts[b] > 0
            self.ref_counts[b] -= 1
            if self.ref_counts[b] == 0:
                self.free_blocks.append(b)


def test_cow_fork_for_append_then_append(gpu):
    L, P, hkv, d = 3, 24, 4, 64
    alloc = _Allocator(P)
    pool = _pool6(gpu, torch.bfloat16, L, P, hkv, d, 9)
    # A and B share two full pages and a partial third (11 rows); C is alone
    shared = alloc.allocate(3)
    tables = [list(shared), list(shared), alloc.allocate(2)]
    alloc.incref(shared)  # B's references
    alloc.incref(shared[2:])  # the radix cache's reference to the partial page
    lens = [43, 43, 20]
    before = O.to_bits(pool)
    forks = cow.fork_for_append(alloc, tables, lens, pool)
    # A forks (ref 3), B forks too (ref 2 left, the cache still holds it), C is not shared
    assert [(i, old) for i, old, _ in forks] == [(0, shared[2]), (1, shared[2])]
    new_a, new_b = forks[0][2], forks[1][2]
    assert tables[0][:2] == tables[1][:2] == shared[:2]
    assert tables[0][2] == new_a and tables[1][2] == new_b
    assert alloc.ref_counts[shared[2]] == 1
    want, _, _ = O.fork_pages(before, [shared[2]] * 2, [new_a, new_b], [11, 11])
    assert np.array_equal(O.to_bits(pool), want)
    # the appends that follow write the forks, leaving the shared page alone
    rows = torch.ones((2, hkv, d), dtype=torch.bfloat16, device=gpu)
    meta = decode_metadata([tables[0], tables[1]], [44, 44])
    for l in range(L):
        pagedattn.append_paged_kv_cache(rows, rows * 2, i32(meta.batch_indices, gpu),
                                        i32(meta.positions, gpu), pool[l],
                                        i32(meta.kv_indices, gpu), i32(meta.kv_indptr, gpu),
                                        i32(meta.kv_last_page_len, gpu), kv_layout="HND")
    after = O.to_bits(pool)
    assert np.array_equal(after[:, shared[2]], before[:, shared[2]])
    one = O.to_bits(rows[0])
    for p in (new_a, new_b):
        assert np.array_equal(after[:, p, 0, :, 11], np.broadcast_to(one, (L, hkv, d)))
    # a second call finds nothing left to fork
    assert cow.fork_for_append(alloc, tables, [44, 44, 20], pool) == []
