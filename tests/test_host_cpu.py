"""CPU-only checks of the host side: the C-ABI library loads and exports
every symbol include/pagedattn.h declares, host-side validation rejects bad
metadata before touching a device, the metadata builders follow the step
executor's rules, and the workload generators / work formulas are right."""

import ctypes
import math
import os
import re

import numpy as np
import pytest
import torch

import pagedattn
from pagedattn import _lib
from pagedattn import workloads as W
from pagedattn.metadata import decode_metadata, prefill_metadata

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pagedattn.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pagedattn_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _declared_functions()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
        assert name in _lib.EXPORTED, f"{name} has no ctypes signature"
    assert lib.pagedattn_abi_version() == 1


def _plan_call(indptr, last, hq=32, hkv=4, d=64, page=16, ws=1 << 20, bsz=None):
    lib = _lib.lib()
    plan = lib.pagedattn_plan_create()
    indptr = np.asarray(indptr, np.int32)
    last = np.asarray(last, np.int32)
    bsz = len(last) if bsz is None else bsz
    # the workspace pointer is never dereferenced when validation fails
    rc = lib.pagedattn_decode_plan(plan, indptr.ctypes.data, last.ctypes.data, bsz, hq, hkv, d,
                                   page, 0, 4096, ws, None)
    msg = lib.pagedattn_last_error().decode()
    lib.pagedattn_plan_destroy(plan)
    return rc, msg


@pytest.mark.parametrize("indptr,last,kw,code,needle", [
    ([0, 3, 2], [5, 5], {}, 1, "monotone"),
    ([0, 2, 4], [0, 5], {}, 1, "kv_last_page_len"),
    ([0, 2, 4], [5, 17], {}, 1, "kv_last_page_len"),
    ([0, 2], [5], {"page": 32}, 2, "page_size"),
    ([0, 2], [5], {"d": 96}, 2, "head_dim"),
    ([0, 2], [5], {"hq": 30, "hkv": 4}, 1, "multiple"),
    ([0, 2], [5], {"hq": 96, "hkv": 4}, 2, "group size"),
])
def test_plan_validation(indptr, last, kw, code, needle):
    rc, msg = _plan_call(indptr, last, **kw)
    assert rc == code and needle in msg, (rc, msg)


def test_plan_workspace_too_small():
    lens = [16 * 100] * 64
    indptr = np.concatenate([[0], np.cumsum([100] * 64)])
    rc, msg = _plan_call(indptr, [16] * 64, ws=512)
    # the partition needs more than 512 bytes: rejected before any upload
    assert rc == 3 and "workspace" in msg


def test_abi_rejects_bad_arguments_without_device():
    lib = _lib.lib()
    rc = lib.pagedattn_append_paged_kv_cache(None, None, 0, 0, 0, 0, 7, None, None, 1, None, 7,
                                             None, 1, None, 1, None, None, 1, 4, 64, 16, None,
                                             None)
    assert rc == 2 and "dtype" in lib.pagedattn_last_error().decode()
    rc = lib.pagedattn_decode_run(None, None, 0, 0, 1, None, 1, None, 0, None, 0, None, None,
                                  None, None, ctypes.c_float(1.0), None)
    assert rc == 5
    rc = lib.pagedattn_copy_bytes(None, None, 15, None)
    assert rc == 1


def test_wrappers_require_device_tensors():
    ws = torch.zeros(1024, dtype=torch.uint8)
    with pytest.raises(ValueError, match="device"):
        pagedattn.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    with pytest.raises(NotImplementedError, match="HND"):
        pagedattn.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")


def test_decode_metadata_rules():
    tables = [[5, 6, 7], [1], [2, 3]]
    m = decode_metadata(tables, [33, 16, 17])
    assert m.kv_indptr.tolist() == [0, 3, 4, 6]
    assert m.kv_last_page_len.tolist() == [1, 16, 1]
    assert m.positions.tolist() == [32, 15, 16]
    # the reference passes whole tables: a reserved extra page overstates kv_len
    m2 = decode_metadata([[5, 6, 7], [1, 9], [2, 3]], [33, 16, 17], trim_tables=False)
    lens = (np.diff(m2.kv_indptr) - 1) * 16 + m2.kv_last_page_len
    assert lens.tolist() == [33, 32, 17]
    m3 = decode_metadata([[5, 6, 7], [1, 9], [2, 3]], [33, 16, 17])
    lens3 = (np.diff(m3.kv_indptr) - 1) * 16 + m3.kv_last_page_len
    assert lens3.tolist() == [33, 16, 17]


def test_prefill_metadata_rules():
    m = prefill_metadata([[4, 5, 6], [7, 8]], [16, 0], [20, 17])
    assert m.qo_indptr.tolist() == [0, 20, 37]
    assert m.kv_indptr.tolist() == [0, 3, 5]
    assert m.kv_indices.tolist() == [4, 5, 6, 7, 8]
    assert m.kv_last_page_len.tolist() == [4, 1]
    assert m.positions[:3].tolist() == [16, 17, 18] and m.positions[20] == 0
    with pytest.raises(ValueError):
        prefill_metadata([[1]], [16], [5])


def _pages_used(meta):
    return [meta.kv_indices[meta.kv_indptr[b]:meta.kv_indptr[b + 1]].tolist()
            for b in range(meta.batch_size)]


def test_workloads_shapes():
    w = W.tinyllama_decode_small(0)
    assert (w.hq, w.hkv, w.d, w.num_pages) == (32, 4, 64, 256)
    assert w.meta.seq_lens.min() >= 64 and w.meta.seq_lens.max() <= 512
    used = [p for t in _pages_used(w.meta) for p in t]
    assert len(used) == len(set(used)) and max(used) < 256
    w2 = W.tinyllama_decode(0)
    need = sum(math.ceil(n / 16) for n in w2.meta.seq_lens)
    assert w2.num_pages == math.ceil(1.2 * need) and w2.meta.batch_size == 256
    used2 = [p for t in _pages_used(w2.meta) for p in t]
    assert len(used2) == len(set(used2)) == need
    w3 = W.llama3_8b_prefill(0)
    tabs = _pages_used(w3.meta)
    for gi, pre in enumerate(w3.extra["prefixes"]):
        assert pre % 16 == 0
        grp = tabs[4 * gi:4 * gi + 4]
        for t in grp:  # the group shares its prefix pages
            assert t[:pre // 16] == grp[0][:pre // 16]
    qo = np.diff(w3.meta.qo_indptr)
    assert qo.min() >= 64 and qo.max() <= 512
    w4 = W.llama3_8b_long_decode(0)
    assert w4.split_pages == 256
    dec, pre = W.llama3_70b_mixed_fp8(0)
    assert dec.meta.batch_size == 128 and pre.meta.batch_size == 4
    assert np.diff(pre.meta.qo_indptr).tolist() == [1024] * 4
    used_d = {p for t in _pages_used(dec.meta) for p in t}
    used_p = {p for t in _pages_used(pre.meta) for p in t}
    assert not used_d & used_p
    assert max(used_d | used_p) < dec.num_pages


def test_work_formulas_brute_force():
    w = W.llama3_8b_prefill(1)
    m = w.meta
    pairs = 0
    for b in range(m.batch_size):
        qo = int(m.qo_indptr[b + 1] - m.qo_indptr[b])
        kv = int(m.seq_lens[b])
        for i in range(qo):
            pairs += sum(1 for j in range(kv) if j <= kv - qo + i)
    assert W.prefill_flops(w) == 4 * w.hq * w.d * pairs
    d = W.tinyllama_decode_small(0)
    want = (int(d.meta.seq_lens.sum()) * 4 * 64 * 2 * 2 + 8 * 32 * 64 * 4
            + 4 * (len(d.meta.kv_indices) + 17))
    assert W.decode_bytes(d, 2) == want


def test_bytes_per_block_and_sizing():
    from pagedattn import capacity as C
    # the reference's rule (capacity.py:16-32): layers x 2 x heads x block x dim x element size
    assert C.bytes_per_block(16, 32, 8, 128, torch.bfloat16) == 32 * 2 * 8 * 16 * 128 * 2
    assert C.bytes_per_block(16, 22, 4, 64, torch.float16) == 22 * 2 * 4 * 16 * 64 * 2
    # e4m3: one byte per element plus an fp32 scale per (layer, K|V, head)
    assert C.bytes_per_block(16, 80, 8, 128, torch.float8_e4m3fn) == \
        80 * 2 * 8 * 16 * 128 + 80 * 2 * 8 * 4
    per = C.bytes_per_block(16, 32, 8, 128, torch.bfloat16)
    free = 100 * 1024 ** 3
    usable = free - max(2 * 1024 ** 3, int(free * 0.15))
    assert C.blocks_for_free_bytes(free, 16, 32, 8, 128, torch.bfloat16) == usable // per
    with pytest.raises(RuntimeError, match="need at least"):
        C.blocks_for_free_bytes(3 * 1024 ** 3, 16, 32, 8, 128, torch.bfloat16, min_blocks=10 ** 6)
    assert C.estimate_num_blocks(torch.device("cpu"), 16, 32, 8, 128, torch.bfloat16) == -1


class _FakeAllocator:
    def __init__(self, n):
        self.free_blocks = list(range(n))
        self.ref_counts = [0] * n

    def allocate(self, n):
        if len(self.free_blocks) < n:
            raise RuntimeError("Not enough free KV blocks")
        out, self.free_blocks = self.free_blocks[:n], self.free_blocks[n:]
        for b in out:
            self.ref_counts[b] = 1
        return out

    def decref(self, blocks):
        for b in blocks:
            self.ref_counts[b] -= 1
            if self.ref_counts[b] == 0:
                self.free_blocks.append(b)


def test_cow_fork_decisions(monkeypatch):
    from pagedattn import cow
    calls = []
    monkeypatch.setattr(cow.ops, "fork_pages",
                        lambda pool, src, dst, valid_tokens=None, kv_scales=None:
                        calls.append((list(src), list(dst), list(valid_tokens))))
    a = _FakeAllocator(10)
    t_shared = a.allocate(2)            # [0, 1]
    for b in t_shared:
        a.ref_counts[b] = 2             # shared by sequences 0 and 1
    tables = [list(t_shared), list(t_shared), a.allocate(1), list(t_shared[:1])]
    a.ref_counts[0] += 1                # sequence 3 shares page 0 too
    # seq 0: next token in shared partial page 1 -> fork; seq 1: page 1 now
    # held by seq 1 alone -> no fork; seq 2: own page; seq 3: page 0 full -> no fork
    forks = cow.fork_for_append(a, tables, [20, 20, 3, 16], None)
    assert forks == [(0, 1, 3)]
    assert calls == [([1], [3], [4])]
    assert tables[0] == [0, 3] and tables[1] == [0, 1]
    assert a.ref_counts[1] == 1 and a.ref_counts[3] == 1
    with pytest.raises(RuntimeError, match="Not enough"):
        a2 = _FakeAllocator(1)
        p = a2.allocate(1)
        a2.ref_counts[p[0]] = 2
        cow.fork_for_append(a2, [p], [5], None)
