"""pagedattn_decode_run_noalloc (the decode entry point that allocates
nothing: its split partials live in the library's static device array)
against pagedattn_decode_run with a device-side plan, through the C ABI:
the same kernels over the same partition, so outputs and log-sum-exp must
be equal bit for bit.  Two calls in a row, the second on a smaller batch
(the array keeps the first call's contents), then one with an e4m3 pool."""

import math

import numpy as np
import pytest
import torch

import pagedattn
from pagedattn import _lib

from paged_cases import decode_case, i32, oracle_decode, rel_err, workspace

pytestmark = pytest.mark.gpu


def _run_noalloc(meta, pool, q, hq, hkv, d, scales=None):
    lib = _lib.lib()
    bsz = len(meta.kv_last_page_len)
    dev = q.device
    out = torch.full((bsz, hq, d), float("nan"), dtype=q.dtype, device=dev)
    lse = torch.full((bsz, hq), float("nan"), dtype=torch.float32, device=dev)
    indptr = i32(meta.kv_indptr, dev)
    ind = i32(meta.kv_indices, dev)
    last = i32(meta.kv_last_page_len, dev)
    rc = lib.pagedattn_decode_run_noalloc(
        bsz, hq, hkv, d, 16, q.data_ptr(), q.stride(0), q.stride(1), _lib.dtype_code(q.dtype),
        pool.data_ptr(), _lib.dtype_code(pool.dtype),
        None if scales is None else scales.data_ptr(), pool.shape[0], ind.data_ptr(),
        ind.numel(), indptr.data_ptr(), last.data_ptr(), out.data_ptr(), lse.data_ptr(),
        1.0 / math.sqrt(d), _lib.stream_of(dev))
    assert rc == 0, lib.pagedattn_last_error()
    torch.cuda.synchronize()
    return out, lse


def _run_device_plan(gpu, meta, pool, q, hq, hkv, d, scales=None):
    w = pagedattn.BatchDecodeWithPagedKVCacheWrapper(workspace(gpu), "HND")
    w.plan(i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu), i32(meta.kv_last_page_len, gpu),
           hq, hkv, d, 16, q_data_type=q.dtype, device_plan=True)
    out, lse = w.run(q, pool, kv_scales=scales, return_lse=True)
    torch.cuda.synchronize()
    return out, lse


def test_noalloc_decode_equals_device_plan(gpu):
    rng = np.random.default_rng(91)
    hq, hkv, d = 64, 8, 128
    # a large batch first (many cut sequences: every share slot written),
    # then a smaller one over the partials the first left behind
    for lens in (rng.integers(1, 6000, 96).tolist(), rng.integers(1, 900, 7).tolist()):
        meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=len(lens))
        ref_o, ref_l = _run_device_plan(gpu, meta, pool, q, hq, hkv, d)
        out, lse = _run_noalloc(meta, pool, q, hq, hkv, d)
        assert torch.equal(out, ref_o)
        assert torch.equal(lse, ref_l)
        # and the oracle's answer, on a few sequences
        rows = sorted({0, len(lens) - 1, int(np.argmax(lens))})
        o_ref, _ = oracle_decode(meta, pool, q, batch=rows)
        assert rel_err(out, o_ref, rows=rows) <= 2e-2


def test_noalloc_decode_e4m3_and_small_heads(gpu):
    rng = np.random.default_rng(92)
    hq, hkv, d = 32, 4, 64
    lens = rng.integers(1, 3000, 40).tolist()
    meta, pool16, q = decode_case(gpu, lens, hq, hkv, d, seed=5)
    pool, scales = pagedattn.quantize_pages_e4m3(pool16)
    ref_o, ref_l = _run_device_plan(gpu, meta, pool, q, hq, hkv, d, scales)
    out, lse = _run_noalloc(meta, pool, q, hq, hkv, d, scales)
    assert torch.equal(out, ref_o)
    assert torch.equal(lse, ref_l)
