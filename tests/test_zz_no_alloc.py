"""pagedattn_decode_run_noalloc (the decode entry point that allocates
nothing: its split partials live in the library's static device array)
against pagedattn_decode_run with a device-side plan, through the C ABI:
the same kernels over the same partition, so outputs and log-sum-exp must
be equal bit for bit.  Two calls in a row, the second on a smaller batch
(the array keeps the first call's contents), then one with an e4m3 pool.
The call leaves the device's free memory unchanged, and a call captured in
a HIP graph replays to the eager call's bits."""

import math

import numpy as np
import pytest
import torch

import pagedattn
from pagedattn import _lib

from paged_cases import decode_case, i32, oracle_decode, rel_err, workspace

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _split_device_plan(monkeypatch):
    # the entry point runs the split device partition: compare with that one
    monkeypatch.setenv("PAGEDATTN_DECODE_SHARED", "0")


def _noalloc_call(meta_dev, pool, q, hq, hkv, d, out, lse, scales=None):
    """One pagedattn_decode_run_noalloc call on the current stream, on
    device tensors made beforehand (indptr, indices, last page lengths)."""
    lib = _lib.lib()
    indptr, ind, last = meta_dev
    bsz = last.numel()
    return lib.pagedattn_decode_run_noalloc(
        bsz, hq, hkv, d, 16, q.data_ptr(), q.stride(0), q.stride(1), _lib.dtype_code(q.dtype),
        pool.data_ptr(), _lib.dtype_code(pool.dtype),
        None if scales is None else scales.data_ptr(), pool.shape[0], ind.data_ptr(),
        ind.numel(), indptr.data_ptr(), last.data_ptr(), out.data_ptr(), lse.data_ptr(),
        1.0 / math.sqrt(d), _lib.stream_of(q.device))


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


def test_noalloc_allocates_nothing_and_replays_from_a_graph(gpu):
    rng = np.random.default_rng(93)
    hq, hkv, d = 32, 8, 128
    lens = rng.integers(1, 5000, 48).tolist()
    meta, pool, q = decode_case(gpu, lens, hq, hkv, d, seed=9)
    meta_dev = (i32(meta.kv_indptr, gpu), i32(meta.kv_indices, gpu),
                i32(meta.kv_last_page_len, gpu))
    bsz = len(lens)
    out = torch.empty((bsz, hq, d), dtype=q.dtype, device=gpu)
    lse = torch.empty((bsz, hq), dtype=torch.float32, device=gpu)
    assert _noalloc_call(meta_dev, pool, q, hq, hkv, d, out, lse) == 0  # per-device set-up
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(gpu)[0]
    assert _noalloc_call(meta_dev, pool, q, hq, hkv, d, out, lse) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(gpu)[0] == free0
    want_o, want_l = out.clone(), lse.clone()

    # capture the call in a graph (its output buffers at fixed addresses) and
    # replay it, with eager work and synchronisation between replays
    g_out = torch.full_like(out, float("nan"))
    g_lse = torch.full_like(lse, float("nan"))
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = _noalloc_call(meta_dev, pool, q, hq, hkv, d, g_out, g_lse)
    assert rc == 0, _lib.lib().pagedattn_last_error()
    torch.cuda.current_stream(gpu).wait_stream(side)
    for rep in range(3):
        g_out.fill_(float("nan"))
        g_lse.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_out, want_o), rep
        assert torch.equal(g_lse, want_l), rep
        # eager work between replays
        assert _noalloc_call(meta_dev, pool, q, hq, hkv, d, out, lse) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, want_o)
