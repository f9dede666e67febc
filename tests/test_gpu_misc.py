"""GPU parity of the small kernels: batch positions, page append (bf16,
fp16, e4m3), the e4m3 pool builder and RoPE, against the CPU oracle.
Integer and byte results must be bit-exact."""

import numpy as np
import pytest
import torch

import oracle as O
import pagedattn
from pagedattn import _lib
from pagedattn.metadata import decode_metadata, prefill_metadata

from paged_cases import i32, random_tables, strided_rows

pytestmark = pytest.mark.gpu


def test_one_hip_runtime(gpu):
    # the library must bind to torch's HIP runtime, not load a second one
    assert len(_lib.loaded_hip_runtimes()) == 1, _lib.loaded_hip_runtimes()
    assert _lib.lib().pagedattn_device_cu_count() > 0


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_batch_indices_positions(gpu, seed):
    rng = np.random.default_rng(seed)
    bsz = int(rng.integers(1, 40))
    counts = rng.integers(0, 600, size=bsz)
    counts[0] = 0  # an empty append range
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    lens = (counts + rng.integers(0, 5000, size=bsz)).astype(np.int32)
    nnz = int(indptr[-1])
    bi, pos = pagedattn.get_batch_indices_positions(i32(indptr, gpu), i32(lens, gpu), nnz)
    ebi, epos = O.batch_indices_positions(indptr, lens, nnz)
    assert np.array_equal(bi.cpu().numpy(), ebi)
    assert np.array_equal(pos.cpu().numpy(), epos)


def _append_case(gpu, dtype, seed, prefill):
    rng = np.random.default_rng(seed)
    hkv, d = 4, 64
    if prefill:
        computed = [0, 16, 35, 100]
        chunks = [17, 1, 64, 29]
        lens = [c + n for c, n in zip(computed, chunks)]
        tables, num_pages = random_tables(rng, lens, extra_pages=5)
        meta = prefill_metadata(tables, computed, chunks)
    else:
        lens = rng.integers(1, 300, size=37).tolist()
        tables, num_pages = random_tables(rng, lens, extra_pages=5)
        meta = decode_metadata(tables, lens)
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    pool = torch.randn((num_pages, 2, hkv, 16, d), generator=g, device=gpu,
                       dtype=torch.float32).to(dtype)
    nnz = meta.nnz
    # k and v are strided views of one fused projection, as in the engine
    qkv = torch.randn((nnz, (8 + 2 * hkv) * d), generator=g, device=gpu,
                      dtype=torch.float32).to(dtype)
    k = qkv[:, 8 * d:(8 + hkv) * d].view(nnz, hkv, d)
    v = qkv[:, (8 + hkv) * d:].view(nnz, hkv, d)
    return meta, pool, k, v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("prefill", [False, True])
def test_append_bit_exact(gpu, dtype, prefill):
    meta, pool, k, v = _append_case(gpu, dtype, 3, prefill)
    before = O.to_bits(pool)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    pagedattn.append_paged_kv_cache(k, v, i32(meta.batch_indices, gpu), i32(meta.positions, gpu),
                                    pool, i32(meta.kv_indices, gpu), i32(meta.kv_indptr, gpu),
                                    i32(meta.kv_last_page_len, gpu), kv_layout="HND",
                                    error_flag=err)
    want, skipped = O.append_pages(before, O.to_bits(k), O.to_bits(v), meta.batch_indices,
                                   meta.positions, meta.kv_indices, meta.kv_indptr)
    assert skipped == 0 and int(err.item()) == 0
    assert np.array_equal(O.to_bits(pool), want)


def test_append_bad_metadata_is_skipped_and_counted(gpu):
    meta, pool, k, v = _append_case(gpu, torch.bfloat16, 4, False)
    bi = meta.batch_indices.copy()
    pos = meta.positions.copy()
    bi[0] = 1000  # no such sequence
    pos[1] = pos[1] + 16 * 50  # past the end of its table
    pos[2] = -3
    before = O.to_bits(pool)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    pagedattn.append_paged_kv_cache(k, v, i32(bi, gpu), i32(pos, gpu), pool,
                                    i32(meta.kv_indices, gpu), i32(meta.kv_indptr, gpu),
                                    i32(meta.kv_last_page_len, gpu), kv_layout="HND",
                                    error_flag=err)
    want, skipped = O.append_pages(before, O.to_bits(k), O.to_bits(v), bi, pos,
                                   meta.kv_indices, meta.kv_indptr)
    assert skipped == 3 and int(err.item()) == 3
    assert np.array_equal(O.to_bits(pool), want)


def test_quantize_pages_bit_exact(gpu):
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    for d in (64, 128):
        pool = torch.randn((50, 2, 8, 16, d), generator=g, device=gpu).to(torch.bfloat16)
        pool[3, 1, 2] = 0
        pool[7, 0, 0, 3, 5] = 200.0  # an outlier sets the block scale
        q8, scales = pagedattn.quantize_pages_e4m3(pool)
        bits, ref_scales = O.quantize_pages(pool.cpu())
        assert torch.equal(scales.cpu(), ref_scales)
        assert np.array_equal(O.to_bits(q8), bits)


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16])
def test_append_e4m3_bit_exact(gpu, src):
    meta, pool, k, v = _append_case(gpu, src, 6, True)
    q8, scales = pagedattn.quantize_pages_e4m3(pool)
    # scale some rows up so the clamp at +-448 is exercised
    k = k * 40
    before = O.to_bits(q8)
    pagedattn.append_paged_kv_cache(k, v, i32(meta.batch_indices, gpu), i32(meta.positions, gpu),
                                    q8, i32(meta.kv_indices, gpu), i32(meta.kv_indptr, gpu),
                                    i32(meta.kv_last_page_len, gpu), kv_layout="HND",
                                    kv_scales=scales)
    want, skipped = O.append_pages_e4m3(before, scales.cpu(), k.cpu(), v.cpu(),
                                        meta.batch_indices, meta.positions, meta.kv_indices,
                                        meta.kv_indptr)
    assert skipped == 0
    assert np.array_equal(O.to_bits(q8), want)


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_rope", [False, True])
def test_append_e4m3_fixed_scale_counts(gpu, src, with_rope):
    # fixed-scale e4m3 appends (stand-alone and RoPE-fused) count every
    # skipped token in error_flag[0] and every clamped 8-element piece in
    # error_flag[1]; blocks with a zero or infinite scale get zero codes and
    # are counted as clamped too
    meta, pool, k, v = _append_case(gpu, src, 16, True)
    q8, scales = pagedattn.quantize_pages_e4m3(pool)
    pages = meta.kv_indices
    scales[int(pages[0]), 0, 1] = 0.0
    scales[int(pages[3]), 1, 2] = float("inf")
    k = (k.float() * 40).to(src)
    bi = meta.batch_indices.copy()
    pos = meta.positions.copy()
    bi[5] = 999
    pos[7] = -1
    g = torch.Generator(device=gpu)
    g.manual_seed(17)
    q = torch.randn((meta.nnz, 8, k.shape[2]), generator=g, device=gpu).to(src)
    before = O.to_bits(q8)
    ka = k.clone()
    if with_rope:
        qa = q.clone()
        pagedattn.apply_rope_pos_ids_inplace(qa, ka, i32(pos, gpu), rope_theta=1e4,
                                             rope_scale=1.0)
    want, skipped = O.append_pages_e4m3(before, scales.cpu(), ka.cpu().float(), v.cpu().float(),
                                        bi, pos, meta.kv_indices, meta.kv_indptr)
    clamped = O.e4m3_clamped_pieces(ka.cpu().float(), v.cpu().float(), scales.cpu(), bi, pos,
                                    meta.kv_indices, meta.kv_indptr, q8.shape[0])
    assert skipped == 2 and clamped > 2 * (k.shape[2] // 8)
    err = torch.zeros(2, dtype=torch.int32, device=gpu)
    args = (i32(bi, gpu), i32(pos, gpu), q8, i32(meta.kv_indices, gpu),
            i32(meta.kv_indptr, gpu), i32(meta.kv_last_page_len, gpu))
    if with_rope:
        pagedattn.rope_append_paged_kv_cache(q, k, v, *args, kv_layout="HND", rope_scale=1.0,
                                             rope_theta=1e4, kv_scales=scales, error_flag=err)
    else:
        pagedattn.append_paged_kv_cache(k, v, *args, kv_layout="HND", kv_scales=scales,
                                        error_flag=err)
    torch.cuda.synchronize()
    assert np.array_equal(O.to_bits(q8), want)
    assert err.tolist() == [skipped, clamped]


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -100)))
    return torch.pow(2.0, e - 7)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("theta,scale,interleave", [(10000.0, 1.0, False),
                                                    (500000.0, 1.0, False),
                                                    (10000.0, 4.0, True)])
def test_rope(gpu, dtype, theta, scale, interleave):
    g = torch.Generator(device=gpu)
    g.manual_seed(7)
    n, hq, hkv, d = 300, 32, 8, 128
    qkv = torch.randn((n, (hq + 2 * hkv) * d), generator=g, device=gpu).to(dtype)
    q = qkv[:, :hq * d].view(n, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(n, hkv, d)
    pos = torch.randint(0, 131072, (n,), generator=g, device=gpu, dtype=torch.int32)
    q0, k0 = q.float().cpu(), k.float().cpu()
    v_before = qkv[:, (hq + hkv) * d:].clone()
    pagedattn.apply_rope_pos_ids_inplace(q, k, pos, interleave=interleave, rope_scale=scale,
                                         rope_theta=theta)
    rq = O.rope(q0, pos.cpu().numpy(), theta, scale, interleave=interleave)
    rk = O.rope(k0, pos.cpu().numpy(), theta, scale, interleave=interleave)
    # within one ulp of the 16-bit result (fp32 sin/cos vs fp64 angles)
    tol = (_bf16_ulp(rq) if dtype == torch.bfloat16 else rq.abs() * 2.0 ** -10) + 1e-5
    assert bool(((q.float().cpu() - rq).abs() <= tol).all())
    tolk = (_bf16_ulp(rk) if dtype == torch.bfloat16 else rk.abs() * 2.0 ** -10) + 1e-5
    assert bool(((k.float().cpu() - rk).abs() <= tolk).all())
    assert torch.equal(qkv[:, (hq + hkv) * d:], v_before)  # v untouched


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("prefill", [False, True])
@pytest.mark.parametrize("fp8", [False, True])
def test_rope_append_equals_separate(gpu, dtype, prefill, fp8):
    # one launch == apply_rope_pos_ids_inplace then append_paged_kv_cache,
    # bit for bit: rotated q and k in place and the pool
    meta, pool, k, v = _append_case(gpu, dtype, 5, prefill)
    hq = 8
    g = torch.Generator(device=gpu)
    g.manual_seed(6)
    q = strided_rows(meta.nnz, hq, pool.shape[-1], dtype, gpu, g, lead=0, tail=8)
    scales = None
    if fp8:
        pool, scales = pagedattn.quantize_pages_e4m3(pool)
    pos = meta.positions.copy()
    bi = meta.batch_indices.copy()
    bi[0] = 1000  # a token the append must skip (and count); RoPE still rotates it
    args = dict(kv_layout="HND", kv_scales=scales)
    q_a, k_a, pool_a = q.clone(), k.clone(), pool.clone()
    err_a = torch.zeros(2, dtype=torch.int32, device=gpu)
    pagedattn.apply_rope_pos_ids_inplace(q_a, k_a, i32(pos, gpu), rope_theta=500000.0,
                                         rope_scale=2.0)
    pagedattn.append_paged_kv_cache(k_a, v, i32(bi, gpu), i32(pos, gpu), pool_a,
                                    i32(meta.kv_indices, gpu), i32(meta.kv_indptr, gpu),
                                    i32(meta.kv_last_page_len, gpu), error_flag=err_a, **args)
    q_b, k_b, pool_b = q.clone(), k.clone(), pool.clone()
    err_b = torch.zeros(2, dtype=torch.int32, device=gpu)
    pagedattn.rope_append_paged_kv_cache(q_b, k_b, v, i32(bi, gpu), i32(pos, gpu), pool_b,
                                         i32(meta.kv_indices, gpu), i32(meta.kv_indptr, gpu),
                                         i32(meta.kv_last_page_len, gpu), rope_scale=2.0,
                                         rope_theta=500000.0, error_flag=err_b, **args)
    torch.cuda.synchronize()
    assert torch.equal(q_a, q_b)
    assert torch.equal(k_a, k_b)
    assert np.array_equal(O.to_bits(pool_a), O.to_bits(pool_b))
    # the skipped token, plus (e4m3) the 8-element pieces clamped at +-448:
    # new rows are not bounded by the pool's per-page amax scales
    clamped = 0
    if fp8:
        clamped = O.e4m3_clamped_pieces(k_a.cpu().float(), v.cpu().float(), scales.cpu(), bi,
                                        pos, meta.kv_indices, meta.kv_indptr, pool.shape[0])
    assert err_a.tolist() == err_b.tolist() == [1, clamped]
