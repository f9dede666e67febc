"""Pins the CPU oracle (oracle/paged_ref.py) before GPU results are compared
with it: closed forms, pure-Python loops, fp64 brute-force golden vectors
(tests/golden/), invariants, transformers' RoPE, and planted mistakes that
these pins must catch."""

import math
import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_small.npz")


# -----------------------------------------------------------------------------
# metadata

def test_kv_lengths_closed_form():
    indptr = [0, 1, 1, 4, 6]
    last = [3, 9, 16, 1]
    assert O.kv_lengths(indptr, last).tolist() == [3, 0, 16 * 2 + 16, 16 + 1]


def _positions_loop(indptr, lens, nnz):
    bi = [0] * nnz
    po = [0] * nnz
    for b in range(len(lens)):
        n = indptr[b + 1] - indptr[b]
        for j in range(indptr[b], indptr[b + 1]):
            bi[j] = b
            po[j] = lens[b] - n + (j - indptr[b])
    return bi, po


def test_batch_positions_loop():
    rng = np.random.default_rng(1)
    for _ in range(20):
        bsz = int(rng.integers(1, 9))
        counts = rng.integers(0, 40, size=bsz)
        indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        lens = counts + rng.integers(0, 500, size=bsz)
        bi, po = O.batch_indices_positions(indptr, lens, int(indptr[-1]))
        ebi, epo = _positions_loop(indptr.tolist(), lens.tolist(), int(indptr[-1]))
        assert bi.tolist() == ebi and po.tolist() == epo


def test_batch_positions_match_caller():
    # the caller's own position_ids (step_executor.py:149-152) equal the oracle's
    from pagedattn.metadata import prefill_metadata
    computed, chunks = [0, 32, 7], [5, 17, 1]
    tables = [[0, 1], [2, 3, 4, 5], [6]]
    m = prefill_metadata(tables, computed, chunks)
    bi, po = O.batch_indices_positions(m.qo_indptr, m.seq_lens, m.nnz)
    assert po.tolist() == m.positions.tolist()
    assert bi.tolist() == m.batch_indices.tolist()


# -----------------------------------------------------------------------------
# append / gather

def _rand_pool(rng, p, h, d):
    return rng.integers(0, 2**16, size=(p, 2, h, 16, d), dtype=np.uint16)


def test_append_loop():
    rng = np.random.default_rng(2)
    p, h, d = 12, 2, 8
    pool = _rand_pool(rng, p, h, d)
    indptr = np.array([0, 3, 5, 9], dtype=np.int32)
    ind = rng.permutation(p)[:9].astype(np.int32)
    n = 30
    bi = rng.integers(0, 3, size=n).astype(np.int32)
    pos = rng.integers(0, 48, size=n).astype(np.int32)
    # make (b, pos) unique so the scatter has no write conflicts
    key = np.unique(bi.astype(np.int64) * 1000 + pos, return_index=True)[1]
    bi, pos = bi[key], pos[key]
    bi[0] = 7  # out of range batch
    pos[1] = 16 * 9  # beyond its table
    k = rng.integers(0, 2**16, size=(len(bi), h, d), dtype=np.uint16)
    v = rng.integers(0, 2**16, size=(len(bi), h, d), dtype=np.uint16)
    got, skipped = O.append_pages(pool, k, v, bi, pos, ind, indptr)
    want = pool.copy()
    sk = 0
    for j in range(len(bi)):
        b, ps = int(bi[j]), int(pos[j])
        if not (0 <= b < 3):
            sk += 1
            continue
        it = int(indptr[b]) + ps // 16
        if it >= int(indptr[b + 1]):
            sk += 1
            continue
        page = int(ind[it])
        for hh in range(h):
            for t in range(d):
                want[page, 0, hh, ps % 16, t] = k[j, hh, t]
                want[page, 1, hh, ps % 16, t] = v[j, hh, t]
    assert skipped == sk >= 1
    assert np.array_equal(got, want)


def test_append_untouched():
    rng = np.random.default_rng(3)
    p, h, d = 6, 1, 4
    pool = np.full((p, 2, h, 16, d), 0xBEEF, dtype=np.uint16)
    indptr = np.array([0, 2], dtype=np.int32)
    ind = np.array([4, 1], dtype=np.int32)
    k = np.zeros((3, h, d), dtype=np.uint16)
    v = np.ones((3, h, d), dtype=np.uint16)
    got, _ = O.append_pages(pool, k, v, np.zeros(3, np.int32), np.array([0, 17, 31], np.int32),
                            ind, indptr)
    changed = np.argwhere(got != pool)
    touched = {(int(a), int(b_), int(c)) for a, b_, _, c, _ in changed}
    assert touched == {(4, 0, 0), (4, 1, 0), (1, 0, 1), (1, 1, 1), (1, 0, 15), (1, 1, 15)}


def test_append_gather_roundtrip():
    rng = np.random.default_rng(4)
    p, h, d = 10, 2, 8
    pool = torch.randn(p, 2, h, 16, d).to(torch.bfloat16)
    bits = O.to_bits(pool)
    lens = [5, 33]
    indptr = np.array([0, 1, 4], dtype=np.int32)
    ind = np.array([7, 2, 9, 0], dtype=np.int32)
    last = np.array([5, 1], dtype=np.int32)
    bi = np.array([0] * 5 + [1] * 33, dtype=np.int32)
    pos = np.array(list(range(5)) + list(range(33)), dtype=np.int32)
    k = torch.randn(len(bi), h, d).to(torch.bfloat16)
    v = torch.randn(len(bi), h, d).to(torch.bfloat16)
    newbits, skipped = O.append_pages(bits, O.to_bits(k), O.to_bits(v), bi, pos, ind, indptr)
    assert skipped == 0
    newpool = O.from_bits(newbits, torch.bfloat16).reshape(pool.shape)
    for b in range(2):
        kk, vv = O.gather_pages(newpool, indptr, ind, last, b)
        sel = bi == b
        assert kk.shape[0] == lens[b]
        assert torch.equal(kk, k[torch.from_numpy(sel)].float())
        assert torch.equal(vv, v[torch.from_numpy(sel)].float())


def test_gather_permutation():
    # relabelling physical pages (pool and tables together) changes nothing
    rng = np.random.default_rng(5)
    pool = torch.randn(8, 2, 2, 16, 4)
    indptr = np.array([0, 3], dtype=np.int32)
    ind = np.array([5, 0, 6], dtype=np.int32)
    last = np.array([9], dtype=np.int32)
    perm = rng.permutation(8)
    inv = np.argsort(perm)
    pool2 = pool[torch.from_numpy(inv)]  # page x moves to slot perm[x]
    ind2 = perm[ind].astype(np.int32)
    k1, v1 = O.gather_pages(pool, indptr, ind, last, 0)
    k2, v2 = O.gather_pages(pool2, indptr, ind2, last, 0)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert k1.shape[0] == 2 * 16 + 9


# -----------------------------------------------------------------------------
# fp8

def _all_finite_e4m3():
    bits = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(bits).view(torch.float8_e4m3fn).float()
    ok = torch.isfinite(vals).numpy()
    return bits[ok], vals[torch.from_numpy(ok)]


def test_e4m3_roundtrip_exact():
    bits, vals = _all_finite_e4m3()
    enc = O.e4m3_encode(vals, 1.0)
    # +0 and -0 both keep their sign bit
    assert np.array_equal(enc, bits)
    assert torch.equal(O.e4m3_decode(bits, 1.0), vals)
    assert float(vals.abs().max()) == O.E4M3_MAX


def test_e4m3_rounding_ties():
    # 1 + 1/16 lies halfway between 1 and 1.125: ties go to the even mantissa (1.0);
    # 1 + 3/16 lies between 1.125 and 1.25: tie goes to 1.25 (even)
    x = torch.tensor([1.0625, 1.1875, 1000.0, -1000.0, 2.0 ** -10, 0.0])
    dec = O.e4m3_decode(O.e4m3_encode(x, 1.0), 1.0)
    assert dec.tolist() == [1.0, 1.25, 448.0, -448.0, 0.0, 0.0]
    # scaling: x / scale is what is rounded
    assert O.e4m3_decode(O.e4m3_encode(torch.tensor([3.0]), 2.0), 2.0).item() == 3.0


def test_quantize_pages_scale():
    pool = torch.randn(3, 2, 2, 16, 8).to(torch.bfloat16)
    pool[1, 1, 0] = 0  # an all-zero block gets scale 1
    bits, scales = O.quantize_pages(pool)
    assert scales[1, 1, 0].item() == 1.0
    amax = pool.float().abs().amax(dim=(3, 4))
    nz = amax > 0
    assert torch.equal(scales[nz], amax[nz] / 448.0)
    dec = O.e4m3_decode(bits, scales[..., None, None])
    # the amax element of every block encodes to +-448 and decodes to +-amax
    # (up to the rounding of 448 * (amax / 448) in fp32)
    assert int(np.abs(bits.astype(np.int16) & 0x7F).max()) == 0x7E
    assert torch.allclose(dec.abs().amax(dim=(3, 4))[nz], amax[nz], rtol=2.0 ** -22, atol=0)
    # dequantised values are within half an e4m3 ulp (relative 2^-4) of the source
    err = (dec - pool.float()).abs()
    bound = torch.maximum(pool.float().abs() * 2.0 ** -4, scales[..., None, None] * 2.0 ** -10)
    assert bool((err <= bound + 1e-12).all())


# fixed-scale e4m3 append and e4m3 gather, pinned element by element: the
# e4m3fn value of a code is computed from its bit fields, and rounding is a
# brute-force search for the nearest code (ties to the even mantissa), so
# neither pin goes through torch's float8 conversion that the oracle uses.

def _e4m3_value(code: int) -> float:
    """OCP e4m3fn: sign, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0
    is subnormal (m / 8 * 2^-6); S.1111.111 is NaN; no infinities."""
    sign = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 0xF, code & 0x7
    if e == 0xF and m == 0x7:
        return math.nan
    if e == 0:
        return sign * (m / 8.0) * 2.0 ** -6
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


_E4M3_POS = [(_e4m3_value(c), c) for c in range(0x7F)]  # 0 .. 448, increasing


def _e4m3_round(y: float) -> int:
    """Code of the e4m3fn value nearest to y after clamping to +-448; a tie
    takes the even code (round to nearest even); the sign of y is kept (-0
    included)."""
    neg = math.copysign(1.0, y) < 0
    a = min(abs(y), 448.0)
    best = None
    for val, code in _E4M3_POS:
        d = abs(val - a)
        if best is None or d < best[0] or (d == best[0] and code % 2 == 0):
            best = (d, code)
    return best[1] | (0x80 if neg else 0)


def test_e4m3_bitfield_table_matches_torch():
    # the bit-field decoder itself agrees with the float8 dtype on all 256 codes
    vals = torch.from_numpy(np.arange(256, dtype=np.uint8)).view(torch.float8_e4m3fn).float()
    for c in range(256):
        want = float(vals[c])
        got = _e4m3_value(c)
        assert (math.isnan(got) and math.isnan(want)) or got == want, c


def _append_e4m3_loop(pool, scales, k, v, bi, pos, ind, indptr, kscale_kind=0, vscale_kind=1,
                      head_shift=0):
    """Per-element restatement of the fixed-scale e4m3 append; the keyword
    arguments plant mistakes (which scale a kind reads, a head offset)."""
    out = pool.copy()
    n_pages, _, h_n, _, d = pool.shape
    skipped = 0
    clamped = 0
    for j in range(len(bi)):
        b, ps = int(bi[j]), int(pos[j])
        if not (0 <= b < len(indptr) - 1) or ps < 0:
            skipped += 1
            continue
        it = int(indptr[b]) + ps // 16
        if it >= int(indptr[b + 1]) or it >= len(ind):
            skipped += 1
            continue
        page = int(ind[it])
        if not (0 <= page < n_pages):
            skipped += 1
            continue
        for kind, src, skind in ((0, k, kscale_kind), (1, v, vscale_kind)):
            for h in range(h_n):
                s = np.float32(scales[page, skind, (h + head_shift) % h_n])
                ok = bool(s > 0) and math.isfinite(float(s))
                for c0 in range(0, d, 8):
                    piece_bad = not ok
                    for t in range(c0, c0 + 8):
                        if ok:
                            y = np.float32(np.float32(src[j, h, t]) / s)
                            piece_bad |= not (abs(float(y)) <= 448.0)
                            out[page, kind, h, ps % 16, t] = _e4m3_round(float(y))
                        else:
                            out[page, kind, h, ps % 16, t] = 0
                    clamped += int(piece_bad)
    return out, skipped, clamped


def _e4m3_append_case(seed=6):
    rng = np.random.default_rng(seed)
    p, h, d = 7, 3, 16
    pool = rng.integers(0, 256, size=(p, 2, h, 16, d), dtype=np.uint8)
    pool[pool & 0x7F == 0x7F] = 0  # no NaN codes in the starting pool
    scales = torch.from_numpy(
        np.ldexp(1.0, rng.integers(-6, 3, size=(p, 2, h))).astype(np.float32)
        * rng.choice([1.0, 0.75, 1.3], size=(p, 2, h)).astype(np.float32))
    scales[2, 1, 0] = 0.0       # a fresh page: zero codes, counted
    scales[4, 0, 2] = math.inf  # not finite: zero codes, counted
    indptr = np.array([0, 2, 4, 6], dtype=np.int32)
    ind = np.array([3, 2, 5, 4, 0, 6], dtype=np.int32)
    bi = np.array([0, 0, 1, 1, 2, 2, 5, 1], dtype=np.int32)  # batch 5 is out of range
    pos = np.array([0, 17, 3, 30, 9, 16, 0, 40], dtype=np.int32)  # 40 is past seq 1's pages
    n = len(bi)
    k = torch.from_numpy(rng.normal(size=(n, h, d)).astype(np.float32)).to(torch.bfloat16)
    v = torch.from_numpy(rng.normal(size=(n, h, d)).astype(np.float32)).to(torch.bfloat16)
    # exact ties of e4m3 rounding and values past the clamp
    k[0, 0, :4] = torch.tensor([1.0625, 1.1875, -1.0625, 0.0]) * float(scales[3, 0, 0])
    k[1, 1, 5] = 1000.0 * float(scales[2, 0, 1])
    v[2, 2, 8] = -600.0 * float(scales[5, 1, 2])
    return pool, scales, k.float(), v.float(), bi, pos, ind, indptr


def test_append_e4m3_loop():
    pool, scales, k, v, bi, pos, ind, indptr = _e4m3_append_case()
    want, want_skip, want_clamp = _append_e4m3_loop(pool, scales.numpy(), k.numpy(), v.numpy(),
                                                    bi, pos, ind, indptr)
    got, skipped = O.append_pages_e4m3(pool, scales, k, v, bi, pos, ind, indptr)
    assert skipped == want_skip == 2
    assert np.array_equal(got, want)
    clamped = O.e4m3_clamped_pieces(k, v, scales, bi, pos, ind, indptr, pool.shape[0])
    # two over-range values, a zero scale and an infinite scale (2 pieces each)
    assert clamped == want_clamp
    assert clamped >= 2 + 2 + 2


def test_gather_e4m3_loop():
    pool, scales, k, v, bi, pos, ind, indptr = _e4m3_append_case(7)
    bits, _ = O.append_pages_e4m3(pool, scales, k, v, bi, pos, ind, indptr)
    last = np.array([16, 16, 7], dtype=np.int32)
    f8 = torch.from_numpy(bits).view(torch.float8_e4m3fn)
    for b in range(3):
        kk, vv = O.gather_pages(f8, indptr, ind, last, b, scales)
        n_tok = (indptr[b + 1] - indptr[b] - 1) * 16 + last[b]
        assert kk.shape[0] == n_tok
        for i in range(n_tok):
            page = int(ind[indptr[b] + i // 16])
            for kind, got in ((0, kk), (1, vv)):
                for h in range(bits.shape[2]):
                    s = np.float32(scales[page, kind, h])
                    for t in range(bits.shape[4]):
                        want = float(np.float32(_e4m3_value(int(bits[page, kind, h, i % 16,
                                                                          t]))) * s)
                        g = float(got[i, h, t])
                        # zero codes times an infinite scale are NaN on both sides
                        assert g == want or (math.isnan(g) and math.isnan(want)), (b, i, h, t)


def test_e4m3_clamped_pieces_loop():
    pool, scales, k, v, bi, pos, ind, indptr = _e4m3_append_case(8)
    k = k * 40.0  # many pieces past +-448 * scale
    _, _, want = _append_e4m3_loop(pool, scales.numpy(), k.numpy(), v.numpy(), bi, pos, ind,
                                   indptr)
    assert O.e4m3_clamped_pieces(k, v, scales, bi, pos, ind, indptr, pool.shape[0]) == want > 6


def test_e4m3_pins_catch_planted_mistakes():
    pool, scales, k, v, bi, pos, ind, indptr = _e4m3_append_case()
    ref, _, _ = _append_e4m3_loop(pool, scales.numpy(), k.numpy(), v.numpy(), bi, pos, ind,
                                  indptr)
    # K and V scales swapped, or the scale of the neighbouring head, change bytes
    for kw in ({"kscale_kind": 1, "vscale_kind": 0}, {"head_shift": 1}, {"head_shift": -1}):
        bad, _, _ = _append_e4m3_loop(pool, scales.numpy(), k.numpy(), v.numpy(), bi, pos, ind,
                                      indptr, **kw)
        assert not np.array_equal(bad, ref), kw
    # a gather that dequantises with the V scale for K, or head h + 1's scale
    f8 = torch.from_numpy(ref).view(torch.float8_e4m3fn)
    last = np.array([16, 16, 16], dtype=np.int32)
    k0, _ = O.gather_pages(f8, indptr, ind, last, 0, scales)
    sw = scales[:, [1, 0]].contiguous()
    k_bad, _ = O.gather_pages(f8, indptr, ind, last, 0, sw)
    assert not torch.equal(k_bad, k0)
    k_bad2, _ = O.gather_pages(f8, indptr, ind, last, 0, scales.roll(1, dims=2))
    assert not torch.equal(k_bad2, k0)


# -----------------------------------------------------------------------------
# attention

def _dense_pool(k, v):
    """Pool + tables holding dense k/v [L, H, D] in pages 1..n (page 0 unused)."""
    L, h, d = k.shape
    npg = max(1, math.ceil(L / 16))
    pool = torch.zeros(npg + 1, 2, h, 16, d, dtype=k.dtype)
    for j in range(L):
        pool[1 + j // 16, 0, :, j % 16] = k[j]
        pool[1 + j // 16, 1, :, j % 16] = v[j]
    indptr = np.array([0, npg], dtype=np.int32)
    ind = np.arange(1, npg + 1, dtype=np.int32)
    last = np.array([(L % 16) or 16], dtype=np.int32)
    return pool, indptr, ind, last


def test_attention_kv_len_one():
    q = torch.randn(1, 4, 8)
    k = torch.randn(1, 2, 8)
    v = torch.randn(1, 2, 8)
    out, lse = O.attention(q, k, v, causal=False)
    assert torch.allclose(out[0], v[0].repeat_interleave(2, 0), atol=1e-6)
    s = (q[0] * k[0].repeat_interleave(2, 0)).sum(-1) / math.sqrt(8)
    assert torch.allclose(lse[0], s, atol=1e-5)


def test_attention_equal_v_rows_and_zero_q():
    k = torch.randn(37, 2, 8)
    row = torch.randn(2, 8)
    v = row[None].repeat(37, 1, 1)
    out, _ = O.attention(torch.randn(3, 4, 8), k, v, causal=False)
    assert torch.allclose(out, row.repeat_interleave(2, 0)[None].expand(3, 4, 8), atol=1e-5)
    v2 = torch.randn(37, 2, 8)
    out0, lse0 = O.attention(torch.zeros(1, 4, 8), k, v2, causal=False)
    assert torch.allclose(out0[0], v2.mean(0).repeat_interleave(2, 0), atol=1e-5)
    assert torch.allclose(lse0, torch.full_like(lse0, math.log(37)), atol=1e-5)


def test_attention_mha_matches_sdpa():
    q = torch.randn(7, 4, 16)
    k = torch.randn(30, 4, 16)
    v = torch.randn(30, 4, 16)
    out, _ = O.attention(q, k, v, causal=False)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1)).transpose(0, 1)
    assert torch.allclose(out, ref, atol=1e-5)


def test_attention_square_causal_matches_sdpa():
    q = torch.randn(19, 2, 8)
    k = torch.randn(19, 2, 8)
    v = torch.randn(19, 2, 8)
    out, _ = O.attention(q, k, v, causal=True)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), is_causal=True).transpose(0, 1)
    assert torch.allclose(out, ref, atol=1e-5)


def test_chunked_prefill_equals_incremental_decode():
    # row i of a causal chunk of n rows over L keys equals decoding that row
    # over the first L - n + i + 1 keys (bottom-right alignment)
    q = torch.randn(5, 4, 8)
    k = torch.randn(23, 2, 8)
    v = torch.randn(23, 2, 8)
    out, lse = O.attention(q, k, v, causal=True)
    for i in range(5):
        n = 23 - 5 + i + 1
        o1, l1 = O.attention(q[i:i + 1], k[:n], v[:n], causal=False)
        assert torch.allclose(out[i], o1[0], atol=1e-5)
        assert torch.allclose(lse[i], l1[0], atol=1e-5)


def _load_golden():
    z = np.load(GOLDEN, allow_pickle=False)
    cases = {}
    for key in z.files:
        name, field = key.split("/")
        cases.setdefault(name, {})[field] = z[key]
    return cases


@pytest.mark.parametrize("name", ["decode_gqa", "prefill_causal", "prefill_full",
                                  "prefill_mha_short_kv"])
def test_attention_golden(name):
    c = _load_golden()[name]
    pool = torch.from_numpy(c["pool"])
    q = torch.from_numpy(c["q"])
    out, lse = O.prefill(q.double(), c["qo_indptr"], pool, c["kv_indptr"], c["kv_indices"],
                         c["kv_last_page_len"], causal=bool(c["causal"]))
    # oracle computes in fp32: compare at fp32 accuracy
    want_o = torch.from_numpy(c["out"])
    want_l = torch.from_numpy(c["lse"])
    assert torch.allclose(out.double(), want_o, atol=2e-6), (out.double() - want_o).abs().max()
    fin = torch.isfinite(want_l)
    assert torch.equal(torch.isfinite(lse), fin)
    assert torch.allclose(lse.double()[fin], want_l[fin], atol=2e-6)


def test_decode_golden_through_decode_entry():
    c = _load_golden()["decode_gqa"]
    pool = torch.from_numpy(c["pool"]).float()
    q = torch.from_numpy(c["q"]).float()
    out, lse = O.decode(q, pool, c["kv_indptr"], c["kv_indices"], c["kv_last_page_len"])
    assert torch.allclose(out.double(), torch.from_numpy(c["out"]), atol=2e-6)
    assert torch.allclose(lse.double(), torch.from_numpy(c["lse"]), atol=2e-6)


@pytest.mark.parametrize("chunk", [1, 7, 16, 100, 1000])
def test_merge_identity(chunk):
    q = torch.randn(1, 8, 16)
    k = torch.randn(131, 2, 16)
    v = torch.randn(131, 2, 16)
    o, l = O.attention(q, k, v, causal=False)
    parts = O.split_attention(q, k, v, chunk)
    mo, ml = O.merge_states([p[0] for p in parts], [p[1] for p in parts])
    assert torch.allclose(mo, o, atol=1e-5) and torch.allclose(ml, l, atol=1e-5)
    so, sl = O.merge_states([o], [l])
    assert torch.allclose(so, o) and torch.allclose(sl, l)


def test_paged_equals_dense():
    k = torch.randn(45, 2, 8)
    v = torch.randn(45, 2, 8)
    q = torch.randn(1, 4, 8)
    pool, indptr, ind, last = _dense_pool(k, v)
    po, pl = O.decode(q, pool, indptr, ind, last)
    do, dl = O.attention(q, k, v, causal=False)
    assert torch.allclose(po, do, atol=1e-6) and torch.allclose(pl, dl, atol=1e-6)


# -----------------------------------------------------------------------------
# RoPE

def test_rope_matches_transformers():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    n, h, d = 40, 3, 64
    theta = 500000.0
    x = torch.randn(n, h, d)
    pos = torch.randint(0, 131072, (n,))
    inv_freq = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = pos.double()[:, None] * inv_freq[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    cos, sin = emb.cos()[None], emb.sin()[None]  # [1, n, d]
    xt = x.double().transpose(0, 1)[None]  # [1, h, n, d]
    ref, _ = apply_rotary_pos_emb(xt, xt, cos, sin, unsqueeze_dim=1)
    got = O.rope(x, pos.numpy(), theta)
    assert torch.allclose(got.double(), ref[0].transpose(0, 1), atol=1e-5)


def test_rope_is_rotation():
    x = torch.randn(9, 2, 16)
    pos = np.arange(9) * 1000
    for inter in (False, True):
        y = O.rope(x, pos, 10000.0, scale=2.0, interleave=inter)
        assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), atol=1e-5)
        assert torch.allclose(y[0], x[0])  # position 0 is the identity
    # linear scaling: (pos, scale) == (pos / scale, 1)
    assert torch.allclose(O.rope(x, pos, 1e4, scale=4.0), O.rope(x, pos / 4.0, 1e4), atol=1e-6)
    # partial rotary: dims >= rotary_dim untouched
    y = O.rope(x, pos, 1e4, rotary_dim=8)
    assert torch.equal(y[..., 8:], x[..., 8:])


def _rope_interleaved_via_rotate_half(x, pos, theta, scale=1.0, rotary_dim=None):
    """Interleaved RoPE (pairs 2i, 2i+1) written as rotate-half RoPE (pairs i,
    i + rd/2) of the de-interleaved vector: gather the rotary dims in the order
    0, 2, 4, ..., 1, 3, 5, ..., rotate, and scatter them back."""
    rd = rotary_dim or x.shape[-1]
    perm = torch.cat([torch.arange(0, rd, 2), torch.arange(1, rd, 2)])
    xd = x.clone()
    xd[..., :rd] = x[..., perm]
    yd = O.rope(xd, pos, theta, scale=scale, rotary_dim=rd)
    y = yd.clone()
    y[..., perm] = yd[..., :rd]
    return y


def _rope_interleaved_negative_angle(x, pos, theta):
    """A plausible mistake: the interleaved pairs rotated by -angle (the sign
    of sin flipped)."""
    d = x.shape[-1]
    i = torch.arange(d // 2, dtype=torch.float64)
    ang = torch.as_tensor(np.asarray(pos), dtype=torch.float64)[:, None] * theta ** (-(2.0 * i) / d)
    c, s = torch.cos(ang).float()[:, None, :], torch.sin(ang).float()[:, None, :]
    a, b = x[..., 0::2].float(), x[..., 1::2].float()
    y = x.float().clone()
    y[..., 0::2] = a * c + b * s
    y[..., 1::2] = b * c - a * s
    return y


def test_rope_interleave_closed_form():
    # the rotate-half form is pinned against transformers above; the
    # interleaved form must equal it on the de-interleaved vector, for full and
    # partial rotary dims and with linear position scaling
    x = torch.randn(33, 3, 64)
    pos = np.random.default_rng(5).integers(0, 131072, 33)
    for rd, scale in ((None, 1.0), (32, 1.0), (None, 8.0)):
        got = O.rope(x, pos, 500000.0, scale=scale, rotary_dim=rd, interleave=True)
        want = _rope_interleaved_via_rotate_half(x, pos, 500000.0, scale=scale, rotary_dim=rd)
        assert torch.allclose(got, want, atol=1e-6), (rd, scale)
    # planted: a rotation by -angle keeps the norm and the position-0 identity
    # (what test_rope_is_rotation checks) but fails the closed form
    bad = _rope_interleaved_negative_angle(x, pos, 500000.0)
    assert torch.allclose(bad.norm(dim=-1), x.norm(dim=-1), atol=1e-4)
    assert not torch.allclose(bad, _rope_interleaved_via_rotate_half(x, pos, 500000.0), atol=1e-3)
    # planted: pairs (i, i + D/2) instead of (2i, 2i+1) also fails it
    wrong_pairs = O.rope(x, pos, 500000.0, interleave=False)
    assert not torch.allclose(wrong_pairs, _rope_interleaved_via_rotate_half(x, pos, 500000.0),
                              atol=1e-3)


# -----------------------------------------------------------------------------
# planted mistakes: each plausible bug in a copy of the oracle fails a pin

def _attention_top_left(q, k, v, causal):
    n, L = q.shape[0], k.shape[0]
    g = q.shape[1] // k.shape[1]
    s = torch.einsum("nhd,lhd->hnl", q, k.repeat_interleave(g, 1)) / math.sqrt(q.shape[2])
    if causal:
        s = s.masked_fill(torch.arange(L)[None, :] > torch.arange(n)[:, None], float("-inf"))
    return torch.einsum("hnl,lhd->nhd", s.softmax(-1), v.repeat_interleave(g, 1))


def _attention_wrong_gqa(q, k, v, causal):
    hq, hkv = q.shape[1], k.shape[1]
    idx = torch.arange(hq) % hkv  # h % Hkv instead of h // g
    s = torch.einsum("nhd,lhd->hnl", q, k[:, idx]) / math.sqrt(q.shape[2])
    return torch.einsum("hnl,lhd->nhd", s.softmax(-1), v[:, idx])


def test_pins_catch_planted_mistakes():
    c = _load_golden()["prefill_causal"]
    pool = torch.from_numpy(c["pool"])
    q = torch.from_numpy(c["q"])
    want = torch.from_numpy(c["out"])
    qo = c["qo_indptr"]
    k, v = O.gather_pages(pool, c["kv_indptr"], c["kv_indices"], c["kv_last_page_len"], 0,
                          dtype=torch.float64)
    rows = slice(int(qo[0]), int(qo[1]))
    bad = _attention_top_left(q[rows], k, v, True)
    assert not torch.allclose(bad, want[rows], atol=1e-3)
    c2 = _load_golden()["decode_gqa"]
    pool2 = torch.from_numpy(c2["pool"])
    k2, v2 = O.gather_pages(pool2, c2["kv_indptr"], c2["kv_indices"], c2["kv_last_page_len"], 2,
                            dtype=torch.float64)
    bad2 = _attention_wrong_gqa(torch.from_numpy(c2["q"])[2:3], k2, v2, False)
    assert not torch.allclose(bad2, torch.from_numpy(c2["out"])[2:3], atol=1e-3)
    # a merge that forgets to rescale by e^{lse_c - lse} breaks the split identity
    qq = torch.randn(1, 4, 8)
    kk, vv = torch.randn(50, 2, 8), torch.randn(50, 2, 8)
    o, _ = O.attention(qq, kk, vv, causal=False)
    parts = O.split_attention(qq, kk, vv, 16)
    naive = torch.stack([p[0] for p in parts]).mean(0)
    assert not torch.allclose(naive, o, atol=1e-3)
