"""Pins of the oracle's KV write path: the power-of-two scale rule, the e4m3
running-amax append and the copy-on-write page fork.  Each pin is an
independent computation (a brute-force search, a pure-Python loop, a
one-shot versus incremental identity) chosen so that a plausible mistake in
the oracle fails it; the planted-mistake test at the end shows that."""

import numpy as np
import pytest
import torch

import oracle as O

PAGE = O.PAGE


# -----------------------------------------------------------------------------
# pow2_scale

def _pow2_brute(a: float) -> float:
    if a <= 0:
        return 0.0
    for k in range(-126, 130):
        if 448.0 * 2.0 ** k >= a:  # exact in float64
            return 2.0 ** k
    raise AssertionError(a)


def test_pow2_scale_brute():
    rng = np.random.default_rng(0)
    vals = [0.0, 448.0, 224.0, 1.0, 3.5, 7.0, 1e-30, 1e-40, 3.0e38]
    for k in range(-20, 20):
        b = np.float32(448.0 * 2.0 ** k)
        vals += [float(b), float(np.nextafter(b, np.float32(np.inf))),
                 float(np.nextafter(b, np.float32(0)))]
    vals += list((rng.standard_normal(200) * 10.0 ** rng.integers(-6, 6, 200)).astype(
        np.float32).__abs__())
    a = np.asarray(vals, dtype=np.float32)
    got = O.pow2_scale(a)
    want = np.asarray([_pow2_brute(float(x)) for x in a], dtype=np.float64)
    # below 448 * 2^-126 the rule clamps to 2^-126
    want = np.where((a > 0) & (want < 2.0 ** -126), 2.0 ** -126, want)
    np.testing.assert_array_equal(got.astype(np.float64), want)


# -----------------------------------------------------------------------------
# running-amax append

def _pool(num_pages, hkv, d, fill=0x5A):
    return np.full((num_pages, 2, hkv, PAGE, d), fill, dtype=np.uint8)


def _seq_meta(tables):
    indptr = np.concatenate([[0], np.cumsum([len(t) for t in tables])]).astype(np.int32)
    return np.concatenate(tables).astype(np.int32), indptr


def _append_calls(pool, scales, rows_k, rows_v, tables, chunks, fn):
    """Append the rows of each sequence in the given per-call chunk sizes
    (chunks[c][b] tokens of sequence b in call c), in calls of all sequences."""
    ind, indptr = _seq_meta(tables)
    done = [0] * len(tables)
    for sizes in chunks:
        bi, pos, ks, vs = [], [], [], []
        for b, n in enumerate(sizes):
            for i in range(n):
                bi.append(b)
                pos.append(done[b] + i)
                ks.append(rows_k[b][done[b] + i])
                vs.append(rows_v[b][done[b] + i])
            done[b] += n
        if not bi:
            continue
        pool, scales, skipped = fn(pool, scales, torch.stack(ks), torch.stack(vs), bi, pos, ind,
                                   indptr)
        assert skipped == 0
    return pool, scales


def _normal_rows(rng, n, hkv, d):
    """Values with |x| in [0.25, 4): every e4m3 code they get stays normal
    under any scale the running rule can reach for them."""
    mag = rng.uniform(0.25, 4.0, size=(n, hkv, d))
    sign = rng.choice([-1.0, 1.0], size=(n, hkv, d))
    return torch.from_numpy(mag * sign).to(torch.bfloat16)


def test_running_append_one_shot_equals_incremental():
    rng = np.random.default_rng(1)
    hkv, d = 2, 16
    tables = [[3, 0], [1, 4]]
    n_tok = [27, 20]
    ks = [_normal_rows(rng, n, hkv, d) for n in n_tok]
    vs = [_normal_rows(rng, n, hkv, d) for n in n_tok]
    # make later rows larger so that scales grow mid-page
    for b in range(2):
        ks[b][5:] *= 2
        vs[b][11:] *= 4
    fn = O.append_pages_e4m3_running
    s0 = torch.zeros(5, 2, hkv)
    one, s_one = _append_calls(_pool(5, hkv, d), s0, ks, vs, tables, [n_tok], fn)
    inc, s_inc = _append_calls(_pool(5, hkv, d), s0, ks, vs, tables,
                               [[1, 1]] * 20 + [[1, 0]] * 7, fn)
    mixed, s_mix = _append_calls(_pool(5, hkv, d), s0, ks, vs, tables,
                                 [[5, 3], [9, 9], [13, 8]], fn)
    for pool, sc in ((inc, s_inc), (mixed, s_mix)):
        assert torch.equal(sc, s_one)
        np.testing.assert_array_equal(pool[[0, 1, 3, 4]][:, :, :, :], one[[0, 1, 3, 4]])
    # page 0 holds rows 16..26 of sequence 0, page 4 rows 16..19 of sequence 1:
    # slots past them were never written
    assert (one[0, :, :, 11:] == 0x5A).all() and (one[4, :, :, 4:] == 0x5A).all()


def test_running_append_fresh_page_equals_direct():
    rng = np.random.default_rng(2)
    hkv, d = 3, 32
    k = torch.from_numpy(rng.standard_normal((16, hkv, d)) * 3).to(torch.bfloat16)
    v = torch.from_numpy(rng.standard_normal((16, hkv, d)) * 0.01).to(torch.bfloat16)
    pool, sc, _ = O.append_pages_e4m3_running(_pool(2, hkv, d), torch.full((2, 2, hkv), 9.0),
                                              k, v, [0] * 16, list(range(16)), [1], [0, 1])
    for kind, x in ((0, k), (1, v)):
        for h in range(hkv):
            blk = x[:, h].float()
            s = _pow2_brute(float(blk.abs().max()))
            assert sc[1, kind, h].item() == s
            want = (blk / s).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            np.testing.assert_array_equal(pool[1, kind, h], want)
    assert (pool[0] == 0x5A).all() and (sc[0] == 9.0).all()


def test_running_amax_scale_bounds():
    rng = np.random.default_rng(3)
    hkv, d = 2, 16
    tables = [[0, 1, 2]]
    x = torch.from_numpy(rng.standard_normal((40, hkv, d)) * np.exp(
        rng.uniform(-3, 3, size=(40, 1, 1)))).to(torch.bfloat16)
    pool, sc = _append_calls(_pool(3, hkv, d), torch.zeros(3, 2, hkv), [x], [x * 0.5], tables,
                             [[7], [1], [9], [3], [12], [8]], O.append_pages_e4m3_running)
    for p in range(3):
        rows = x[16 * p:16 * p + 16]
        n = rows.shape[0]
        for kind, src in ((0, rows), (1, rows * 0.5)):
            for h in range(hkv):
                s = sc[p, kind, h].item()
                amax = src[:, h].float().abs().max().item()
                assert s == _pow2_brute(amax), (p, kind, h)
                dec = O.e4m3_decode(pool[p, kind, h, :n], s)
                err = (dec - src[:, h].float()).abs()
                # e4m3: 3 mantissa bits (half-ulp 2^-4 relative) + subnormal
                # step 2^-9 * s, plus one extra rounding for re-encoded rows
                bound = 2 * (src[:, h].float().abs() * 2.0 ** -4 + s * 2.0 ** -9)
                assert bool((err <= bound).all()), (p, kind, h, float((err - bound).max()))


def test_running_append_skips_bad_metadata():
    hkv, d = 1, 16
    k = torch.ones(4, hkv, d, dtype=torch.bfloat16)
    pool, sc, skipped = O.append_pages_e4m3_running(
        _pool(2, hkv, d), torch.zeros(2, 2, hkv), k, k, [0, 0, 5, 0], [0, 1, 0, 40], [1],
        [0, 1])
    assert skipped == 2
    assert sc[1, 0, 0].item() == 2.0 ** -8  # 448 * 2^-9 < 1 <= 448 * 2^-8
    code_256 = torch.tensor([256.0]).to(torch.float8_e4m3fn).view(torch.uint8).item()
    assert (pool[1, :, :, :2] == code_256).all() and (pool[1, :, :, 2:] == 0x5A).all()


# -----------------------------------------------------------------------------
# fork

def _fork_loop(pool, src, dst, valid, scales):
    out = pool.copy()
    sc = scales.clone() if scales is not None else None
    L, P, _, H, _, D = pool.shape
    skipped = 0
    for f in range(len(src)):
        s, d, n = src[f], dst[f], (valid[f] if valid is not None else PAGE)
        if not (0 <= s < P and 0 <= d < P and 0 <= n <= PAGE):
            skipped += 1
            continue
        for l in range(L):
            for kind in range(2):
                for h in range(H):
                    for r in range(n):
                        for e in range(D):
                            out[l, d, kind, h, r, e] = pool[l, s, kind, h, r, e]
                    if sc is not None:
                        sc[l, d, kind, h] = scales[l, s, kind, h]
    return out, sc, skipped


def test_fork_pages_loop():
    rng = np.random.default_rng(4)
    pool = rng.integers(0, 256, size=(3, 6, 2, 2, PAGE, 8), dtype=np.uint8)
    scales = torch.from_numpy(rng.random((3, 6, 2, 2)).astype(np.float32))
    src, dst, valid = [0, 2, 9, 1], [3, 5, 4, 4], [7, 16, 3, 17]
    got = O.fork_pages(pool, src, dst, valid, scales)
    want = _fork_loop(pool, src, dst, valid, scales)
    np.testing.assert_array_equal(got[0], want[0])
    assert torch.equal(got[1], want[1]) and got[2] == want[2] == 2


def test_fork_then_gather():
    rng = np.random.default_rng(5)
    pool = torch.from_numpy(rng.standard_normal((2, 5, 2, 2, PAGE, 8))).to(torch.bfloat16)
    bits = O.to_bits(pool)
    out, _, _ = O.fork_pages(bits, [1], [4], [9])
    forked = O.from_bits(out, torch.bfloat16)
    for l in range(2):
        k0, v0 = O.gather_pages(pool[l], [0, 1], [1], [9], 0)
        k1, v1 = O.gather_pages(forked[l], [0, 1], [4], [9], 0)
        assert torch.equal(k0, k1) and torch.equal(v0, v1)
    assert torch.equal(forked[:, :4], pool[:, :4])
    assert torch.equal(forked[:, 4, :, :, 9:], pool[:, 4, :, :, 9:])


# -----------------------------------------------------------------------------
# planted mistakes: each must fail a pin above

def _running_without_requant(pool_bits, scales, k, v, bi, pos, ind, indptr):
    """Planted mistake: the scale grows but the rows already in the page keep
    their old codes."""
    out, sc, skipped = O.append_pages_e4m3_running(pool_bits, scales, k, v, bi, pos, ind, indptr)
    ok, page_id, slot = O.paged_ref._append_targets(bi, pos, ind, indptr, pool_bits.shape[0])
    for t in range(len(bi)):
        if ok[t]:
            out[page_id[t], :, :, :slot[t]] = pool_bits[page_id[t], :, :, :slot[t]]
    return out, sc, skipped


def test_pins_catch_planted_kvwrite_mistakes():
    rng = np.random.default_rng(1)
    hkv, d = 1, 16
    ks = [_normal_rows(rng, 16, hkv, d)]
    ks[0][8:] *= 8
    s0 = torch.zeros(1, 2, hkv)
    one, _ = _append_calls(_pool(1, hkv, d), s0, ks, ks, [[0]], [[16]],
                           _running_without_requant)
    inc, _ = _append_calls(_pool(1, hkv, d), s0, ks, ks, [[0]], [[1]] * 16,
                           _running_without_requant)
    assert not np.array_equal(one, inc)
