"""Writes tests/golden/attention_small.npz: paged attention known answers
computed by brute force in pure-Python float64 loops (no torch, no numpy
linear algebra), independent of the oracle in oracle/paged_ref.py.

Each case is a tiny HND pool [P, 2, Hkv, 16, D], block tables, ragged query
rows and the expected outputs / log-sum-exp per (row, head).  The mask is
the bottom-right causal mask of src/models/llama.py:218-222 (row i of a
sequence with qo rows and kv keys sees key j iff j <= kv - qo + i).

Run:  python tests/golden/make_golden.py
"""

import math
import os
import random

import numpy as np

PAGE = 16


def brute_case(rng, hq, hkv, d, qo_lens, kv_lens, causal, num_pages):
    g = hq // hkv
    pool = [[[[[rng.gauss(0.0, 1.0) for _ in range(d)] for _ in range(PAGE)]
              for _ in range(hkv)] for _ in range(2)] for _ in range(num_pages)]
    perm = list(range(num_pages))
    rng.shuffle(perm)
    tables, at = [], 0
    for n in kv_lens:
        k = (n + PAGE - 1) // PAGE
        tables.append(perm[at:at + k])
        at += k
    assert at <= num_pages
    nrows = sum(qo_lens)
    q = [[[rng.gauss(0.0, 1.0) for _ in range(d)] for _ in range(hq)] for _ in range(nrows)]
    out = [[[0.0] * d for _ in range(hq)] for _ in range(nrows)]
    lse = [[0.0] * hq for _ in range(nrows)]
    scale = 1.0 / math.sqrt(d)
    row0 = 0
    for b, (nq, nk) in enumerate(zip(qo_lens, kv_lens)):
        for i in range(nq):
            for h in range(hq):
                kh = h // g
                s = []
                for j in range(nk):
                    if causal and j > nk - nq + i:
                        continue
                    page = tables[b][j // PAGE]
                    krow = pool[page][0][kh][j % PAGE]
                    s.append((j, scale * sum(q[row0 + i][h][t] * krow[t] for t in range(d))))
                if not s:
                    lse[row0 + i][h] = -math.inf
                    continue
                m = max(v for _, v in s)
                den = sum(math.exp(v - m) for _, v in s)
                lse[row0 + i][h] = m + math.log(den)
                o = [0.0] * d
                for j, v in s:
                    page = tables[b][j // PAGE]
                    vrow = pool[page][1][kh][j % PAGE]
                    w = math.exp(v - m) / den
                    for t in range(d):
                        o[t] += w * vrow[t]
                out[row0 + i][h] = o
        row0 += nq
    indptr = [0]
    flat = []
    for t in tables:
        flat.extend(t)
        indptr.append(len(flat))
    last = [(n % PAGE) or PAGE if n > 0 else 1 for n in kv_lens]
    qo_indptr = [0]
    for n in qo_lens:
        qo_indptr.append(qo_indptr[-1] + n)
    return {
        "pool": np.array(pool, dtype=np.float64),
        "q": np.array(q, dtype=np.float64),
        "kv_indptr": np.array(indptr, dtype=np.int32),
        "kv_indices": np.array(flat, dtype=np.int32),
        "kv_last_page_len": np.array(last, dtype=np.int32),
        "qo_indptr": np.array(qo_indptr, dtype=np.int32),
        "causal": np.array(int(causal)),
        "out": np.array(out, dtype=np.float64),
        "lse": np.array(lse, dtype=np.float64),
    }


CASES = {
    # decode: one row per sequence, GQA 2:1, partial and exactly-full pages
    "decode_gqa": dict(hq=4, hkv=2, d=8, qo_lens=[1, 1, 1, 1], kv_lens=[1, 16, 23, 40],
                       causal=False, num_pages=8),
    # chunked prefill after a cached prefix, GQA 4:1, bottom-right causal
    "prefill_causal": dict(hq=4, hkv=1, d=8, qo_lens=[3, 5, 1], kv_lens=[20, 5, 17],
                           causal=True, num_pages=6),
    # same shapes without the mask
    "prefill_full": dict(hq=4, hkv=1, d=8, qo_lens=[3, 5, 1], kv_lens=[20, 5, 17],
                         causal=False, num_pages=6),
    # MHA, a query chunk longer than its kv (leading rows see nothing)
    "prefill_mha_short_kv": dict(hq=2, hkv=2, d=4, qo_lens=[6], kv_lens=[4], causal=True,
                                 num_pages=1),
}


def main():
    rng = random.Random(20261201)
    arrays = {}
    for name, cfg in CASES.items():
        for k, v in brute_case(rng, **cfg).items():
            arrays[f"{name}/{k}"] = v
        arrays[f"{name}/heads"] = np.array([cfg["hq"], cfg["hkv"], cfg["d"]], dtype=np.int32)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attention_small.npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path, len(arrays), "arrays")


if __name__ == "__main__":
    main()
