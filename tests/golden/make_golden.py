"""Writes tests/golden/golden.npz: tiny known-answer cases for the oracle.

The reference ships no golden vectors (its tests draw CUDA randn on the fly),
so these fixtures are computed here by brute-force enumeration in float64
plain Python, independently of oracle/attention_ref.py:
  * every (query, key) pair is visited explicitly; visibility is decided per
    pair by the conditions of the reference kernels
    (dense causal j <= i + Sk - Sq: tests/test_compare_ref.py:22,
     _kernels_forward.py:135-144; paged: _kernels_paged.py:274-308;
     decode: _kernels_paged.py:450-451);
  * page resolution walks the block table slot by slot
    (_kernels_paged.py:265-272);
  * gradients are central finite differences of the brute-force forward.
Run: python tests/golden/make_golden.py   (deterministic; numpy only)
"""
from __future__ import annotations

import math
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def softmax_row(scores):
    """scores: list of visible logits (already scaled); returns (weights, lse)."""
    if not scores:
        return [], -math.inf
    m = max(scores)
    e = [math.exp(s - m) for s in scores]
    tot = sum(e)
    return [x / tot for x in e], m + math.log(tot)


def brute_dense(q, k, v, scale, causal):
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    g = H // Hk
    out = np.zeros((B, Sq, H, D))
    lse = np.full((B, H, Sq), -np.inf)
    for b in range(B):
        for h in range(H):
            hk = h // g
            for i in range(Sq):
                keys = [j for j in range(Sk) if (not causal) or j <= i + Sk - Sq]
                sc = [scale * sum(q[b, i, h, d] * k[b, j, hk, d] for d in range(D)) for j in keys]
                w, l = softmax_row(sc)
                lse[b, h, i] = l
                for wj, j in zip(w, keys):
                    for d in range(D):
                        out[b, i, h, d] += wj * v[b, j, hk, d]
    return out, lse


def fd_grads(q, k, v, dout, scale, causal, eps=1e-6):
    def loss(qq, kk, vv):
        o, _ = brute_dense(qq, kk, vv, scale, causal)
        return float((o * dout).sum())

    grads = []
    for idx, t in enumerate((q, k, v)):
        g = np.zeros_like(t)
        it = np.nditer(t, flags=["multi_index"])
        for _ in it:
            mi = it.multi_index
            args_p = [q.copy(), k.copy(), v.copy()]
            args_m = [q.copy(), k.copy(), v.copy()]
            args_p[idx][mi] += eps
            args_m[idx][mi] -= eps
            g[mi] = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        grads.append(g)
    return grads


def resolve(cache, bt_row, pos, page):
    lp = pos // page
    slot = pos - lp * page
    return cache[bt_row[lp], slot]


def brute_paged(q, kc, vc, bt, seq_lens, qsl, pkl, scale, causal, wq, wk):
    T, Hq, D = q.shape
    page, Hkv = kc.shape[1], kc.shape[2]
    g = Hq // Hkv
    out = np.zeros((T, Hq, D))
    lse = np.full((Hq, T), -np.inf)
    for b in range(bt.shape[0]):
        for t in range(qsl[b + 1] - qsl[b]):
            row = qsl[b] + t
            for h in range(Hq):
                hk = h // g
                keys = []
                for n in range(seq_lens[b]):
                    ok = True
                    if causal:
                        ok = n <= pkl[b] + t
                        if ok and wq > 0:
                            ok = t < n + wq
                        if ok and wk > 0:
                            ok = n < t + wk
                    if ok:
                        keys.append(n)
                sc = [scale * sum(q[row, h, d] * resolve(kc, bt[b], n, page)[hk, d]
                                  for d in range(D)) for n in keys]
                w, l = softmax_row(sc)
                lse[h, row] = l
                for wj, n in zip(w, keys):
                    out[row, h] += wj * resolve(vc, bt[b], n, page)[hk]
    return out, lse


def main():
    rng = np.random.default_rng(20260101)
    data = {}

    cases = {
        "dense_nc": dict(B=1, Sq=5, Sk=7, H=2, Hk=1, D=4, causal=False, scale=0.37),
        "dense_c_skgt": dict(B=2, Sq=4, Sk=6, H=2, Hk=2, D=4, causal=True, scale=0.5),
        "dense_c_sqgt": dict(B=1, Sq=6, Sk=3, H=1, Hk=1, D=4, causal=True, scale=0.5),
    }
    for name, c in cases.items():
        q = rng.standard_normal((c["B"], c["Sq"], c["H"], c["D"]))
        k = rng.standard_normal((c["B"], c["Sk"], c["Hk"], c["D"]))
        v = rng.standard_normal((c["B"], c["Sk"], c["Hk"], c["D"]))
        o, l = brute_dense(q, k, v, c["scale"], c["causal"])
        data.update({f"{name}/q": q, f"{name}/k": k, f"{name}/v": v, f"{name}/out": o,
                     f"{name}/lse": l, f"{name}/scale": np.float64(c["scale"]),
                     f"{name}/causal": np.int32(c["causal"])})

    # backward: causal, GQA, Sk > Sq
    q = rng.standard_normal((1, 4, 2, 3))
    k = rng.standard_normal((1, 5, 1, 3))
    v = rng.standard_normal((1, 5, 1, 3))
    dout = rng.standard_normal((1, 4, 2, 3))
    dq, dk, dv = fd_grads(q, k, v, dout, 0.6, True)
    data.update({"bwd/q": q, "bwd/k": k, "bwd/v": v, "bwd/dout": dout, "bwd/dq": dq,
                 "bwd/dk": dk, "bwd/dv": dv, "bwd/scale": np.float64(0.6),
                 "bwd/causal": np.int32(1)})

    # paged: 2 sequences, page 4, scattered pool of 6 pages, padding -1
    page, Hq, Hkv, D = 4, 4, 2, 4
    q_lens, seq_lens, prefix = [3, 5], [7, 5], [4, 0]
    pool = 6
    perm = rng.permutation(pool)
    bt = np.full((2, 3), -1, dtype=np.int32)
    bt[0, :2] = perm[:2]
    bt[1, :2] = perm[2:4]
    kc = rng.standard_normal((pool, page, Hkv, D))
    vc = rng.standard_normal((pool, page, Hkv, D))
    qsl = np.array([0, 3, 8], dtype=np.int32)
    q = rng.standard_normal((8, Hq, D))
    for tag, causal, wq, wk in (("c", True, -1, -1), ("nc", False, -1, -1), ("win", True, 3, 2)):
        o, l = brute_paged(q, kc, vc, bt, seq_lens, qsl, prefix, 0.45, causal, wq, wk)
        data.update({f"paged_{tag}/out": o, f"paged_{tag}/lse": l,
                     f"paged_{tag}/causal": np.int32(causal), f"paged_{tag}/wq": np.int32(wq),
                     f"paged_{tag}/wk": np.int32(wk)})
    data.update({"paged/q": q, "paged/k_cache": kc, "paged/v_cache": vc, "paged/block_table": bt,
                 "paged/seq_lens": np.array(seq_lens, dtype=np.int32),
                 "paged/query_start_loc": qsl,
                 "paged/prefix_kv_lens": np.array(prefix, dtype=np.int32),
                 "paged/scale": np.float64(0.45)})

    # decode: 3 sequences, MQA (Hkv = 1), page 4
    seq_lens = [1, 6, 9]
    pool = 7
    perm = rng.permutation(pool)
    bt = np.full((3, 3), -1, dtype=np.int32)
    bt[0, :1] = perm[:1]
    bt[1, :2] = perm[1:3]
    bt[2, :3] = perm[3:6]
    kc = rng.standard_normal((pool, 4, 1, 4))
    vc = rng.standard_normal((pool, 4, 1, 4))
    qd = rng.standard_normal((3, 4, 4))
    o = np.zeros((3, 4, 4))
    l = np.full((3, 4), -np.inf)
    for b in range(3):
        qsl_b = np.array([0, 1], dtype=np.int32)
        ob, lb = brute_paged(qd[b:b + 1], kc, vc, bt[b:b + 1], [seq_lens[b]], qsl_b, [0], 0.5,
                             False, -1, -1)
        o[b], l[b] = ob[0], lb[:, 0]
    data.update({"decode/q": qd, "decode/k_cache": kc, "decode/v_cache": vc,
                 "decode/block_table": bt, "decode/seq_lens": np.array(seq_lens, dtype=np.int32),
                 "decode/scale": np.float64(0.5), "decode/out": o, "decode/lse": l})

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({len(data)} arrays)")


if __name__ == "__main__":
    main()
