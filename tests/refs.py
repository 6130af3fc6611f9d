"""Independent numpy references used to pin the oracle and to check the GPU
path: float64 closed forms and exact integer arithmetic. They follow the
documented semantics, not the oracle's code, so a dropped term, a wrong
index or a transposed operand in either shows up as a mismatch."""

import math

import numpy as np


def ref_decode(q, k, v, lens=None):
    """float64 softmax(q k^T / sqrt(D)) v per (b, h) with kv head h // G
    (reference tests/test_attention.py:26-45 conventions)."""
    b, hq, d = q.shape
    _, hkv, t, _ = k.shape
    group = hq // hkv
    out = np.zeros((b, hq, d), dtype=np.float64)
    for bi in range(b):
        length = t if lens is None else int(lens[bi])
        if length == 0:
            continue
        for h in range(hq):
            kv = h // group
            s = k[bi, kv, :length].astype(np.float64) @ q[bi, h].astype(np.float64)
            s /= math.sqrt(d)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[bi, h] = p @ v[bi, kv, :length].astype(np.float64)
    return out


def materialize_paged(k_pool, table, width=None):
    """[Nb,Hkv,P,D] pool + [B,S] table -> contiguous [B,Hkv,S*P,D] cache."""
    nb, hkv, page, d = k_pool.shape
    b, s = table.shape
    width = s if width is None else width
    out = np.zeros((b, hkv, width * page, d), dtype=k_pool.dtype)
    for bi in range(b):
        for j in range(width):
            out[bi, :, j * page:(j + 1) * page] = k_pool[table[bi, j]]
    return out


def ref_decode_paged(q, k_pool, v_pool, table, lens=None):
    kc = materialize_paged(k_pool, table)
    vc = materialize_paged(v_pool, table)
    return ref_decode(q, kc, vc, lens)


def ref_qgemm_i32(a, b):
    return a.astype(np.int64) @ b.astype(np.int64).T


def ref_qgemm(a, sa, b, sb):
    """exact int accumulation, f32(sa*sb) scale, one f32 product
    (reference tests/test_qgemm.py:21-23)."""
    acc = ref_qgemm_i32(a, b)
    assert np.abs(acc).max(initial=0) < 2**31
    return acc.astype(np.int32).astype(np.float32) * (np.float32(sa) * np.float32(sb))


def ref_qgemm_pc(a, sa, b, sb):
    """per-channel: f32(sa * sb[j]) then one product
    (reference tests/test_qgemm_perchannel.py:25-30)."""
    acc = ref_qgemm_i32(a, b)
    scales = np.float32(sa) * np.asarray(sb, dtype=np.float32)
    return acc.astype(np.int32).astype(np.float32) * scales


def ref_prefill(q, k, v, causal=True, rows=None):
    """float64 prefill attention (reference tests/test_attention.py:155-173
    conventions): query row i of [B,Hq,S,D] attends to key rows [0, i]
    (causal) or all S rows, kv head h // G. rows: optional subset of query
    rows (the others stay 0)."""
    b, hq, s, d = q.shape
    hkv = k.shape[1]
    group = hq // hkv
    out = np.zeros((b, hq, s, d), dtype=np.float64)
    rows = range(s) if rows is None else rows
    for bi in range(b):
        for h in range(hq):
            kv = h // group
            kd = k[bi, kv].astype(np.float64)
            vd = v[bi, kv].astype(np.float64)
            for i in rows:
                lim = i + 1 if causal else s
                sc = kd[:lim] @ q[bi, h, i].astype(np.float64) / math.sqrt(d)
                p = np.exp(sc - sc.max())
                p /= p.sum()
                out[bi, h, i] = p @ vd[:lim]
    return out


def ref_quantize(x):
    """float32 closed form of the symmetric quantizer, with numpy rounding
    (np.rint: half to even)."""
    x = np.asarray(x, dtype=np.float32)
    m = np.float32(np.abs(x).max(initial=0.0))
    scale = np.float32(m / np.float32(127.0)) if m > 0 else np.float32(1.0)
    inv = np.float32(np.float32(1.0) / scale)
    q = np.clip(np.rint(x * inv), -127, 127).astype(np.int8)
    return q, float(scale)


def ref_rmsnorm(x, w, eps, residual=None):
    v = x.astype(np.float64) if residual is None else x.astype(np.float64) + residual
    inv = 1.0 / np.sqrt((v ** 2).mean(axis=-1, keepdims=True) + eps)
    return v * inv * w


def ref_rope(x, theta, pos_offset, neox, positions=None):
    seq, dim = x.shape
    y = np.zeros((seq, dim), dtype=np.float64)
    xd = x.astype(np.float64)
    for r in range(seq):
        pos = (r if positions is None else positions[r]) + pos_offset
        for j in range(dim // 2):
            a = pos * theta ** (-2.0 * j / dim)
            c, s = math.cos(a), math.sin(a)
            i1, i2 = (j, j + dim // 2) if neox else (2 * j, 2 * j + 1)
            y[r, i1] = xd[r, i1] * c - xd[r, i2] * s
            y[r, i2] = xd[r, i1] * s + xd[r, i2] * c
    return y


def ref_swiglu(g, u):
    g = g.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


def bf16_round(a):
    """Round float32 values to bfloat16 (nearest-even) and back to float32."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(
        torch.bfloat16).float().numpy()


def f16_round(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def splitmix_uniform(seed):
    """splitmix64 finalised to a float32 in [0, 1), in Python integers
    (reference cuda_util.cuh:69-76)."""
    mask = (1 << 64) - 1
    z = (seed + 0x9E3779B97F4A7C15) & mask
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
    z ^= z >> 31
    return float(np.float32((z >> 11) * (1.0 / 9007199254740992.0)))


def ref_topp(logits, p, t=1.0, seed=0):
    """float64 nucleus sampling with the reference's order and cut rule:
    returns (token, margin), margin = the smallest distance (relative to the
    total mass) between the cut or draw threshold and a prefix boundary -
    a small margin means float rounding may legitimately move the token."""
    inv_t = np.float32(1.0) / np.float32(t)
    v = (np.asarray(logits, np.float32) * inv_t).astype(np.float32)
    idx = np.arange(v.size)
    order = np.lexsort((idx, -v.astype(np.float64)))
    m = np.exp(v[order].astype(np.float64) - float(v[order[0]]))
    cum = np.cumsum(m)
    total = cum[-1]
    thr = p * total
    k = int(np.searchsorted(cum, thr, side="left"))
    k = min(k, v.size - 1)
    nucleus = cum[k]
    margin = min(abs(cum[k] - thr), abs(thr - (cum[k - 1] if k else 0.0))) / total
    target = splitmix_uniform(seed) * nucleus
    j = int(np.searchsorted(cum[:k + 1], target, side="left"))
    j = min(j, k)
    margin = min(margin, abs(cum[j] - target) / total,
                 abs(target - (cum[j - 1] if j else 0.0)) / total)
    return int(order[j]), margin
