"""TEST INFRASTRUCTURE - NOT PART OF THE PRODUCT.

CPU oracle for the decode hot path: ctypes bindings to ``oracle.cpp``, a
plain C++ restatement of the reference's single-threaded ``*_cpu``
functions (fusedtok 2.5.0; citations in oracle.cpp). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may use
it, as the checker or as the timed CPU baseline; ``fusedtok_amd`` never
imports it.

Every function takes and returns numpy arrays (float32 / int8 / int32,
C-contiguous) and raises ValueError on the reference's invalid-argument
paths.

Parity pinning: every function here is checked in ``tests/test_oracle.py``
against the reference tests' known-answer cases and against independent
float64 / integer numpy references (closed forms, brute force); see the
docstrings there. No function is left unpinned.
"""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build():
    """Compile the oracle with its Makefile (g++; seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.or_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _call(fn, *args):
    lib = _load()
    st = getattr(lib, fn)(*args)
    if st != 0:
        raise ValueError(lib.or_last_error().decode())


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


def attention_decode(q, k, v, lens=None):
    """attention_decode_cpu: q [B,Hq,D], k/v [B,Hkv,T,D] -> [B,Hq,D] f32."""
    q, k, v, lens = _f32(q), _f32(k), _f32(v), _i32(lens)
    b, hq, d = q.shape
    _, hkv, t, _ = k.shape
    out = np.zeros((b, hq, d), np.float32)
    _call("or_attention_decode", _p(q), _p(k), _p(v), _p(lens), _p(out),
          b, hq, hkv, t, d)
    return out


def attention_prefill(q, k, v, causal=True):
    """attention_prefill_cpu: q [B,Hq,S,D], k/v [B,Hkv,S,D] -> [B,Hq,S,D] f32."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, hq, s, d = q.shape
    hkv = k.shape[1]
    out = np.zeros((b, hq, s, d), np.float32)
    _call("or_attention_prefill", _p(q), _p(k), _p(v), _p(out), b, hq, hkv, s, d,
          1 if causal else 0)
    return out


def attention_decode_paged(q, k_pool, v_pool, table, lens=None):
    """attention_decode_paged_cpu: pools [Nb,Hkv,P,D], table [B,S]."""
    q, k_pool, v_pool = _f32(q), _f32(k_pool), _f32(v_pool)
    table, lens = _i32(table), _i32(lens)
    b, hq, d = q.shape
    nb, hkv, page, _ = k_pool.shape
    out = np.zeros((b, hq, d), np.float32)
    _call("or_attention_decode_paged", _p(q), _p(k_pool), _p(v_pool),
          _p(table), _p(lens), _p(out), b, hq, hkv, page, table.shape[1], nb, d)
    return out


def kv_append_paged(k_pool, v_pool, table, k_new, v_new, lens):
    """kv_append_paged_cpu, in place on (copies of nothing: the pools given).
    Any element type (byte-exact copies)."""
    assert k_pool.flags["C_CONTIGUOUS"] and v_pool.flags["C_CONTIGUOUS"]
    k_new = np.ascontiguousarray(k_new, dtype=k_pool.dtype)
    v_new = np.ascontiguousarray(v_new, dtype=k_pool.dtype)
    table, lens = _i32(table), _i32(lens)
    nb, hkv, page, d = k_pool.shape
    b = k_new.shape[0]
    _call("or_kv_append_paged", _p(k_new), _p(v_new), _p(table), _p(lens),
          _p(k_pool), _p(v_pool), b, hkv, d, page, table.shape[1], nb,
          k_pool.itemsize)


def kv_append(k_cache, v_cache, k_new, v_new, lens):
    """kv_append_cpu, in place."""
    assert k_cache.flags["C_CONTIGUOUS"] and v_cache.flags["C_CONTIGUOUS"]
    k_new = np.ascontiguousarray(k_new, dtype=k_cache.dtype)
    v_new = np.ascontiguousarray(v_new, dtype=k_cache.dtype)
    lens = _i32(lens)
    b, hkv, t, d = k_cache.shape
    _call("or_kv_append", _p(k_new), _p(v_new), _p(lens), _p(k_cache),
          _p(v_cache), b, hkv, d, t, k_cache.itemsize)


def quantize_int8(x):
    """quantize_int8_cpu -> (q int8, scale float)."""
    x = _f32(x)
    q = np.empty(x.shape, np.int8)
    s = ctypes.c_float(0.0)
    _call("or_quantize_int8", _p(x), ctypes.c_longlong(x.size), _p(q),
          ctypes.byref(s))
    return q, float(s.value)


def dequantize_int8(q, scale):
    """dequantize_int8_cpu -> float32 q * scale."""
    q = np.ascontiguousarray(q, np.int8)
    x = np.empty(q.shape, np.float32)
    _call("or_dequantize_int8", _p(q), ctypes.c_longlong(q.size),
          ctypes.c_float(scale), _p(x))
    return x


def qadd_int8(qa, sa, qb, sb):
    """quantize_int8(f32(qa*sa) + f32(qb*sb)) -> (q int8, scale float)."""
    qa = np.ascontiguousarray(qa, np.int8)
    qb = np.ascontiguousarray(qb, np.int8)
    assert qa.shape == qb.shape
    q = np.empty(qa.shape, np.int8)
    s = ctypes.c_float(0.0)
    _call("or_qadd_int8", _p(qa), _p(qb), ctypes.c_longlong(qa.size),
          ctypes.c_float(sa), ctypes.c_float(sb), _p(q), ctypes.byref(s))
    return q, float(s.value)


def qgemm_i32(a, b):
    """Exact int32 accumulators A_q . B_q^T."""
    a = np.ascontiguousarray(a, np.int8)
    b = np.ascontiguousarray(b, np.int8)
    m, k = a.shape
    n = b.shape[0]
    acc = np.zeros((m, n), np.int32)
    _call("or_qgemm_i32", _p(a), _p(b), m, n, k, _p(acc))
    return acc


def qgemm(a, sa, b, sb):
    """qgemm_cpu: float(acc) * f32(sa * sb)."""
    a = np.ascontiguousarray(a, np.int8)
    b = np.ascontiguousarray(b, np.int8)
    m, k = a.shape
    n = b.shape[0]
    y = np.zeros((m, n), np.float32)
    _call("or_qgemm", _p(a), _p(b), m, n, k, ctypes.c_float(sa),
          ctypes.c_float(sb), _p(y))
    return y


def qgemm_perchannel(a, sa, b, sb):
    """qgemm_perchannel_cpu: float(acc) * f32(sa * sb[j])."""
    a = np.ascontiguousarray(a, np.int8)
    b = np.ascontiguousarray(b, np.int8)
    sb = _f32(sb)
    m, k = a.shape
    n = b.shape[0]
    y = np.zeros((m, n), np.float32)
    _call("or_qgemm_perchannel", _p(a), _p(b), _p(sb), m, n, k,
          ctypes.c_float(sa), _p(y))
    return y


def rmsnorm(x, w, residual=None, eps=1e-6):
    """rmsnorm_cpu over the last dim of a 1-D/2-D array."""
    x = _f32(x)
    w = _f32(w)
    r = None if residual is None else _f32(residual)
    rows, cols = (1, x.shape[0]) if x.ndim == 1 else x.shape
    y = np.empty_like(x)
    _call("or_rmsnorm", _p(x), _p(w), _p(r), rows, cols, ctypes.c_float(eps),
          _p(y))
    return y


def rope(x, theta=10000.0, pos_offset=0, neox=False):
    """rope_cpu / rope_neox_cpu on x [seq, dim]."""
    x = _f32(x)
    seq, dim = x.shape
    y = np.empty_like(x)
    _call("or_rope", _p(x), seq, dim, ctypes.c_float(theta), pos_offset,
          1 if neox else 0, _p(y))
    return y


def swiglu(g, u):
    """swiglu_cpu."""
    g = _f32(g)
    u = _f32(u)
    y = np.empty_like(g)
    _call("or_swiglu", _p(g), _p(u), ctypes.c_longlong(g.size), _p(y))
    return y


def rmsnorm_blocked(x, w, residual=None, eps=1e-6):
    """RMSNorm in the GPU kernels' summation order (cols % 4 == 0)."""
    x = _f32(x)
    w = _f32(w)
    r = None if residual is None else _f32(residual)
    rows, cols = (1, x.shape[0]) if x.ndim == 1 else x.shape
    y = np.empty_like(x)
    _call("or_rmsnorm_blocked", _p(x), _p(w), _p(r), rows, cols,
          ctypes.c_float(eps), _p(y))
    return y


def rmsnorm_quant(x, w, residual=None, eps=1e-6):
    """rmsnorm_blocked -> quantize_int8 over the whole output."""
    x = _f32(x)
    w = _f32(w)
    r = None if residual is None else _f32(residual)
    rows, cols = (1, x.shape[0]) if x.ndim == 1 else x.shape
    q = np.empty(x.shape, np.int8)
    s = ctypes.c_float(0.0)
    _call("or_rmsnorm_quant", _p(x), _p(w), _p(r), rows, cols,
          ctypes.c_float(eps), _p(q), ctypes.byref(s))
    return q, float(s.value)


def swiglu_quant(g, u):
    """swiglu_cpu -> quantize_int8 on [rows, cols] gate / up (any row
    stride: the arrays may be column slices of one [rows, 2*cols] array)."""
    g = np.asarray(g, dtype=np.float32)
    u = np.asarray(u, dtype=np.float32)
    rows, cols = g.shape
    both = np.ascontiguousarray(np.concatenate([g, u], axis=1))
    q = np.empty((rows, cols), np.int8)
    s = ctypes.c_float(0.0)
    gp = both.ctypes.data
    up = gp + cols * 4
    _call("or_swiglu_quant", ctypes.c_void_p(gp), ctypes.c_void_p(up), rows,
          cols, ctypes.c_longlong(2 * cols), _p(q), ctypes.byref(s))
    return q, float(s.value)


def rope_kv_append_paged(qkv, q_heads, kv_heads, k_pool, v_pool, table, lens,
                         theta=10000.0, pos_offset=0, neox=False):
    """rope (q and k heads of sequence b at position lens[b] + pos_offset),
    then kv_append_paged of the rotated k and the v heads. qkv is
    [batch, (q_heads + 2 * kv_heads) * dim] float32; returns q_out
    [batch, q_heads, dim] and updates the pools in place."""
    qkv = _f32(qkv)
    batch = qkv.shape[0]
    dim = qkv.shape[1] // (q_heads + 2 * kv_heads)
    heads = qkv.reshape(batch, q_heads + 2 * kv_heads, dim)
    lens = _i32(lens)
    rot = np.empty((batch, q_heads + kv_heads, dim), np.float32)
    for b in range(batch):
        for h in range(q_heads + kv_heads):
            rot[b, h] = rope(heads[b, h][None, :], theta,
                             int(lens[b]) + pos_offset, neox)[0]
    kv_append_paged(k_pool, v_pool, table, rot[:, q_heads:],
                    np.ascontiguousarray(heads[:, q_heads + kv_heads:]), lens)
    return rot[:, :q_heads].copy()


# ---------------------------------------------------------------------------
# post-logits sampling
# ---------------------------------------------------------------------------


def splitmix_uniform(seed):
    """The shared sampler RNG: splitmix64 finalised to a float in [0, 1)."""
    lib = _load()
    lib.or_splitmix_uniform.restype = ctypes.c_float
    return float(lib.or_splitmix_uniform(ctypes.c_ulonglong(seed)))


def argmax_batched(x):
    """argmax_batched_cpu: [rows, n] f32 -> int64 [rows] (earliest index on ties)."""
    x = _f32(x)
    rows, n = x.shape
    out = np.zeros(rows, np.int64)
    _call("or_argmax_batched", _p(x), rows, n, _p(out))
    return out


def repetition_penalty(logits, ids, penalty):
    """repetition_penalty_cpu: each distinct id once, from the original logit."""
    logits = _f32(logits)
    ids = np.ascontiguousarray(ids, np.int64)
    y = np.empty_like(logits)
    _call("or_repetition_penalty", _p(logits), logits.size, _p(ids), ids.size,
          ctypes.c_float(penalty), _p(y))
    return y


def sample_topp(logits, p, temperature=1.0, seed=0):
    """sample_topp_cpu -> token id."""
    logits = _f32(logits)
    out = ctypes.c_longlong(0)
    _call("or_sample_topp", _p(logits), logits.size, ctypes.c_float(p),
          ctypes.c_float(temperature), ctypes.c_ulonglong(seed), ctypes.byref(out))
    return int(out.value)


def decode_step_batched(logits, ids, offs, penalty, p, temperature, seeds):
    """Per row: repetition_penalty over ids[offs[r]:offs[r+1]], then
    sample_topp with seeds[r]. offs=None: no ids."""
    logits = _f32(logits)
    rows, n = logits.shape
    ids = np.ascontiguousarray(np.zeros(0) if ids is None else ids, np.int64)
    offs_a = None if offs is None else np.ascontiguousarray(offs, np.int64)
    seeds = np.ascontiguousarray(seeds, np.uint64)
    out = np.zeros(rows, np.int64)
    _call("or_decode_step_batched", _p(logits), rows, n, _p(ids), _p(offs_a),
          ctypes.c_float(penalty), ctypes.c_float(p), ctypes.c_float(temperature),
          _p(seeds), _p(out))
    return out
