"""fusedtok_amd: the fusedtok decode hot path, native to AMD MI355X (gfx950).

The public functions keep fusedtok 2.5.0's names, signatures and error
contract for the decode hot path (reference python/fusedtok/__init__.py):

- ``attention_decode`` / ``attention_decode_paged``: flash-decoding GQA
  attention over contiguous / paged KV caches (f32, bf16, fp16 storage);
- ``attention_prefill``: causal / bidirectional attention over a fresh
  sequence's S query rows (the step before decode);
- ``kv_append`` / ``kv_append_paged``: one fresh token's K/V rows per
  sequence written in place at position ``lens[b]``;
- ``quantize_int8``: symmetric per-tensor INT8 quantize; ``dequantize_int8``
  and the fused dequantize-add-requantize ``qadd_int8``;
- ``qgemm`` / ``qgemm_perchannel``: W8A8 GEMM with exact int32 accumulation;
- ``rmsnorm`` (+ residual), ``rope`` (interleaved / NeoX, ``pos_offset``),
  ``swiglu``;
- the post-logits step: ``argmax`` / ``argmax_batched`` (greedy),
  ``sample_topp`` / ``sample_topp_batched`` and ``decode_step`` /
  ``decode_step_batched`` (repetition penalty -> temperature -> nucleus
  sampling, deterministic per seed).

Execution paths:

- torch tensors on the GPU -> zero-copy: the HIP kernels read and write the
  tensors' memory through ``data_ptr()`` on the current torch stream, with no
  host synchronisation (``quantize_int8`` syncs once to return its Python
  float scale, as the reference does).
- host inputs (numpy arrays, CPU torch tensors) -> staged: uploaded, run on
  the GPU, downloaded. This replaces both of the reference's host paths; the
  ``cuda=`` keyword is accepted for compatibility. There is no CPU fallback:
  without a HIP device, host inputs raise RuntimeError.

Validation happens before any device work, with the reference's contract:
TypeError for dtype / device-family problems, ValueError for shapes and
values, RuntimeError for HIP failures. Device-resident ``lens`` and block
tables are trusted (never read back); host-origin ones are range-checked.

Build additions (not in the reference): fp16 storage for ``rmsnorm``,
``rope`` and ``swiglu``; bf16 / fp16 input to ``quantize_int8`` and a
device-resident scale (``device_scale=True``); bf16 / fp16 GEMM outputs
(``out_dtype=``) and a device scale operand; ``qgemm_i32`` (raw int32
accumulators); per-row RoPE positions (``positions=``); the fused
decode-chain steps ``rmsnorm_quant``, ``swiglu_quant`` and
``rope_kv_append_paged`` (GPU tensors only).
"""

import numpy as np

# torch first: its bundled HIP runtime (libamdhip64.so, soname
# libamdhip64.so.7) must be the one loaded in this process, so that the
# library's own libamdhip64.so.7 dependency binds to it by soname. Loading the
# library first would pull in a second HIP runtime from /opt/rocm; two
# runtimes in one process do not share devices or stream handles.
import torch

try:
    from . import _fusedtok
except ImportError as exc:  # pragma: no cover - exercised by packaging
    raise ImportError(
        "fusedtok_amd: the native extension is not built. Run "
        "`python -c 'import __graft_entry__ as g; g.build()'` from the "
        "repository root (needs hipcc for gfx950)."
    ) from exc

__version__ = "0.1.0"

__all__ = [
    "cuda_available",
    "rmsnorm",
    "rope",
    "swiglu",
    "quantize_int8",
    "dequantize_int8",
    "qadd_int8",
    "qgemm",
    "qgemm_perchannel",
    "qgemm_i32",
    "attention_decode",
    "attention_decode_paged",
    "attention_prefill",
    "kv_append",
    "kv_append_paged",
    "rmsnorm_quant",
    "rmsnorm_qgemm",
    "swiglu_quant",
    "rope_kv_append_paged",
    "argmax",
    "argmax_batched",
    "sample_topp",
    "sample_topp_batched",
    "decode_step",
    "decode_step_batched",
]

# C-ABI dtype codes (include/fusedtok_amd.h)
_DT_F32, _DT_BF16, _DT_F16 = 0, 1, 2
_DT_CODE = {torch.float32: _DT_F32, torch.bfloat16: _DT_BF16,
            torch.float16: _DT_F16}
_HALF = (torch.bfloat16, torch.float16)


def cuda_available():
    """True if a usable HIP device is present (reference fusedtok.cu:34-37)."""
    return _fusedtok.cuda_available()


# ---------------------------------------------------------------------------
# dispatch helpers
# ---------------------------------------------------------------------------


def _is_torch(x):
    return torch.is_tensor(x)


def _on_gpu(x):
    return torch.is_tensor(x) and x.is_cuda


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _require_gpu(t, name):
    if not _on_gpu(t):
        raise TypeError(f"{name} must be a GPU tensor when the primary input "
                        "is on the GPU")


def _check_contiguous(t, name):
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_dtype(t, name, allowed):
    if not t.is_cuda:
        raise TypeError(f"{name} must be a GPU tensor (got a CPU tensor on "
                        "the zero-copy path)")
    if t.dtype not in allowed:
        names = ", ".join(str(d).replace("torch.", "") for d in allowed)
        raise TypeError(f"{name} must be one of ({names}), got {t.dtype}")
    _check_contiguous(t, name)


_FLOAT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _launcher(base, dtype):
    if dtype is torch.bfloat16:
        return getattr(_fusedtok, base + "_bf16")
    if dtype is torch.float16:
        return getattr(_fusedtok, base + "_fp16")
    return getattr(_fusedtok, base)


def _need_device():
    if not _fusedtok.cuda_available():
        raise RuntimeError(
            "fusedtok_amd runs on the GPU only: no HIP device is available "
            "for these host inputs (there is no CPU fallback)")
    return torch.device("cuda", torch.cuda.current_device())


def _host_f32(x, name):
    """Host-origin input -> float32 C-contiguous numpy array."""
    if _is_torch(x):
        if x.is_cuda:
            raise TypeError(f"{name} is a GPU tensor while another input is "
                            "host-side; move all inputs to the same device")
        x = x.detach()
        if x.dtype is not torch.float32:
            x = x.to(torch.float32)
        return np.ascontiguousarray(x.numpy())
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _upload(arr, device):
    return torch.from_numpy(np.ascontiguousarray(arr)).to(device)


# Small per-call int64 arguments (token histories, offsets, seeds) travel in
# one non-blocking copy from a ring of pinned host buffers: a pageable copy
# per array made every call wait for the GPU to drain before the host could
# prepare the next one. A slot is refilled only after the copy that read it
# has completed (its event).
_PIN_RING = []
_PIN_SLOTS = 4
_pin_next = [0]


def _upload_i64(arrays, device):
    """Host int64 numpy arrays -> device int64 tensors (views of one
    buffer), ordered on the current stream."""
    sizes = [int(a.size) for a in arrays]
    total = max(1, sum(sizes))
    if len(_PIN_RING) < _PIN_SLOTS:
        _PIN_RING.append([torch.empty(0, dtype=torch.int64), None])
    slot = _PIN_RING[_pin_next[0] % len(_PIN_RING)]
    _pin_next[0] += 1
    if slot[1] is not None:
        slot[1].synchronize()
    if slot[0].numel() < total:
        slot[0] = torch.empty(max(total, 2 * slot[0].numel(), 1024), dtype=torch.int64,
                              pin_memory=True)
    host = slot[0].numpy()
    at = 0
    for a, k in zip(arrays, sizes):
        host[at:at + k] = a.reshape(-1)
        at += k
    dev = torch.empty(total, dtype=torch.int64, device=device)
    dev.copy_(slot[0][:total], non_blocking=True)
    ev = torch.cuda.Event()
    ev.record(torch.cuda.current_stream(device))
    slot[1] = ev
    out, at = [], 0
    for k in sizes:
        out.append(dev[at:at + k])
        at += k
    return out


def _result(res_t, like):
    """Staged result back to the caller's family (torch CPU or numpy)."""
    out = res_t.cpu()
    return out if _is_torch(like) else out.numpy()


def _host_int_array(t, name):
    """Host-origin integer values as numpy, or None for a GPU tensor."""
    if _is_torch(t):
        if t.is_cuda:
            return None
        host = t.detach().cpu().numpy()
    else:
        host = np.asarray(t)
    if host.size and not np.issubdtype(host.dtype, np.integer):
        raise TypeError(f"{name} must hold integer values (got dtype {host.dtype})")
    return host


def _host_lens_checked(lens, batch, limit, upper_inclusive=True):
    host = _host_int_array(lens, "lens")
    if host is None:
        return None
    host = np.ascontiguousarray(host, dtype=np.int32)
    if host.ndim != 1 or host.shape[0] != batch:
        raise ValueError("lens must be 1-D with batch entries")
    bracket = "]" if upper_inclusive else ")"
    if host.size and (host.min() < 0 or host.max() > limit
                      or (not upper_inclusive and host.max() == limit)):
        raise ValueError(f"lens entries must be in [0, {limit}{bracket}")
    return host


def _lens_tensor(lens, batch, limit, device, upper_inclusive=True):
    host = _host_lens_checked(lens, batch, limit, upper_inclusive)
    if host is not None:
        return torch.from_numpy(host).to(device)
    lt = lens
    if lt.dtype is not torch.int32:
        lt = lt.to(torch.int32)
    if not lt.is_contiguous():
        lt = lt.contiguous()
    if lt.ndim != 1 or lt.numel() != batch:
        raise ValueError("lens must be 1-D with batch entries")
    return lt


def _host_table_checked(table, batch, nblocks):
    host = _host_int_array(table, "block_table")
    if host is None:
        return None
    host = np.ascontiguousarray(host, dtype=np.int32)
    if host.ndim != 2 or host.shape[0] != batch:
        raise ValueError("block_table must be [B, S] with batch rows")
    if host.size and (host.min() < 0 or host.max() >= nblocks):
        raise ValueError(f"block_table entries must be in [0, {nblocks})")
    return host


def _table_tensor(table, batch, nblocks, device):
    host = _host_table_checked(table, batch, nblocks)
    if host is not None:
        return torch.from_numpy(host).to(device)
    bt = table
    if bt.dtype is not torch.int32:
        bt = bt.to(torch.int32)
    if not bt.is_contiguous():
        bt = bt.contiguous()
    if bt.ndim != 2 or bt.shape[0] != batch:
        raise ValueError("block_table must be [B, S] with batch rows")
    return bt


def _rows_cols(shape):
    if len(shape) == 1:
        return 1, shape[0]
    if len(shape) == 2:
        return shape[0], shape[1]
    raise ValueError("expected a 1-D or 2-D tensor")


# ---------------------------------------------------------------------------
# swiglu (reference __init__.py:498-539)
# ---------------------------------------------------------------------------


def swiglu(gate, up, *, cuda=False):
    """SwiGLU activation: ``silu(gate) * up`` = ``gate / (1 + exp(-gate)) * up``."""
    if _on_gpu(gate):
        _require_gpu(up, "up")
        _check_dtype(gate, "gate", _FLOAT_DTYPES)
        _check_dtype(up, "up", _FLOAT_DTYPES)
        if gate.dtype is not up.dtype:
            raise TypeError("inputs must have the same dtype")
        if gate.shape != up.shape:
            raise ValueError("inputs must have the same shape")
        out = torch.empty_like(gate)
        _launcher("swiglu_launch", gate.dtype)(
            gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(),
            _stream())
        return out
    g = _host_f32(gate, "gate")
    u = _host_f32(up, "up")
    if g.shape != u.shape:
        raise ValueError("inputs must have the same shape")
    dev = _need_device()
    res = swiglu(_upload(g, dev), _upload(u, dev))
    return _result(res, gate)


# ---------------------------------------------------------------------------
# rmsnorm (reference __init__.py:547-590)
# ---------------------------------------------------------------------------


def rmsnorm(x, weight, *, residual=None, eps=1e-6, cuda=False):
    """RMSNorm, optionally fused with a residual add:

    ``y = (x + r) * rsqrt(mean((x + r)^2) + eps) * weight``

    x: [rows, cols] or [cols]; weight: [cols] (float32; bf16/fp16 weights
    are upcast); residual: same shape and dtype as x.
    """
    if _on_gpu(x):
        _check_dtype(x, "x", _FLOAT_DTYPES)
        _require_gpu(weight, "weight")
        if weight.dtype is not torch.float32:
            weight = weight.to(torch.float32)
        if not weight.is_contiguous():
            weight = weight.contiguous()
        rows, cols = _rows_cols(x.shape)
        if weight.ndim != 1 or weight.numel() != cols:
            raise ValueError("weight must be 1-D with cols entries")
        r_ptr = None
        if residual is not None:
            _require_gpu(residual, "residual")
            _check_dtype(residual, "residual", _FLOAT_DTYPES)
            if residual.dtype is not x.dtype:
                raise TypeError("residual must have the same dtype as x")
            if residual.shape != x.shape:
                raise ValueError("residual must have the same shape as x")
            r_ptr = residual.data_ptr()
        out = torch.empty_like(x)
        _launcher("rmsnorm_launch", x.dtype)(
            x.data_ptr(), weight.data_ptr(), r_ptr, out.data_ptr(), rows, cols,
            float(eps), _stream())
        return out
    arr_x = _host_f32(x, "x")
    arr_w = _host_f32(weight, "weight")
    rows, cols = _rows_cols(arr_x.shape)
    if arr_w.ndim != 1 or arr_w.shape[0] != cols:
        raise ValueError("weight.size() must equal cols")
    arr_r = None
    if residual is not None:
        arr_r = _host_f32(residual, "residual")
        if arr_r.shape != arr_x.shape:
            raise ValueError("x.size() must equal rows * cols (residual shape)")
    if cols == 0:
        raise ValueError("rows must be >= 0 and cols must be > 0")
    dev = _need_device()
    res = rmsnorm(_upload(arr_x, dev), _upload(arr_w, dev),
                  residual=None if arr_r is None else _upload(arr_r, dev),
                  eps=eps)
    return _result(res, x)


# ---------------------------------------------------------------------------
# rope (reference __init__.py:645-702)
# ---------------------------------------------------------------------------


def rope(q, k=None, *, theta=10000.0, pos_offset=0, neox=False, cuda=False,
         positions=None, rows_per_position=1):
    """Rotary position embedding on (q, k).

    q, k: [seq, dim] with even dim. ``neox=False`` rotates interleaved pairs
    (2j, 2j+1); ``neox=True`` rotates the row halves (j, j + dim/2). Row r
    sits at position ``r + pos_offset``; pair j turns by
    ``position * theta^(-2j/dim)``. Returns ``(q_rot, k_rot)`` (None if k is).

    Build addition: ``positions`` (a GPU int32 vector) with
    ``rows_per_position`` places row r at ``positions[r // rows_per_position]
    + pos_offset`` - e.g. q viewed as [B*Hq, D] with ``rows_per_position=Hq``
    and per-sequence positions.
    """
    if _on_gpu(q):
        _check_dtype(q, "q", _FLOAT_DTYPES)
        if q.ndim != 2:
            raise ValueError("q must be 2-D [seq, dim]")
        seq, dim = q.shape
        if dim % 2:
            raise ValueError("dim must be even (RoPE pairs elements)")
        if pos_offset < 0:
            raise ValueError("pos_offset must be >= 0")
        k_out = None
        if k is not None:
            _require_gpu(k, "k")
            _check_dtype(k, "k", _FLOAT_DTYPES)
            if k.dtype is not q.dtype:
                raise TypeError("k must have the same dtype as q")
            if k.shape != q.shape:
                raise ValueError("k must have the same shape as q")
        pos_ptr = None
        if positions is not None:
            _require_gpu(positions, "positions")
            if positions.dtype is not torch.int32:
                raise TypeError("positions must be int32")
            _check_contiguous(positions, "positions")
            if rows_per_position < 1:
                raise ValueError("rows_per_position must be >= 1")
            if positions.numel() * rows_per_position < seq:
                raise ValueError("positions must cover every row")
            pos_ptr = positions.data_ptr()
        q_out = torch.empty_like(q)
        if k is not None:
            k_out = torch.empty_like(k)
        code = _DT_CODE[q.dtype]
        for src, dst in ((q, q_out), (k, k_out)):
            if src is None:
                continue
            if pos_ptr is None and rows_per_position == 1:
                if q.dtype is torch.float32:
                    _fusedtok.rope_launch(bool(neox), src.data_ptr(), dst.data_ptr(),
                                          seq, dim, float(theta), int(pos_offset),
                                          _stream())
                else:
                    base = "rope_neox_launch" if neox else "rope_launch"
                    _launcher(base, q.dtype)(src.data_ptr(), dst.data_ptr(), seq,
                                             dim, float(theta), int(pos_offset),
                                             _stream())
            else:
                _fusedtok.rope_launch_ex(src.data_ptr(), dst.data_ptr(), code, seq,
                                         dim, float(theta), int(pos_offset),
                                         pos_ptr, int(rows_per_position),
                                         bool(neox), _stream())
        return q_out, k_out
    arr_q = _host_f32(q, "q")
    arr_k = None if k is None else _host_f32(k, "k")
    if arr_q.ndim != 2:
        raise ValueError("q must be 2-D [seq, dim]")
    if arr_q.shape[1] % 2:
        raise ValueError("dim must be even (RoPE pairs elements)")
    if pos_offset < 0:
        raise ValueError("pos_offset must be >= 0")
    if arr_k is not None and arr_k.shape != arr_q.shape:
        raise ValueError("k.size() must equal q.size()")
    dev = _need_device()
    qr, kr = rope(_upload(arr_q, dev),
                  None if arr_k is None else _upload(arr_k, dev),
                  theta=theta, pos_offset=pos_offset, neox=neox)
    return _result(qr, q), (None if kr is None else _result(kr, q))


# ---------------------------------------------------------------------------
# attention (reference __init__.py:710-788, 849-940)
# ---------------------------------------------------------------------------


def attention_decode(q, k_cache, v_cache, lens=None, *, cuda=False):
    """Single-token causal attention with GQA over a contiguous KV cache:

    ``out[b, h] = softmax(q[b,h] . K[b,kv(h)]^T / sqrt(D)) . V[b,kv(h)]``

    q: [B, Hq, D]; k_cache / v_cache: [B, Hkv, T, D]; lens: [B] valid lengths
    (<= T; None = all rows). q head h reads kv head ``h // (Hq // Hkv)``.
    Length-0 sequences give zero rows. Storage f32 / bf16 / fp16; softmax and
    accumulators are float32; the output matches the input dtype.
    """
    if _on_gpu(q):
        for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
            _check_dtype(t, name, _FLOAT_DTYPES)
        for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
            if t.dtype is not q.dtype:
                raise TypeError(f"{name} must have the same dtype as q")
        if q.ndim != 3 or k_cache.ndim != 4 or v_cache.ndim != 4:
            raise ValueError("q must be [B, Hq, D]; k/v caches [B, Hkv, T, D]")
        b, hq, d = q.shape
        b2, hkv, t_rows, d2 = k_cache.shape
        if (b2, d2) != (b, d) or v_cache.shape != k_cache.shape:
            raise ValueError("k_cache/v_cache must match q's batch and dim")
        if hq < 1 or hkv < 1:
            raise ValueError("head counts must be >= 1")
        if hq % hkv:
            raise ValueError("q heads must be a multiple of kv heads")
        lens_ptr = None
        if lens is not None:
            lens_ptr = _lens_tensor(lens, b, t_rows, q.device)
        out = torch.empty((b, hq, d), dtype=q.dtype, device=q.device)
        if b * hq > 0:
            _launcher("attention_decode_launch", q.dtype)(
                q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                None if lens_ptr is None else lens_ptr.data_ptr(), out.data_ptr(),
                b, hq, hkv, t_rows, d, _stream())
        return out
    arr_q = _host_f32(q, "q")
    arr_k = _host_f32(k_cache, "k_cache")
    arr_v = _host_f32(v_cache, "v_cache")
    if arr_q.ndim != 3 or arr_k.ndim != 4 or arr_v.ndim != 4:
        raise ValueError("q must be [B, Hq, D]; k/v caches [B, Hkv, T, D]")
    b, hq, d = arr_q.shape
    b2, hkv, t_rows, d2 = arr_k.shape
    if (b2, d2) != (b, d) or arr_v.shape != arr_k.shape:
        raise ValueError("k_cache/v_cache must match q's batch and dim")
    if hkv < 1 or hq < 1:
        raise ValueError("head counts must be >= 1")
    if hq % hkv:
        raise ValueError("q heads must be a multiple of kv heads")
    if d % 4 or d > 512:
        raise ValueError("dim must be a multiple of 4 and at most 512")
    arr_l = None
    if lens is not None:
        arr_l = _host_lens_checked(lens, b, t_rows)
        if arr_l is None:
            raise TypeError("lens must be a host array on this path")
    dev = _need_device()
    res = attention_decode(_upload(arr_q, dev), _upload(arr_k, dev),
                           _upload(arr_v, dev),
                           None if arr_l is None else _upload(arr_l, dev))
    return _result(res, q)


def attention_prefill(q, k, v, causal=True, *, cuda=False):
    """Prefill (fresh-sequence) attention over S query rows:

    ``out[b, h, i] = softmax(q[b,h,i] . K[b,kv(h)]^T / sqrt(D)) . V[b,kv(h)]``
    where query row i attends to key rows ``[0, i]`` (``causal=True``) or to
    all S rows (``causal=False``). q: [B, Hq, S, D]; k / v: [B, Hkv, S, D];
    out: [B, Hq, S, D] in q's dtype (f32 / bf16 / fp16 storage, float32
    softmax and accumulators). GQA as :func:`attention_decode`; D a multiple
    of 4, at most 512 (reference ``__init__.py:791-846``).
    """
    if _on_gpu(q):
        for name, t in (("q", q), ("k", k), ("v", v)):
            _check_dtype(t, name, _FLOAT_DTYPES)
        for name, t in (("k", k), ("v", v)):
            if t.dtype is not q.dtype:
                raise TypeError(f"{name} must have the same dtype as q")
        if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
            raise ValueError("q/k/v must be [B, heads, S, D]")
        b, hq, s, d = q.shape
        b2, hkv, s2, d2 = k.shape
        if (b2, s2, d2) != (b, s, d) or v.shape != k.shape:
            raise ValueError("k/v must match q's batch, seq and dim")
        if hq < 1 or hkv < 1:
            raise ValueError("head counts must be >= 1")
        if hq % hkv:
            raise ValueError("q heads must be a multiple of kv heads")
        out = torch.empty((b, hq, s, d), dtype=q.dtype, device=q.device)
        if b * hq * s > 0:
            _launcher("attention_prefill_launch", q.dtype)(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                b, hq, hkv, s, d, bool(causal), _stream())
        return out
    arr_q = _host_f32(q, "q")
    arr_k = _host_f32(k, "k")
    arr_v = _host_f32(v, "v")
    if arr_q.ndim != 4 or arr_k.ndim != 4 or arr_v.ndim != 4:
        raise ValueError("q/k/v must be [B, heads, S, D]")
    b, hq, s, d = arr_q.shape
    b2, hkv, s2, d2 = arr_k.shape
    if (b2, s2, d2) != (b, s, d) or arr_v.shape != arr_k.shape:
        raise ValueError("k/v must match q's batch, seq and dim")
    if hq < 1 or hkv < 1:
        raise ValueError("head counts must be >= 1")
    if hq % hkv:
        raise ValueError("q heads must be a multiple of kv heads")
    if d % 4 or d > 512:
        raise ValueError("dim must be a multiple of 4 and at most 512")
    dev = _need_device()
    res = attention_prefill(_upload(arr_q, dev), _upload(arr_k, dev),
                            _upload(arr_v, dev), causal)
    return _result(res, q)


def attention_decode_paged(q, k_pool, v_pool, block_table, lens=None, *,
                           cuda=False):
    """Single-token GQA attention over a PAGED KV cache.

    k_pool / v_pool: [Nb, Hkv, P, D]; block_table: [B, S] int; token t of
    sequence b is ``pool[block_table[b, t // P], kv, t % P]``; lens: [B]
    (None = S * P rows each). GQA group sizes 1/2/4/8/16. Host-origin table
    and lens values are validated; GPU-resident ones are trusted.
    """
    if _on_gpu(q):
        for name, t in (("q", q), ("k_pool", k_pool), ("v_pool", v_pool)):
            _check_dtype(t, name, _FLOAT_DTYPES)
        for name, t in (("k_pool", k_pool), ("v_pool", v_pool)):
            if t.dtype is not q.dtype:
                raise TypeError(f"{name} must have the same dtype as q")
        if q.ndim != 3 or k_pool.ndim != 4 or v_pool.ndim != 4:
            raise ValueError("q must be [B, Hq, D]; pools [Nb, Hkv, P, D]")
        b, hq, d = q.shape
        nb, hkv, page, d2 = k_pool.shape
        if d2 != d or v_pool.shape != k_pool.shape:
            raise ValueError("pools must match q's dim and each other")
        if hq < 1 or hkv < 1:
            raise ValueError("head counts must be >= 1")
        if hq % hkv:
            raise ValueError("q heads must be a multiple of kv heads")
        if hq // hkv not in (1, 2, 4, 8, 16):
            raise ValueError("paged decode supports GQA group sizes "
                             "1/2/4/8/16 (use attention_decode otherwise)")
        bt = _table_tensor(block_table, b, nb, q.device)
        s_width = bt.shape[1]
        lt = None
        if lens is not None:
            lt = _lens_tensor(lens, b, s_width * page, q.device)
        out = torch.empty((b, hq, d), dtype=q.dtype, device=q.device)
        if b * hq > 0:
            _launcher("attention_decode_paged_launch", q.dtype)(
                q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), bt.data_ptr(),
                None if lt is None else lt.data_ptr(), out.data_ptr(),
                b, hq, hkv, page, s_width, d, _stream())
        return out
    arr_q = _host_f32(q, "q")
    arr_k = _host_f32(k_pool, "k_pool")
    arr_v = _host_f32(v_pool, "v_pool")
    if arr_q.ndim != 3 or arr_k.ndim != 4 or arr_v.ndim != 4:
        raise ValueError("q must be [B, Hq, D]; pools [Nb, Hkv, P, D]; "
                         "block_table [B, S]")
    b, hq, d = arr_q.shape
    nb, hkv, page, d2 = arr_k.shape
    arr_t = _host_table_checked(block_table, b, nb)
    if arr_t is None:
        raise TypeError("block_table must be a host array on this path")
    if d2 != d or arr_v.shape != arr_k.shape:
        raise ValueError("pools must match q's dim and each other")
    if hkv < 1 or hq < 1:
        raise ValueError("head counts must be >= 1")
    if hq % hkv:
        raise ValueError("q heads must be a multiple of kv heads")
    if hq // hkv not in (1, 2, 4, 8, 16):
        raise ValueError("paged decode supports GQA group sizes "
                         "1/2/4/8/16 (use attention_decode otherwise)")
    if d % 4 or d > 512:
        raise ValueError("dim must be a multiple of 4 and at most 512")
    arr_l = None
    if lens is not None:
        arr_l = _host_lens_checked(lens, b, arr_t.shape[1] * page)
        if arr_l is None:
            raise TypeError("lens must be a host array on this path")
    dev = _need_device()
    res = attention_decode_paged(
        _upload(arr_q, dev), _upload(arr_k, dev), _upload(arr_v, dev),
        _upload(arr_t, dev), None if arr_l is None else _upload(arr_l, dev))
    return _result(res, q)


# ---------------------------------------------------------------------------
# kv append (reference __init__.py:943-1112)
# ---------------------------------------------------------------------------


def _host_inplace_f32(arr, name):
    raw = arr.numpy() if _is_torch(arr) else arr
    if not isinstance(raw, np.ndarray) or raw.dtype != np.float32 \
            or not raw.flags["C_CONTIGUOUS"]:
        raise TypeError(f"{name} must be a float32 C-contiguous array "
                        "(in-place op; conversion would drop writes)")
    return raw


def kv_append_paged(k_pool, v_pool, block_table, k_new, v_new, lens, *,
                    cuda=False):
    """Write one fresh token's K/V rows per sequence into the paged pools,
    in place: ``k_new[b]`` lands at block ``block_table[b, lens[b] // P]``,
    offset ``lens[b] % P``. lens is required (values in [0, S*P)). Returns
    None."""
    if _on_gpu(k_pool):
        for name, t in (("k_pool", k_pool), ("v_pool", v_pool),
                        ("k_new", k_new), ("v_new", v_new)):
            _check_dtype(t, name, _FLOAT_DTYPES)
        for name, t in (("v_pool", v_pool), ("k_new", k_new), ("v_new", v_new)):
            if t.dtype is not k_pool.dtype:
                raise TypeError(f"{name} must have the pool dtype")
        if k_pool.ndim != 4 or v_pool.ndim != 4:
            raise ValueError("pools must be [Nb, Hkv, P, D]")
        if k_new.ndim != 3 or v_new.ndim != 3:
            raise ValueError("k_new/v_new must be [B, Hkv, D]")
        nb, hkv, page, d = k_pool.shape
        b, hkv2, d2 = k_new.shape
        if (hkv2, d2) != (hkv, d) or v_pool.shape != k_pool.shape \
                or v_new.shape != k_new.shape:
            raise ValueError("k/v operands must match the pool layout")
        if b == 0:
            return None
        bt = _table_tensor(block_table, b, nb, k_pool.device)
        lt = _lens_tensor(lens, b, bt.shape[1] * page, k_pool.device,
                          upper_inclusive=False)
        _launcher("kv_append_paged_launch", k_pool.dtype)(
            k_new.data_ptr(), v_new.data_ptr(), bt.data_ptr(), lt.data_ptr(),
            k_pool.data_ptr(), v_pool.data_ptr(), b, hkv, d, page, bt.shape[1],
            _stream())
        return None
    kp = _host_inplace_f32(k_pool, "k_pool")
    vp = _host_inplace_f32(v_pool, "v_pool")
    kn = _host_f32(k_new, "k_new")
    vn = _host_f32(v_new, "v_new")
    if kp.ndim != 4 or kn.ndim != 3:
        raise ValueError("pools [Nb,Hkv,P,D]; k_new [B,Hkv,D]")
    nb, hkv, page, d = kp.shape
    b = kn.shape[0]
    if kn.shape != (b, hkv, d) or vp.shape != kp.shape or vn.shape != kn.shape:
        raise ValueError("k/v operands must match the pool layout")
    arr_t = _host_table_checked(block_table, b, nb)
    if arr_t is None:
        raise TypeError("block_table must be a host array on this path")
    arr_l = _host_lens_checked(lens, b, arr_t.shape[1] * page,
                               upper_inclusive=False)
    if arr_l is None:
        raise TypeError("lens must be a host array on this path")
    if d % 4:
        raise ValueError("dim must be a multiple of 4")
    if b == 0:
        return None
    dev = _need_device()
    kp_d, vp_d = _upload(kp, dev), _upload(vp, dev)
    kv_append_paged(kp_d, vp_d, _upload(arr_t, dev), _upload(kn, dev),
                    _upload(vn, dev), _upload(arr_l, dev))
    np.copyto(kp, kp_d.cpu().numpy())
    np.copyto(vp, vp_d.cpu().numpy())
    return None


def kv_append(k_cache, v_cache, k_new, v_new, lens, *, cuda=False):
    """Write one fresh token's K/V rows per sequence into the contiguous
    caches [B, Hkv, T, D] at row ``lens[b]`` (in place; lens in [0, T)).
    Returns None."""
    if _on_gpu(k_cache):
        for name, t in (("k_cache", k_cache), ("v_cache", v_cache),
                        ("k_new", k_new), ("v_new", v_new)):
            _check_dtype(t, name, _FLOAT_DTYPES)
        for name, t in (("v_cache", v_cache), ("k_new", k_new),
                        ("v_new", v_new)):
            if t.dtype is not k_cache.dtype:
                raise TypeError(f"{name} must have the cache dtype")
        if k_cache.ndim != 4 or v_cache.ndim != 4:
            raise ValueError("caches must be [B, Hkv, T, D]")
        if k_new.ndim != 3 or v_new.ndim != 3:
            raise ValueError("k_new/v_new must be [B, Hkv, D]")
        b, hkv, t_rows, d = k_cache.shape
        if tuple(k_new.shape) != (b, hkv, d) or v_cache.shape != k_cache.shape \
                or v_new.shape != k_new.shape:
            raise ValueError("k/v operands must match the cache layout")
        if b == 0:
            return None
        lt = _lens_tensor(lens, b, t_rows, k_cache.device, upper_inclusive=False)
        _launcher("kv_append_launch", k_cache.dtype)(
            k_new.data_ptr(), v_new.data_ptr(), lt.data_ptr(), k_cache.data_ptr(),
            v_cache.data_ptr(), b, hkv, d, t_rows, _stream())
        return None
    kc = _host_inplace_f32(k_cache, "k_cache")
    vc = _host_inplace_f32(v_cache, "v_cache")
    kn = _host_f32(k_new, "k_new")
    vn = _host_f32(v_new, "v_new")
    if kc.ndim != 4 or kn.ndim != 3:
        raise ValueError("caches [B,Hkv,T,D]; k_new [B,Hkv,D]")
    b, hkv, t_rows, d = kc.shape
    if kn.shape != (b, hkv, d) or vc.shape != kc.shape or vn.shape != kn.shape:
        raise ValueError("k/v operands must match the cache layout")
    arr_l = _host_lens_checked(lens, b, t_rows, upper_inclusive=False)
    if arr_l is None:
        raise TypeError("lens must be a host array on this path")
    if d % 4:
        raise ValueError("dim must be a multiple of 4")
    if b == 0:
        return None
    dev = _need_device()
    kc_d, vc_d = _upload(kc, dev), _upload(vc, dev)
    kv_append(kc_d, vc_d, _upload(kn, dev), _upload(vn, dev), _upload(arr_l, dev))
    np.copyto(kc, kc_d.cpu().numpy())
    np.copyto(vc, vc_d.cpu().numpy())
    return None


# ---------------------------------------------------------------------------
# INT8 (reference __init__.py:1402-1425, 1476-1599)
# ---------------------------------------------------------------------------


def quantize_int8(x, *, device_scale=False):
    """Symmetric per-tensor INT8 quantization.

    ``scale = max(|x|) / 127`` (1.0 for all-zero input);
    ``q = clamp(rint(x * (1 / scale)), -127, 127)``. Returns ``(q, scale)``
    with scale a Python float. Build additions: bf16 / fp16 GPU input, and
    ``device_scale=True`` returns the scale as a 1-element GPU float32 tensor
    without synchronising the stream.
    """
    if _on_gpu(x):
        _check_dtype(x, "x", _FLOAT_DTYPES)
        q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
        scale = torch.empty(1, dtype=torch.float32, device=x.device)
        if x.numel() == 0:
            scale.fill_(1.0)   # all-zero (here: empty) input -> scale 1.0
        if x.dtype is torch.float32:
            _fusedtok.quantize_launch(x.data_ptr(), q.data_ptr(), scale.data_ptr(),
                                      x.numel(), _stream())
        else:
            _fusedtok.quantize_launch_ex(x.data_ptr(), _DT_CODE[x.dtype],
                                         q.data_ptr(), scale.data_ptr(),
                                         x.numel(), _stream())
        if device_scale:
            return q, scale
        return q, float(scale)
    arr = _host_f32(x, "x")
    dev = _need_device()
    q, s = quantize_int8(_upload(arr, dev))
    return (q.cpu() if _is_torch(x) else q.cpu().numpy()), s


def _dev_scale(s, name):
    """Python float -> (float, None); 1-element GPU float32 tensor -> (0.0, ptr)."""
    if _on_gpu(s):
        if s.dtype is not torch.float32 or s.numel() != 1:
            raise TypeError(f"a device {name} must be a 1-element float32 tensor")
        return 0.0, s.data_ptr()
    if _is_torch(s):
        s = s.item()
    return float(s), None


def dequantize_int8(q, scale, *, out_dtype=None):
    """Dequantize int8: ``x = q * scale`` in float32 (one rounding).

    Takes the UNPACKED pair from :func:`quantize_int8`
    (``dequantize_int8(*quantize_int8(x))``), as the reference
    (``__init__.py:1428-1449``). Build additions: ``scale`` may be the
    1-element GPU tensor of ``quantize_int8(..., device_scale=True)``, and
    ``out_dtype`` bf16 / fp16 stores the float32 value rounded to
    nearest-even (GPU path).
    """
    if _on_gpu(q):
        if q.dtype is not torch.int8:
            raise TypeError(f"q must be int8, got {q.dtype}")
        _check_contiguous(q, "q")
        odt = torch.float32 if out_dtype is None else out_dtype
        if odt not in _DT_CODE:
            raise TypeError("out_dtype must be float32, bfloat16 or float16")
        sc, sc_ptr = _dev_scale(scale, "scale")
        x = torch.empty(q.shape, dtype=odt, device=q.device)
        if q.numel():
            if odt is torch.float32 and sc_ptr is None:
                _fusedtok.dequantize_launch(q.data_ptr(), x.data_ptr(), sc, q.numel(),
                                            _stream())
            else:
                _fusedtok.dequantize_launch_ex(q.data_ptr(), sc, sc_ptr, x.data_ptr(),
                                               _DT_CODE[odt], q.numel(), _stream())
        return x
    if _is_torch(q):
        if q.dtype is not torch.int8:
            raise TypeError(f"q must be int8, got {q.dtype}")
        arr = q.detach().numpy()
    else:
        arr = np.asarray(q)
        if arr.size and not np.issubdtype(arr.dtype, np.integer):
            raise TypeError(f"q must be int8, got {arr.dtype}")
    dev = _need_device()
    x = dequantize_int8(_upload(np.ascontiguousarray(arr, dtype=np.int8), dev),
                        float(scale))
    return _result(x, q)


def qadd_int8(qa, sa, qb, sb, *, device_scale=False):
    """Fused dequantize-add-requantize of two int8 tensors:
    ``v = f32(qa * sa) + f32(qb * sb)``, requantized with v's own per-tensor
    scale. Returns ``(qy, out_scale)``, equal bit for bit to
    ``quantize_int8(dequantize_int8(qa, sa) + dequantize_int8(qb, sb))``.
    GPU int8 tensors only (TypeError otherwise, as the reference's
    ``__init__.py:1452-1473``). Build additions: ``sa`` / ``sb`` may be
    1-element GPU float32 tensors, and ``device_scale=True`` returns
    out_scale as one without synchronising the stream.
    """
    if not (_on_gpu(qa) and _on_gpu(qb)):
        raise TypeError("qadd_int8 needs GPU int8 tensors")
    if qa.dtype is not torch.int8 or qb.dtype is not torch.int8:
        raise TypeError("inputs must be int8")
    _check_contiguous(qa, "qa")
    _check_contiguous(qb, "qb")
    if qa.shape != qb.shape:
        raise ValueError("inputs must have the same shape")
    fa, pa = _dev_scale(sa, "sa")
    fb, pb = _dev_scale(sb, "sb")
    qy = torch.empty(qa.shape, dtype=torch.int8, device=qa.device)
    out_scale = torch.empty(1, dtype=torch.float32, device=qa.device)
    n = qa.numel()
    if n == 0:
        out_scale.fill_(1.0)   # no values: the all-zero scale
    elif pa is None and pb is None:
        _fusedtok.qadd_launch(qa.data_ptr(), qb.data_ptr(), fa, fb, qy.data_ptr(),
                              out_scale.data_ptr(), n, _stream())
    else:
        _fusedtok.qadd_launch_ex(qa.data_ptr(), qb.data_ptr(), fa, fb, pa, pb,
                                 qy.data_ptr(), out_scale.data_ptr(), n, _stream())
    if device_scale:
        return qy, out_scale
    return qy, float(out_scale)


# ---------------------------------------------------------------------------
# fused decode-chain steps (build additions; GPU tensors only). The
# reference runs these as separate ops (rmsnorm -> quantize_int8,
# swiglu -> quantize_int8, rope -> kv_append_paged); each fused op returns
# exactly what this library's unfused chain returns.
# ---------------------------------------------------------------------------


def _gpu_only(t, name):
    if not _on_gpu(t):
        raise TypeError(f"{name} must be a GPU tensor (fused ops have no "
                        "host path)")


def rmsnorm_quant(x, weight, *, residual=None, eps=1e-6, device_scale=False):
    """``quantize_int8(rmsnorm(x, weight, residual=residual, eps=eps))`` with
    the RMSNorm output kept in float32 registers: returns ``(q, scale)``, q
    int8 of x's shape, bit-identical to the unfused float32 chain. cols must
    be a multiple of 4. ``device_scale=True`` returns the scale as a
    1-element GPU float32 tensor without synchronising."""
    _gpu_only(x, "x")
    _check_dtype(x, "x", _FLOAT_DTYPES)
    _require_gpu(weight, "weight")
    if weight.dtype is not torch.float32:
        weight = weight.to(torch.float32)
    if not weight.is_contiguous():
        weight = weight.contiguous()
    rows, cols = _rows_cols(x.shape)
    if weight.ndim != 1 or weight.numel() != cols:
        raise ValueError("weight must be 1-D with cols entries")
    r_ptr = None
    if residual is not None:
        _require_gpu(residual, "residual")
        _check_dtype(residual, "residual", _FLOAT_DTYPES)
        if residual.dtype is not x.dtype:
            raise TypeError("residual must have the same dtype as x")
        if residual.shape != x.shape:
            raise ValueError("residual must have the same shape as x")
        r_ptr = residual.data_ptr()
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    # the kernel writes the scale; an empty input has none to compute (1.0,
    # as quantize_int8), set here so the common path launches no fill kernel
    scale = torch.empty(1, dtype=torch.float32, device=x.device)
    if rows == 0:
        scale.fill_(1.0)
    _fusedtok.rmsnorm_quant_launch(x.data_ptr(), _DT_CODE[x.dtype],
                                   weight.data_ptr(), r_ptr, q.data_ptr(),
                                   scale.data_ptr(), rows, cols, float(eps),
                                   _stream())
    return (q, scale) if device_scale else (q, float(scale))


def rmsnorm_qgemm(x, weight, b_q, b_scales, *, residual=None, eps=1e-6, out_dtype=None):
    """BASELINE config 2's chain in one call: ``q, s = rmsnorm_quant(x,
    weight, residual=residual, eps=eps)`` then ``qgemm_perchannel(q, s, b_q,
    b_scales, out_dtype=out_dtype)``, bit for bit. Returns ``(y, q, scale)``
    with the scale a 1-element GPU float32 tensor (no synchronisation). One
    row with K <= 4096 runs as one launch (every workgroup of the GEMV
    normalises and quantises the row itself); other shapes run the two
    ops. ``b_scales`` per-channel [N] (a float for per-tensor)."""
    _gpu_only(x, "x")
    _check_dtype(x, "x", _FLOAT_DTYPES)
    _require_gpu(weight, "weight")
    if weight.dtype is not torch.float32:
        weight = weight.to(torch.float32)
    if not weight.is_contiguous():
        weight = weight.contiguous()
    if not x.is_contiguous():
        x = x.contiguous()
    rows, k = _rows_cols(x.shape)
    if weight.ndim != 1 or weight.numel() != k:
        raise ValueError("weight must be 1-D with K entries")
    if k % 4 != 0:
        raise ValueError("rmsnorm_qgemm: K must be a multiple of 4")
    _require_gpu(b_q, "b_q")
    if b_q.dtype is not torch.int8 or b_q.ndim != 2 or b_q.shape[1] != k:
        raise ValueError("b_q must be int8 [N, K]")
    if not b_q.is_contiguous():
        b_q = b_q.contiguous()
    n = b_q.shape[0]
    sb_vec, sb = None, 0.0
    if _is_torch(b_scales) or isinstance(b_scales, (list, tuple, np.ndarray)):
        if not _is_torch(b_scales):
            b_scales = torch.as_tensor(np.asarray(b_scales, dtype=np.float32), device=x.device)
        if b_scales.ndim != 1 or b_scales.numel() != n:
            raise ValueError("b_scales must be 1-D with N entries")
        b_scales = b_scales.to(device=x.device, dtype=torch.float32).contiguous()
        sb_vec = b_scales.data_ptr()
    else:
        sb = float(b_scales)
    r_ptr = None
    if residual is not None:
        _require_gpu(residual, "residual")
        if residual.dtype is not x.dtype or residual.shape != x.shape:
            raise ValueError("residual must match x in dtype and shape")
        if not residual.is_contiguous():
            residual = residual.contiguous()   # kept alive until the launch
        r_ptr = residual.data_ptr()
    odt = torch.float32 if out_dtype is None else out_dtype
    if odt not in _OUT_CODES:
        raise TypeError("out_dtype must be float32, bfloat16 or float16")
    y = torch.empty((rows, n), dtype=odt, device=x.device)
    q = torch.empty((rows, k), dtype=torch.int8, device=x.device)
    scale = torch.empty(1, dtype=torch.float32, device=x.device)
    if rows == 0:
        scale.fill_(1.0)
        return y, q, scale
    _fusedtok.rmsnorm_qgemm_launch(x.data_ptr(), _DT_CODE[x.dtype], weight.data_ptr(), r_ptr,
                                   float(eps), b_q.data_ptr(), sb_vec, sb, y.data_ptr(),
                                   _OUT_CODES[odt], q.data_ptr(), scale.data_ptr(), rows, n,
                                   k, _stream())
    return y, q, scale


def swiglu_quant(gate, up, *, device_scale=False):
    """``quantize_int8(swiglu(gate, up))`` without the float intermediate:
    returns ``(q, scale)`` with q a dense int8 [rows, cols]. gate and up are
    [rows, cols] (or 1-D) GPU tensors of one dtype whose rows may be strided
    alike, e.g. ``h[:, :f]`` and ``h[:, f:]`` of one gate|up GEMM output."""
    _gpu_only(gate, "gate")
    _require_gpu(up, "up")
    for name, t in (("gate", gate), ("up", up)):
        if t.dtype not in _FLOAT_DTYPES:
            raise TypeError(f"{name} must be float32, bfloat16 or float16")
    if up.dtype is not gate.dtype:
        raise TypeError("up must have the same dtype as gate")
    if gate.shape != up.shape:
        raise ValueError("gate and up must have the same shape")
    if gate.ndim == 1:
        gate, up = gate.reshape(1, -1), up.reshape(1, -1)
    if gate.ndim != 2:
        raise ValueError("gate and up must be 1-D or 2-D")
    rows, cols = gate.shape
    ld = gate.stride(0) if rows > 1 else cols
    if rows > 0 and cols > 0:
        if gate.stride(1) != 1 or up.stride(1) != 1 or \
                (rows > 1 and up.stride(0) != ld):
            raise ValueError("gate and up must have unit column stride and "
                             "the same row stride")
    q = torch.empty((rows, cols), dtype=torch.int8, device=gate.device)
    scale = torch.empty(1, dtype=torch.float32, device=gate.device)
    if rows * cols == 0:
        scale.fill_(1.0)
    _fusedtok.swiglu_quant_launch(gate.data_ptr(), up.data_ptr(),
                                  _DT_CODE[gate.dtype], q.data_ptr(),
                                  scale.data_ptr(), rows, cols, ld, _stream())
    return (q, scale) if device_scale else (q, float(scale))


def rope_kv_append_paged(qkv, q_heads, kv_heads, k_pool, v_pool, block_table,
                         lens, *, theta=10000.0, pos_offset=0, neox=False):
    """The decode token's RoPE and paged KV append in one launch.

    qkv: [B, (q_heads + 2 * kv_heads) * D] (rows may be strided), holding
    each sequence's q heads, then its k heads, then its v heads. Sequence b's
    token sits at position ``lens[b] + pos_offset``: returns the rotated q
    [B, q_heads, D]; the rotated k heads and the v heads are written in place
    into slot ``lens[b]`` of the pools [Nb, kv_heads, P, D]. Equal to
    ``rope(q, positions=lens)`` plus ``kv_append_paged(..., rope(k), v, lens)``.
    lens is not advanced."""
    _gpu_only(qkv, "qkv")
    for name, t in (("qkv", qkv), ("k_pool", k_pool), ("v_pool", v_pool)):
        _require_gpu(t, name)
        if t.dtype not in _FLOAT_DTYPES:
            raise TypeError(f"{name} must be float32, bfloat16 or float16")
    for name, t in (("k_pool", k_pool), ("v_pool", v_pool)):
        if t.dtype is not qkv.dtype:
            raise TypeError(f"{name} must have the qkv dtype")
        _check_contiguous(t, name)
    if int(q_heads) < 1 or int(kv_heads) < 1:
        raise ValueError("q_heads and kv_heads must be >= 1")
    if q_heads % kv_heads:
        raise ValueError("q_heads must be a multiple of kv_heads")
    if k_pool.ndim != 4 or v_pool.shape != k_pool.shape:
        raise ValueError("pools must be [Nb, Hkv, P, D] of one shape")
    nb, hkv, page, d = k_pool.shape
    if hkv != kv_heads:
        raise ValueError("kv_heads must equal the pools' head count")
    if qkv.ndim != 2 or qkv.shape[1] != (q_heads + 2 * kv_heads) * d:
        raise ValueError("qkv must be [B, (q_heads + 2 * kv_heads) * D]")
    if d % 2:
        raise ValueError("dim must be even (RoPE pairs elements)")
    if int(pos_offset) < 0:
        raise ValueError("pos_offset must be >= 0")
    b = qkv.shape[0]
    q_out = torch.empty((b, q_heads, d), dtype=qkv.dtype, device=qkv.device)
    if b == 0:
        return q_out
    if qkv.stride(1) != 1:
        raise ValueError("qkv rows must be contiguous")
    bt = _table_tensor(block_table, b, nb, qkv.device)
    lt = _lens_tensor(lens, b, bt.shape[1] * page, qkv.device,
                      upper_inclusive=False)
    _fusedtok.rope_kv_append_paged_launch(
        qkv.data_ptr(), _DT_CODE[qkv.dtype], qkv.stride(0) if b > 1 else qkv.shape[1],
        lt.data_ptr(), bt.data_ptr(), q_out.data_ptr(), k_pool.data_ptr(),
        v_pool.data_ptr(), b, q_heads, kv_heads, d, page, bt.shape[1],
        float(theta), int(pos_offset), bool(neox), _stream())
    return q_out


def _qgemm_gpu_operands(a_q, b_q):
    if not _on_gpu(b_q):
        raise TypeError("both operands must be GPU int8 tensors")
    if a_q.dtype is not torch.int8 or b_q.dtype is not torch.int8:
        raise TypeError("operands must be int8")
    _check_contiguous(a_q, "a_q")
    _check_contiguous(b_q, "b_q")
    if a_q.ndim != 2 or b_q.ndim != 2:
        raise ValueError("operands must be 2-D [rows, K]")
    m, k = a_q.shape
    n, k2 = b_q.shape
    if k != k2:
        raise ValueError("inner dimensions must match")
    return m, n, k


def _int8_host(arr, name):
    if _is_torch(arr):
        if arr.is_cuda:
            raise TypeError(f"{name} must be a host tensor on this path")
        arr = arr.detach().numpy()
    a = np.asarray(arr)
    if a.size and not np.issubdtype(a.dtype, np.integer):
        raise TypeError(f"{name} must be an integer array, got {a.dtype}")
    return np.ascontiguousarray(a, dtype=np.int8)


_OUT_CODES = {torch.float32: _DT_F32, torch.bfloat16: _DT_BF16,
              torch.float16: _DT_F16}


def _scale_arg(a_scale, device):
    """Host float -> (float, None); GPU tensor -> (0.0, device pointer)."""
    if _on_gpu(a_scale):
        t = a_scale
        if t.dtype is not torch.float32 or t.numel() != 1:
            raise TypeError("a device a_scale must be a 1-element float32 tensor")
        return 0.0, t
    return float(a_scale), None


def qgemm(a_q, a_scale, b_q, b_scale, *, cuda=False, out_dtype=None):
    """INT8 matmul, exact int32 accumulation:
    ``y[M, N] = (A_q[M, K] @ B_q[N, K]^T) * f32(a_scale * b_scale)``.

    Output float32 (build addition: ``out_dtype`` bf16 / fp16 on the GPU
    path, the float32 value rounded to nearest-even; ``a_scale`` may be a
    1-element GPU tensor, e.g. from ``quantize_int8(..., device_scale=True)``).
    """
    if _on_gpu(a_q):
        m, n, k = _qgemm_gpu_operands(a_q, b_q)
        odt = torch.float32 if out_dtype is None else out_dtype
        if odt not in _OUT_CODES:
            raise TypeError("out_dtype must be float32, bfloat16 or float16")
        y = torch.empty((m, n), dtype=odt, device=a_q.device)
        sa, sa_t = _scale_arg(a_scale, a_q.device)
        if m > 0 and n > 0:
            if odt is torch.float32 and sa_t is None:
                _fusedtok.qgemm_launch(a_q.data_ptr(), b_q.data_ptr(), y.data_ptr(),
                                       m, n, k, sa, float(b_scale), _stream())
            else:
                _fusedtok.qgemm_launch_ex(
                    a_q.data_ptr(), b_q.data_ptr(), None, float(b_scale), sa,
                    None if sa_t is None else sa_t.data_ptr(), y.data_ptr(),
                    _OUT_CODES[odt], m, n, k, _stream())
        return y
    a = _int8_host(a_q, "a_q")
    b = _int8_host(b_q, "b_q")
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("operands must be 2-D [rows, K]")
    if a.shape[1] != b.shape[1]:
        raise ValueError("inner dimensions must match")
    dev = _need_device()
    y = qgemm(_upload(a, dev), float(a_scale), _upload(b, dev), float(b_scale))
    return _result(y, a_q)


def qgemm_perchannel(a_q, a_scale, b_q, b_scales, *, cuda=False, out_dtype=None):
    """INT8 matmul with per-output-channel weight scales (W8A8):
    ``y[M, N] = (A_q @ B_q^T) * f32(a_scale * b_scales[j])``; bit-identical to
    the reference CPU path in float32. Build additions as in :func:`qgemm`.
    """
    if _on_gpu(a_q):
        m, n, k = _qgemm_gpu_operands(a_q, b_q)
        if not _is_torch(b_scales):
            b_scales = torch.as_tensor(np.asarray(b_scales, dtype=np.float32),
                                       device=a_q.device)
        if b_scales.ndim != 1 or b_scales.numel() != n:
            raise ValueError("b_scales must be 1-D with n entries")
        if b_scales.dtype is not torch.float32:
            b_scales = b_scales.to(torch.float32)
        if not b_scales.is_contiguous():
            b_scales = b_scales.contiguous()
        if not b_scales.is_cuda:
            b_scales = b_scales.to(a_q.device)
        odt = torch.float32 if out_dtype is None else out_dtype
        if odt not in _OUT_CODES:
            raise TypeError("out_dtype must be float32, bfloat16 or float16")
        y = torch.empty((m, n), dtype=odt, device=a_q.device)
        sa, sa_t = _scale_arg(a_scale, a_q.device)
        if m > 0 and n > 0:
            if odt is torch.float32 and sa_t is None:
                _fusedtok.qgemm_perchannel_launch(
                    a_q.data_ptr(), b_q.data_ptr(), b_scales.data_ptr(),
                    y.data_ptr(), m, n, k, sa, _stream())
            else:
                _fusedtok.qgemm_launch_ex(
                    a_q.data_ptr(), b_q.data_ptr(), b_scales.data_ptr(), 0.0, sa,
                    None if sa_t is None else sa_t.data_ptr(), y.data_ptr(),
                    _OUT_CODES[odt], m, n, k, _stream())
        return y
    a = _int8_host(a_q, "a_q")
    b = _int8_host(b_q, "b_q")
    sb = np.ascontiguousarray(np.asarray(b_scales, dtype=np.float32))
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("operands must be 2-D [rows, K]")
    if a.shape[1] != b.shape[1]:
        raise ValueError("inner dimensions must match")
    if sb.ndim != 1 or sb.shape[0] != b.shape[0]:
        raise ValueError("b_scales must be 1-D with n entries")
    dev = _need_device()
    y = qgemm_perchannel(_upload(a, dev), float(a_scale), _upload(b, dev),
                         _upload(sb, dev))
    return _result(y, a_q)


def qgemm_i32(a_q, b_q):
    """Build addition (test hook): the exact int32 accumulators
    ``A_q @ B_q^T`` through the same kernels as the float paths."""
    if _on_gpu(a_q):
        m, n, k = _qgemm_gpu_operands(a_q, b_q)
        acc = torch.empty((m, n), dtype=torch.int32, device=a_q.device)
        if m > 0 and n > 0:
            _fusedtok.qgemm_i32_launch(a_q.data_ptr(), b_q.data_ptr(),
                                       acc.data_ptr(), m, n, k, _stream())
        return acc
    a = _int8_host(a_q, "a_q")
    b = _int8_host(b_q, "b_q")
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[1]:
        raise ValueError("operands must be 2-D [rows, K] with matching K")
    dev = _need_device()
    return _result(qgemm_i32(_upload(a, dev), _upload(b, dev)), a_q)


# ---------------------------------------------------------------------------
# post-logits sampling (reference __init__.py:1120-1176, 1602-1632,
# 2292-2316, 2366-2540; sampling.cu, topk.cu)
# ---------------------------------------------------------------------------


def _logits_f32(t, name="logits"):
    if not t.is_cuda:
        raise TypeError(f"{name} must be a GPU tensor (got a CPU tensor on the "
                        "zero-copy path)")
    if t.dtype is not torch.float32:
        raise TypeError(f"{name} must be float32, got {t.dtype}")
    _check_contiguous(t, name)


def _sampling_params(p, temperature, penalty=1.0):
    if not penalty > 0.0:
        raise ValueError("penalty must be > 0")
    if not 0.0 < p <= 1.0:
        raise ValueError("p must be in (0, 1]")
    if not temperature > 0.0:
        raise ValueError("temperature must be > 0")


def _host_logits(x, ndim, what):
    arr = _host_f32(x, "logits")
    if arr.ndim != ndim:
        raise ValueError(what)
    return arr


def _ids_arg(ids, vocab, device, name="sampled_ids"):
    """1-D int64 ids on `device`: host values range-checked against
    [0, vocab) (ValueError); a GPU tensor is trusted (the kernels drop
    out-of-range entries) - the reference's boundary (__init__.py:322-343)."""
    if _on_gpu(ids):
        it = ids if ids.dtype is torch.int64 else ids.to(torch.int64)
        if not it.is_contiguous():
            it = it.contiguous()
        if it.ndim != 1:
            raise ValueError(f"{name} must be 1-D")
        return it
    host = _host_int_array(ids, name)
    host = np.ascontiguousarray(host, dtype=np.int64)
    if host.ndim != 1:
        raise ValueError(f"{name} must be 1-D")
    if host.size and (host.min() < 0 or host.max() >= vocab):
        raise ValueError(f"{name} values must be in [0, {vocab})")
    return torch.from_numpy(host).to(device)


def _batch_seeds(seeds, rows, name="seeds"):
    """None -> 0..rows-1; else one non-negative integer per row
    (reference __init__.py:370-395)."""
    if seeds is None:
        return np.arange(rows, dtype=np.int64)
    if _is_torch(seeds):
        seeds = seeds.detach().cpu().numpy()
    arr = np.asarray(seeds)
    if arr.dtype.kind not in "iu":
        raise TypeError(f"{name} must contain integers")
    if arr.ndim != 1:
        raise ValueError(f"{name} must be 1-D")
    if arr.shape[0] != rows:
        raise ValueError(f"{name} must have one entry per row")
    out = np.ascontiguousarray(arr, dtype=np.int64)
    if out.size and out.min() < 0:
        raise ValueError(f"{name} values must be in [0, 2**63)")
    return out


def _batch_ids(sampled_ids, ids_offsets, rows, n):
    """Per-row histories -> (flat int64 ids, int64 offsets), host side:
    ragged sequences, a 2-D array (every row contributes all columns), or
    flat ids plus ids_offsets (reference __init__.py:2415-2481)."""
    if ids_offsets is not None:
        if _is_torch(sampled_ids):
            sampled_ids = sampled_ids.detach().cpu().numpy()
        if _is_torch(ids_offsets):
            ids_offsets = ids_offsets.detach().cpu().numpy()
        ids = np.ascontiguousarray(sampled_ids)
        if ids.ndim != 1:
            raise ValueError("sampled_ids with ids_offsets must be a flat 1-D array")
        offs = np.ascontiguousarray(ids_offsets)
        if offs.ndim != 1 or offs.size != rows + 1:
            raise ValueError("ids_offsets must be 1-D with rows + 1 entries")
        if ids.size and not np.issubdtype(ids.dtype, np.integer):
            raise TypeError("sampled_ids entries must be integers")
        if offs.size and not np.issubdtype(offs.dtype, np.integer):
            raise TypeError("ids_offsets entries must be integers")
        ids = ids.astype(np.int64, copy=False)
        offs = offs.astype(np.int64, copy=False)
        if offs[0] != 0 or offs[-1] != ids.size or (np.diff(offs) < 0).any():
            raise ValueError("ids_offsets must start at 0, end at len(sampled_ids) "
                             "and be non-decreasing")
    elif isinstance(sampled_ids, (list, tuple)):
        if len(sampled_ids) != rows:
            raise ValueError("sampled_ids must have one entry per row")
        flat, offs = [], [0]
        for row_ids in sampled_ids:
            row = np.asarray(row_ids)
            if row.size and not np.issubdtype(row.dtype, np.integer):
                raise TypeError("sampled_ids entries must be integers")
            flat.extend(int(i) for i in row.reshape(-1))
            offs.append(len(flat))
        ids = np.asarray(flat, dtype=np.int64)
        offs = np.asarray(offs, dtype=np.int64)
    else:
        arr = sampled_ids
        if _is_torch(arr):
            arr = arr.detach().cpu().numpy()
        arr = np.asarray(arr)
        if arr.ndim != 2:
            raise ValueError("sampled_ids must be per-row sequences, a 2-D array, "
                             "or flat ids plus ids_offsets")
        if arr.shape[0] != rows:
            raise ValueError("sampled_ids must have one entry per row")
        if arr.size and not np.issubdtype(arr.dtype, np.integer):
            raise TypeError("sampled_ids entries must be integers")
        ids = np.ascontiguousarray(arr, dtype=np.int64).reshape(-1)
        offs = np.arange(rows + 1, dtype=np.int64) * arr.shape[1]
    if ids.size and (ids.min() < 0 or ids.max() >= n):
        raise ValueError(f"sampled_ids values must be in [0, {n})")
    return ids, offs


def argmax(x, *, cuda=False):
    """Index of the largest element (earliest index on ties)."""
    if _on_gpu(x):
        _logits_f32(x, "x")
        if x.ndim != 1:
            raise ValueError("x must be 1-D for argmax")
        if x.numel() == 0:
            raise ValueError("argmax of empty input")
        out = torch.empty(1, dtype=torch.int32, device=x.device)
        _fusedtok.argmax_launch(x.data_ptr(), x.numel(), out.data_ptr(), _stream())
        return int(out.item())
    arr = _host_f32(x, "x")
    if arr.ndim != 1:
        raise ValueError("x must be 1-D for argmax")
    if arr.size == 0:
        raise ValueError("argmax of empty input")
    return argmax(_upload(arr, _need_device()))


def argmax_batched(x, *, cuda=False):
    """Row-wise argmax of ``[rows, vocab]`` float32 logits, earliest index on
    ties; one launch. GPU input: an int64 GPU tensor, no host sync."""
    if _on_gpu(x):
        _logits_f32(x, "x")
        if x.ndim != 2:
            raise ValueError("x must be 2-D [rows, vocab] for argmax_batched")
        if x.shape[1] == 0:
            raise ValueError("argmax of empty input")
        rows, n = x.shape
        out = torch.empty(rows, dtype=torch.int64, device=x.device)
        if rows:
            _fusedtok.argmax_batched_launch(x.data_ptr(), rows, n, out.data_ptr(), _stream())
        return out
    arr = _host_f32(x, "x")
    if arr.ndim != 2:
        raise ValueError("x must be 2-D [rows, vocab] for argmax_batched")
    if arr.shape[1] == 0:
        raise ValueError("argmax of empty input")
    return _result(argmax_batched(_upload(arr, _need_device())), x)


def sample_topp(logits, p, *, temperature=1.0, seed=0, cuda=False):
    """Fused nucleus sampling: softmax of ``logits / temperature``, truncated
    to the smallest top-p nucleus, inverse-CDF draw at a splitmix hash
    uniform of ``seed``. Deterministic per seed. Returns the token id."""
    _sampling_params(p, temperature)
    if _on_gpu(logits):
        _logits_f32(logits)
        if logits.ndim != 1:
            raise ValueError("logits must be 1-D")
        if logits.numel() == 0:
            raise ValueError("sample of empty logits")
        out = torch.empty(1, dtype=torch.int64, device=logits.device)
        _fusedtok.sample_topp_launch(logits.data_ptr(), logits.numel(), float(p),
                                     float(temperature), int(seed), out.data_ptr(), _stream())
        return int(out.item())
    arr = _host_logits(logits, 1, "logits must be 1-D")
    if arr.size == 0:
        raise ValueError("sample of empty logits")
    return sample_topp(_upload(arr, _need_device()), p, temperature=temperature, seed=seed)


def _seeds_dev(seeds, rows, device):
    s = _batch_seeds(seeds, rows)
    return _upload_i64([s], device)[0]   # int64 bits = the uint64 seeds


def sample_topp_batched(logits, p, *, temperature=1.0, seeds=None, cuda=False,
                        device_out=False):
    """Nucleus sampling of every row of ``[rows, vocab]`` float32 logits (each
    row split across CUs when there are fewer rows than CUs). ``seeds``: one
    per row (None: 0..rows-1).
    Returns int64 tokens on the host (the reference's contract); build
    addition ``device_out=True`` returns them as a GPU tensor, no sync."""
    _sampling_params(p, temperature)
    if _on_gpu(logits):
        _logits_f32(logits)
        if logits.ndim != 2:
            raise ValueError("logits must be 2-D [rows, vocab]")
        rows, n = logits.shape
        sd = _seeds_dev(seeds, rows, logits.device)
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
        if rows:
            if n == 0:
                raise ValueError("sample of empty logits")
            _fusedtok.sample_topp_batched_launch(logits.data_ptr(), rows, n, float(p),
                                                 float(temperature), sd.data_ptr(),
                                                 out.data_ptr(), _stream())
        return out if device_out else out.cpu()
    arr = _host_logits(logits, 2, "logits must be 2-D [rows, vocab]")
    res = sample_topp_batched(_upload(arr, _need_device()), p, temperature=temperature,
                              seeds=seeds)
    return res if _is_torch(logits) else res.numpy()


def decode_step(logits, sampled_ids, penalty=1.0, *, p=0.9, temperature=1.0, seed=0,
                cuda=False):
    """Fused decode step: CTRL repetition penalty over ``sampled_ids`` (each
    distinct id once), then ``/ temperature``, then nucleus sampling, in one
    launch. Returns the token id; deterministic per seed."""
    _sampling_params(p, temperature, penalty)
    if _on_gpu(logits):
        _logits_f32(logits)
        if logits.ndim != 1:
            raise ValueError("logits must be 1-D")
        n = logits.numel()
        if n == 0:
            raise ValueError("sample of empty logits")
        ids = _ids_arg(sampled_ids, n, logits.device)
        out = torch.empty(1, dtype=torch.int64, device=logits.device)
        _fusedtok.decode_step_launch(logits.data_ptr(), ids.data_ptr() if ids.numel() else None,
                                     n, ids.numel(), float(penalty), float(p),
                                     float(temperature), int(seed), out.data_ptr(), _stream())
        return int(out.item())
    arr = _host_logits(logits, 1, "logits must be 1-D")
    if arr.size == 0:
        raise ValueError("sample of empty logits")
    dev = _need_device()
    ids = _ids_arg(sampled_ids, arr.size, dev)
    return decode_step(_upload(arr, dev), ids, penalty, p=p, temperature=temperature,
                       seed=seed)


def decode_step_batched(logits, sampled_ids, penalty=1.0, *, p=0.9, temperature=1.0,
                        seeds=None, ids_offsets=None, cuda=False, device_out=False):
    """The fused decode step for every row of ``[rows, vocab]`` float32
    logits (each row split across CUs when there are fewer rows than CUs).
    ``sampled_ids``: per-row histories (ragged sequences, a 2-D array, or
    flat ids with ``ids_offsets``). Returns int64 tokens on the host (the reference's
    contract); build addition ``device_out=True`` keeps them on the GPU."""
    _sampling_params(p, temperature, penalty)
    if _on_gpu(logits):
        _logits_f32(logits)
        if logits.ndim != 2:
            raise ValueError("logits must be 2-D [rows, vocab]")
        rows, n = logits.shape
        ids, offs = _batch_ids(sampled_ids, ids_offsets, rows, n)
        ids_t, offs_t, sd = _upload_i64([ids, offs, _batch_seeds(seeds, rows)],
                                        logits.device)
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
        if rows:
            if n == 0:
                raise ValueError("sample of empty logits")
            _fusedtok.decode_step_batched_launch(
                logits.data_ptr(), rows, n, ids_t.data_ptr() if ids.size else None,
                offs_t.data_ptr(), float(penalty), float(p), float(temperature),
                sd.data_ptr(), out.data_ptr(), _stream())
        return out if device_out else out.cpu()
    arr = _host_logits(logits, 2, "logits must be 2-D [rows, vocab]")
    res = decode_step_batched(_upload(arr, _need_device()), sampled_ids, penalty, p=p,
                              temperature=temperature, seeds=seeds, ids_offsets=ids_offsets)
    return res if _is_torch(logits) else res.numpy()
