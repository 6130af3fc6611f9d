"""fusedtok_amd: the fusedtok decode hot path, native to AMD MI355X (gfx950).

The public functions keep fusedtok 2.5.0's names, signatures and error
contract for the decode hot path (reference python/fusedtok/__init__.py,
stubs __init__.pyi:99-107,208-236):

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

How a call runs: each op states its operands once, as a contract
(``_contract.py``: symbolic shapes, element types, in-place operands, and
rules over the shape symbols). One validator checks every call against its
contract before any device work. GPU tensors then go to the HIP kernels
zero-copy, through ``data_ptr()`` on the current torch stream and without a
host sync. ``quantize_int8`` syncs once to return its Python float scale, as
the reference does. Host inputs (numpy arrays, CPU tensors) are uploaded,
run through the same op on the GPU, and brought back, which replaces both of
the reference's host paths; the ``cuda=`` keyword is accepted for
compatibility. There is no CPU fallback: without a HIP device, host inputs
raise RuntimeError. Errors follow the reference: TypeError for dtype /
device-family problems, ValueError for shapes and values, RuntimeError for
HIP failures. Device-resident ``lens`` and block tables are trusted (never
read back); host-origin ones are range-checked.

Build additions (not in the reference): fp16 storage for ``rmsnorm``,
``rope`` and ``swiglu``; bf16 / fp16 input to ``quantize_int8`` and a
device-resident scale (``device_scale=True``); bf16 / fp16 GEMM outputs
(``out_dtype=``) and a device scale operand; ``qgemm_i32`` (raw int32
accumulators); per-row RoPE positions (``positions=``); the fused
decode-chain steps ``rmsnorm_quant``, ``rmsnorm_qgemm``, ``swiglu_quant``
and ``rope_kv_append_paged`` (GPU tensors only).
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

from ._contract import FLOATS as _FLOATS
from ._contract import INT8 as _INT8
from ._contract import Arr as _Arr
from ._contract import Contract as _Contract
from ._contract import Idx as _Idx
from ._contract import Rule as _Rule
from . import _sampling_args as _sargs

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
    "attention_decode_paged_quant",
    "attention_decode_paged_append",
    "attention_prefill",
    "kv_append",
    "kv_append_paged",
    "rmsnorm_quant",
    "rmsnorm_qgemm",
    "swiglu_quant",
    "rope_kv_append_paged",
    "qgemm_rope_kv_append_paged",
    "qgemm_rmsnorm_quant",
    "qgemm_swiglu_quant",
    "DecodeLayer",
    "DecodeStack",
    "argmax",
    "argmax_batched",
    "sample_topp",
    "sample_topp_batched",
    "decode_step",
    "decode_step_batched",
]

# element-type codes of the C ABI (include/fusedtok_amd.h: FT_DT_*) and the
# name suffix of each storage type's pybind entry (reference bindings.cpp:
# `<op>_launch`, `<op>_launch_bf16`, `<op>_launch_fp16`)
_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
_SUFFIX = {torch.float32: "", torch.bfloat16: "_bf16", torch.float16: "_fp16"}


def _native(entry, dtype):
    return getattr(_fusedtok, entry + _SUFFIX[dtype])


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _out_dtype(out_dtype):
    dt = torch.float32 if out_dtype is None else out_dtype
    if dt not in _CODE:
        raise TypeError("out_dtype must be float32, bfloat16 or float16")
    return dt


def _scale_operand(s, what):
    """A scale given as a Python number or as a 1-element GPU float32 tensor
    (e.g. a device-resident quantize scale): returns (value, device pointer),
    one of them unused."""
    if torch.is_tensor(s) and s.is_cuda:
        if s.dtype is not torch.float32 or s.numel() != 1:
            raise TypeError(f"a device {what} must be a 1-element float32 tensor")
        return 0.0, s.data_ptr()
    return float(s.item() if torch.is_tensor(s) else s), None


def cuda_available():
    """True if a usable HIP device is present (reference fusedtok.cu:34-37)."""
    return _fusedtok.cuda_available()


# ---------------------------------------------------------------------------
# contracts shared by several ops
# ---------------------------------------------------------------------------

_HEADS = _Rule(lambda c: c.Hq >= 1 and c.Hkv >= 1, "head counts must be >= 1")
_GQA = _Rule(lambda c: c.Hq % c.Hkv == 0, "q heads must be a multiple of kv heads")
_PAGED_GROUP = _Rule(lambda c: c.Hq // c.Hkv in (1, 2, 4, 8, 16),
                     "paged decode supports GQA group sizes 1/2/4/8/16 "
                     "(use attention_decode otherwise)")
# the kernels check D themselves; a host call checks it before its upload
_DIM_HOST = _Rule(lambda c: c.D % 4 == 0 and c.D <= 512,
                  "dim must be a multiple of 4 and at most 512")
_DIM4_HOST = _Rule(lambda c: c.D % 4 == 0, "dim must be a multiple of 4")

_LENS_WHAT = "lens must be 1-D with batch entries"
_TABLE_WHAT = "block_table must be [B, S] with batch rows"


def _table(optional=False):
    return _Idx("block_table", "B S", lambda c: c.Nb, open_bound=True,
                optional=optional, what=_TABLE_WHAT)


# ---------------------------------------------------------------------------
# elementwise and row ops: swiglu, rmsnorm, rope
# ---------------------------------------------------------------------------

_SWIGLU = _Contract(
    _Arr("gate"),
    _Arr("up", "=gate", same_dtype="gate", mismatch="inputs must have the same shape"))


def swiglu(gate, up, *, cuda=False):
    """SwiGLU activation: ``silu(gate) * up`` = ``gate / (1 + exp(-gate)) * up``
    (reference ``__init__.py:537-539``, ``activations.cu:501-521``)."""
    c = _SWIGLU.bind(gate=gate, up=up)
    if not c.on_gpu:
        return c.staged(swiglu)
    out = torch.empty_like(c.gate)
    _native("swiglu_launch", c.gate.dtype)(c.ptr("gate"), c.ptr("up"), out.data_ptr(),
                                           c.gate.numel(), _stream())
    return out


_RMSNORM = _Contract(
    _Arr("x", "rows? cols", rank_msg="expected a 1-D or 2-D tensor"),
    _Arr("weight", "cols", (torch.float32,), upcast=True,
         mismatch="weight must be 1-D with cols entries"),
    _Arr("residual", "=x", same_dtype="x", optional=True,
         mismatch="residual must have the same shape as x"),
    rules=(_Rule(lambda c: c.cols > 0, "rows must be >= 0 and cols must be > 0"),))


def rmsnorm(x, weight, *, residual=None, eps=1e-6, cuda=False):
    """RMSNorm, optionally fused with a residual add:

    ``y = (x + r) * rsqrt(mean((x + r)^2) + eps) * weight``

    x: [rows, cols] or [cols]; weight: [cols] (float32; bf16/fp16 weights
    are upcast); residual: same shape and dtype as x (reference
    ``__init__.py:555-598``, ``rmsnorm.cu:110-153``).
    """
    c = _RMSNORM.bind(x=x, weight=weight, residual=residual)
    if not c.on_gpu:
        return c.staged(lambda **a: rmsnorm(a["x"], a["weight"], residual=a["residual"],
                                            eps=eps))
    out = torch.empty_like(c.x)
    _native("rmsnorm_launch", c.x.dtype)(c.ptr("x"), c.ptr("weight"), c.ptr("residual"),
                                         out.data_ptr(), c.rows, c.cols, float(eps),
                                         _stream())
    return out


_ROPE = _Contract(
    _Arr("q", "seq dim", rank_msg="q must be 2-D [seq, dim]"),
    _Arr("k", "=q", same_dtype="q", optional=True, mismatch="k must have the same shape as q"),
    rules=(_Rule(lambda c: c.dim % 2 == 0, "dim must be even (RoPE pairs elements)"),
           _Rule(lambda c: c.pos_offset >= 0, "pos_offset must be >= 0")))


def rope(q, k=None, *, theta=10000.0, pos_offset=0, neox=False, cuda=False,
         positions=None, rows_per_position=1):
    """Rotary position embedding on (q, k).

    q, k: [seq, dim] with even dim. ``neox=False`` rotates interleaved pairs
    (2j, 2j+1); ``neox=True`` rotates the row halves (j, j + dim/2). Row r
    sits at position ``r + pos_offset``; pair j turns by
    ``position * theta^(-2j/dim)``. Returns ``(q_rot, k_rot)`` (None if k is)
    (reference ``__init__.py:645-702``, ``rope.cu:175-345``).

    Build addition: ``positions`` (a GPU int32 vector) with
    ``rows_per_position`` places row r at ``positions[r // rows_per_position]
    + pos_offset`` - e.g. q viewed as [B*Hq, D] with ``rows_per_position=Hq``
    and per-sequence positions.
    """
    c = _ROPE.bind(q=q, k=k, pos_offset=pos_offset)
    if not c.on_gpu:
        return c.staged(lambda **a: rope(a["q"], a["k"], theta=theta,
                                         pos_offset=pos_offset, neox=neox))
    pos_ptr = None
    if positions is not None:
        if not (torch.is_tensor(positions) and positions.is_cuda):
            raise TypeError("positions must be a GPU tensor when the primary input is "
                            "on the GPU")
        if positions.dtype is not torch.int32:
            raise TypeError("positions must be int32")
        if not positions.is_contiguous():
            raise ValueError("positions must be contiguous")
        if rows_per_position < 1:
            raise ValueError("rows_per_position must be >= 1")
        if positions.numel() * rows_per_position < c.seq:
            raise ValueError("positions must cover every row")
        pos_ptr = positions.data_ptr()
    per_row = pos_ptr is not None or rows_per_position != 1
    rotated = []
    for src in (c.q, c.k):
        if src is None:
            rotated.append(None)
            continue
        dst = torch.empty_like(src)
        if per_row:
            _fusedtok.rope_launch_ex(src.data_ptr(), dst.data_ptr(), _CODE[src.dtype], c.seq,
                                     c.dim, float(theta), int(pos_offset), pos_ptr,
                                     int(rows_per_position), bool(neox), _stream())
        elif src.dtype is torch.float32:
            # the reference's f32 entry takes the layout flag first
            _fusedtok.rope_launch(bool(neox), src.data_ptr(), dst.data_ptr(), c.seq, c.dim,
                                  float(theta), int(pos_offset), _stream())
        else:
            entry = "rope_neox_launch" if neox else "rope_launch"
            _native(entry, src.dtype)(src.data_ptr(), dst.data_ptr(), c.seq, c.dim,
                                      float(theta), int(pos_offset), _stream())
        rotated.append(dst)
    return rotated[0], rotated[1]


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

_DECODE = _Contract(
    _Arr("q", "B Hq D"),
    _Arr("k_cache", "B Hkv T D", same_dtype="q",
         mismatch="k_cache/v_cache must match q's batch and dim"),
    _Arr("v_cache", "=k_cache", same_dtype="q",
         mismatch="k_cache/v_cache must match q's batch and dim"),
    _Idx("lens", "B", lambda c: c.T, optional=True, what=_LENS_WHAT),
    rank_msg="q must be [B, Hq, D]; k/v caches [B, Hkv, T, D]",
    rules=(_HEADS, _GQA), host_rules=(_DIM_HOST,))


def attention_decode(q, k_cache, v_cache, lens=None, *, cuda=False):
    """Single-token causal attention with GQA over a contiguous KV cache:

    ``out[b, h] = softmax(q[b,h] . K[b,kv(h)]^T / sqrt(D)) . V[b,kv(h)]``

    q: [B, Hq, D]; k_cache / v_cache: [B, Hkv, T, D]; lens: [B] valid lengths
    (<= T; None = all rows). q head h reads kv head ``h // (Hq // Hkv)``.
    Length-0 sequences give zero rows. Storage f32 / bf16 / fp16; softmax and
    accumulators are float32; the output matches the input dtype (reference
    ``__init__.py:710-788``, ``attention.cu:1468-1585``).
    """
    c = _DECODE.bind(q=q, k_cache=k_cache, v_cache=v_cache, lens=lens)
    if not c.on_gpu:
        return c.staged(attention_decode)
    out = torch.empty((c.B, c.Hq, c.D), dtype=c.q.dtype, device=c.device)
    if c.B * c.Hq:
        _native("attention_decode_launch", c.q.dtype)(
            c.ptr("q"), c.ptr("k_cache"), c.ptr("v_cache"), c.ptr("lens"), out.data_ptr(),
            c.B, c.Hq, c.Hkv, c.T, c.D, _stream())
    return out


_PREFILL = _Contract(
    _Arr("q", "B Hq S D"),
    _Arr("k", "B Hkv S D", same_dtype="q", mismatch="k/v must match q's batch, seq and dim"),
    _Arr("v", "=k", same_dtype="q", mismatch="k/v must match q's batch, seq and dim"),
    rank_msg="q/k/v must be [B, heads, S, D]",
    rules=(_HEADS, _GQA), host_rules=(_DIM_HOST,))


def attention_prefill(q, k, v, causal=True, *, cuda=False):
    """Prefill (fresh-sequence) attention over S query rows:

    ``out[b, h, i] = softmax(q[b,h,i] . K[b,kv(h)]^T / sqrt(D)) . V[b,kv(h)]``
    where query row i attends to key rows ``[0, i]`` (``causal=True``) or to
    all S rows (``causal=False``). q: [B, Hq, S, D]; k / v: [B, Hkv, S, D];
    out: [B, Hq, S, D] in q's dtype (f32 / bf16 / fp16 storage, float32
    softmax and accumulators). GQA as :func:`attention_decode`; D a multiple
    of 4, at most 512 (reference ``__init__.py:791-846``).
    """
    c = _PREFILL.bind(q=q, k=k, v=v)
    if not c.on_gpu:
        return c.staged(lambda **a: attention_prefill(a["q"], a["k"], a["v"], causal))
    out = torch.empty((c.B, c.Hq, c.S, c.D), dtype=c.q.dtype, device=c.device)
    if c.B * c.Hq * c.S:
        _native("attention_prefill_launch", c.q.dtype)(
            c.ptr("q"), c.ptr("k"), c.ptr("v"), out.data_ptr(), c.B, c.Hq, c.Hkv, c.S,
            c.D, bool(causal), _stream())
    return out


_DECODE_PAGED = _Contract(
    _Arr("q", "B Hq D"),
    _Arr("k_pool", "Nb Hkv P D", same_dtype="q",
         mismatch="pools must match q's dim and each other"),
    _Arr("v_pool", "=k_pool", same_dtype="q",
         mismatch="pools must match q's dim and each other"),
    _table(),
    _Idx("lens", "B", lambda c: c.S * c.P, optional=True, what=_LENS_WHAT),
    rank_msg="q must be [B, Hq, D]; pools [Nb, Hkv, P, D]",
    rules=(_HEADS, _GQA, _PAGED_GROUP), host_rules=(_DIM_HOST,))


def attention_decode_paged(q, k_pool, v_pool, block_table, lens=None, *,
                           cuda=False):
    """Single-token GQA attention over a PAGED KV cache.

    k_pool / v_pool: [Nb, Hkv, P, D]; block_table: [B, S] int; token t of
    sequence b is ``pool[block_table[b, t // P], kv, t % P]``; lens: [B]
    (None = S * P rows each). GQA group sizes 1/2/4/8/16. Host-origin table
    and lens values are validated; GPU-resident ones are trusted (reference
    ``__init__.py:849-940``, ``attention.cu:1791-1915``).
    """
    c = _DECODE_PAGED.bind(q=q, k_pool=k_pool, v_pool=v_pool, block_table=block_table,
                           lens=lens)
    if not c.on_gpu:
        return c.staged(attention_decode_paged)
    out = torch.empty((c.B, c.Hq, c.D), dtype=c.q.dtype, device=c.device)
    if c.B * c.Hq:
        _native("attention_decode_paged_launch", c.q.dtype)(
            c.ptr("q"), c.ptr("k_pool"), c.ptr("v_pool"), c.ptr("block_table"),
            c.ptr("lens"), out.data_ptr(), c.B, c.Hq, c.Hkv, c.P, c.S, c.D, _stream())
    return out


def attention_decode_paged_quant(q, k_pool, v_pool, block_table, lens=None, *,
                                 device_scale=False):
    """``out = attention_decode_paged(q, k_pool, v_pool, block_table, lens)``
    and ``quantize_int8(out)`` in one call, bit for bit: returns ``(out,
    codes, scale)`` with codes int8 of out's shape (the o_proj GEMM's input).
    On the split-stream attention path the attention kernels also keep the
    max |out| of each (sequence, head), so the quantize is a single launch.
    GPU tensors only; ``device_scale=True`` returns the scale as a 1-element
    GPU float32 tensor without synchronising. Build addition: the reference
    runs the two launches one after the other."""
    c = _DECODE_PAGED.bind(q=q, k_pool=k_pool, v_pool=v_pool, block_table=block_table,
                           lens=lens)
    if not c.on_gpu:
        raise TypeError("attention_decode_paged_quant takes GPU tensors (fused ops have no "
                        "host path)")
    out = torch.empty((c.B, c.Hq, c.D), dtype=c.q.dtype, device=c.device)
    codes = torch.empty((c.B, c.Hq, c.D), dtype=torch.int8, device=c.device)
    scale = torch.empty(1, dtype=torch.float32, device=c.device)
    if c.B * c.Hq == 0:
        scale.fill_(1.0)   # no values: the all-zero scale
    else:
        _fusedtok.attention_decode_paged_quant_launch(
            c.ptr("q"), c.ptr("k_pool"), c.ptr("v_pool"), c.ptr("block_table"),
            c.ptr("lens"), out.data_ptr(), _CODE[c.q.dtype], codes.data_ptr(),
            scale.data_ptr(), c.B, c.Hq, c.Hkv, c.P, c.S, c.D, _stream())
    return (out, codes, scale) if device_scale else (out, codes, float(scale))


# ---------------------------------------------------------------------------
# KV append (in place)
# ---------------------------------------------------------------------------

_NEW_KV_MISMATCH = "k/v operands must match the pool layout"

_APPEND_PAGED = _Contract(
    _Arr("k_pool", "Nb Hkv P D", inplace=True),
    _Arr("v_pool", "=k_pool", same_dtype="k_pool", inplace=True, mismatch=_NEW_KV_MISMATCH),
    _Arr("k_new", "B Hkv D", same_dtype="k_pool", mismatch=_NEW_KV_MISMATCH,
         rank_msg="k_new/v_new must be [B, Hkv, D]"),
    _Arr("v_new", "=k_new", same_dtype="k_pool", mismatch=_NEW_KV_MISMATCH),
    _table(),
    _Idx("lens", "B", lambda c: c.S * c.P, open_bound=True, what=_LENS_WHAT),
    rank_msg="pools must be [Nb, Hkv, P, D]", host_rules=(_DIM4_HOST,))


def kv_append_paged(k_pool, v_pool, block_table, k_new, v_new, lens, *,
                    cuda=False):
    """Write one fresh token's K/V rows per sequence into the paged pools,
    in place: ``k_new[b]`` lands at block ``block_table[b, lens[b] // P]``,
    offset ``lens[b] % P``. lens is required (values in [0, S*P)). Returns
    None (reference ``__init__.py:943-1027``, ``attention.cu:1924-1966``)."""
    c = _APPEND_PAGED.bind(k_pool=k_pool, v_pool=v_pool, k_new=k_new, v_new=v_new,
                           block_table=block_table, lens=lens)
    if c.B == 0:
        return None
    if not c.on_gpu:
        c.staged(kv_append_paged)
        return None
    _native("kv_append_paged_launch", c.k_pool.dtype)(
        c.ptr("k_new"), c.ptr("v_new"), c.ptr("block_table"), c.ptr("lens"),
        c.ptr("k_pool"), c.ptr("v_pool"), c.B, c.Hkv, c.D, c.P, c.S, _stream())
    return None


_DECODE_APPEND = _Contract(
    _Arr("q", "B Hq D"),
    _Arr("k_pool", "Nb Hkv P D", same_dtype="q", inplace=True,
         mismatch="pools must match q's dim and each other"),
    _Arr("v_pool", "=k_pool", same_dtype="q", inplace=True,
         mismatch="pools must match q's dim and each other"),
    _Arr("k_new", "B Hkv D", same_dtype="q", mismatch=_NEW_KV_MISMATCH,
         rank_msg="k_new/v_new must be [B, Hkv, D]"),
    _Arr("v_new", "=k_new", same_dtype="q", mismatch=_NEW_KV_MISMATCH),
    _table(),
    _Idx("lens", "B", lambda c: c.S * c.P, open_bound=True, what=_LENS_WHAT),
    rank_msg="q must be [B, Hq, D]; pools [Nb, Hkv, P, D]",
    rules=(_HEADS, _GQA, _PAGED_GROUP), host_rules=(_DIM_HOST,))


def attention_decode_paged_append(q, k_pool, v_pool, block_table, k_new, v_new, lens):
    """One decode step over a paged cache: ``kv_append_paged(k_pool, v_pool,
    block_table, k_new, v_new, lens)`` then ``attention_decode_paged(q,
    k_pool, v_pool, block_table, lens + 1)``, in one call (lens is not
    modified). GPU tensors only. For bf16 / fp16 with D = 128 the decode
    kernel attends the cached tokens and its combine kernel folds the fresh token into each row's log-sum-exp merge
    (in float32: the output equals the two ops' within the attention
    tolerance) and writes it into the pools (bit for bit), one launch
    fewer; other shapes run the two ops. Build addition: the
    reference runs the two ops (``attention.cu:1924-1966``, then
    ``attention.cu:1785-1900``)."""
    c = _DECODE_APPEND.bind(q=q, k_pool=k_pool, v_pool=v_pool, k_new=k_new, v_new=v_new,
                            block_table=block_table, lens=lens)
    if not c.on_gpu:
        raise TypeError("attention_decode_paged_append takes GPU tensors (fused ops have no "
                        "host path)")
    out = torch.empty((c.B, c.Hq, c.D), dtype=c.q.dtype, device=c.device)
    if c.B:
        _fusedtok.attention_decode_paged_append_launch(
            c.ptr("q"), c.ptr("k_pool"), c.ptr("v_pool"), c.ptr("block_table"),
            c.ptr("k_new"), c.ptr("v_new"), c.ptr("lens"), out.data_ptr(),
            _CODE[c.q.dtype], c.B, c.Hq, c.Hkv, c.P, c.S, c.D, _stream())
    return out


_APPEND = _Contract(
    _Arr("k_cache", "B Hkv T D", inplace=True),
    _Arr("v_cache", "=k_cache", same_dtype="k_cache", inplace=True,
         mismatch="k/v operands must match the cache layout"),
    _Arr("k_new", "B Hkv D", same_dtype="k_cache",
         mismatch="k/v operands must match the cache layout",
         rank_msg="k_new/v_new must be [B, Hkv, D]"),
    _Arr("v_new", "=k_new", same_dtype="k_cache",
         mismatch="k/v operands must match the cache layout"),
    _Idx("lens", "B", lambda c: c.T, open_bound=True, what=_LENS_WHAT),
    rank_msg="caches must be [B, Hkv, T, D]", host_rules=(_DIM4_HOST,))


def kv_append(k_cache, v_cache, k_new, v_new, lens, *, cuda=False):
    """Write one fresh token's K/V rows per sequence into the contiguous
    caches [B, Hkv, T, D] at row ``lens[b]`` (in place; lens in [0, T)).
    Returns None (reference ``__init__.py:1030-1112``,
    ``attention.cu:1985-2035``)."""
    c = _APPEND.bind(k_cache=k_cache, v_cache=v_cache, k_new=k_new, v_new=v_new, lens=lens)
    if c.B == 0:
        return None
    if not c.on_gpu:
        c.staged(kv_append)
        return None
    _native("kv_append_launch", c.k_cache.dtype)(
        c.ptr("k_new"), c.ptr("v_new"), c.ptr("lens"), c.ptr("k_cache"), c.ptr("v_cache"),
        c.B, c.Hkv, c.D, c.T, _stream())
    return None


# ---------------------------------------------------------------------------
# INT8: quantize, dequantize, qadd
# ---------------------------------------------------------------------------

_QUANT = _Contract(_Arr("x"))


def quantize_int8(x, *, device_scale=False):
    """Symmetric per-tensor INT8 quantization.

    ``scale = max(|x|) / 127`` (1.0 for all-zero input);
    ``q = clamp(rint(x * (1 / scale)), -127, 127)``. Returns ``(q, scale)``
    with scale a Python float (reference ``__init__.py:1402-1425``,
    ``quantize.cu:153-215``). Build additions: bf16 / fp16 GPU input, and
    ``device_scale=True`` returns the scale as a 1-element GPU float32 tensor
    without synchronising the stream.
    """
    c = _QUANT.bind(x=x)
    if not c.on_gpu:
        return c.staged(lambda **a: quantize_int8(a["x"]))
    q = torch.empty(c.x.shape, dtype=torch.int8, device=c.device)
    scale = torch.empty(1, dtype=torch.float32, device=c.device)
    n = c.x.numel()
    if n == 0:
        scale.fill_(1.0)   # no values: the all-zero scale
    if c.x.dtype is torch.float32:
        _fusedtok.quantize_launch(c.ptr("x"), q.data_ptr(), scale.data_ptr(), n, _stream())
    else:
        _fusedtok.quantize_launch_ex(c.ptr("x"), _CODE[c.x.dtype], q.data_ptr(),
                                     scale.data_ptr(), n, _stream())
    return (q, scale) if device_scale else (q, float(scale))


_DEQUANT = _Contract(_Arr("q", "*", _INT8, dtype_msg="q must be int8"))


def dequantize_int8(q, scale, *, out_dtype=None):
    """Dequantize int8: ``x = q * scale`` in float32 (one rounding).

    Takes the UNPACKED pair from :func:`quantize_int8`
    (``dequantize_int8(*quantize_int8(x))``), as the reference
    (``__init__.py:1428-1449``). Build additions: ``scale`` may be the
    1-element GPU tensor of ``quantize_int8(..., device_scale=True)``, and
    ``out_dtype`` bf16 / fp16 stores the float32 value rounded to
    nearest-even (GPU path).
    """
    c = _DEQUANT.bind(q=q)
    if not c.on_gpu:
        return c.staged(lambda **a: dequantize_int8(a["q"], float(scale)))
    odt = _out_dtype(out_dtype)
    value, dev_ptr = _scale_operand(scale, "scale")
    x = torch.empty(c.q.shape, dtype=odt, device=c.device)
    n = c.q.numel()
    if n == 0:
        return x
    if odt is torch.float32 and dev_ptr is None:
        _fusedtok.dequantize_launch(c.ptr("q"), x.data_ptr(), value, n, _stream())
    else:
        _fusedtok.dequantize_launch_ex(c.ptr("q"), value, dev_ptr, x.data_ptr(), _CODE[odt],
                                       n, _stream())
    return x


_QADD = _Contract(
    _Arr("qa", "*", _INT8, dtype_msg="inputs must be int8"),
    _Arr("qb", "=qa", _INT8, dtype_msg="inputs must be int8",
         mismatch="inputs must have the same shape"),
    host=False)


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
    if not (torch.is_tensor(qa) and qa.is_cuda and torch.is_tensor(qb) and qb.is_cuda):
        raise TypeError("qadd_int8 needs GPU int8 tensors")
    c = _QADD.bind(qa=qa, qb=qb)
    fa, pa = _scale_operand(sa, "sa")
    fb, pb = _scale_operand(sb, "sb")
    qy = torch.empty(c.qa.shape, dtype=torch.int8, device=c.device)
    out_scale = torch.empty(1, dtype=torch.float32, device=c.device)
    n = c.qa.numel()
    if n == 0:
        out_scale.fill_(1.0)
    elif pa is None and pb is None:
        _fusedtok.qadd_launch(c.ptr("qa"), c.ptr("qb"), fa, fb, qy.data_ptr(),
                              out_scale.data_ptr(), n, _stream())
    else:
        _fusedtok.qadd_launch_ex(c.ptr("qa"), c.ptr("qb"), fa, fb, pa, pb, qy.data_ptr(),
                                 out_scale.data_ptr(), n, _stream())
    return (qy, out_scale) if device_scale else (qy, float(out_scale))


# ---------------------------------------------------------------------------
# W8A8 GEMM
# ---------------------------------------------------------------------------


def _gemm_contract(with_scales):
    ops = [_Arr("a_q", "M K", _INT8, dtype_msg="a_q must be an int8 array"),
           _Arr("b_q", "N K", _INT8, dtype_msg="b_q must be an int8 array",
                mismatch="inner dimensions must match")]
    if with_scales:
        ops.append(_Arr("b_scales", "N", (torch.float32,), upcast=True,
                        mismatch="b_scales must be 1-D with n entries"))
    return _Contract(*ops, rank_msg="operands must be 2-D [rows, K]")


_GEMM = _gemm_contract(False)
_GEMM_PC = _gemm_contract(True)


def _gemm_out(c, out_dtype):
    return torch.empty((c.M, c.N), dtype=_out_dtype(out_dtype), device=c.device)


def qgemm(a_q, a_scale, b_q, b_scale, *, cuda=False, out_dtype=None):
    """INT8 matmul, exact int32 accumulation:
    ``y[M, N] = (A_q[M, K] @ B_q[N, K]^T) * f32(a_scale * b_scale)``
    (reference ``__init__.py:1476-1536``, ``qgemm.cu:612-703``).

    Output float32 (build addition: ``out_dtype`` bf16 / fp16 on the GPU
    path, the float32 value rounded to nearest-even; ``a_scale`` may be a
    1-element GPU tensor, e.g. from ``quantize_int8(..., device_scale=True)``).
    """
    c = _GEMM.bind(a_q=a_q, b_q=b_q)
    if not c.on_gpu:
        return c.staged(lambda **a: qgemm(a["a_q"], float(a_scale), a["b_q"],
                                          float(b_scale)))
    y = _gemm_out(c, out_dtype)
    sa, sa_ptr = _scale_operand(a_scale, "a_scale")
    if c.M and c.N:
        if y.dtype is torch.float32 and sa_ptr is None:
            _fusedtok.qgemm_launch(c.ptr("a_q"), c.ptr("b_q"), y.data_ptr(), c.M, c.N, c.K,
                                   sa, float(b_scale), _stream())
        else:
            _fusedtok.qgemm_launch_ex(c.ptr("a_q"), c.ptr("b_q"), None, float(b_scale), sa,
                                      sa_ptr, y.data_ptr(), _CODE[y.dtype], c.M, c.N, c.K,
                                      _stream())
    return y


def qgemm_perchannel(a_q, a_scale, b_q, b_scales, *, cuda=False, out_dtype=None):
    """INT8 matmul with per-output-channel weight scales (W8A8):
    ``y[M, N] = (A_q @ B_q^T) * f32(a_scale * b_scales[j])``; bit-identical to
    the reference CPU path in float32 (reference ``__init__.py:1539-1599``,
    ``qgemm.cu:640-652``). Build additions as in :func:`qgemm`.
    """
    if torch.is_tensor(a_q) and a_q.is_cuda and not torch.is_tensor(b_scales):
        b_scales = torch.as_tensor(np.asarray(b_scales, dtype=np.float32), device=a_q.device)
    elif torch.is_tensor(a_q) and a_q.is_cuda and not b_scales.is_cuda:
        b_scales = b_scales.to(a_q.device)
    c = _GEMM_PC.bind(a_q=a_q, b_q=b_q, b_scales=b_scales)
    if not c.on_gpu:
        return c.staged(lambda **a: qgemm_perchannel(a["a_q"], float(a_scale), a["b_q"],
                                                     a["b_scales"]))
    y = _gemm_out(c, out_dtype)
    sa, sa_ptr = _scale_operand(a_scale, "a_scale")
    if c.M and c.N:
        if y.dtype is torch.float32 and sa_ptr is None:
            _fusedtok.qgemm_perchannel_launch(c.ptr("a_q"), c.ptr("b_q"), c.ptr("b_scales"),
                                              y.data_ptr(), c.M, c.N, c.K, sa, _stream())
        else:
            _fusedtok.qgemm_launch_ex(c.ptr("a_q"), c.ptr("b_q"), c.ptr("b_scales"), 0.0, sa,
                                      sa_ptr, y.data_ptr(), _CODE[y.dtype], c.M, c.N, c.K,
                                      _stream())
    return y


def qgemm_i32(a_q, b_q):
    """Build addition (test hook): the exact int32 accumulators
    ``A_q @ B_q^T`` through the same kernels as the float paths."""
    c = _GEMM.bind(a_q=a_q, b_q=b_q)
    if not c.on_gpu:
        return c.staged(qgemm_i32)
    acc = torch.empty((c.M, c.N), dtype=torch.int32, device=c.device)
    if c.M and c.N:
        _fusedtok.qgemm_i32_launch(c.ptr("a_q"), c.ptr("b_q"), acc.data_ptr(), c.M, c.N, c.K,
                                   _stream())
    return acc


# ---------------------------------------------------------------------------
# fused decode-chain steps (build additions; GPU tensors only). The
# reference runs these as separate ops (rmsnorm -> quantize_int8,
# swiglu -> quantize_int8, rope -> kv_append_paged); each fused op returns
# exactly what this library's unfused chain returns.
# ---------------------------------------------------------------------------

_RMS_Q = _Contract(
    _Arr("x", "rows? cols", rank_msg="expected a 1-D or 2-D tensor"),
    _Arr("weight", "cols", (torch.float32,), upcast=True,
         mismatch="weight must be 1-D with cols entries"),
    _Arr("residual", "=x", same_dtype="x", optional=True,
         mismatch="residual must have the same shape as x"),
    host=False)


def rmsnorm_quant(x, weight, *, residual=None, eps=1e-6, device_scale=False):
    """``quantize_int8(rmsnorm(x, weight, residual=residual, eps=eps))`` with
    the RMSNorm output kept in float32 registers: returns ``(q, scale)``, q
    int8 of x's shape. The codes are those of the float32 chain: equal to
    ``quantize_int8(rmsnorm(...))`` bit for bit for float32 x. For bf16 /
    fp16 x the unfused chain rounds y to x's dtype before quantising and its
    codes can differ from these by one step. cols must be a multiple of 4.
    ``device_scale=True`` returns the scale as a 1-element GPU float32 tensor
    without synchronising."""
    c = _RMS_Q.bind(x=x, weight=weight, residual=residual)
    q = torch.empty(c.x.shape, dtype=torch.int8, device=c.device)
    # the kernel writes the scale; an empty input has none to compute (1.0,
    # as quantize_int8), set here so the common path launches no fill kernel
    scale = torch.empty(1, dtype=torch.float32, device=c.device)
    if c.rows == 0:
        scale.fill_(1.0)
    _fusedtok.rmsnorm_quant_launch(c.ptr("x"), _CODE[c.x.dtype], c.ptr("weight"),
                                   c.ptr("residual"), q.data_ptr(), scale.data_ptr(),
                                   c.rows, c.cols, float(eps), _stream())
    return (q, scale) if device_scale else (q, float(scale))


_RMS_QGEMM = _Contract(
    _Arr("x", "M? K", rank_msg="expected a 1-D or 2-D tensor"),
    _Arr("weight", "K", (torch.float32,), upcast=True,
         mismatch="weight must be 1-D with K entries"),
    _Arr("b_q", "N K", _INT8, dtype_msg="b_q must be int8 [N, K]",
         mismatch="b_q must be int8 [N, K]"),
    _Arr("residual", "=x", same_dtype="x", optional=True,
         mismatch="residual must match x in dtype and shape"),
    rules=(_Rule(lambda c: c.K % 4 == 0, "rmsnorm_qgemm: K must be a multiple of 4"),),
    host=False)


def rmsnorm_qgemm(x, weight, b_q, b_scales, *, residual=None, eps=1e-6, out_dtype=None):
    """BASELINE config 2's chain in one call: ``q, s = rmsnorm_quant(x,
    weight, residual=residual, eps=eps)`` then ``qgemm_perchannel(q, s, b_q,
    b_scales, out_dtype=out_dtype)``, bit for bit. Returns ``(y, q, scale)``
    with the scale a 1-element GPU float32 tensor (no synchronisation). One
    row with K <= 4096 runs as one launch (every workgroup of the GEMV
    normalises and quantises the row itself); other shapes run the two
    ops. ``b_scales`` per-channel [N] (a float for per-tensor)."""
    if torch.is_tensor(x) and x.is_cuda and not x.is_contiguous():
        x = x.contiguous()
    if torch.is_tensor(residual) and residual.is_cuda and not residual.is_contiguous():
        residual = residual.contiguous()
    c = _RMS_QGEMM.bind(x=x, weight=weight, b_q=b_q, residual=residual)
    sb_ptr, sb = None, 0.0
    if torch.is_tensor(b_scales) or isinstance(b_scales, (list, tuple, np.ndarray)):
        vec = torch.as_tensor(b_scales, dtype=torch.float32, device=c.device).contiguous()
        if vec.ndim != 1 or vec.numel() != c.N:
            raise ValueError("b_scales must be 1-D with N entries")
        b_scales = vec
        sb_ptr = vec.data_ptr()
    else:
        sb = float(b_scales)
    odt = _out_dtype(out_dtype)
    y = torch.empty((c.M, c.N), dtype=odt, device=c.device)
    q = torch.empty((c.M, c.K), dtype=torch.int8, device=c.device)
    scale = torch.empty(1, dtype=torch.float32, device=c.device)
    if c.M == 0:
        scale.fill_(1.0)
        return y, q, scale
    _fusedtok.rmsnorm_qgemm_launch(c.ptr("x"), _CODE[c.x.dtype], c.ptr("weight"),
                                   c.ptr("residual"), float(eps), c.ptr("b_q"), sb_ptr, sb,
                                   y.data_ptr(), _CODE[odt], q.data_ptr(), scale.data_ptr(),
                                   c.M, c.N, c.K, _stream())
    return y, q, scale


def swiglu_quant(gate, up, *, device_scale=False):
    """``quantize_int8(swiglu(gate, up))`` without the float intermediate:
    returns ``(q, scale)`` with q a dense int8 [rows, cols]. gate and up are
    [rows, cols] (or 1-D) GPU tensors of one dtype whose rows may be strided
    alike, e.g. ``h[:, :f]`` and ``h[:, f:]`` of one gate|up GEMM output."""
    for name, t in (("gate", gate), ("up", up)):
        if not (torch.is_tensor(t) and t.is_cuda):
            raise TypeError(f"{name} must be a GPU tensor (fused ops have no host path)")
        if t.dtype not in _FLOATS:
            raise TypeError(f"{name} must be float32, bfloat16 or float16")
    if up.dtype is not gate.dtype:
        raise TypeError("up must have the same dtype as gate")
    if gate.shape != up.shape:
        raise ValueError("gate and up must have the same shape")
    g2 = gate.reshape(1, -1) if gate.ndim == 1 else gate
    u2 = up.reshape(1, -1) if up.ndim == 1 else up
    if g2.ndim != 2:
        raise ValueError("gate and up must be 1-D or 2-D")
    rows, cols = g2.shape
    ld = g2.stride(0) if rows > 1 else cols
    if rows * cols and (g2.stride(1) != 1 or u2.stride(1) != 1
                        or (rows > 1 and u2.stride(0) != ld)):
        raise ValueError("gate and up must have unit column stride and the same row stride")
    q = torch.empty((rows, cols), dtype=torch.int8, device=gate.device)
    scale = torch.empty(1, dtype=torch.float32, device=gate.device)
    if rows * cols == 0:
        scale.fill_(1.0)
    _fusedtok.swiglu_quant_launch(g2.data_ptr(), u2.data_ptr(), _CODE[gate.dtype], q.data_ptr(),
                                  scale.data_ptr(), rows, cols, ld, _stream())
    return (q, scale) if device_scale else (q, float(scale))


_ROPE_KV = _Contract(
    _Arr("k_pool", "Nb Hkv P D", rank_msg="pools must be [Nb, Hkv, P, D] of one shape"),
    _Arr("v_pool", "=k_pool", same_dtype="k_pool",
         mismatch="pools must be [Nb, Hkv, P, D] of one shape"),
    _table(),
    _Idx("lens", "B", lambda c: c.S * c.P, open_bound=True, what=_LENS_WHAT),
    host=False)


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
    if not (torch.is_tensor(qkv) and qkv.is_cuda):
        raise TypeError("qkv must be a GPU tensor (fused ops have no host path)")
    if qkv.dtype not in _FLOATS:
        raise TypeError("qkv must be float32, bfloat16 or float16")
    for name, t in (("k_pool", k_pool), ("v_pool", v_pool)):
        if torch.is_tensor(t) and t.is_cuda and t.dtype is not qkv.dtype:
            raise TypeError(f"{name} must have the qkv dtype")
    q_heads, kv_heads = int(q_heads), int(kv_heads)
    if q_heads < 1 or kv_heads < 1:
        raise ValueError("q_heads and kv_heads must be >= 1")
    if q_heads % kv_heads:
        raise ValueError("q_heads must be a multiple of kv_heads")
    if int(pos_offset) < 0:
        raise ValueError("pos_offset must be >= 0")
    rows = qkv.shape[0] if qkv.ndim == 2 else -1
    # the pools bind Nb Hkv P D; the table and lens bind B against qkv's rows
    if qkv.ndim == 2 and rows == 0:
        d0 = k_pool.shape[-1] if k_pool.ndim == 4 else 0
        return torch.empty((0, q_heads, d0), dtype=qkv.dtype, device=qkv.device)
    c = _ROPE_KV.bind(k_pool=k_pool, v_pool=v_pool, block_table=block_table, lens=lens)
    if c.Hkv != kv_heads:
        raise ValueError("kv_heads must equal the pools' head count")
    if qkv.ndim != 2 or qkv.shape[1] != (q_heads + 2 * kv_heads) * c.D or rows != c.B:
        raise ValueError("qkv must be [B, (q_heads + 2 * kv_heads) * D]")
    if c.D % 2:
        raise ValueError("dim must be even (RoPE pairs elements)")
    if qkv.stride(1) != 1:
        raise ValueError("qkv rows must be contiguous")
    q_out = torch.empty((c.B, q_heads, c.D), dtype=qkv.dtype, device=qkv.device)
    _fusedtok.rope_kv_append_paged_launch(
        qkv.data_ptr(), _CODE[qkv.dtype], qkv.stride(0) if c.B > 1 else qkv.shape[1],
        c.ptr("lens"), c.ptr("block_table"), q_out.data_ptr(), c.ptr("k_pool"),
        c.ptr("v_pool"), c.B, q_heads, kv_heads, c.D, c.P, c.S, float(theta),
        int(pos_offset), bool(neox), _stream())
    return q_out


def _device_scale(a_scale, device):
    """The GEMM's activation scale as a 1-element GPU float32 tensor."""
    _, ptr = _scale_operand(a_scale, "a_scale")
    if ptr is not None:
        return a_scale
    return torch.tensor([float(a_scale.item() if torch.is_tensor(a_scale) else a_scale)],
                        dtype=torch.float32, device=device)


def _fused_gemm_operands(a_q, w_q, w_scales, name):
    if not all(torch.is_tensor(t) and t.is_cuda for t in (a_q, w_q)):
        raise TypeError(f"{name}: a_q and w_q must be GPU tensors (fused ops have no host path)")
    if not torch.is_tensor(w_scales):
        w_scales = torch.as_tensor(np.asarray(w_scales, dtype=np.float32), device=a_q.device)
    return _GEMM_PC.bind(a_q=a_q, b_q=w_q, b_scales=w_scales.to(a_q.device))


def qgemm_rope_kv_append_paged(a_q, a_scale, w_q, w_scales, q_heads, kv_heads, k_pool,
                               v_pool, block_table, lens, *, theta=10000.0, pos_offset=0,
                               neox=False):
    """The QKV projection and the decode token's RoPE + paged KV append:
    ``qkv = qgemm_perchannel(a_q, a_scale, w_q, w_scales, out_dtype=pool
    dtype)`` then ``rope_kv_append_paged(qkv, ...)``, bit for bit. Returns
    ``(q_rot, qkv)``. A K-split GEMM's partial sums are folded by the RoPE
    kernel itself, so the chain is two launches."""
    g = _fused_gemm_operands(a_q, w_q, w_scales, "qgemm_rope_kv_append_paged")
    if not (torch.is_tensor(k_pool) and k_pool.is_cuda and k_pool.dtype in _FLOATS):
        raise TypeError("k_pool must be a float32, bfloat16 or float16 GPU tensor")
    q_heads, kv_heads = int(q_heads), int(kv_heads)
    if q_heads < 1 or kv_heads < 1 or q_heads % kv_heads:
        raise ValueError("q_heads and kv_heads must be >= 1, q_heads a multiple of kv_heads")
    if int(pos_offset) < 0:
        raise ValueError("pos_offset must be >= 0")
    c = _ROPE_KV.bind(k_pool=k_pool, v_pool=v_pool, block_table=block_table, lens=lens)
    if c.Hkv != kv_heads:
        raise ValueError("kv_heads must equal the pools' head count")
    if g.N != (q_heads + 2 * kv_heads) * c.D or g.M != c.B:
        raise ValueError("w_q must be [(q_heads + 2 * kv_heads) * D, K] and a_q [B, K]")
    if c.D % 2:
        raise ValueError("dim must be even (RoPE pairs elements)")
    dt = k_pool.dtype
    qkv = torch.empty((c.B, g.N), dtype=dt, device=k_pool.device)
    q_out = torch.empty((c.B, q_heads, c.D), dtype=dt, device=k_pool.device)
    if c.B:
        sa = _device_scale(a_scale, k_pool.device)
        _fusedtok.qgemm_rope_kv_append_paged_launch(
            g.ptr("a_q"), sa.data_ptr(), g.ptr("b_q"), g.ptr("b_scales"), g.K, _CODE[dt],
            qkv.data_ptr(), c.ptr("lens"), c.ptr("block_table"), q_out.data_ptr(),
            c.ptr("k_pool"), c.ptr("v_pool"), c.B, q_heads, kv_heads, c.D, c.P, c.S,
            float(theta), int(pos_offset), bool(neox), _stream())
    return q_out, qkv


def qgemm_rmsnorm_quant(a_q, a_scale, w_q, w_scales, weight, *, residual=None, eps=1e-6,
                        out_dtype=None, device_scale=False):
    """A projection followed by the next RMSNorm's quantize: ``y =
    qgemm_perchannel(a_q, a_scale, w_q, w_scales, out_dtype=out_dtype)`` then
    ``q, s = rmsnorm_quant(y, weight, residual=residual, eps=eps)``, bit for
    bit. Returns ``(y, q, scale)``. A K-split GEMM's partial sums are folded
    by the RMSNorm row pass (which stores y), so the chain is three launches
    instead of four. ``device_scale=True`` returns the scale as a 1-element
    GPU float32 tensor without synchronising."""
    g = _fused_gemm_operands(a_q, w_q, w_scales, "qgemm_rmsnorm_quant")
    dt = _out_dtype(out_dtype)
    if g.N % 4:
        raise ValueError("qgemm_rmsnorm_quant: N must be a multiple of 4")
    w = torch.as_tensor(weight).to(device=a_q.device, dtype=torch.float32).contiguous()
    if w.shape != (g.N,):
        raise ValueError("weight must be 1-D with N entries")
    if residual is not None:
        if not (torch.is_tensor(residual) and residual.is_cuda and residual.dtype is dt
                and residual.shape == (g.M, g.N)):
            raise ValueError("residual must be a GPU tensor of y's dtype and shape [M, N]")
        residual = residual.contiguous()
    y = torch.empty((g.M, g.N), dtype=dt, device=a_q.device)
    q = torch.empty((g.M, g.N), dtype=torch.int8, device=a_q.device)
    scale = torch.empty(1, dtype=torch.float32, device=a_q.device)
    if g.M == 0 or g.N == 0:
        scale.fill_(1.0)
    else:
        sa = _device_scale(a_scale, a_q.device)
        _fusedtok.qgemm_rmsnorm_quant_launch(
            g.ptr("a_q"), sa.data_ptr(), g.ptr("b_q"), g.ptr("b_scales"), _CODE[dt],
            y.data_ptr(), None if residual is None else residual.data_ptr(), w.data_ptr(),
            float(eps), q.data_ptr(), scale.data_ptr(), g.M, g.N, g.K, _stream())
    return (y, q, scale) if device_scale else (y, q, float(scale))


def qgemm_swiglu_quant(a_q, a_scale, w_q, w_scales, *, out_dtype=None, device_scale=False):
    """The gate/up projection followed by the SwiGLU's quantize: ``h =
    qgemm_perchannel(a_q, a_scale, w_q, w_scales, out_dtype=out_dtype)``
    with ``w_q`` = [2 * inter, K] (gate rows, then up rows), then ``q, s =
    swiglu_quant(h[:, :inter], h[:, inter:])``, bit for bit. Returns ``(h,
    q, scale)``. Where the GEMM runs unsplit on the skinny kernel (16 < M <=
    64), its epilogue takes the SwiGLU maximum, so the chain is two launches
    instead of three. ``device_scale=True`` returns the scale as a
    1-element GPU float32 tensor without synchronising."""
    g = _fused_gemm_operands(a_q, w_q, w_scales, "qgemm_swiglu_quant")
    dt = _out_dtype(out_dtype)
    if g.N % 2:
        raise ValueError("qgemm_swiglu_quant: w_q must have an even row count (gate | up)")
    inter = g.N // 2
    h = torch.empty((g.M, g.N), dtype=dt, device=a_q.device)
    q = torch.empty((g.M, inter), dtype=torch.int8, device=a_q.device)
    scale = torch.empty(1, dtype=torch.float32, device=a_q.device)
    if g.M == 0 or inter == 0:
        scale.fill_(1.0)
    else:
        sa = _device_scale(a_scale, a_q.device)
        _fusedtok.qgemm_swiglu_quant_launch(
            g.ptr("a_q"), sa.data_ptr(), g.ptr("b_q"), g.ptr("b_scales"), _CODE[dt],
            h.data_ptr(), q.data_ptr(), scale.data_ptr(), g.M, inter, g.K, _stream())
    return (h, q, scale) if device_scale else (h, q, float(scale))


# ---------------------------------------------------------------------------
# post-logits sampling (reference __init__.py:1120-1176, 1602-1632,
# 2292-2316, 2366-2540; sampling.cu, topk.cu). Argument normalisation lives
# in _sampling_args.py; these wrappers allocate outputs and launch.
# ---------------------------------------------------------------------------

_ROW = _Contract(_Arr("logits", "n", (torch.float32,), rank_msg="logits must be 1-D",
                      dtype_msg="logits must be float32"))
_ROWS = _Contract(_Arr("logits", "rows n", (torch.float32,),
                       rank_msg="logits must be 2-D [rows, vocab]",
                       dtype_msg="logits must be float32"))
_X1 = _Contract(_Arr("x", "n", (torch.float32,), rank_msg="x must be 1-D for argmax",
                     dtype_msg="x must be float32"))
_X2 = _Contract(_Arr("x", "rows n", (torch.float32,),
                     rank_msg="x must be 2-D [rows, vocab] for argmax_batched",
                     dtype_msg="x must be float32"))


def argmax(x, *, cuda=False):
    """Index of the largest element (earliest index on ties)."""
    c = _X1.bind(x=x)
    if c.n == 0:
        raise ValueError("argmax of empty input")
    if not c.on_gpu:
        return c.staged(lambda **a: argmax(a["x"]))
    out = torch.empty(1, dtype=torch.int32, device=c.device)
    _fusedtok.argmax_launch(c.ptr("x"), c.n, out.data_ptr(), _stream())
    return int(out.item())


def argmax_batched(x, *, cuda=False):
    """Row-wise argmax of ``[rows, vocab]`` float32 logits, earliest index on
    ties; one launch. GPU input: an int64 GPU tensor, no host sync."""
    c = _X2.bind(x=x)
    if c.n == 0:
        raise ValueError("argmax of empty input")
    if not c.on_gpu:
        return c.staged(lambda **a: argmax_batched(a["x"]))
    out = torch.empty(c.rows, dtype=torch.int64, device=c.device)
    if c.rows:
        _fusedtok.argmax_batched_launch(c.ptr("x"), c.rows, c.n, out.data_ptr(), _stream())
    return out


def sample_topp(logits, p, *, temperature=1.0, seed=0, cuda=False):
    """Fused nucleus sampling: softmax of ``logits / temperature``, truncated
    to the smallest top-p nucleus, inverse-CDF draw at a splitmix hash
    uniform of ``seed``. Deterministic per seed. Returns the token id."""
    _sargs.check_params(p, temperature)
    c = _ROW.bind(logits=logits)
    if c.n == 0:
        raise ValueError("sample of empty logits")
    if not c.on_gpu:
        return c.staged(lambda **a: sample_topp(a["logits"], p, temperature=temperature,
                                                seed=seed))
    out = torch.empty(1, dtype=torch.int64, device=c.device)
    _fusedtok.sample_topp_launch(c.ptr("logits"), c.n, float(p), float(temperature),
                                 int(seed), out.data_ptr(), _stream())
    return int(out.item())


def sample_topp_batched(logits, p, *, temperature=1.0, seeds=None, cuda=False,
                        device_out=False):
    """Nucleus sampling of every row of ``[rows, vocab]`` float32 logits (each
    row split across CUs when there are fewer rows than CUs). ``seeds``: one
    per row (None: 0..rows-1).
    Returns int64 tokens on the host (the reference's contract); build
    addition ``device_out=True`` returns them as a GPU tensor, no sync."""
    _sargs.check_params(p, temperature)
    c = _ROWS.bind(logits=logits)
    if not c.on_gpu:
        return c.staged(lambda **a: sample_topp_batched(a["logits"], p,
                                                        temperature=temperature,
                                                        seeds=seeds))
    seed_vec = _sargs.seed_vector(seeds, c.rows)
    out = torch.empty(c.rows, dtype=torch.int64, device=c.device)
    if c.rows:
        if c.n == 0:
            raise ValueError("sample of empty logits")
        _sargs.launch_with_int64(
            [seed_vec], c.device, _fusedtok.host_device_address,
            lambda a: _fusedtok.sample_topp_batched_launch(
                c.ptr("logits"), c.rows, c.n, float(p), float(temperature), a[0],
                out.data_ptr(), _stream()))
    return out if device_out else out.cpu()


def decode_step(logits, sampled_ids, penalty=1.0, *, p=0.9, temperature=1.0, seed=0,
                cuda=False):
    """Fused decode step: CTRL repetition penalty over ``sampled_ids`` (each
    distinct id once), then ``/ temperature``, then nucleus sampling, in one
    launch. Returns the token id; deterministic per seed."""
    _sargs.check_params(p, temperature, penalty)
    c = _ROW.bind(logits=logits)
    if c.n == 0:
        raise ValueError("sample of empty logits")
    device = c.device if c.on_gpu else None
    ids = _sargs.history_1d(sampled_ids, c.n, device)
    if not c.on_gpu:
        return c.staged(lambda **a: decode_step(a["logits"], ids, penalty, p=p,
                                                temperature=temperature, seed=seed))
    out = torch.empty(1, dtype=torch.int64, device=c.device)
    _fusedtok.decode_step_launch(c.ptr("logits"), ids.data_ptr() if ids.numel() else None,
                                 c.n, ids.numel(), float(penalty), float(p),
                                 float(temperature), int(seed), out.data_ptr(), _stream())
    return int(out.item())


def decode_step_batched(logits, sampled_ids, penalty=1.0, *, p=0.9, temperature=1.0,
                        seeds=None, ids_offsets=None, cuda=False, device_out=False):
    """The fused decode step for every row of ``[rows, vocab]`` float32
    logits (each row split across CUs when there are fewer rows than CUs).
    ``sampled_ids``: per-row histories (ragged sequences, a 2-D array, or
    flat ids with ``ids_offsets``). Returns int64 tokens on the host (the
    reference's contract); build addition ``device_out=True`` keeps them on
    the GPU."""
    _sargs.check_params(p, temperature, penalty)
    c = _ROWS.bind(logits=logits)
    if not c.on_gpu:
        return c.staged(lambda **a: decode_step_batched(
            a["logits"], sampled_ids, penalty, p=p, temperature=temperature, seeds=seeds,
            ids_offsets=ids_offsets))
    flat, offsets = _sargs.histories_csr(sampled_ids, ids_offsets, c.rows, c.n)
    seed_vec = _sargs.seed_vector(seeds, c.rows)
    out = torch.empty(c.rows, dtype=torch.int64, device=c.device)
    if c.rows:
        if c.n == 0:
            raise ValueError("sample of empty logits")
        # histories, offsets and seeds read in place from pinned host memory
        _sargs.launch_with_int64(
            [flat, offsets, seed_vec], c.device, _fusedtok.host_device_address,
            lambda a: _fusedtok.decode_step_batched_launch(
                c.ptr("logits"), c.rows, c.n, a[0] if flat.size else None, a[1],
                float(penalty), float(p), float(temperature), a[2], out.data_ptr(),
                _stream()))
    return out if device_out else out.cpu()


from .layer import DecodeLayer, DecodeStack  # noqa: E402  (uses the loaded extension)
