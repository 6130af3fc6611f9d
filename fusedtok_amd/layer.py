"""DecodeLayer: one Llama-shaped W8A8 decode layer as a native object
(csrc/layer.hip, C ABI ft_decode_layer_*), with a HIP-graph capture of the
whole layer.

The reference has no layer op; a decode layer there is its ops called one by
one (rmsnorm -> quantize_int8 -> qgemm_perchannel -> rope -> kv_append_paged
-> attention_decode_paged -> quantize_int8 -> qgemm_perchannel -> rmsnorm ->
quantize_int8 -> qgemm_perchannel -> swiglu -> quantize_int8 ->
qgemm_perchannel). This object runs the same chain through this library's
fused ops, every step bit-identical to the unfused op chain:

    q1, s1   = rmsnorm_quant(x, norm1, eps)
    q, qkv   = qgemm_rope_kv_append_paged(q1, s1, w_qkv, s_qkv, ...)  (slot lens)
    att, qa, sa = attention_decode_paged_quant(q, pools, table, lens + 1)
    o, q2, s2   = qgemm_rmsnorm_quant(qa, sa, w_o, s_o, norm2, residual=x)
    h        = qgemm_perchannel(q2, s2, w_gu, s_gu)        (gate rows, then up)
    q3, s3   = swiglu_quant(h[:, :inter], h[:, inter:])
    y        = qgemm_perchannel(q3, s3, w_down, s_down)

Capture follows the library's graph contract (reference
docs/en/execution.md:73-103): ``capture`` runs one warm-up forward (which
sizes the scratch buffers for the shape and makes the same writes a replay
makes), then records the forward; a replay reads the captured tensors'
current contents, so new inputs are written in place before ``replay``.
"""

import torch

from . import _fusedtok

_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _stream():
    return torch.cuda.current_stream().cuda_stream


class DecodeLayer:
    """A W8A8 decode layer on the current GPU.

    Weights (GPU tensors, kept referenced by the layer): ``norm1``, ``norm2``
    float [hidden]; ``w_qkv`` int8 [(q_heads + 2 kv_heads) * head_dim, hidden]
    with per-channel ``s_qkv``; ``w_o`` int8 [hidden, q_heads * head_dim];
    ``w_gu`` int8 [2 * inter, hidden] (gate rows, then up rows); ``w_down``
    int8 [hidden, inter]; each with its float32 per-channel scales.
    Activations and the KV pools are ``dtype``; the activation buffers hold
    up to ``max_batch`` rows.
    """

    def __init__(self, *, norm1, w_qkv, s_qkv, w_o, s_o, norm2, w_gu, s_gu, w_down, s_down,
                 q_heads, kv_heads, page, max_batch, dtype=torch.bfloat16, eps=1e-5,
                 theta=10000.0, neox=True, pos_offset=0):
        if dtype not in _CODES:
            raise TypeError("dtype must be float32, bfloat16 or float16")
        dev = w_qkv.device if torch.is_tensor(w_qkv) else None
        if dev is None or dev.type != "cuda":
            raise TypeError("DecodeLayer weights must be GPU tensors")

        def f32(t, name, shape):
            t = torch.as_tensor(t).to(device=dev, dtype=torch.float32).contiguous()
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} must have shape {shape}")
            return t

        def i8(t, name, shape):
            if not (torch.is_tensor(t) and t.is_cuda and t.dtype is torch.int8):
                raise TypeError(f"{name} must be an int8 GPU tensor")
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} must have shape {shape}")
            return t.contiguous()

        hq, hkv = int(q_heads), int(kv_heads)
        if hq < 1 or hkv < 1 or hq % hkv:
            raise ValueError("q_heads must be a positive multiple of kv_heads")
        hidden = int(w_qkv.shape[1])
        if w_o.ndim != 2 or w_o.shape[1] % hq:
            raise ValueError("w_o must be [hidden, q_heads * head_dim]")
        d = int(w_o.shape[1]) // hq
        inter = int(w_down.shape[1]) if w_down.ndim == 2 else -1
        nqkv = (hq + 2 * hkv) * d
        self._w = dict(
            norm1=f32(norm1, "norm1", (hidden,)), norm2=f32(norm2, "norm2", (hidden,)),
            w_qkv=i8(w_qkv, "w_qkv", (nqkv, hidden)), s_qkv=f32(s_qkv, "s_qkv", (nqkv,)),
            w_o=i8(w_o, "w_o", (hidden, hq * d)), s_o=f32(s_o, "s_o", (hidden,)),
            w_gu=i8(w_gu, "w_gu", (2 * inter, hidden)), s_gu=f32(s_gu, "s_gu", (2 * inter,)),
            w_down=i8(w_down, "w_down", (hidden, inter)),
            s_down=f32(s_down, "s_down", (hidden,)))
        self.hidden, self.q_heads, self.kv_heads, self.head_dim = hidden, hq, hkv, d
        self.inter, self.page, self.max_batch, self.dtype = inter, int(page), int(max_batch), dtype
        self.device = dev
        w = self._w
        with torch.cuda.device(dev):
            self._h = _fusedtok.decode_layer_create(
                hidden, hq, hkv, d, inter, int(page), int(max_batch), _CODES[dtype],
                float(eps), float(theta), bool(neox), int(pos_offset),
                w["norm1"].data_ptr(), w["norm2"].data_ptr(), w["w_qkv"].data_ptr(),
                w["s_qkv"].data_ptr(), w["w_o"].data_ptr(), w["s_o"].data_ptr(),
                w["w_gu"].data_ptr(), w["s_gu"].data_ptr(), w["w_down"].data_ptr(),
                w["s_down"].data_ptr())
        self._captured = None

    def _operands(self, x, k_pool, v_pool, block_table, lens, out):
        def gpu(t, name, dtype):
            if not (torch.is_tensor(t) and t.is_cuda and t.device == self.device):
                raise TypeError(f"{name} must be a tensor on {self.device}")
            if t.dtype is not dtype:
                raise TypeError(f"{name} must be {dtype}")
            if not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous")
            return t
        x = gpu(x, "x", self.dtype)
        if x.ndim != 2 or x.shape[1] != self.hidden:
            raise ValueError("x must be [batch, hidden]")
        b = int(x.shape[0])
        if b > self.max_batch:
            raise ValueError("batch exceeds the layer's max_batch")
        pool_shape = (self.kv_heads, self.page, self.head_dim)
        for name, p in (("k_pool", k_pool), ("v_pool", v_pool)):
            gpu(p, name, self.dtype)
            if p.ndim != 4 or tuple(p.shape[1:]) != pool_shape:
                raise ValueError(f"{name} must be [blocks, kv_heads, page, head_dim]")
        gpu(block_table, "block_table", torch.int32)
        if block_table.ndim != 2 or block_table.shape[0] != b or block_table.shape[1] < 1:
            raise ValueError("block_table must be int32 [batch, width >= 1]")
        gpu(lens, "lens", torch.int32)
        if tuple(lens.shape) != (b,):
            raise ValueError("lens must be int32 [batch]")
        if out is None:
            out = torch.empty_like(x)
        else:
            gpu(out, "out", self.dtype)
            if out.shape != x.shape:
                raise ValueError("out must have x's shape")
        return (x, out, k_pool, v_pool, block_table, lens), b, int(block_table.shape[1])

    def _ptrs(self, ops):
        return [t.data_ptr() for t in ops]

    def forward(self, x, k_pool, v_pool, block_table, lens, *, out=None):
        """One decode step of the layer: returns y [batch, hidden]; appends
        each sequence's K/V at slot lens[b] of the pools (lens not advanced)."""
        ops, b, width = self._operands(x, k_pool, v_pool, block_table, lens, out)
        _fusedtok.decode_layer_forward(self._h, *self._ptrs(ops), b, width, _stream())
        return ops[1]

    __call__ = forward

    def capture(self, x, k_pool, v_pool, block_table, lens, *, out=None):
        """Warm-up forward, then record the layer into a HIP graph bound to
        these tensors (kept referenced until the next capture). Returns the
        output tensor every replay writes."""
        ops, b, width = self._operands(x, k_pool, v_pool, block_table, lens, out)
        _fusedtok.decode_layer_capture(self._h, *self._ptrs(ops), b, width, _stream())
        self._captured = ops
        return ops[1]

    def replay(self):
        """Launch the captured layer on the current stream."""
        if self._captured is None:
            raise RuntimeError("DecodeLayer.replay: nothing captured")
        _fusedtok.decode_layer_replay(self._h, _stream())
        return self._captured[1]

    def close(self):
        h = getattr(self, "_h", None)
        if h:
            # refused (ValueError, the layer left open) while a stack uses it
            _fusedtok.decode_layer_destroy(h)
        self._h = None
        self._captured = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DecodeStack:
    """Layers chained in one forward: ``y = layers[-1](... layers[0](x))``,
    the same results as calling the layers one after another, bit for bit.
    Where a layer's down GEMM splits K, the next layer's first RMSNorm row
    pass folds its partial sums (csrc/layer.hip, C ABI ft_decode_stack_*):
    one launch per chained layer fewer than the layer objects called one by
    one. ``capture`` records the whole chain into one HIP graph.

    The layers (DecodeLayer objects on one device with one dtype and hidden
    size) are kept referenced; a layer may appear more than once, and closing
    a layer raises ValueError while a stack using it is open. Each layer
    has its own KV pools (``k_pools`` / ``v_pools``: sequences of tensors,
    one per layer); the block table and lens are shared.
    """

    def __init__(self, layers):
        layers = list(layers)
        if not layers or not all(isinstance(L, DecodeLayer) for L in layers):
            raise TypeError("DecodeStack needs a non-empty sequence of DecodeLayer objects")
        first = layers[0]
        for L in layers[1:]:
            if (L.device != first.device or L.dtype is not first.dtype
                    or L.hidden != first.hidden):
                raise ValueError("DecodeStack layers must share the device, dtype and hidden size")
        if any(L._h is None for L in layers):
            raise ValueError("DecodeStack: a layer has been closed")
        self.layers = layers
        self.device, self.dtype, self.hidden = first.device, first.dtype, first.hidden
        self.max_batch = min(L.max_batch for L in layers)
        with torch.cuda.device(self.device):
            self._h = _fusedtok.decode_stack_create([L._h for L in layers])
        self._captured = None

    def _operands(self, x, k_pools, v_pools, block_table, lens, out):
        k_pools, v_pools = list(k_pools), list(v_pools)
        n = len(self.layers)
        if len(k_pools) != n or len(v_pools) != n:
            raise ValueError(f"k_pools and v_pools must hold one pool per layer ({n})")
        ops = None
        for L, kp, vp in zip(self.layers, k_pools, v_pools):
            ops, b, width = L._operands(x, kp, vp, block_table, lens, out)
            out = ops[1]
        return ops[0], ops[1], k_pools, v_pools, ops[4], ops[5], b, width

    def _args(self, x, k_pools, v_pools, block_table, lens, out):
        if self._h is None or any(L._h is None for L in self.layers):
            raise RuntimeError("DecodeStack: the stack or one of its layers has been closed")
        x, y, kps, vps, table, ln, b, width = self._operands(x, k_pools, v_pools, block_table,
                                                             lens, out)
        if b > self.max_batch:
            raise ValueError("batch exceeds the stack's max_batch")
        return (x, y, kps, vps, table, ln), (
            x.data_ptr(), y.data_ptr(), [t.data_ptr() for t in kps],
            [t.data_ptr() for t in vps], table.data_ptr(), ln.data_ptr(), b, width)

    def forward(self, x, k_pools, v_pools, block_table, lens, *, out=None):
        """One decode step through every layer: returns y [batch, hidden];
        each layer appends its sequence's K/V at slot lens[b] of its own
        pools (lens not advanced)."""
        keep, args = self._args(x, k_pools, v_pools, block_table, lens, out)
        _fusedtok.decode_stack_forward(self._h, *args, _stream())
        return keep[1]

    __call__ = forward

    def capture(self, x, k_pools, v_pools, block_table, lens, *, out=None):
        """Warm-up forward, then the chain recorded into one HIP graph bound
        to these tensors (kept referenced until the next capture). Returns
        the output tensor every replay writes."""
        keep, args = self._args(x, k_pools, v_pools, block_table, lens, out)
        _fusedtok.decode_stack_capture(self._h, *args, _stream())
        self._captured = keep
        return keep[1]

    def replay(self):
        """Launch the captured chain on the current stream."""
        if self._h is None or any(L._h is None for L in self.layers):
            raise RuntimeError("DecodeStack: the stack or one of its layers has been closed")
        if self._captured is None:
            raise RuntimeError("DecodeStack.replay: nothing captured")
        _fusedtok.decode_stack_replay(self._h, _stream())
        return self._captured[1]

    def close(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            _fusedtok.decode_stack_destroy(h)
        self._captured = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
