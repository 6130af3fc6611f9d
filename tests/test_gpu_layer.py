"""GPU tests of the DecodeLayer object (csrc/layer.hip, C ABI
ft_decode_layer_*):
  - its forward equals this library's unfused op chain bit for bit (output
    and KV pools), at a toy shape and at BASELINE config 4 (Llama-3-8B
    layer, batch 64, context 8192, uniform and ragged lengths). The chain
    is a Llama block: r = x + o_proj(attention) and y = r + mlp(norm2(r)),
    each residual add rounded to the activation dtype as a model's tensors
    are;
  - the captured HIP graph replays equal the eager forward, with eager work
    between replays, and a replay after the inputs are rewritten in place
    recomputes (the library's capture contract, reference
    docs/en/execution.md:73-103 and tests/test_attention.py:482-550);
  - the float32 layer against the CPU oracle's op chain (oracle/): the GEMMs
    and RMSNorm are exact there, RoPE and attention are not (device trig,
    summation order), so a quantize downstream may move a code by one step:
    the output is compared at 1e-2 of its largest magnitude;
  - argument errors."""

import numpy as np
import pytest
import torch

import fusedtok_amd as ft
import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"

TOY = dict(b=4, hq=8, hkv=2, d=64, hidden=512, inter=768, page=16, lens=[5, 300, 17, 100])
C4 = dict(b=64, hq=32, hkv=8, d=128, hidden=4096, inter=14336, page=16, lens=[8192] * 64)
EPS, THETA = 1e-5, 500000.0


def make_case(cfg, dt, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    b, hq, hkv, d = cfg["b"], cfg["hq"], cfg["hkv"], cfg["d"]
    hid, inter, page = cfg["hidden"], cfg["inter"], cfg["page"]

    def wq(rows, cols):
        return (torch.randint(-127, 128, (rows, cols), device=DEV, generator=gen,
                              dtype=torch.int32).to(torch.int8),
                (torch.rand((rows,), device=DEV, generator=gen) * 9e-3 + 1e-3).float())
    w = {}
    w["norm1"] = (torch.rand((hid,), device=DEV, generator=gen) + 0.5).float()
    w["norm2"] = (torch.rand((hid,), device=DEV, generator=gen) + 0.5).float()
    w["w_qkv"], w["s_qkv"] = wq((hq + 2 * hkv) * d, hid)
    w["w_o"], w["s_o"] = wq(hid, hq * d)
    w["w_gu"], w["s_gu"] = wq(2 * inter, hid)
    w["w_down"], w["s_down"] = wq(hid, inter)
    lens = torch.tensor(cfg["lens"], dtype=torch.int32, device=DEV)
    npg = (max(cfg["lens"]) + 1 + page - 1) // page
    rng = np.random.default_rng(seed)
    pool = b * npg + 3
    table = torch.from_numpy(rng.permutation(pool)[: b * npg].reshape(b, npg)
                             .astype(np.int32)).to(DEV)
    kp = torch.randn((pool, hkv, page, d), device=DEV, generator=gen).to(dt)
    vp = torch.randn((pool, hkv, page, d), device=DEV, generator=gen).to(dt)
    x = torch.randn((b, hid), device=DEV, generator=gen).to(dt)
    return w, x, kp, vp, table, lens


def op_chain(cfg, w, x, kp, vp, table, lens, dt):
    """The layer as this library's unfused ops (the reference's op order)."""
    b, hq, hkv, d, inter = cfg["b"], cfg["hq"], cfg["hkv"], cfg["d"], cfg["inter"]
    q1, s1 = ft.rmsnorm_quant(x, w["norm1"], eps=EPS, device_scale=True)
    qkv = ft.qgemm_perchannel(q1, s1, w["w_qkv"], w["s_qkv"], out_dtype=dt)
    qr = ft.rope_kv_append_paged(qkv, hq, hkv, kp, vp, table, lens, theta=THETA, neox=True)
    att = ft.attention_decode_paged(qr, kp, vp, table, lens + 1)
    qa, sa = ft.quantize_int8(att.reshape(b, hq * d), device_scale=True)
    o = ft.qgemm_perchannel(qa, sa, w["w_o"], w["s_o"], out_dtype=dt)
    q2, s2 = ft.rmsnorm_quant(o, w["norm2"], residual=x, eps=EPS, device_scale=True)
    res = (o.float() + x.float()).to(dt)  # residual stream after attention
    h = ft.qgemm_perchannel(q2, s2, w["w_gu"], w["s_gu"], out_dtype=dt)
    q3, s3 = ft.swiglu_quant(h[:, :inter], h[:, inter:], device_scale=True)
    d = ft.qgemm_perchannel(q3, s3, w["w_down"], w["s_down"], out_dtype=dt)
    return (d.float() + res.float()).to(dt)


def make_layer(cfg, w, dt, max_batch=None):
    return ft.DecodeLayer(q_heads=cfg["hq"], kv_heads=cfg["hkv"], page=cfg["page"],
                          max_batch=max_batch or cfg["b"], dtype=dt, eps=EPS, theta=THETA,
                          neox=True, **w)


def raw(t):
    return t.cpu().view(torch.int32 if t.dtype is torch.float32 else torch.int16).numpy()


# config 4's batch with ragged context lengths (uniform in [512, 8192])
C4R = dict(C4, lens=[int(v) for v in np.random.default_rng(404).integers(512, 8193, 64)])


@pytest.mark.parametrize("name,dt", [("toy", torch.float32), ("toy", torch.bfloat16),
                                     ("toy", torch.float16), ("c4", torch.bfloat16),
                                     ("c4r", torch.bfloat16)])
def test_layer_forward_equals_the_op_chain(name, dt):
    cfg = {"toy": TOY, "c4": C4, "c4r": C4R}[name]
    w, x, kp, vp, table, lens = make_case(cfg, dt, 11)
    kp_ref, vp_ref = kp.clone(), vp.clone()
    y_ref = op_chain(cfg, w, x, kp_ref, vp_ref, table, lens, dt)
    layer = make_layer(cfg, w, dt, max_batch=cfg["b"] + 5)
    for rep in range(2):
        y = layer(x, kp, vp, table, lens)
        torch.cuda.synchronize()
        assert np.array_equal(raw(y), raw(y_ref)), f"{name} rep {rep}: y differs"
    assert torch.equal(kp, kp_ref) and torch.equal(vp, vp_ref)
    # a smaller batch through the same buffers
    b2 = cfg["b"] // 2
    sub = dict(cfg, b=b2, lens=cfg["lens"][:b2])
    y2_ref = op_chain(sub, w, x[:b2], kp_ref, vp_ref, table[:b2].contiguous(), lens[:b2], dt)
    y2 = layer(x[:b2], kp, vp, table[:b2].contiguous(), lens[:b2].contiguous())
    torch.cuda.synchronize()
    assert np.array_equal(raw(y2), raw(y2_ref))
    layer.close()


def test_layer_graph_replays_and_rewritten_inputs():
    dt = torch.bfloat16
    w, x, kp, vp, table, lens = make_case(TOY, dt, 12)
    layer = make_layer(TOY, w, dt)
    ref = layer(x, kp.clone(), vp.clone(), table, lens).clone()
    y = layer.capture(x, kp, vp, table, lens)
    torch.cuda.synchronize()
    assert torch.equal(y, ref), "warm-up of the capture differs"
    for rep in range(3):
        y.zero_()
        layer.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {rep} differs from the eager layer"
        eager = layer(x, kp.clone(), vp.clone(), table, lens)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager, ref)
    # new inputs written in place: the replay recomputes from them
    gen = torch.Generator(device=DEV).manual_seed(99)
    x.copy_(torch.randn(x.shape, device=DEV, generator=gen).to(dt))
    lens.copy_(torch.tensor([7, 290, 3, 150], dtype=torch.int32, device=DEV))
    kp2, vp2 = kp.clone(), vp.clone()
    ref2 = layer(x, kp2, vp2, table, lens).clone()
    layer.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, ref2)
    assert torch.equal(kp, kp2) and torch.equal(vp, vp2)
    assert not torch.equal(ref2, ref)
    layer.close()


def test_layer_float32_against_the_oracle_chain():
    cfg, dt = TOY, torch.float32
    w, x, kp, vp, table, lens = make_case(cfg, dt, 13)
    b, hq, hkv, d, inter = cfg["b"], cfg["hq"], cfg["hkv"], cfg["d"], cfg["inter"]
    h = {k: v.cpu().numpy() for k, v in w.items()}
    xh, kph, vph = x.cpu().numpy(), kp.cpu().numpy(), vp.cpu().numpy()
    tbl, ln = table.cpu().numpy(), lens.cpu().numpy()
    layer = make_layer(cfg, w, dt)
    y = layer(x, kp, vp, table, lens).cpu().numpy()

    q1, s1 = oracle.rmsnorm_quant(xh, h["norm1"], None, EPS)
    qkv = oracle.qgemm_perchannel(q1, s1, h["w_qkv"], h["s_qkv"])
    qr = oracle.rope_kv_append_paged(qkv, hq, hkv, kph, vph, tbl, ln, THETA, 0, True)
    att = oracle.attention_decode_paged(qr, kph, vph, tbl, ln + 1)
    qa, sa = oracle.quantize_int8(att.reshape(b, hq * d))
    o = oracle.qgemm_perchannel(qa, sa, h["w_o"], h["s_o"])
    q2, s2 = oracle.rmsnorm_quant(o, h["norm2"], xh, EPS)
    res = o + xh
    gu = oracle.qgemm_perchannel(q2, s2, h["w_gu"], h["s_gu"])
    q3, s3 = oracle.swiglu_quant(gu[:, :inter], gu[:, inter:])
    y_ref = oracle.qgemm_perchannel(q3, s3, h["w_down"], h["s_down"]) + res

    # RoPE on the device against the host's float64 trig: within an ulp or two
    np.testing.assert_allclose(kp.cpu().numpy(), kph, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(vp.cpu().numpy(), vph, rtol=0, atol=0)
    err = np.abs(y - y_ref).max() / np.abs(y_ref).max()
    assert err <= 1e-2, err
    layer.close()


def test_layer_argument_errors():
    dt = torch.bfloat16
    w, x, kp, vp, table, lens = make_case(TOY, dt, 14)
    layer = make_layer(TOY, w, dt, max_batch=2)
    with pytest.raises(ValueError, match="max_batch"):
        layer(x, kp, vp, table, lens)
    with pytest.raises(TypeError, match="x must be"):
        layer(x[:2].float(), kp, vp, table[:2], lens[:2])
    with pytest.raises(ValueError, match="k_pool must be"):
        layer(x[:2].contiguous(), kp[:, :, :8].contiguous(), vp, table[:2].contiguous(),
              lens[:2].contiguous())
    with pytest.raises(RuntimeError, match="nothing captured"):
        layer.replay()
    with pytest.raises(ValueError, match="w_o must"):
        ft.DecodeLayer(q_heads=3, kv_heads=1, page=16, max_batch=1, dtype=dt, **w)
    bad = dict(w, s_o=w["s_o"][:-1])
    with pytest.raises(ValueError, match="s_o must have shape"):
        ft.DecodeLayer(q_heads=8, kv_heads=2, page=16, max_batch=1, dtype=dt, **bad)
    layer.close()


# ---------------------------------------------------------------------------
# DecodeStack: layers chained in one forward (ft_decode_stack_*)
# ---------------------------------------------------------------------------
# 20 rows take the skinny GEMM with a K split of the down projection (3
# partials, folded by the next layer's RMSNorm row pass); 4 rows the decode
# GEMM (never split: the plain hand-over)
MID = dict(b=20, hq=8, hkv=2, d=64, hidden=512, inter=768, page=16,
           lens=[5, 300, 17, 100, 64, 1, 250, 33, 80, 9, 120, 7, 40, 200, 2, 150, 60, 11, 90, 30])
# the same rows with a longer down projection: split 8 (one batch of 8
# partial loads) and split 16 (the fold loops over batches of 8)
MID8 = dict(MID, inter=2048)
MID16 = dict(MID, inter=4096)


def make_stack_case(cfg, dt, n_layers, seed):
    w0, x, kp, vp, table, lens = make_case(cfg, dt, seed)
    ws, kps, vps = [w0], [kp], [vp]
    for i in range(1, n_layers):
        w, _, kpi, vpi, _, _ = make_case(cfg, dt, seed + 100 * i)
        ws.append(w)
        kps.append(kpi)
        vps.append(vpi)
    return ws, x, kps, vps, table, lens


@pytest.mark.parametrize("name,dt,n", [("toy", torch.bfloat16, 3), ("mid", torch.float32, 3),
                                       ("mid", torch.bfloat16, 4), ("mid", torch.float16, 2),
                                       ("c4", torch.bfloat16, 2), ("mid", torch.bfloat16, 1),
                                       ("mid8", torch.bfloat16, 2), ("mid16", torch.float32, 2),
                                       ("mid16", torch.float16, 3)])
def test_stack_equals_the_layers_called_in_turn(name, dt, n):
    cfg = {"toy": TOY, "mid": MID, "mid8": MID8, "mid16": MID16, "c4": C4}[name]
    ws, x, kps, vps, table, lens = make_stack_case(cfg, dt, n, 21)
    layers = [make_layer(cfg, w, dt) for w in ws]
    kps_ref, vps_ref = [t.clone() for t in kps], [t.clone() for t in vps]
    cur = x
    for L, kp, vp in zip(layers, kps_ref, vps_ref):
        cur = L(cur, kp, vp, table, lens)
    torch.cuda.synchronize()
    y_ref = cur.clone()
    stack = ft.DecodeStack(layers)
    for rep in range(2):
        y = stack(x, kps, vps, table, lens)
        torch.cuda.synchronize()
        assert np.array_equal(raw(y), raw(y_ref)), f"{name} n={n} rep {rep}: y differs"
    for i in range(n):
        assert torch.equal(kps[i], kps_ref[i]) and torch.equal(vps[i], vps_ref[i]), f"pools {i}"
    # a layer used twice in one stack (shared weights, separate pools)
    if n >= 2:
        twice = ft.DecodeStack([layers[0], layers[0]])
        kp2 = [kps[0].clone(), kps[1].clone()]
        vp2 = [vps[0].clone(), vps[1].clone()]
        kq = [t.clone() for t in kp2]
        vq = [t.clone() for t in vp2]
        y1 = layers[0](x, kq[0], vq[0], table, lens)
        y2_ref = layers[0](y1, kq[1], vq[1], table, lens).clone()
        y2 = twice(x, kp2, vp2, table, lens)
        torch.cuda.synchronize()
        assert np.array_equal(raw(y2), raw(y2_ref))
        twice.close()
    stack.close()
    for L in layers:
        L.close()


def test_stack_graph_replays_and_rewritten_inputs():
    dt = torch.bfloat16
    ws, x, kps, vps, table, lens = make_stack_case(MID, dt, 3, 31)
    layers = [make_layer(MID, w, dt) for w in ws]
    stack = ft.DecodeStack(layers)
    ref = stack(x, [t.clone() for t in kps], [t.clone() for t in vps], table, lens).clone()
    y = stack.capture(x, kps, vps, table, lens)
    torch.cuda.synchronize()
    assert torch.equal(y, ref), "warm-up of the capture differs"
    for rep in range(3):
        y.zero_()
        stack.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {rep} differs from the eager stack"
        eager = stack(x, [t.clone() for t in kps], [t.clone() for t in vps], table, lens)
        torch.cuda.synchronize()
        assert torch.equal(eager, ref)
    gen = torch.Generator(device=DEV).manual_seed(98)
    x.copy_(torch.randn(x.shape, device=DEV, generator=gen).to(dt))
    ref2 = stack(x, [t.clone() for t in kps], [t.clone() for t in vps], table, lens).clone()
    stack.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, ref2) and not torch.equal(ref2, ref)
    stack.close()
    for L in layers:
        L.close()


def test_stack_argument_errors():
    dt = torch.bfloat16
    ws, x, kps, vps, table, lens = make_stack_case(TOY, dt, 2, 41)
    layers = [make_layer(TOY, w, dt) for w in ws]
    with pytest.raises(TypeError, match="non-empty sequence"):
        ft.DecodeStack([])
    other = make_layer(TOY, {k: (v.float() if v.dtype is torch.bfloat16 else v)
                             for k, v in ws[0].items()}, torch.float32)
    with pytest.raises(ValueError, match="share the device, dtype and hidden"):
        ft.DecodeStack([layers[0], other])
    stack = ft.DecodeStack(layers)
    with pytest.raises(ValueError, match="one pool per layer"):
        stack(x, kps[:1], vps[:1], table, lens)
    with pytest.raises(RuntimeError, match="nothing captured"):
        stack.replay()
    stack.capture(x, kps, vps, table, lens)
    # the stack holds its layers: closing one is refused while the stack
    # (and the graph it captured) may still use the layer's buffers
    with pytest.raises(ValueError, match="still used by a decode stack"):
        layers[1].close()
    stack.replay()
    torch.cuda.synchronize()
    stack.close()
    with pytest.raises(RuntimeError, match="has been closed"):
        stack(x, kps, vps, table, lens)
    with pytest.raises(RuntimeError, match="has been closed"):
        stack.replay()
    layers[1].close()
    layers[0].close()
    other.close()


def test_stack_max_batch_is_the_smallest_and_empty_batches():
    # the stack's hand-over buffers hold the smallest max_batch of its
    # layers; a larger batch is refused before anything runs, an empty
    # batch returns an empty output
    dt = torch.bfloat16
    ws, x, kps, vps, table, lens = make_stack_case(TOY, dt, 2, 51)
    big = make_layer(TOY, ws[0], dt, max_batch=8)
    small = make_layer(TOY, ws[1], dt, max_batch=TOY["b"])
    stack = ft.DecodeStack([big, small])
    assert stack.max_batch == TOY["b"]
    kq, vq = [t.clone() for t in kps], [t.clone() for t in vps]
    y1 = big(x, kq[0], vq[0], table, lens)
    y_ref = small(y1, kq[1], vq[1], table, lens).clone()
    y = stack(x, kps, vps, table, lens)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    x5 = torch.cat([x, x[:1]])
    with pytest.raises(ValueError, match="max_batch"):
        stack(x5, kps, vps, torch.cat([table, table[:1]]), torch.cat([lens, lens[:1]]))
    y0 = stack(x[:0], kps, vps, table[:0], lens[:0])
    assert y0.shape == (0, TOY["hidden"])
    stack.close()
    big.close()
    small.close()
