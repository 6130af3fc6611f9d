"""GPU parity at the BASELINE workloads themselves, against the CPU oracle.

Each test builds one of BASELINE.json's configs at its full size, runs it
through the public API (the same calls bench.py times) and checks the
result against the oracle on the same inputs:

  C1   contiguous fp16 decode, B=1, Hq=Hkv=32, T=4096: every head of the one
       row against the oracle on the fp16-rounded inputs, and against a
       float64 softmax(QK^T)V.
  C5a  W8A8 GEMM M=4096 K=8192 N=28672, per-channel scales, bf16 out:
       sampled rows (one per 256-row tile band and the edges) over all 28672
       columns, and sampled columns (one per 256-column tile band) over all
       4096 rows. int32 accumulators bit-exact; the bf16 output equal to the
       oracle's float32 value rounded once.
  C5b  paged bf16 decode, B=8, Hq=64, Hkv=8, 131072 tokens per row (every
       row spans many stream segments): every row against the oracle.
  C4   Llama-3-8B W8A8 decode layer, B=64, context 8192, stage by stage:
       each stage's GPU input is handed to the oracle for that stage, every
       row of every stage.

Tolerances: int8 codes, scales and int32
accumulators bit-exact; half-precision GEMM outputs equal to the f32 oracle
value rounded once; half-precision attention |err| <= 2e-3 + 1e-2 * |ref|
against the oracle run on the half-rounded inputs. The SwiGLU codes may
differ by one step from the oracle's (device expf against the host's).
"""

import numpy as np
import pytest
import torch

import fusedtok_amd as ft
import oracle
from tests import refs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def assert_half_close(got, ref, what=""):
    err = np.abs(got - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert err.max(initial=-1) <= 0, (
        f"{what}: max |err| {np.abs(got - ref).max():.3e} exceeds 2e-3 + 1e-2|ref|")


def f32(x):
    return x.float().cpu().numpy()


def sub_pool(pool, table_row, npg):
    """The pages of one sequence, in table order, as float32 host arrays."""
    idx = torch.from_numpy(table_row[:npg].astype(np.int64)).to(pool.device)
    return pool[idx].float().cpu().numpy()


def paged_row_ref(q_row, kp, vp, table_row, length, page):
    """Oracle decode of one sequence through a table over its own pages."""
    npg = (length + page - 1) // page
    sub_tbl = np.arange(npg, dtype=np.int32)[None, :]
    return oracle.attention_decode_paged(q_row, sub_pool(kp, table_row, npg),
                                         sub_pool(vp, table_row, npg), sub_tbl,
                                         np.array([length], np.int32))


# ---------------------------------------------------------------------------
# config 1: contiguous fp16 decode
# ---------------------------------------------------------------------------


def test_c1_contiguous_fp16_b1_h32_t4096():
    b, h, t_rows, d = 1, 32, 4096, 128
    rng = np.random.default_rng(1)
    q = rng.standard_normal((b, h, d)).astype(np.float32)
    k = rng.standard_normal((b, h, t_rows, d)).astype(np.float32)
    v = rng.standard_normal((b, h, t_rows, d)).astype(np.float32)
    f16 = torch.float16
    qt, kt, vt = (torch.from_numpy(a).to(DEV, f16) for a in (q, k, v))
    out = ft.attention_decode(qt, kt, vt)
    torch.cuda.synchronize()
    got = f32(out)
    qr, kr, vr = f32(qt), f32(kt), f32(vt)
    assert_half_close(got, oracle.attention_decode(qr, kr, vr), "C1 vs oracle")
    # float64 softmax(QK^T / sqrt(D)) V on the same fp16-rounded inputs
    s = np.einsum("bhd,bhtd->bht", qr.astype(np.float64), kr.astype(np.float64)) / np.sqrt(d)
    p = np.exp(s - s.max(-1, keepdims=True))
    ref64 = np.einsum("bht,bhtd->bhd", p / p.sum(-1, keepdims=True), vr.astype(np.float64))
    assert_half_close(got, ref64, "C1 vs float64")


# ---------------------------------------------------------------------------
# config 5a: the prefill-sized W8A8 GEMM
# ---------------------------------------------------------------------------


def test_c5a_gemm_4096x8192x28672_bf16_sampled_rows_and_columns():
    m, k, n = 4096, 8192, 28672
    gen = torch.Generator(device=DEV).manual_seed(5)
    a = torch.randint(-127, 128, (m, k), device=DEV, generator=gen,
                      dtype=torch.int32).to(torch.int8)
    b = torch.randint(-127, 128, (n, k), device=DEV, generator=gen,
                      dtype=torch.int32).to(torch.int8)
    sb = (torch.rand((n,), device=DEV, generator=gen) * 9e-3 + 1e-3).float()
    sa = 0.0123
    y = ft.qgemm_perchannel(a, sa, b, sb, out_dtype=torch.bfloat16)
    acc = ft.qgemm_i32(a, b)
    torch.cuda.synchronize()
    a_h, b_h, sb_h = a.cpu().numpy(), b.cpu().numpy(), sb.cpu().numpy()
    # one row in every 256-row tile band (at a varying offset) plus the edges
    rows = sorted({0, 1, 255, 256, 2047, 2048, 4094, 4095}
                  | {256 * i + (37 * i) % 256 for i in range(16)})
    ref = oracle.qgemm_perchannel(a_h[rows], sa, b_h, sb_h)
    np.testing.assert_array_equal(acc[rows].cpu().numpy(), oracle.qgemm_i32(a_h[rows], b_h))
    assert torch.equal(y[rows].cpu(), torch.from_numpy(ref).to(torch.bfloat16))
    # one column in every 256-column tile band, over every row
    cols = sorted({0, n - 1} | {256 * j + (53 * j) % 256 for j in range(n // 256)})
    ref_c = oracle.qgemm_perchannel(a_h, sa, b_h[cols], sb_h[cols])
    np.testing.assert_array_equal(acc[:, cols].cpu().numpy(),
                                  oracle.qgemm_i32(a_h, b_h[cols]))
    assert torch.equal(y[:, cols].cpu(), torch.from_numpy(ref_c).to(torch.bfloat16))


# ---------------------------------------------------------------------------
# config 5b: long-context paged decode
# ---------------------------------------------------------------------------


def test_c5b_paged_bf16_b8_hq64_ctx131072_every_row():
    b, hq, hkv, d, page, ctx = 8, 64, 8, 128, 16, 131072
    npg = ctx // page
    pool = b * npg + 64
    rng = np.random.default_rng(51)
    table = rng.permutation(pool)[: b * npg].reshape(b, npg).astype(np.int32)
    gen = torch.Generator(device=DEV).manual_seed(51)
    bf = torch.bfloat16
    kp = torch.empty((pool, hkv, page, d), dtype=bf, device=DEV)
    vp = torch.empty((pool, hkv, page, d), dtype=bf, device=DEV)
    for pl in (kp, vp):
        flat = pl.view(pool, -1)
        for s in range(0, pool, 8192):
            e = min(pool, s + 8192)
            flat[s:e].copy_(torch.randn((e - s, flat.shape[1]), device=DEV, generator=gen))
    q = torch.randn((b, hq, d), device=DEV, generator=gen).to(bf)
    lens = np.full(b, ctx, np.int32)
    lens[5] = ctx - 4095  # one row ending inside a page and a segment
    out = ft.attention_decode_paged(q, kp, vp, torch.from_numpy(table).to(DEV),
                                    torch.from_numpy(lens).to(DEV))
    torch.cuda.synchronize()
    got = f32(out)
    for bi in range(b):
        ref = paged_row_ref(f32(q[bi:bi + 1]), kp, vp, table[bi], int(lens[bi]), page)
        assert_half_close(got[bi:bi + 1], ref, f"C5b row {bi} len {lens[bi]}")


# ---------------------------------------------------------------------------
# config 4: one W8A8 decode layer, stage by stage
# ---------------------------------------------------------------------------


def test_c4_decode_layer_stage_by_stage():
    bsz, ctx, hid, hq, hkv, d, inter = 64, 8192, 4096, 32, 8, 128, 14336
    page, eps, theta = 16, 1e-5, 500000.0
    bf = torch.bfloat16
    gen = torch.Generator(device=DEV).manual_seed(4)

    def wq(rows, cols):
        return (torch.randint(-127, 128, (rows, cols), device=DEV, generator=gen,
                              dtype=torch.int32).to(torch.int8),
                (torch.rand((rows,), device=DEV, generator=gen) * 9e-3 + 1e-3).float())
    wn1 = (torch.rand((hid,), device=DEV, generator=gen) + 0.5).float()
    wn2 = (torch.rand((hid,), device=DEV, generator=gen) + 0.5).float()
    w_qkv, w_o = wq((hq + 2 * hkv) * d, hid), wq(hid, hq * d)
    w_gu, w_down = wq(2 * inter, hid), wq(hid, inter)
    npg = (ctx + 1 + page - 1) // page
    pool = bsz * npg + 64
    rng = np.random.default_rng(4)
    table = rng.permutation(pool)[: bsz * npg].reshape(bsz, npg).astype(np.int32)
    table_t = torch.from_numpy(table).to(DEV)
    kp = torch.randn((pool, hkv, page, d), device=DEV, generator=gen, dtype=bf)
    vp = torch.randn((pool, hkv, page, d), device=DEV, generator=gen, dtype=bf)
    lens = np.full(bsz, ctx, np.int32)
    lens[::7] -= np.arange(len(lens[::7]), dtype=np.int32) * 97  # ragged rows
    lens_t = torch.from_numpy(lens).to(DEV)
    x = torch.randn((bsz, hid), device=DEV, generator=gen).to(bf)

    def gemm_ref_rows(q_act, s_act, w, rows):
        return oracle.qgemm_perchannel(q_act.cpu().numpy()[rows], float(s_act),
                                       w[0].cpu().numpy(), w[1].cpu().numpy())

    def check_gemm(y, q_act, s_act, w, rows, what):
        ref = gemm_ref_rows(q_act, s_act, w, rows)
        assert torch.equal(y[rows].cpu(), torch.from_numpy(ref).to(bf)), what

    # 1. RMSNorm -> quantize
    q1, s1 = ft.rmsnorm_quant(x, wn1, eps=eps, device_scale=True)
    eq, es = oracle.rmsnorm_quant(f32(x), wn1.cpu().numpy(), None, eps)
    np.testing.assert_array_equal(q1.cpu().numpy(), eq)
    assert float(s1) == es
    # 2. QKV GEMM (every row)
    qkv = ft.qgemm_perchannel(q1, s1, *w_qkv, out_dtype=bf)
    check_gemm(qkv, q1, s1, w_qkv, list(range(bsz)), "QKV GEMM")
    # 3. NeoX RoPE at position lens[b] + paged append of k, v
    qkv_h = f32(qkv)
    slot_pages = table[np.arange(bsz), lens // page]
    qr = ft.rope_kv_append_paged(qkv, hq, hkv, kp, vp, table_t, lens_t,
                                 theta=theta, pos_offset=0, neox=True)
    torch.cuda.synchronize()
    sub_k = np.zeros((bsz, hkv, page, d), np.float32)
    sub_v = np.zeros_like(sub_k)
    sub_tbl = np.zeros((bsz, npg), np.int32)
    sub_tbl[np.arange(bsz), lens // page] = np.arange(bsz)
    q_ref = oracle.rope_kv_append_paged(qkv_h, hq, hkv, sub_k, sub_v, sub_tbl, lens,
                                        theta=theta, pos_offset=0, neox=True)
    # one bf16 rounding of the float32 rotation (at most one bf16 step apart)
    np.testing.assert_allclose(f32(qr), refs.bf16_round(q_ref), rtol=1e-2, atol=1e-6)
    sel = torch.from_numpy(slot_pages.astype(np.int64)).to(DEV)
    in_pg = torch.from_numpy((lens % page).astype(np.int64)).to(DEV)
    k_slot = f32(kp[sel, :, in_pg])   # [bsz, hkv, d]
    v_slot = f32(vp[sel, :, in_pg])
    k_ref = refs.bf16_round(sub_k[np.arange(bsz), :, lens % page])
    np.testing.assert_allclose(k_slot, k_ref, rtol=1e-2, atol=1e-6)
    np.testing.assert_array_equal(v_slot, sub_v[np.arange(bsz), :, lens % page])
    # 4. paged decode over lens + 1 tokens (every row)
    att = ft.attention_decode_paged(qr, kp, vp, table_t, lens_t + 1)
    torch.cuda.synchronize()
    got = f32(att)
    for bi in range(bsz):
        ref = paged_row_ref(f32(qr[bi:bi + 1]), kp, vp, table[bi], int(lens[bi]) + 1, page)
        assert_half_close(got[bi:bi + 1], ref, f"C4 decode row {bi}")
    # 5. quantize the attention output
    qa, sa = ft.quantize_int8(att.reshape(bsz, hq * d), device_scale=True)
    eqa, esa = oracle.quantize_int8(got.reshape(bsz, hq * d))
    np.testing.assert_array_equal(qa.cpu().numpy(), eqa)
    assert float(sa) == esa
    # 6. o_proj GEMM (every row)
    o = ft.qgemm_perchannel(qa, sa, *w_o, out_dtype=bf)
    check_gemm(o, qa, sa, w_o, list(range(bsz)), "o_proj GEMM")
    # 7. RMSNorm(+residual) -> quantize
    q2, s2 = ft.rmsnorm_quant(o, wn2, residual=x, eps=eps, device_scale=True)
    eq2, es2 = oracle.rmsnorm_quant(f32(o), wn2.cpu().numpy(), f32(x), eps)
    np.testing.assert_array_equal(q2.cpu().numpy(), eq2)
    assert float(s2) == es2
    # 8. gate/up GEMM (every row: 7.5 G MACs, ~3 s of oracle time)
    h = ft.qgemm_perchannel(q2, s2, *w_gu, out_dtype=bf)
    check_gemm(h, q2, s2, w_gu, list(range(bsz)), "gate/up GEMM")
    # 9. SwiGLU -> quantize: within one code step of the oracle
    q3, s3 = ft.swiglu_quant(h[:, :inter], h[:, inter:], device_scale=True)
    h_h = f32(h)
    eq3, es3 = oracle.swiglu_quant(h_h[:, :inter], h_h[:, inter:])
    assert abs(float(s3) - es3) <= 1e-6 * es3
    assert np.abs(q3.cpu().numpy().astype(np.int32) - eq3.astype(np.int32)).max() <= 1
    # 10. down GEMM (every row), on the GPU's codes and scale
    yd = ft.qgemm_perchannel(q3, s3, *w_down, out_dtype=bf)
    check_gemm(yd, q3, s3, w_down, list(range(bsz)), "down GEMM")
