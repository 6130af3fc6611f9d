"""GPU parity of the fused decode-chain steps (rmsnorm_quant, swiglu_quant,
rope_kv_append_paged, attention_decode_paged_quant, qgemm_rope_kv_append_paged,
qgemm_rmsnorm_quant):
  - against the CPU oracle on the same seeded inputs: int8 codes and the
    scale bit-exact for rmsnorm_quant (the oracle follows the kernel's
    summation order); within one code step for swiglu_quant (device expf vs
    the host's); RoPE within 1e-6 (f32) / one storage ulp (bf16, fp16);
  - against this library's unfused GPU chain (rmsnorm -> quantize_int8,
    swiglu -> quantize_int8, rope(positions=lens) -> kv_append_paged,
    attention_decode_paged -> quantize_int8, qgemm_perchannel ->
    rope_kv_append_paged, qgemm_perchannel -> rmsnorm_quant): bit-exact,
    which is the fused ops' contract, on split and unsplit GEMMs."""

import numpy as np
import pytest
import torch

import fusedtok_amd as ft
import oracle
from tests import refs

pytestmark = pytest.mark.gpu
DEV = "cuda"
ALL = [torch.float32, torch.bfloat16, torch.float16]


def t(a, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return x if dtype is None else x.to(dtype)


def as_f32(x):
    return x.float().cpu().numpy()


def raw(x):
    if x.dtype is torch.float32:
        return x.cpu().view(torch.int32).numpy()
    return x.cpu().view(torch.int16).numpy()


# ---------------------------------------------------------------------------
# rmsnorm_quant
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("rows,cols", [(1, 4096), (8, 4096), (16, 4096), (5, 1028),
                                       (3, 8), (2, 5000)])
@pytest.mark.parametrize("with_res", [False, True])
def test_rmsnorm_quant_matches_oracle_and_chain(dt, rows, cols, with_res):
    rng = np.random.default_rng(rows * 7919 + cols + with_res)
    x = t(rng.standard_normal((rows, cols)).astype(np.float32) * 2, dt)
    w = t(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    r = t(rng.standard_normal((rows, cols)).astype(np.float32), dt) if with_res else None
    q, s = ft.rmsnorm_quant(x, w, residual=r, eps=1e-5)
    eq, es = oracle.rmsnorm_quant(as_f32(x), w.cpu().numpy(),
                                  None if r is None else as_f32(r), 1e-5)
    np.testing.assert_array_equal(q.cpu().numpy(), eq)
    assert s == es
    # unfused GPU chain on float32 storage
    y = ft.rmsnorm(x.float(), w, residual=None if r is None else r.float(), eps=1e-5)
    np.testing.assert_array_equal(
        y.cpu().numpy(), oracle.rmsnorm_blocked(as_f32(x), w.cpu().numpy(),
                                                None if r is None else as_f32(r), 1e-5))
    q2, s2 = ft.quantize_int8(y)
    np.testing.assert_array_equal(q.cpu().numpy(), q2.cpu().numpy())
    assert s == s2


@pytest.mark.parametrize("rows", [1, 3])
def test_rmsnorm_qgemm_without_output_columns_still_quantises(rows):
    # b_q [0, K]: no GEMM output, but the codes and the scale are returned
    # as rmsnorm_quant writes them
    rng = np.random.default_rng(rows)
    x = t(rng.standard_normal((rows, 256)).astype(np.float32), torch.float16)
    w = t(rng.uniform(0.5, 1.5, 256).astype(np.float32))
    b = torch.empty((0, 256), dtype=torch.int8, device=DEV)
    sb = torch.empty((0,), dtype=torch.float32, device=DEV)
    y, q, s = ft.rmsnorm_qgemm(x, w, b, sb, eps=1e-5, out_dtype=torch.float16)
    q2, s2 = ft.rmsnorm_quant(x, w, eps=1e-5, device_scale=True)
    assert y.shape == (rows, 0)
    assert torch.equal(q, q2) and torch.equal(s, s2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(1, 4096), (16, 4096), (64, 4096), (3, 1028)])
def test_rmsnorm_quant_vs_half_storage_chain(dt, rows, cols):
    # The fused op quantises the float32 RMSNorm result. The unfused chain on
    # half storage first rounds y to bf16 / fp16 (rmsnorm's output dtype),
    # then quantises: y and the scale each move by at most one half-precision
    # rounding (relative 2^-8 for bf16, 2^-11 for fp16), so a code of
    # magnitude <= 127 moves by less than 127 * 2 * 2^-8 < 1 before rint, and
    # the two codes differ by at most one step. That is the bound between the
    # fused op and the reference's half-storage chain (rmsnorm.cu:110-130 ->
    # quantize.cu:153-186 on the rounded y); exact agreement with that chain
    # is not claimed.
    rng = np.random.default_rng(rows * 13 + cols)
    x = t(rng.standard_normal((rows, cols)).astype(np.float32) * 2, dt)
    w = t(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    r = t(rng.standard_normal((rows, cols)).astype(np.float32), dt)
    for res in (None, r):
        q, s = ft.rmsnorm_quant(x, w, residual=res, eps=1e-5)
        y_half = ft.rmsnorm(x, w, residual=res, eps=1e-5)
        assert y_half.dtype is dt
        q_half, s_half = ft.quantize_int8(y_half)
        diff = np.abs(q.cpu().numpy().astype(np.int32) - q_half.cpu().numpy().astype(np.int32))
        assert diff.max() <= 1
        rel = 2.0 ** -8 if dt is torch.bfloat16 else 2.0 ** -11
        assert abs(s - s_half) <= rel * s * (1 + 1e-6)


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("rows,cols", [(1, 4096), (2, 12), (3, 4096), (4, 4096),
                                       (4, 1000), (1, 4)])
def test_rmsnorm_quant_one_launch_matches_two_launch_path(dt, rows, cols, tuning):
    # up to 4 rows of up to 4096 columns run as one workgroup; FT_RMSQ_SPLIT=1
    # forces the per-row + fold/quantize kernels. Both must agree bit for bit.
    rng = np.random.default_rng(rows * 131 + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 3
    x[rows // 2, : cols // 3] *= 40.0
    x = t(x, dt)
    w = t(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    r = t(rng.standard_normal((rows, cols)).astype(np.float32), dt)
    for res in (None, r):
        q1, s1 = ft.rmsnorm_quant(x, w, residual=res, eps=1e-5)
        tuning("FT_RMSQ_SPLIT", 1)
        q2, s2 = ft.rmsnorm_quant(x, w, residual=res, eps=1e-5)
        tuning.clear("FT_RMSQ_SPLIT")
        np.testing.assert_array_equal(q1.cpu().numpy(), q2.cpu().numpy())
        assert s1 == s2


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("rows,cols", [(17, 4096), (20, 12), (64, 4096), (64, 4),
                                       (257, 1028), (1000, 512), (4096, 64)])
def test_rmsnorm_quant_grid_launch_matches_two_launches(dt, rows, cols, tuning):
    # From 17 rows of at most 4096 columns, rmsnorm_quant is one launch: the
    # tensor maximum is folded inside it through device-scope atomics
    # (grid_max). FT_GRID_SYNC=1 forces the row pass + fold/quantize pair.
    # Eight calls go back to back with no host sync, each with its largest
    # value in another row, so a workgroup that read a stale maximum would
    # show as a wrong scale or wrong codes.
    rng = np.random.default_rng(rows * 17 + cols)
    w = t(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    base = rng.standard_normal((rows, cols)).astype(np.float32)
    xs, rs = [], []
    for i in range(8):
        a = base.copy()
        a[(i * 7919) % rows, (i * 31) % cols] = 50.0 + 10 * i
        xs.append(t(a, dt))
        rs.append(t(rng.standard_normal((rows, cols)).astype(np.float32), dt))
    for with_res in (False, True):
        got = [ft.rmsnorm_quant(x, w, residual=r if with_res else None, eps=1e-5,
                                device_scale=True) for x, r in zip(xs, rs)]
        tuning("FT_GRID_SYNC", 1)
        ref = [ft.rmsnorm_quant(x, w, residual=r if with_res else None, eps=1e-5,
                                device_scale=True) for x, r in zip(xs, rs)]
        tuning.clear("FT_GRID_SYNC")
        for i, ((q1, s1), (q2, s2)) in enumerate(zip(got, ref)):
            assert torch.equal(s1, s2), f"call {i}: scale"
            assert torch.equal(q1, q2), f"call {i}: codes"
    # and against the oracle for the last call
    eq, es = oracle.rmsnorm_quant(as_f32(xs[-1]), w.cpu().numpy(), as_f32(rs[-1]), 1e-5)
    np.testing.assert_array_equal(got[-1][0].cpu().numpy(), eq)
    assert float(got[-1][1]) == es


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("rows,n,k,res", [(1, 11008, 4096, False), (1, 777, 1024, True),
                                          (1, 5, 48, True), (1, 300, 4112, False),
                                          (3, 300, 512, True),
                                          # N > 64 * CUs: the GEMV's grid-stride
                                          # second pass reloads its weight rows
                                          (1, 28672, 4096, True)])
@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16, torch.float32])
def test_rmsnorm_qgemm_equals_the_two_ops(dt, rows, n, k, res, odt, tuning):
    # one row with K <= 4096 runs as one launch (the GEMV normalises and
    # quantises the row in every workgroup); the codes, the scale and the
    # output must equal rmsnorm_quant followed by qgemm_perchannel
    rng = np.random.default_rng(rows * 31 + n + k + res)
    x = t(rng.standard_normal((rows, k)).astype(np.float32) * 2, dt)
    w = t(rng.uniform(0.5, 1.5, k).astype(np.float32))
    r = t(rng.standard_normal((rows, k)).astype(np.float32), dt) if res else None
    b = t(rng.integers(-127, 128, (n, k)).astype(np.int8))
    sb = t(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    y, q, s = ft.rmsnorm_qgemm(x, w, b, sb, residual=r, eps=1e-5, out_dtype=odt)
    q2, s2 = ft.rmsnorm_quant(x, w, residual=r, eps=1e-5, device_scale=True)
    y2 = ft.qgemm_perchannel(q2, s2, b, sb, out_dtype=odt)
    assert torch.equal(q, q2) and torch.equal(s, s2) and torch.equal(y, y2)
    eq, es = oracle.rmsnorm_quant(as_f32(x), w.cpu().numpy(), None if r is None else as_f32(r),
                                  1e-5)
    np.testing.assert_array_equal(q.cpu().numpy(), eq)
    assert float(s) == es
    ref = oracle.qgemm_perchannel(eq, es, b.cpu().numpy(), sb.cpu().numpy())
    assert torch.equal(y.cpu(), torch.from_numpy(ref).to(odt))
    # the two-op path of the same entry point, and a per-tensor weight scale
    tuning("FT_RMSQ_GEMV_SPLIT", 1)
    y3, q3, s3 = ft.rmsnorm_qgemm(x, w, b, sb, residual=r, eps=1e-5, out_dtype=odt)
    tuning.clear("FT_RMSQ_GEMV_SPLIT")
    assert torch.equal(y3, y) and torch.equal(q3, q) and torch.equal(s3, s)
    yt, _, _ = ft.rmsnorm_qgemm(x, w, b, 0.004, residual=r, eps=1e-5, out_dtype=odt)
    assert torch.equal(yt, ft.qgemm(q2, s2, b, 0.004, out_dtype=odt))


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("rows,n,k,res", [
    # C2's shape at 2, 8 and 16 rows (one-workgroup normalisation up to 4
    # rows, the row + quantize kernels above; the decode GEMMs)
    (2, 11008, 4096, False), (8, 11008, 4096, True), (16, 11008, 4096, False),
    (16, 28672, 4096, True),
    # K = 512, N not a multiple of 16, few column tiles
    (5, 1000, 512, True), (13, 4000, 2048, False),
    (16, 40, 1024, True), (4, 17, 4096, False), (3, 300, 512, True),
    (7, 300, 4608, False), (9, 64, 1000, True), (17, 64, 512, False)])
def test_rmsnorm_qgemm_several_rows_equals_the_two_ops(dt, rows, n, k, res, tuning):
    # more than one row: the codes, the scale and the output must equal
    # rmsnorm_quant followed by qgemm_perchannel and the oracle chain
    odt = {torch.float32: torch.bfloat16, torch.bfloat16: torch.float16,
           torch.float16: torch.float16}[dt]
    rng = np.random.default_rng(rows * 37 + n + k + res)
    x = rng.standard_normal((rows, k)).astype(np.float32) * 2
    x[rows // 2, : k // 5] *= 30.0  # one row dominates the tensor maximum
    x = t(x, dt)
    w = t(rng.uniform(0.5, 1.5, k).astype(np.float32))
    r = t(rng.standard_normal((rows, k)).astype(np.float32), dt) if res else None
    b = t(rng.integers(-127, 128, (n, k)).astype(np.int8))
    sb = t(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    y, q, s = ft.rmsnorm_qgemm(x, w, b, sb, residual=r, eps=1e-5, out_dtype=odt)
    q2, s2 = ft.rmsnorm_quant(x, w, residual=r, eps=1e-5, device_scale=True)
    y2 = ft.qgemm_perchannel(q2, s2, b, sb, out_dtype=odt)
    assert torch.equal(q, q2) and torch.equal(s, s2) and torch.equal(y, y2)
    eq, es = oracle.rmsnorm_quant(as_f32(x), w.cpu().numpy(), None if r is None else as_f32(r),
                                  1e-5)
    np.testing.assert_array_equal(q.cpu().numpy(), eq)
    assert float(s) == es
    cols = np.arange(0, n, max(1, n // 512))  # a column sample keeps the oracle GEMM short
    ref = oracle.qgemm_perchannel(eq, es, np.ascontiguousarray(b.cpu().numpy()[cols]),
                                  np.ascontiguousarray(sb.cpu().numpy()[cols]))
    assert torch.equal(y.cpu()[:, cols], torch.from_numpy(ref).to(odt))
    # the two-step chain of the same entry point, and a per-tensor weight scale
    tuning("FT_RMSQ_GEMV_SPLIT", 1)
    y3, q3, s3 = ft.rmsnorm_qgemm(x, w, b, sb, residual=r, eps=1e-5, out_dtype=odt)
    tuning.clear("FT_RMSQ_GEMV_SPLIT")
    assert torch.equal(y3, y) and torch.equal(q3, q) and torch.equal(s3, s)
    yt, _, _ = ft.rmsnorm_qgemm(x, w, b, 0.004, residual=r, eps=1e-5, out_dtype=odt)
    assert torch.equal(yt, ft.qgemm(q2, s2, b, 0.004, out_dtype=odt))


def test_rmsnorm_quant_device_scale_zero_rows_and_1d():
    rng = np.random.default_rng(3)
    x = t(rng.standard_normal(512).astype(np.float32), torch.bfloat16)
    w = t(np.ones(512, np.float32))
    q, s = ft.rmsnorm_quant(x, w, device_scale=True)
    assert q.shape == (512,) and s.shape == (1,) and s.is_cuda
    q1, s1 = ft.rmsnorm_quant(x, w)
    assert float(s) == s1 and torch.equal(q, q1)
    q0, s0 = ft.rmsnorm_quant(torch.empty((0, 64), device=DEV), t(np.ones(64, np.float32)))
    assert q0.shape == (0, 64) and s0 == 1.0
    with pytest.raises(ValueError):
        ft.rmsnorm_quant(torch.ones((2, 6), device=DEV), torch.ones(6, device=DEV))
    with pytest.raises(TypeError):
        ft.rmsnorm_quant(np.ones((2, 8), np.float32), np.ones(8, np.float32))


def test_rmsnorm_quant_repeatable_over_growing_shapes():
    # the per-row statistics live in a scratch slot that grows; a smaller call
    # after a larger one must not read stale rows
    rng = np.random.default_rng(4)
    w = t(rng.uniform(0.5, 1.5, 2048).astype(np.float32))
    big = t(rng.standard_normal((64, 2048)).astype(np.float32) * 50)
    small = t(rng.standard_normal((3, 2048)).astype(np.float32))
    ft.rmsnorm_quant(big, w)
    q, s = ft.rmsnorm_quant(small, w)
    eq, es = oracle.rmsnorm_quant(small.cpu().numpy(), w.cpu().numpy())
    np.testing.assert_array_equal(q.cpu().numpy(), eq)
    assert s == es


# ---------------------------------------------------------------------------
# swiglu_quant
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("rows,cols", [(1, 11008), (8, 14336), (64, 300), (3, 1), (5, 301)])
def test_swiglu_quant_halves_match_chain_and_oracle(dt, rows, cols):
    rng = np.random.default_rng(rows * 31 + cols)
    h = t((rng.standard_normal((rows, 2 * cols)) * 3).astype(np.float32), dt)
    g, u = h[:, :cols], h[:, cols:]
    q, s = ft.swiglu_quant(g, u)
    # unfused GPU chain on float32 storage
    y = ft.swiglu(g.float().contiguous(), u.float().contiguous())
    q2, s2 = ft.quantize_int8(y)
    np.testing.assert_array_equal(q.cpu().numpy(), q2.cpu().numpy())
    assert s == s2
    # oracle (host expf): scale within rounding, codes within one step
    eq, es = oracle.swiglu_quant(as_f32(g), as_f32(u))
    assert s == pytest.approx(es, rel=1e-6)
    assert np.abs(q.cpu().numpy().astype(int) - eq.astype(int)).max() <= 1


def test_swiglu_quant_contiguous_pair_and_errors():
    rng = np.random.default_rng(8)
    g = t(rng.standard_normal((4, 256)).astype(np.float32), torch.float16)
    u = t(rng.standard_normal((4, 256)).astype(np.float32), torch.float16)
    q, s = ft.swiglu_quant(g, u, device_scale=True)
    q2, s2 = ft.quantize_int8(ft.swiglu(g.float(), u.float()))
    assert torch.equal(q, q2) and float(s) == s2
    with pytest.raises(TypeError):
        ft.swiglu_quant(g, u.float())
    with pytest.raises(ValueError):
        ft.swiglu_quant(g, u[:, :128])
    q0, s0 = ft.swiglu_quant(g[:0], u[:0])
    assert q0.shape == (0, 256) and s0 == 1.0


# ---------------------------------------------------------------------------
# rope_kv_append_paged
# ---------------------------------------------------------------------------


def rope_kv_case(rng, b, hq, hkv, d, lens, page=16, extra=3):
    width = max(1, max((l + 1 + page - 1) // page for l in lens))
    nb = b * width + extra
    qkv = rng.standard_normal((b, (hq + 2 * hkv) * d)).astype(np.float32)
    kp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    vp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    tbl = rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32)
    return qkv, kp, vp, tbl, np.array(lens, np.int32)


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("neox", [False, True])
@pytest.mark.parametrize("off", [0, 5])
def test_rope_kv_append_matches_chain_and_oracle(dt, neox, off):
    rng = np.random.default_rng(100 + 10 * neox + off)
    b, hq, hkv, d, page = 5, 32, 8, 128, 16
    qkv, kp, vp, tbl, lens = rope_kv_case(rng, b, hq, hkv, d, [0, 15, 16, 700, 8191],
                                          page)
    qkv_d = t(qkv, dt)
    kp_d, vp_d = t(kp, dt), t(vp, dt)
    kp_c, vp_c = kp_d.clone(), vp_d.clone()
    tbl_d, lens_d = t(tbl), t(lens)
    qo = ft.rope_kv_append_paged(qkv_d, hq, hkv, kp_d, vp_d, tbl_d, lens_d,
                                 theta=500000.0, pos_offset=off, neox=neox)
    # unfused GPU chain
    qh = qkv_d[:, : hq * d].reshape(b * hq, d).contiguous()
    kh = qkv_d[:, hq * d:(hq + hkv) * d].reshape(b * hkv, d).contiguous()
    vh = qkv_d[:, (hq + hkv) * d:].reshape(b, hkv, d).contiguous()
    qr, _ = ft.rope(qh, theta=500000.0, pos_offset=off, neox=neox, positions=lens_d,
                    rows_per_position=hq)
    kr, _ = ft.rope(kh, theta=500000.0, pos_offset=off, neox=neox, positions=lens_d,
                    rows_per_position=hkv)
    ft.kv_append_paged(kp_c, vp_c, tbl_d, kr.reshape(b, hkv, d), vh, lens_d)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(raw(qo.reshape(b * hq, d)), raw(qr))
    np.testing.assert_array_equal(raw(kp_d), raw(kp_c))
    np.testing.assert_array_equal(raw(vp_d), raw(vp_c))
    # oracle on the storage-rounded inputs
    ek, ev = as_f32(t(kp, dt)), as_f32(t(vp, dt))
    eq = oracle.rope_kv_append_paged(as_f32(qkv_d), hq, hkv, ek, ev, tbl, lens,
                                     500000.0, off, neox)
    if dt is torch.float32:
        tol = dict(rtol=0, atol=1e-6)
    else:
        rnd = refs.bf16_round if dt is torch.bfloat16 else refs.f16_round
        eq, ek = rnd(eq), rnd(ek)
        tol = dict(rtol=1e-2 if dt is torch.bfloat16 else 2e-3, atol=1e-6)
    np.testing.assert_allclose(as_f32(qo), eq, **tol)
    np.testing.assert_allclose(as_f32(kp_d), ek, **tol)
    np.testing.assert_array_equal(as_f32(vp_d), ev)


def test_rope_kv_append_strided_rows_and_errors():
    rng = np.random.default_rng(9)
    b, hq, hkv, d = 3, 8, 2, 64
    qkv, kp, vp, tbl, lens = rope_kv_case(rng, b, hq, hkv, d, [3, 40, 0])
    wide = np.zeros((b, (hq + 2 * hkv) * d + 64), np.float32)
    wide[:, : qkv.shape[1]] = qkv
    kp_a, vp_a = t(kp), t(vp)
    kp_b, vp_b = t(kp), t(vp)
    qa = ft.rope_kv_append_paged(t(qkv), hq, hkv, kp_a, vp_a, t(tbl), t(lens))
    qb = ft.rope_kv_append_paged(t(wide)[:, : qkv.shape[1]], hq, hkv, kp_b, vp_b,
                                 tbl, lens)          # host table / lens
    assert torch.equal(qa, qb) and torch.equal(kp_a, kp_b) and torch.equal(vp_a, vp_b)
    with pytest.raises(ValueError):                   # slot beyond capacity
        ft.rope_kv_append_paged(t(qkv), hq, hkv, kp_a, vp_a, tbl,
                                np.array([3, 40, tbl.shape[1] * 16], np.int32))
    with pytest.raises(ValueError):
        ft.rope_kv_append_paged(t(qkv), hq, 3, kp_a, vp_a, tbl, lens)
    with pytest.raises(TypeError):
        ft.rope_kv_append_paged(t(qkv, torch.bfloat16), hq, hkv, kp_a, vp_a, tbl, lens)


# ---------------------------------------------------------------------------
# a whole W8A8 decode layer (the chain bench.py times as a HIP graph):
# captured once, replayed several times with eager work in between; every
# replay must equal the eager layer bit for bit (all kernels here are
# deterministic: fixed reduction orders, integer GEMM sums)
# ---------------------------------------------------------------------------


# ---------------------------------------------------------------------------
# attention_decode_paged_quant
# ---------------------------------------------------------------------------

# (b, hq, hkv, d, page, lens): C4's decode batch; one long row split over many
# segments (the combine kernel writes the maxima); ragged rows with empty
# ones; group 1 at D = 64 (the generic kernel, quantised in full)
ATTN_Q_CASES = {
    "c4": (32, 32, 8, 128, 16, None),
    "long": (1, 32, 8, 128, 16, [4133]),
    "ragged": (5, 16, 2, 128, 32, [0, 1, 33, 0, 900]),
    "d64": (3, 8, 8, 64, 16, [10, 200, 3]),
}


# the stream path's quantize: "grid", the combine kernel folds the heads'
# maxima (grid_max) and writes the codes; "partials", FT_GRID_SYNC=1: it
# writes the maxima and a second launch the codes; "generic": the generic
# kernels, quantised in full
@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("case", list(ATTN_Q_CASES))
@pytest.mark.parametrize("path", ["grid", "partials", "generic"])
def test_attention_decode_paged_quant_equals_the_two_ops(dt, case, path, tuning):
    generic = path == "generic"
    if generic:
        tuning("FT_ATTN_FORCE_GENERIC", 1)
    if path == "partials":
        tuning("FT_GRID_SYNC", 1)
    rng = np.random.default_rng(sorted(ATTN_Q_CASES).index(case) + 7 * generic)
    b, hq, hkv, d, page, lens = ATTN_Q_CASES[case]
    if lens is None:
        lens = rng.integers(1, 700, b).tolist()
    width = max(1, max((n + page - 1) // page for n in lens))
    nb = b * width + 2
    q = t(rng.standard_normal((b, hq, d)).astype(np.float32), dt)
    kp = t(rng.standard_normal((nb, hkv, page, d)).astype(np.float32), dt)
    vp = t(rng.standard_normal((nb, hkv, page, d)).astype(np.float32), dt)
    tbl = t(rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32))
    ln = t(np.array(lens, np.int32))
    out_ref = ft.attention_decode_paged(q, kp, vp, tbl, ln)
    codes_ref, scale_ref = ft.quantize_int8(out_ref, device_scale=True)
    for rep in range(2):  # the second call reuses the maxima scratch
        out, codes, scale = ft.attention_decode_paged_quant(q, kp, vp, tbl, ln,
                                                            device_scale=True)
        torch.cuda.synchronize()
        assert np.array_equal(raw(out), raw(out_ref)), f"{case} rep {rep}: out differs"
        assert torch.equal(codes, codes_ref), f"{case} rep {rep}: codes differ"
        assert scale.item() == scale_ref.item(), (scale.item(), scale_ref.item())
    empty = torch.tensor([n == 0 for n in lens], device=DEV)
    assert not codes[empty].any()  # empty rows are zero and quantise to 0
    # the scale is max |stored output| / 127 in float32
    expect = np.float32(out_ref.float().abs().max().item()) / np.float32(127.0)
    assert scale.item() == expect


def test_attention_decode_paged_quant_empty_and_errors():
    q = torch.zeros((0, 4, 128), dtype=torch.bfloat16, device=DEV)
    kp = torch.zeros((2, 2, 16, 128), dtype=torch.bfloat16, device=DEV)
    out, codes, scale = ft.attention_decode_paged_quant(
        q, kp, kp, torch.zeros((0, 1), dtype=torch.int32, device=DEV))
    assert out.shape == (0, 4, 128) and codes.shape == (0, 4, 128) and scale == 1.0
    with pytest.raises(TypeError, match="GPU tensors"):
        ft.attention_decode_paged_quant(np.zeros((1, 4, 8), np.float32),
                                        np.zeros((2, 2, 4, 8), np.float32),
                                        np.zeros((2, 2, 4, 8), np.float32),
                                        np.zeros((1, 1), np.int32))


# ---------------------------------------------------------------------------
# GEMM + next step (the K-split partials folded by the next kernel)
# ---------------------------------------------------------------------------

def wq_dev(gen, rows, cols):
    return (torch.randint(-127, 128, (rows, cols), device=DEV, generator=gen,
                          dtype=torch.int32).to(torch.int8),
            (torch.rand((rows,), device=DEV, generator=gen) * 9e-3 + 1e-3).float())


# (b, hq, hkv, d, k, switches): C4's QKV (K split 4 by default); the same
# unsplit; a split of 3 at a toy shape; 9 partials (two load batches) on a
# forced skinny kernel; the M = 1 GEMV (never split)
QKV_CASES = {
    "c4": (64, 32, 8, 128, 4096, {}),
    "c4_unsplit": (64, 32, 8, 128, 4096, {"FT_QGEMM_KSPLIT": 1}),
    "split3": (20, 8, 2, 64, 1024, {"FT_QGEMM_KSPLIT": 3}),
    "split9": (5, 4, 4, 32, 2304, {"FT_QGEMM_KERNEL": 1, "FT_QGEMM_KSPLIT": 9}),
    "gemv": (1, 8, 2, 64, 512, {}),
}


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("case", list(QKV_CASES))
def test_qgemm_rope_kv_append_equals_the_two_ops(dt, case, tuning):
    b, hq, hkv, d, k, sw = QKV_CASES[case]
    for name, v in sw.items():
        tuning(name, v)
    gen = torch.Generator(device=DEV).manual_seed(list(QKV_CASES).index(case))
    rng = np.random.default_rng(list(QKV_CASES).index(case))
    page = 16
    lens = rng.integers(0, 300, b).astype(np.int32)
    width = int(lens.max()) // page + 1
    nb = b * width + 3
    a = torch.randint(-127, 128, (b, k), device=DEV, generator=gen,
                      dtype=torch.int32).to(torch.int8)
    sa = torch.tensor([0.0123], dtype=torch.float32, device=DEV)
    w, ws = wq_dev(gen, (hq + 2 * hkv) * d, k)
    kp = torch.randn((nb, hkv, page, d), device=DEV, generator=gen).to(dt)
    vp = torch.randn((nb, hkv, page, d), device=DEV, generator=gen).to(dt)
    tbl = t(rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32))
    ln = t(lens)
    kp_ref, vp_ref = kp.clone(), vp.clone()
    qkv_ref = ft.qgemm_perchannel(a, sa, w, ws, out_dtype=dt)
    q_ref = ft.rope_kv_append_paged(qkv_ref, hq, hkv, kp_ref, vp_ref, tbl, ln,
                                    theta=500000.0, pos_offset=3, neox=True)
    for rep in range(2):
        q_rot, qkv = ft.qgemm_rope_kv_append_paged(a, sa, w, ws, hq, hkv, kp, vp, tbl, ln,
                                                   theta=500000.0, pos_offset=3, neox=True)
        torch.cuda.synchronize()
        assert np.array_equal(raw(qkv), raw(qkv_ref)), f"{case} rep {rep}: qkv differs"
        assert np.array_equal(raw(q_rot), raw(q_ref)), f"{case} rep {rep}: q differs"
        assert np.array_equal(raw(kp), raw(kp_ref)) and np.array_equal(raw(vp), raw(vp_ref))


# (m, n, k, residual, switches): C4's o_proj (K split 4); the same unsplit;
# 3 rows on a forced split of 9 (the one-launch small-row path of the chain
# against the fold's two passes); rows past 4096 columns (the row kernel's
# loop form); the decode GEMM (never split)
RMSQ_CASES = {
    "c4": (64, 4096, 4096, True, {}),
    "c4_unsplit": (64, 4096, 4096, True, {"FT_QGEMM_KSPLIT": 1}),
    "small_split9": (3, 1024, 2304, False, {"FT_QGEMM_KERNEL": 1, "FT_QGEMM_KSPLIT": 9}),
    "wide": (40, 5000, 512, True, {"FT_QGEMM_KSPLIT": 2}),
    "decode": (8, 2048, 1024, True, {}),
}


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("case", list(RMSQ_CASES))
def test_qgemm_rmsnorm_quant_equals_the_two_ops(dt, case, tuning):
    m, n, k, res, sw = RMSQ_CASES[case]
    for name, v in sw.items():
        tuning(name, v)
    gen = torch.Generator(device=DEV).manual_seed(50 + list(RMSQ_CASES).index(case))
    a = torch.randint(-127, 128, (m, k), device=DEV, generator=gen,
                      dtype=torch.int32).to(torch.int8)
    sa = torch.tensor([0.0031], dtype=torch.float32, device=DEV)
    w, ws = wq_dev(gen, n, k)
    nw = (torch.rand((n,), device=DEV, generator=gen) + 0.5).float()
    r = torch.randn((m, n), device=DEV, generator=gen).to(dt) if res else None
    y_ref = ft.qgemm_perchannel(a, sa, w, ws, out_dtype=dt)
    q_ref, s_ref = ft.rmsnorm_quant(y_ref, nw, residual=r, eps=1e-5, device_scale=True)
    for rep in range(2):
        y, q, s = ft.qgemm_rmsnorm_quant(a, sa, w, ws, nw, residual=r, eps=1e-5, out_dtype=dt,
                                         device_scale=True)
        torch.cuda.synchronize()
        assert np.array_equal(raw(y), raw(y_ref)), f"{case} rep {rep}: y differs"
        assert torch.equal(q, q_ref), f"{case} rep {rep}: codes differ"
        assert s.item() == s_ref.item()


# (m, inter, k, switches) of the gate/up GEMM + swiglu_quant. Per the GEMM
# dispatch rules, the first six run unsplit on the skinny ring kernel with
# the SwiGLU maxima in its epilogue: C4's shape (8 waves, 4 row blocks) at a
# short and at its full K, the same with FT_GRID_SYNC=1 (the epilogue writes
# its maxima and a second launch writes the codes, instead of folding the
# maxima in the launch with grid_max), 40 rows (4 row blocks, 24 rows past
# M), 17 rows (2 row blocks), and 4-wave workgroups (forced). The last three
# take the GEMM + swiglu_quant fallback: a K split (inter too small to fill
# the CUs), the decode GEMM (m <= 16), and inter not a multiple of the
# paired column tile.
SWQ_CASES = {
    "c4": (64, 14336, 512, {}),
    "c4_full_k": (64, 14336, 4096, {}),
    "c4_partials": (64, 14336, 512, {"FT_GRID_SYNC": 1}),
    "rows40": (40, 12288, 256, {}),
    "rows17": (17, 12288, 256, {}),
    "nw4": (64, 6144, 512, {"FT_QGEMM_SK_WAVES": 4}),
    "split": (64, 768, 1024, {}),
    "decode": (8, 12288, 512, {}),
    "odd_tile": (64, 12320, 256, {}),
}


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("case", list(SWQ_CASES))
def test_qgemm_swiglu_quant_equals_the_two_ops(dt, case, tuning):
    m, inter, k, sw = SWQ_CASES[case]
    for name, v in sw.items():
        tuning(name, v)
    gen = torch.Generator(device=DEV).manual_seed(90 + list(SWQ_CASES).index(case))
    a = torch.randint(-127, 128, (m, k), device=DEV, generator=gen,
                      dtype=torch.int32).to(torch.int8)
    sa = torch.tensor([0.0007], dtype=torch.float32, device=DEV)
    w, ws = wq_dev(gen, 2 * inter, k)
    h_ref = ft.qgemm_perchannel(a, sa, w, ws, out_dtype=dt)
    q_ref, s_ref = ft.swiglu_quant(h_ref[:, :inter], h_ref[:, inter:], device_scale=True)
    for rep in range(2):
        h, q, s = ft.qgemm_swiglu_quant(a, sa, w, ws, out_dtype=dt, device_scale=True)
        torch.cuda.synchronize()
        assert np.array_equal(raw(h), raw(h_ref)), f"{case} rep {rep}: h differs"
        assert torch.equal(q, q_ref), f"{case} rep {rep}: codes differ"
        assert s.item() == s_ref.item(), f"{case} rep {rep}: scale differs"


def test_qgemm_swiglu_quant_maximum_from_the_epilogue_and_errors():
    # the SwiGLU maximum sits in one element: a single large activation row
    # entry times a large weight entry (gate) makes one output dominate, so
    # a lost workgroup partial or a wrong gate/up pairing changes the scale
    gen = torch.Generator(device=DEV).manual_seed(7)
    m, inter, k = 64, 14336, 256
    a = torch.randint(-3, 4, (m, k), device=DEV, generator=gen, dtype=torch.int32).to(torch.int8)
    w, ws = wq_dev(gen, 2 * inter, k)
    w = (w // 16).contiguous()
    a[37, 5] = 127
    w[9001, 5] = 127            # gate column 9001
    w[inter + 9001, 5] = -127   # its up partner
    sa = torch.tensor([0.01], dtype=torch.float32, device=DEV)
    h_ref = ft.qgemm_perchannel(a, sa, w, ws, out_dtype=torch.bfloat16)
    q_ref, s_ref = ft.swiglu_quant(h_ref[:, :inter], h_ref[:, inter:])
    h, q, s = ft.qgemm_swiglu_quant(a, sa, w, ws, out_dtype=torch.bfloat16)
    assert s == s_ref and torch.equal(q, q_ref)
    assert q[37, 9001].item() in (-127, 127)
    with pytest.raises(ValueError, match="even row count"):
        ft.qgemm_swiglu_quant(a, sa, w[:-1].contiguous(), ws[:-1].contiguous())


def test_decode_layer_graph_replays_equal_eager():
    dev = torch.device(DEV)
    gen = torch.Generator(device=dev).manual_seed(77)
    b, hq, hkv, d, hid, inter, page = 4, 8, 2, 64, 512, 768, 16
    bf = torch.bfloat16

    def wq(rows, cols):
        return (torch.randint(-127, 128, (rows, cols), device=dev, generator=gen,
                              dtype=torch.int32).to(torch.int8),
                (torch.rand((rows,), device=dev, generator=gen) * 9e-3 + 1e-3).float())
    wn1 = (torch.rand((hid,), device=dev, generator=gen) + 0.5).float()
    wn2 = (torch.rand((hid,), device=dev, generator=gen) + 0.5).float()
    wqkv, wo, wgu, wd = wq((hq + 2 * hkv) * d, hid), wq(hid, hq * d), wq(2 * inter, hid), \
        wq(hid, inter)
    lens = torch.tensor([5, 300, 17, 100], dtype=torch.int32, device=dev)
    npg = (301 + page - 1) // page
    table = torch.arange(b * npg, dtype=torch.int32, device=dev).reshape(b, npg)
    kp = torch.randn((b * npg, hkv, page, d), device=dev, generator=gen, dtype=bf)
    vp = torch.randn((b * npg, hkv, page, d), device=dev, generator=gen, dtype=bf)
    x = torch.randn((b, hid), device=dev, generator=gen).to(bf)

    def layer():
        q1, s1 = ft.rmsnorm_quant(x, wn1, eps=1e-5, device_scale=True)
        qkv = ft.qgemm_perchannel(q1, s1, *wqkv, out_dtype=bf)
        qr = ft.rope_kv_append_paged(qkv, hq, hkv, kp, vp, table, lens,
                                     theta=500000.0, neox=True)
        att = ft.attention_decode_paged(qr, kp, vp, table, lens + 1)
        qa, sa = ft.quantize_int8(att.reshape(b, hq * d), device_scale=True)
        o = ft.qgemm_perchannel(qa, sa, *wo, out_dtype=bf)
        q2, s2 = ft.rmsnorm_quant(o, wn2, residual=x, eps=1e-5, device_scale=True)
        h = ft.qgemm_perchannel(q2, s2, *wgu, out_dtype=bf)
        q3, s3 = ft.swiglu_quant(h[:, :inter], h[:, inter:], device_scale=True)
        return ft.qgemm_perchannel(q3, s3, *wd, out_dtype=bf)

    ref = layer().clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = layer()
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {rep} differs from the eager layer"
        eager = layer()               # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager, ref)
