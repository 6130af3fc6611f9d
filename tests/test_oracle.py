"""Pins the CPU oracle (oracle/oracle.cpp) before it is trusted as the GPU
path's checker. Each oracle function is checked against
  - the reference tests' known-answer cases (file:line cited per test),
  - independent float64 / exact-integer numpy references (tests/refs.py),
  - invariants the mathematics fixes (identity at position 0, norm
    conservation, paged == materialised contiguous bit-for-bit, ...),
  - the committed golden vectors (tests/golden/),
chosen so that a plausible slip (wrong sign, swapped index, dropped term,
transposed operand) fails at least one of them. A deliberately broken copy of
the oracle arithmetic is checked to FAIL these pins (test_pins_catch_*).
"""

import math
import os

import numpy as np
import pytest

import oracle
from tests import refs

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")


# ---------------------------------------------------------------------------
# quantize (reference tests/test_quantize.py)
# ---------------------------------------------------------------------------


def test_quantize_known_answer():
    # test_quantize.py:16-22
    q, s = oracle.quantize_int8(np.array([-2.0, -1.0, 0.0, 1.0, 2.0], np.float32))
    assert s == pytest.approx(2.0 / 127.0)
    assert q.dtype == np.int8
    assert list(q) == [-127, -64, 0, 64, 127]   # 63.5 rounds half-to-even -> 64


def test_quantize_zero_and_extremes():
    q, s = oracle.quantize_int8(np.zeros(8, np.float32))       # test_quantize.py:34-39
    assert s == 1.0 and (q == 0).all()
    q, s = oracle.quantize_int8(np.array([1e30, -1e30], np.float32))  # :42-45
    assert q[0] == 127 and q[1] == -127


def test_quantize_roundtrip_bound_and_closed_form():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(10000).astype(np.float32)
    q, s = oracle.quantize_int8(x)
    assert np.abs(q.astype(np.float32) * s - x).max() <= s * 0.51  # :25-31
    rq, rs = refs.ref_quantize(x)
    assert s == rs
    np.testing.assert_array_equal(q, rq)


def test_quantize_half_even_ties():
    # x * inv lands exactly on k + 0.5 for these values: rint must go to even
    x = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.5], np.float32)
    q, s = oracle.quantize_int8(x)
    assert s == 1.0
    assert list(q) == [127, 0, 2, 2, 0, -2, 4]


def test_dequantize_closed_form_and_roundtrip():
    # dequantize_int8_cpu is q * scale in float32 (quantize.cu:188-193); the
    # reference's round-trip bound test_quantize.py:25-31 goes through it
    rng = np.random.default_rng(0)
    x = rng.standard_normal(10000).astype(np.float32)
    q, s = oracle.quantize_int8(x)
    back = oracle.dequantize_int8(q, s)
    assert back.dtype == np.float32
    assert np.abs(back - x).max() <= s * 0.51
    np.testing.assert_array_equal(back, q.astype(np.float32) * np.float32(s))
    # every code, an awkward scale: exact float32 products
    codes = np.arange(-128, 128, dtype=np.int8)
    sc = np.float32(0.0123456)
    np.testing.assert_array_equal(oracle.dequantize_int8(codes, float(sc)),
                                  codes.astype(np.float64).astype(np.float32) * sc)


def test_qadd_is_the_explicit_pipeline():
    # test_quantize.py:48-66: qadd equals dequant -> add -> requant; here the
    # pipeline is evaluated independently in numpy float32 (two rounded
    # products, a rounded sum) and quantized by the numpy closed form
    rng = np.random.default_rng(1)
    for n in (1, 7, 1000, 65537):
        a = rng.standard_normal(n).astype(np.float32)
        b = (rng.standard_normal(n) * 3).astype(np.float32)
        qa, sa = oracle.quantize_int8(a)
        qb, sb = oracle.quantize_int8(b)
        v = (qa.astype(np.float32) * np.float32(sa)) + (qb.astype(np.float32) * np.float32(sb))
        rq, rs = refs.ref_quantize(v)
        q, s = oracle.qadd_int8(qa, sa, qb, sb)
        assert s == rs
        np.testing.assert_array_equal(q, rq)
        # the reference test's tolerance statement holds too
        assert np.abs(q.astype(np.float32) * s - v).max() <= s * 0.51


def test_qadd_cancellation_and_zero():
    # qa*sa + qb*sb == 0 everywhere: scale 1.0, all codes 0 (make_scale)
    qa = np.array([5, -7, 0, 127], np.int8)
    q, s = oracle.qadd_int8(qa, 0.5, -qa, 0.5)
    assert s == 1.0 and (q == 0).all()
    # one dominant element maps to +-127; the sum saturates nothing else
    q, s = oracle.qadd_int8(np.array([127, 1], np.int8), 1.0,
                            np.array([127, -1], np.int8), 1.0)
    assert s == pytest.approx(254.0 / 127.0) and list(q) == [127, 0]


# ---------------------------------------------------------------------------
# qgemm (reference tests/test_qgemm.py, test_qgemm_perchannel.py)
# ---------------------------------------------------------------------------


def _rand_q(rng, rows, k):
    return rng.integers(-127, 128, size=(rows, k)).astype(np.int8)


@pytest.mark.parametrize("m,n,k", [(1, 8, 16), (3, 5, 7), (65, 63, 33),
                                   (17, 200, 129), (100, 50, 1)])
def test_qgemm_exact(m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    a, b = _rand_q(rng, m, k), _rand_q(rng, n, k)
    np.testing.assert_array_equal(oracle.qgemm_i32(a, b), refs.ref_qgemm_i32(a, b))
    np.testing.assert_array_equal(oracle.qgemm(a, 0.03, b, 0.02),
                                  refs.ref_qgemm(a, 0.03, b, 0.02))
    sb = (10.0 ** rng.uniform(-2.0, 0.3, n)).astype(np.float32)
    np.testing.assert_array_equal(oracle.qgemm_perchannel(a, 0.03, b, sb),
                                  refs.ref_qgemm_pc(a, 0.03, b, sb))


def test_qgemm_extremes_and_k0():
    a = np.full((4, 100), -127, np.int8)    # test_qgemm.py:53-59
    b = np.full((3, 100), -127, np.int8)
    y = oracle.qgemm(a, 1.0, b, 1.0)
    assert (y == 127 * 127 * 100).all()
    z = oracle.qgemm(np.zeros((4, 0), np.int8), 0.5, np.zeros((3, 0), np.int8), 0.25)
    np.testing.assert_array_equal(z, np.zeros((4, 3), np.float32))


def test_qgemm_equal_channel_scales_match_per_tensor():
    # test_qgemm_perchannel.py:73-84
    rng = np.random.default_rng(5)
    a, b = _rand_q(rng, 33, 129), _rand_q(rng, 47, 129)
    np.testing.assert_array_equal(
        oracle.qgemm_perchannel(a, 0.03, b, np.full(47, 0.02, np.float32)),
        oracle.qgemm(a, 0.03, b, np.float32(0.02)))


# ---------------------------------------------------------------------------
# attention (reference tests/test_attention.py, test_attention_paged.py)
# ---------------------------------------------------------------------------

SHAPES = [  # test_attention.py:57-67
    (1, 8, 2, 1, 64, False),
    (1, 32, 8, 517, 128, False),
    (1, 32, 32, 100, 64, False),
    (3, 12, 4, 64, 32, True),
    (2, 6, 3, 33, 8, True),
    (1, 4, 1, 16, 4, True),
    (1, 8, 8, 0, 64, False),
    (2, 4, 4, 0, 32, True),
    (1, 2, 2, 1024, 256, False),
]


def _case(rng, b, hq, hkv, t, d, with_lens):
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    k = rng.standard_normal((b, hkv, t, d)).astype(np.float32)
    v = rng.standard_normal((b, hkv, t, d)).astype(np.float32)
    lens = rng.integers(0, t + 1, size=b).astype(np.int32) if with_lens else None
    return q, k, v, lens


@pytest.mark.parametrize("b,hq,hkv,t,d,with_lens", SHAPES)
def test_decode_matches_float64(b, hq, hkv, t, d, with_lens):
    rng = np.random.default_rng(b * 1000 + hq * 31 + hkv * 7 + t + d)
    q, k, v, lens = _case(rng, b, hq, hkv, t, d, with_lens)
    y = oracle.attention_decode(q, k, v, lens)
    np.testing.assert_allclose(y, refs.ref_decode(q, k, v, lens), rtol=1e-4, atol=1e-5)


def test_decode_gqa_constant_v_and_padding():
    rng = np.random.default_rng(5)   # test_attention.py:82-95
    b, hq, hkv, t, d = 1, 6, 3, 4, 8
    q = np.ones((b, hq, d), np.float32)
    k = np.zeros((b, hkv, t, d), np.float32)
    v = np.broadcast_to(rng.standard_normal((b, hkv, 1, d)).astype(np.float32),
                        (b, hkv, t, d)).copy()
    y = oracle.attention_decode(q, k, v)
    for h in range(hq):
        np.testing.assert_allclose(y[0, h], v[0, h // 2, 0], rtol=1e-6, atol=1e-7)
    # poisoned padding past lens is ignored; len 0 -> zero row (:98-115)
    q, k, v, _ = _case(rng, 2, 8, 4, 16, 32, False)
    lens = np.array([16, 5], np.int32)
    y = oracle.attention_decode(q, k, v, lens)
    k2, v2 = k.copy(), v.copy()
    k2[1, :, 5:] = 1e6
    v2[1, :, 5:] = 1e6
    np.testing.assert_array_equal(oracle.attention_decode(q, k2, v2, lens), y)
    y0 = oracle.attention_decode(q, k, v, np.array([0, 5], np.int32))
    assert (y0[0] == 0).all()


def test_decode_errors():
    q = np.zeros((1, 6, 32), np.float32)
    k = np.zeros((1, 2, 8, 32), np.float32)
    with pytest.raises(ValueError):
        oracle.attention_decode(np.zeros((1, 5, 32), np.float32), k, k)
    with pytest.raises(ValueError):
        oracle.attention_decode(np.zeros((1, 2, 30), np.float32),
                                np.zeros((1, 1, 4, 30), np.float32),
                                np.zeros((1, 1, 4, 30), np.float32))
    with pytest.raises(ValueError):
        oracle.attention_decode(q, k, k, np.array([9], np.int32))


def _paged_case(rng, b, hq, hkv, d, nb, lens, page=16):
    width = max((l + page - 1) // page for l in lens)
    kp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    vp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    tbl = rng.integers(0, nb, (b, width)).astype(np.int32)
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    return q, kp, vp, tbl, np.asarray(lens, np.int32)


def test_paged_equals_materialised_contiguous_bit_exact():
    # test_attention_paged.py:62-70
    rng = np.random.default_rng(41)
    q, kp, vp, tbl, lens = _paged_case(rng, 3, 8, 2, 64, 20, [37, 16, 48])
    out_p = oracle.attention_decode_paged(q, kp, vp, tbl, lens)
    kc, vc = refs.materialize_paged(kp, tbl), refs.materialize_paged(vp, tbl)
    np.testing.assert_array_equal(out_p, oracle.attention_decode(q, kc, vc, lens))
    np.testing.assert_allclose(out_p, refs.ref_decode_paged(q, kp, vp, tbl, lens),
                               rtol=1e-4, atol=1e-5)


def test_paged_single_token_is_v_and_errors():
    rng = np.random.default_rng(43)   # test_attention_paged.py:85-94
    q, kp, vp, tbl, lens = _paged_case(rng, 2, 2, 2, 128, 4, [1, 16])
    out = oracle.attention_decode_paged(q, kp, vp, tbl, lens)
    np.testing.assert_allclose(out[0, 0], vp[tbl[0, 0], 0, 0], atol=1e-6)
    bad = tbl.copy()
    bad[0, 0] = 99
    with pytest.raises(ValueError):
        oracle.attention_decode_paged(q, kp, vp, bad, lens)


PREFILL_SHAPES = [  # reference tests/test_attention.py:176-184
    (1, 4, 2, 1, 32), (1, 8, 8, 5, 64), (2, 6, 3, 17, 16), (1, 32, 8, 40, 128),
    (1, 4, 1, 33, 8), (1, 8, 2, 64, 256), (1, 4, 2, 9, 512),
]


@pytest.mark.parametrize("b,hq,hkv,s,d", PREFILL_SHAPES)
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_matches_float64(b, hq, hkv, s, d, causal):
    # test_attention.py:187-197: rtol 1e-4, atol 1e-5 against float64
    rng = np.random.default_rng(b * 100 + hq * 17 + s * 3 + d + causal)
    q = rng.standard_normal((b, hq, s, d)).astype(np.float32)
    k = rng.standard_normal((b, hkv, s, d)).astype(np.float32)
    v = rng.standard_normal((b, hkv, s, d)).astype(np.float32)
    y = oracle.attention_prefill(q, k, v, causal)
    np.testing.assert_allclose(y, refs.ref_prefill(q, k, v, causal), rtol=1e-4, atol=1e-5)


def test_prefill_first_row_s1_decode_and_errors():
    rng = np.random.default_rng(50)
    # test_attention.py:200-210: causal row 0 attends only to key 0 -> v[0]
    q = rng.standard_normal((1, 4, 9, 32)).astype(np.float32)
    k = rng.standard_normal((1, 2, 9, 32)).astype(np.float32)
    v = rng.standard_normal((1, 2, 9, 32)).astype(np.float32)
    y = oracle.attention_prefill(q, k, v, True)
    for h in range(4):
        np.testing.assert_array_equal(y[0, h, 0], v[0, h // 2, 0])
    # causal row i is the decode step over keys [0, i] (bit-identical loops)
    for i in (3, 8):
        dec = oracle.attention_decode(q[:, :, i], k[:, :, :i + 1], v[:, :, :i + 1])
        np.testing.assert_array_equal(y[:, :, i], dec)
    # bidirectional: every row is the decode step over all S keys
    yb = oracle.attention_prefill(q, k, v, False)
    np.testing.assert_array_equal(yb[:, :, 2], oracle.attention_decode(q[:, :, 2], k, v))
    # test_attention.py:227-238: shape contract
    with pytest.raises(ValueError):
        oracle.attention_prefill(np.zeros((1, 5, 8, 32), np.float32),
                                 np.zeros((1, 2, 8, 32), np.float32),
                                 np.zeros((1, 2, 8, 32), np.float32))
    with pytest.raises(ValueError):
        oracle.attention_prefill(np.zeros((1, 4, 8, 30), np.float32),
                                 np.zeros((1, 2, 8, 30), np.float32),
                                 np.zeros((1, 2, 8, 30), np.float32))


def test_kv_append_copies_and_bounds():
    rng = np.random.default_rng(9)
    b, hkv, t, d = 3, 2, 10, 8
    kc = rng.standard_normal((b, hkv, t, d)).astype(np.float32)
    vc = rng.standard_normal((b, hkv, t, d)).astype(np.float32)
    kn = rng.standard_normal((b, hkv, d)).astype(np.float32)
    vn = rng.standard_normal((b, hkv, d)).astype(np.float32)
    lens = np.array([0, 4, 9], np.int32)
    ek, ev = kc.copy(), vc.copy()
    for bi in range(b):
        ek[bi, :, lens[bi]] = kn[bi]
        ev[bi, :, lens[bi]] = vn[bi]
    oracle.kv_append(kc, vc, kn, vn, lens)
    np.testing.assert_array_equal(kc, ek)
    np.testing.assert_array_equal(vc, ev)
    with pytest.raises(ValueError):
        oracle.kv_append(kc, vc, kn, vn, np.array([0, 4, 10], np.int32))
    # paged
    nb, page = 7, 4
    kp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    vp = kp.copy()
    tbl = np.array([[3, 1, 6], [0, 2, 5], [4, 4, 4]], np.int32)
    plens = np.array([5, 0, 11], np.int32)
    ek = kp.copy()
    for bi in range(b):
        blk, off = tbl[bi, plens[bi] // page], plens[bi] % page
        ek[blk, :, off] = kn[bi]
    oracle.kv_append_paged(kp, vp, tbl, kn, vn, plens)
    np.testing.assert_array_equal(kp, ek)
    with pytest.raises(ValueError):
        oracle.kv_append_paged(kp, vp, tbl, kn, vn, np.array([5, 0, 12], np.int32))


# ---------------------------------------------------------------------------
# rmsnorm / rope / swiglu (reference test_rmsnorm.py, test_rope.py,
# test_swiglu.py)
# ---------------------------------------------------------------------------


def test_rmsnorm_known_answer_and_float64():
    y = oracle.rmsnorm(np.array([[3.0, 4.0]], np.float32), np.ones(2, np.float32),
                       eps=1e-12)   # test_rmsnorm.py:37-43
    inv = 1.0 / math.sqrt(12.5)
    assert y[0] == pytest.approx([3.0 * inv, 4.0 * inv], abs=1e-6)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((8, 257)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 257).astype(np.float32)
    r = rng.uniform(-1, 1, x.shape).astype(np.float32)
    np.testing.assert_allclose(oracle.rmsnorm(x, w, r, eps=1e-5),
                               refs.ref_rmsnorm(x, w, 1e-5, r), rtol=1e-5, atol=1e-6)
    # residual == shifted input (test_rmsnorm.py:54-61)
    np.testing.assert_allclose(oracle.rmsnorm(x, w, r), oracle.rmsnorm(x + r, w),
                               atol=1e-6)


@pytest.mark.parametrize("neox", [False, True])
def test_rope_float64_and_invariants(neox):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((6, 16)).astype(np.float32)
    for off in (0, 7, 8192):
        np.testing.assert_allclose(oracle.rope(x, 10000.0, off, neox),
                                   refs.ref_rope(x, 10000.0, off, neox),
                                   rtol=0, atol=1e-6)
    y = oracle.rope(x, 10000.0, 0, neox)
    np.testing.assert_array_equal(y[0], x[0])          # position 0 = identity
    full = oracle.rope(x, 10000.0, 0, neox)
    np.testing.assert_allclose(oracle.rope(x[2:4], 10000.0, 2, neox), full[2:4],
                               atol=1e-6)              # offset == slice
    half = 8
    a = (x[:, :half], x[:, half:]) if neox else (x[:, 0::2], x[:, 1::2])
    b = (y[:, :half], y[:, half:]) if neox else (y[:, 0::2], y[:, 1::2])
    np.testing.assert_allclose(np.hypot(*b), np.hypot(*a), atol=1e-5)  # norm kept
    np.testing.assert_allclose(oracle.rope(x, 500000.0, 3, neox),
                               refs.ref_rope(x, 500000.0, 3, neox), atol=1e-6)


def test_swiglu_closed_form_and_extremes():
    rng = np.random.default_rng(3)
    g = rng.standard_normal(1000).astype(np.float32) * 4
    u = rng.standard_normal(1000).astype(np.float32)
    np.testing.assert_allclose(oracle.swiglu(g, u), refs.ref_swiglu(g, u),
                               rtol=1e-6, atol=1e-7)
    y = oracle.swiglu(np.array([-100.0, 0.0, 100.0], np.float32),
                      np.array([3.0, 5.0, 2.0], np.float32))
    np.testing.assert_allclose(y, [0.0, 0.0, 200.0], atol=1e-6)


# ---------------------------------------------------------------------------
# fused decode-chain steps: compositions of the pinned functions above, plus
# the GPU-order RMSNorm (rmsnorm_blocked)
# ---------------------------------------------------------------------------


def test_rmsnorm_blocked_exact_on_integer_data_and_close_otherwise():
    rng = np.random.default_rng(12)
    # integer data: every partial sum is exact, so any order gives the same
    # bits -> blocked == sequential reference order, bit for bit
    x = rng.integers(-8, 9, (5, 4096)).astype(np.float32)
    w = rng.integers(1, 4, 4096).astype(np.float32)
    r = rng.integers(-3, 4, x.shape).astype(np.float32)
    np.testing.assert_array_equal(oracle.rmsnorm_blocked(x, w, r, 1e-5),
                                  oracle.rmsnorm(x, w, r, 1e-5))
    # known answer (test_rmsnorm.py:37-43 padded to 4 columns)
    y = oracle.rmsnorm_blocked(np.array([[3.0, 4.0, 0.0, 0.0]], np.float32),
                               np.ones(4, np.float32), eps=1e-12)
    inv = 1.0 / math.sqrt(25.0 / 4)
    assert y[0] == pytest.approx([3.0 * inv, 4.0 * inv, 0, 0], abs=1e-6)
    # random data, ragged chunk counts (cols / 4 not a multiple of 256)
    for cols in (4, 1028, 4096, 5000):
        x = rng.standard_normal((3, cols)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
        np.testing.assert_allclose(oracle.rmsnorm_blocked(x, w),
                                   refs.ref_rmsnorm(x, w, 1e-6), rtol=2e-6, atol=1e-7)
    with pytest.raises(ValueError):
        oracle.rmsnorm_blocked(np.ones((1, 6), np.float32), np.ones(6, np.float32))


def test_rmsnorm_quant_is_the_chain_and_near_the_reference_order():
    rng = np.random.default_rng(13)
    x = rng.standard_normal((4, 2048)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 2048).astype(np.float32)
    r = rng.standard_normal(x.shape).astype(np.float32)
    q, s = oracle.rmsnorm_quant(x, w, r, 1e-5)
    q2, s2 = oracle.quantize_int8(oracle.rmsnorm_blocked(x, w, r, 1e-5))
    np.testing.assert_array_equal(q, q2)
    assert s == s2
    # the reference's own order (rmsnorm_cpu -> quantize_int8_cpu): the sums
    # differ in rounding only, so codes move by at most one step
    q3, s3 = oracle.quantize_int8(oracle.rmsnorm(x, w, r, 1e-5))
    assert s == pytest.approx(s3, rel=1e-5)
    assert np.abs(q.astype(int) - q3.astype(int)).max() <= 1
    # known answer: [3, 4, 0, 0] -> y = [0.6, 0.8, 0, 0] * 2 -> scale 1.6/127
    q, s = oracle.rmsnorm_quant(np.array([[3.0, 4.0, 0.0, 0.0]], np.float32),
                                np.ones(4, np.float32), eps=1e-12)
    assert s == pytest.approx(1.6 / 127, rel=1e-6)
    np.testing.assert_array_equal(q, [[95, 127, 0, 0]])


def test_swiglu_quant_strided_halves_and_closed_form():
    rng = np.random.default_rng(14)
    h = (rng.standard_normal((6, 2 * 300)) * 3).astype(np.float32)
    g, u = h[:, :300], h[:, 300:]
    q, s = oracle.swiglu_quant(g, u)
    q2, s2 = oracle.quantize_int8(oracle.swiglu(np.ascontiguousarray(g),
                                                np.ascontiguousarray(u)))
    np.testing.assert_array_equal(q, q2)
    assert s == s2
    y = refs.ref_swiglu(g, u)
    assert s == pytest.approx(np.abs(y).max() / 127, rel=1e-6)
    np.testing.assert_array_equal(q, np.clip(np.rint(y / s), -127, 127))
    q, s = oracle.swiglu_quant(np.zeros((2, 8), np.float32), np.ones((2, 8), np.float32))
    assert s == 1.0 and not q.any()


@pytest.mark.parametrize("neox", [False, True])
def test_rope_kv_append_oracle_positions_and_slots(neox):
    rng = np.random.default_rng(15 + neox)
    b, hq, hkv, d, page, width = 3, 4, 2, 16, 4, 3
    nb = b * width + 1
    qkv = rng.standard_normal((b, (hq + 2 * hkv) * d)).astype(np.float32)
    kp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    vp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    tbl = rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32)
    lens = np.array([0, 5, 11], np.int32)
    k0, v0 = kp.copy(), vp.copy()
    qo = oracle.rope_kv_append_paged(qkv, hq, hkv, kp, vp, tbl, lens, 10000.0, 7, neox)
    heads = qkv.reshape(b, hq + 2 * hkv, d)
    for i in range(b):
        pos = int(lens[i]) + 7
        np.testing.assert_allclose(qo[i], refs.ref_rope(heads[i, :hq], 10000.0, 0, neox,
                                                        positions=np.full(hq, pos)),
                                   atol=1e-6)
        blk, off = tbl[i, lens[i] // page], lens[i] % page
        np.testing.assert_allclose(kp[blk, :, off],
                                   refs.ref_rope(heads[i, hq:hq + hkv], 10000.0, 0, neox,
                                                 positions=np.full(hkv, pos)), atol=1e-6)
        np.testing.assert_array_equal(vp[blk, :, off], heads[i, hq + hkv:])
        kp[blk, :, off] = k0[blk, :, off]
        vp[blk, :, off] = v0[blk, :, off]
    np.testing.assert_array_equal(kp, k0)      # nothing else written
    np.testing.assert_array_equal(vp, v0)


# ---------------------------------------------------------------------------
# golden vectors (tests/golden/make_golden.py: numpy float64 / exact ints)
# ---------------------------------------------------------------------------


def test_golden_vectors():
    g = np.load(GOLDEN, allow_pickle=False)
    np.testing.assert_allclose(
        oracle.attention_decode(g["dec_q"], g["dec_k"], g["dec_v"], g["dec_lens"]),
        g["dec_out"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(
        oracle.attention_decode_paged(g["pg_q"], g["pg_kp"], g["pg_vp"], g["pg_tbl"],
                                      g["pg_lens"]),
        g["pg_out"], rtol=1e-4, atol=1e-5)
    q, s = oracle.quantize_int8(g["qz_x"])
    np.testing.assert_array_equal(q, g["qz_q"])
    assert s == float(g["qz_scale"])
    np.testing.assert_array_equal(oracle.qgemm_i32(g["gm_a"], g["gm_b"]), g["gm_acc"])
    np.testing.assert_array_equal(
        oracle.qgemm_perchannel(g["gm_a"], float(g["gm_sa"]), g["gm_b"], g["gm_sb"]),
        g["gm_y"])
    np.testing.assert_allclose(oracle.rmsnorm(g["rn_x"], g["rn_w"], g["rn_r"], 1e-5),
                               g["rn_y"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(oracle.rope(g["rp_x"], 10000.0, 8192, True),
                               g["rp_y"], atol=1e-6)
    np.testing.assert_allclose(oracle.swiglu(g["sw_g"], g["sw_u"]), g["sw_y"],
                               rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------------------
# the pins must catch plausible mistakes (planted in a CPU copy, never in
# the product)
# ---------------------------------------------------------------------------


def test_pins_catch_transposed_gqa_mapping():
    rng = np.random.default_rng(11)
    q, k, v, _ = _case(rng, 1, 8, 2, 40, 16, False)
    # wrong mapping h % Hkv instead of h // G changes the answer visibly
    wrong = np.stack([refs.ref_decode(q[:, [h]], k[:, [h % 2]], v[:, [h % 2]])[:, 0]
                      for h in range(8)], axis=1)
    assert not np.allclose(wrong, oracle.attention_decode(q, k, v), atol=1e-3)


def test_pins_catch_round_half_away():
    x = np.array([0.5, 1.5, 2.5, -2.5], np.float32)
    away = np.sign(x) * np.floor(np.abs(x) + 0.5)
    q, _ = oracle.quantize_int8(np.concatenate([x, [127.0]]).astype(np.float32))
    assert not np.array_equal(q[:4], away.astype(np.int8))


# ---------------------------------------------------------------------------
# post-logits sampling (reference tests/test_sampling.py, test_sample_topp.py,
# test_decode_step.py, test_argmax_batched.py)
# ---------------------------------------------------------------------------


def test_splitmix_uniform_matches_integer_restatement():
    for seed in [0, 1, 7, 42, 123, 12345, 2**40 + 3, 2**63 - 1]:
        assert oracle.splitmix_uniform(seed) == refs.splitmix_uniform(seed)
    us = [oracle.splitmix_uniform(s) for s in range(2000)]
    assert min(us) >= 0.0 and max(us) < 1.0 and 0.45 < np.mean(us) < 0.55


def test_argmax_batched_ties_nan_and_numpy():
    # test_sampling.py:79-82 / test_argmax_batched.py:41-53: earliest index
    x = np.array([[1, 3, 3, 2], [5, 5, 1, 0], [-np.inf, -np.inf, -np.inf, -np.inf],
                  [np.nan, 9, 1, 2], [1, np.nan, 7, 7]], np.float32)
    np.testing.assert_array_equal(oracle.argmax_batched(x), [1, 0, 0, 0, 2])
    rng = np.random.default_rng(0)
    y = rng.integers(-5, 5, (64, 300)).astype(np.float32)   # many ties
    np.testing.assert_array_equal(oracle.argmax_batched(y), np.argmax(y, axis=1))


def test_repetition_penalty_closed_form():
    # test_sampling.py:104-125: positive logits divide, negative multiply,
    # zero unchanged, duplicates applied once, empty ids = identity
    x = np.array([2.0, -2.0, 0.0, 4.0], np.float32)
    y = oracle.repetition_penalty(x, [0, 1, 2, 0, 0], 2.0)
    np.testing.assert_array_equal(y, [1.0, -4.0, 0.0, 4.0])
    np.testing.assert_array_equal(oracle.repetition_penalty(x, [], 3.0), x)
    with pytest.raises(ValueError):
        oracle.repetition_penalty(x, [4], 2.0)
    with pytest.raises(ValueError):
        oracle.repetition_penalty(x, [0], 0.0)


def test_sample_topp_known_answers():
    # test_sample_topp.py:37-43: peaked logits at low temperature -> the peak
    peak = np.array([10.0] + [0.0] * 49, np.float32)
    assert {oracle.sample_topp(peak, 0.9, 0.1, s) for s in range(16)} == {0}
    # :45-50: a very high temperature spreads the draws
    assert len({oracle.sample_topp(peak, 1.0, 1e4, s) for s in range(64)}) > 10
    # flat logits, p = 1: the order is the index order and every mass is 1,
    # so the token is the first prefix reaching u * n: ceil(u n) - 1
    flat = np.zeros(32, np.float32)
    for s in range(50):
        u = refs.splitmix_uniform(s)
        assert oracle.sample_topp(flat, 1.0, 1.0, s) == max(0, int(np.ceil(u * 32)) - 1)
    # :99-111: parameter contract
    for args in [(0.0, 1.0), (1.5, 1.0), (0.9, 0.0)]:
        with pytest.raises(ValueError):
            oracle.sample_topp(np.ones(4, np.float32), *args)
    with pytest.raises(ValueError):
        oracle.sample_topp(np.zeros(0, np.float32), 0.9)


def test_sample_topp_matches_float64_reference_and_nucleus():
    # the oracle against an independent float64 restatement of the same rule;
    # a differing token is only allowed where a threshold sits within float32
    # summation error of a prefix boundary
    rng = np.random.default_rng(5)
    for n, scale in [(100, 3.0), (2000, 2.0), (50000, 1.0)]:
        logits = (rng.standard_normal(n) * scale).astype(np.float32)
        for p, t in [(0.9, 1.0), (0.5, 0.7), (1.0, 1.3)]:
            for seed in range(25):
                got = oracle.sample_topp(logits, p, t, seed)
                want, margin = refs.ref_topp(logits, p, t, seed)
                assert got == want or margin < 1e-4, (n, p, t, seed, got, want, margin)
    # test_sample_topp.py:87-96: never outside the nucleus
    logits = (rng.standard_normal(100) * 3).astype(np.float32)
    probs = np.exp(logits.astype(np.float64) - logits.max())
    probs /= probs.sum()
    order = np.argsort(-probs, kind="stable")
    nucleus = set(order[:np.searchsorted(np.cumsum(probs[order]), 0.7) + 1].tolist())
    assert all(oracle.sample_topp(logits, 0.7, 1.0, s) in nucleus for s in range(200))


def test_sample_topp_distribution_matches_softmax():
    # test_sample_topp.py:67-84: frequencies track the renormalised nucleus
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal(8) * 2).astype(np.float32)
    probs = np.exp(logits.astype(np.float64) - logits.max())
    probs /= probs.sum()
    n = 6000
    counts = np.bincount([oracle.sample_topp(logits, 0.95, 1.0, s) for s in range(n)],
                         minlength=8)
    order = np.argsort(-probs)
    keep = order[:np.searchsorted(np.cumsum(probs[order]), 0.95) + 1]
    kp = probs[keep] / probs[keep].sum()
    for tok, pr in zip(keep, kp):
        assert abs(counts[tok] / n - pr) < 5 * np.sqrt(pr * (1 - pr) / n) + 1e-4


def test_decode_step_is_penalty_then_topp():
    # test_decode_step.py:30-60: the composed order; penalty 1.0 or no ids
    # is plain sample_topp; a heavy penalty moves the draw off the top token
    rng = np.random.default_rng(31)
    logits = (rng.standard_normal((3, 900)) * 2).astype(np.float32)
    ids = rng.integers(0, 900, size=(3, 40))
    offs = np.arange(4) * 40
    seeds = np.array([0, 7, 123], np.uint64)
    for pen in (1.0, 1.3, 0.7):
        got = oracle.decode_step_batched(logits, ids.reshape(-1), offs, pen, 0.9, 0.8, seeds)
        for r in range(3):
            want = oracle.sample_topp(oracle.repetition_penalty(logits[r], ids[r], pen),
                                      0.9, 0.8, int(seeds[r]))
            assert got[r] == want
    plain = oracle.decode_step_batched(logits, None, None, 2.0, 0.9, 1.0, seeds)
    for r in range(3):
        assert plain[r] == oracle.sample_topp(logits[r], 0.9, 1.0, int(seeds[r]))
    top = int(np.argmax(logits[0]))
    draws = oracle.decode_step_batched(np.repeat(logits[:1], 40, 0), np.array([top] * 40),
                                       np.arange(41), 100.0, 0.8, 1.0,
                                       np.arange(40, dtype=np.uint64))
    assert top not in set(draws.tolist())
