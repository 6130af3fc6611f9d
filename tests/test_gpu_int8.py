"""GPU parity, bit-exact: INT8 quantize codes and scale, int32 GEMM
accumulators and the float32 GEMM epilogue equal the CPU oracle exactly;
bf16 / fp16 GEMM outputs equal the oracle's float32 value rounded to
nearest-even. Every GEMM kernel is exercised: GEMV (M == 1, or forced up to
8), decode (2 <= M <= 16, 1 / 2 / 4 waves per tile, and the LDS-ring
variant), skinny (M <= 64, with
and without the cross-workgroup K split), tiled, big (M, N >= 256, DMA and
register-staged), scalar fallback (K % 16 != 0) and the K == 0 zero fill."""

import numpy as np
import pytest
import torch

import fusedtok_amd as ft
import oracle
from tests import refs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t(a, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return x if dtype is None else x.to(dtype)


def rand_q(rng, rows, k):
    return rng.integers(-127, 128, size=(rows, k)).astype(np.int8)


# ---------------------------------------------------------------------------
# quantize
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("n", [1, 5, 777, 4096, 65536, 65537, 1 << 20, 3_000_001])
def test_quantize_f32_bit_exact(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 2.5).astype(np.float32)
    q, s = ft.quantize_int8(t(x))
    rq, rs = oracle.quantize_int8(x)
    assert q.dtype == torch.int8 and isinstance(s, float)
    assert s == rs
    np.testing.assert_array_equal(q.cpu().numpy(), rq)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [4096 * 16, 4096 * 64 + 3])
def test_quantize_half_input_bit_exact(dt, n):
    rng = np.random.default_rng(n + 1)
    xt = torch.from_numpy((rng.standard_normal(n) * 3).astype(np.float32)).to(DEV, dt)
    q, s = ft.quantize_int8(xt)
    rq, rs = oracle.quantize_int8(xt.float().cpu().numpy())
    assert s == rs
    np.testing.assert_array_equal(q.cpu().numpy(), rq)


def test_quantize_known_answers_and_device_scale():
    q, s = ft.quantize_int8(t(np.array([-2.0, -1.0, 0.0, 1.0, 2.0], np.float32)))
    assert s == pytest.approx(2.0 / 127.0)
    assert q.cpu().tolist() == [-127, -64, 0, 64, 127]
    q, s = ft.quantize_int8(t(np.zeros(8, np.float32)))
    assert s == 1.0 and (q == 0).all()
    q, s = ft.quantize_int8(t(np.array([1e30, -1e30], np.float32)))
    assert q.cpu().tolist() == [127, -127]
    q, s = ft.quantize_int8(torch.empty(0, device=DEV))   # empty: scale 1.0
    assert s == 1.0 and q.numel() == 0
    x = np.random.default_rng(2).standard_normal((16, 4096)).astype(np.float32)
    q, sd = ft.quantize_int8(t(x), device_scale=True)
    assert sd.is_cuda and sd.dtype == torch.float32 and sd.numel() == 1
    rq, rs = oracle.quantize_int8(x)
    assert float(sd) == rs
    np.testing.assert_array_equal(q.cpu().numpy(), rq)


@pytest.mark.parametrize("n", [1, 3, 4096, 65536, 65537, 1 << 20])
def test_dequantize_bit_exact(n):
    rng = np.random.default_rng(n + 5)
    q = rand_q(rng, 1, n).reshape(n)
    x = ft.dequantize_int8(t(q), 0.0173)
    assert x.dtype == torch.float32
    np.testing.assert_array_equal(x.cpu().numpy(), oracle.dequantize_int8(q, 0.0173))
    # bf16 / fp16 out: the float32 value rounded once; device scale operand
    sd = t(np.array([0.0173], np.float32))
    ref = torch.from_numpy(oracle.dequantize_int8(q, 0.0173))
    for dt in (torch.bfloat16, torch.float16):
        y = ft.dequantize_int8(t(q), sd, out_dtype=dt)
        assert torch.equal(y.cpu(), ref.to(dt))


def test_dequantize_roundtrip_views_and_staged():
    # test_quantize.py:25-31 on the GPU, an odd-offset int8 view (scalar
    # path), and host input staged through the device
    x = np.random.default_rng(0).standard_normal(10001).astype(np.float32)
    q, s = ft.quantize_int8(t(x))
    back = ft.dequantize_int8(q, s).cpu().numpy()
    assert np.abs(back - x).max() <= s * 0.51
    v = ft.dequantize_int8(q[1:], s).cpu().numpy()
    np.testing.assert_array_equal(v, oracle.dequantize_int8(q[1:].cpu().numpy(), s))
    qh = q.cpu().numpy()
    np.testing.assert_array_equal(ft.dequantize_int8(qh, s), oracle.dequantize_int8(qh, s))
    with pytest.raises(TypeError):
        ft.dequantize_int8(t(x), s)                      # float "codes"


@pytest.mark.parametrize("n", [1, 1000, 65536, 65537, 3_000_001])
def test_qadd_bit_exact(n):
    rng = np.random.default_rng(n + 9)
    a = rng.standard_normal(n).astype(np.float32)
    b = (rng.standard_normal(n) * 4).astype(np.float32)
    qa, sa = oracle.quantize_int8(a)
    qb, sb = oracle.quantize_int8(b)
    qy, sy = ft.qadd_int8(t(qa), sa, t(qb), sb)
    rq, rs = oracle.qadd_int8(qa, sa, qb, sb)
    assert isinstance(sy, float) and sy == rs
    np.testing.assert_array_equal(qy.cpu().numpy(), rq)


def test_qadd_device_scales_chain_and_contract():
    # quantize (device scale) -> qadd with device scales -> device out scale:
    # no host sync, same bits as the host-scale call
    rng = np.random.default_rng(11)
    a = rng.standard_normal((64, 4096)).astype(np.float32)
    b = rng.standard_normal((64, 4096)).astype(np.float32)
    qa, sa_d = ft.quantize_int8(t(a), device_scale=True)
    qb, sb_d = ft.quantize_int8(t(b), device_scale=True)
    qy, sy_d = ft.qadd_int8(qa, sa_d, qb, sb_d, device_scale=True)
    assert sy_d.is_cuda and sy_d.numel() == 1
    rq, rs = oracle.qadd_int8(qa.cpu().numpy(), float(sa_d), qb.cpu().numpy(), float(sb_d))
    assert float(sy_d) == rs
    np.testing.assert_array_equal(qy.cpu().numpy(), rq)
    # 1-byte-offset views (scalar path), both sizes of the two-phase split
    for n in (1000, 70001):
        qa1 = qa.reshape(-1)[1:n + 1]
        qb1 = qb.reshape(-1)[1:n + 1]
        qy1, sy1 = ft.qadd_int8(qa1, 0.02, qb1, 0.03)
        rq1, rs1 = oracle.qadd_int8(qa1.cpu().numpy(), 0.02, qb1.cpu().numpy(), 0.03)
        assert sy1 == rs1
        np.testing.assert_array_equal(qy1.cpu().numpy(), rq1)
    # reference contract: GPU int8 only, equal shapes; empty -> scale 1.0
    with pytest.raises(TypeError):
        ft.qadd_int8(np.ones(4, np.int8), 1.0, np.ones(4, np.int8), 1.0)
    with pytest.raises(TypeError):
        ft.qadd_int8(t(a), 1.0, t(b), 1.0)
    with pytest.raises(ValueError):
        ft.qadd_int8(qa, 1.0, qb[:3], 1.0)
    q0, s0 = ft.qadd_int8(qa[:0], 1.0, qb[:0], 1.0)
    assert s0 == 1.0 and q0.numel() == 0


def test_quantize_misaligned_view_and_staged():
    x = np.random.default_rng(3).standard_normal(1001).astype(np.float32)
    xt = t(x)
    q, s = ft.quantize_int8(xt[1:])          # 4-byte offset view: scalar path
    rq, rs = oracle.quantize_int8(x[1:])
    assert s == rs
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    q2, s2 = ft.quantize_int8(x)             # host input -> staged
    rq2, rs2 = oracle.quantize_int8(x)
    assert s2 == rs2 and isinstance(q2, np.ndarray)
    np.testing.assert_array_equal(q2, rq2)


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------

GEMM_SHAPES = [
    (1, 8, 16),            # GEMV, tiny
    (1, 1000, 4096),       # GEMV, decode-like
    (2, 1000, 4096),       # decode kernel, 2 waves per tile
    (3, 5, 7),             # scalar fallback (odd K)
    (8, 11008, 4096),      # BASELINE config 2, M = 8
    (16, 11008, 4096),     # BASELINE config 2, M = 16
    (1, 11008, 4096),      # BASELINE config 2, M = 1
    (33, 300, 1024),       # skinny MT = 4, K split
    (16, 6144, 4096),      # decode kernel, 1 wave per tile
    (64, 4096, 4096),      # BASELINE config 4 o_proj shape
    (64, 512, 14336),      # BASELINE config 4 down-proj K, fewer rows
    (65, 63, 33),          # scalar fallback
    (65, 130, 96),         # tiled, ragged edges
    (128, 256, 512),       # tiled
    (300, 500, 1024),      # tiled, ragged
    (17, 4096, 129),       # scalar fallback, tall N
    (100, 50, 16),         # tiled, single short slab
    (1024, 1024, 1024),    # big tiles (256 x 256)
    (257, 300, 80),        # big tiles, ragged M/N, K not a multiple of 64
    (512, 256, 1040),      # big tiles, K tail
    (256, 256, 128),       # 128-byte-slab kernel, one slab
    (512, 768, 256),       # 128-byte-slab kernel, two slabs (no refill)
    (300, 520, 384),       # 128-byte-slab kernel, ragged M/N, one refill
]


@pytest.mark.parametrize("band", [0, 1, 3])
def test_big_persistent_tiles_bit_exact(band, tuning):
    # 9 x 33 = 297 tiles of 256 x 256 > one workgroup per CU: the persistent
    # 128-byte-slab kernel (8 waves with 16x16x64 MFMAs) walks several tiles
    # per workgroup, with the next tile's first slabs loading during the
    # previous tile's epilogue; the default tile order and two other band
    # heights (a band of 3 leaves a ragged last band). Rows from every
    # 256-row band are checked against the oracle over all columns, so every
    # tile is covered.
    if band:
        tuning("FT_QGEMM_BAND", band)
    rng = np.random.default_rng(77)
    m, n, k = 2304, 8448, 384
    a, b = rand_q(rng, m, k), rand_q(rng, n, k)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    at, bt = t(a), t(b)
    acc = ft.qgemm_i32(at, bt).cpu().numpy()
    y = ft.qgemm_perchannel(at, 0.011, bt, t(sb), out_dtype=torch.bfloat16).cpu()
    rows = sorted({0, 255, 2303} | {256 * bb + (bb * 37) % 256 for bb in range(9)})
    ra = np.ascontiguousarray(a[rows])
    np.testing.assert_array_equal(acc[rows], oracle.qgemm_i32(ra, b))
    ref = torch.from_numpy(oracle.qgemm_perchannel(ra, 0.011, b, sb)).to(torch.bfloat16)
    assert torch.equal(y[rows], ref)


@pytest.mark.parametrize("big", [0, 1, 2])
def test_big_kernels_bit_exact(big, tuning):
    # the three big-tile kernels on one K % 128 == 0 shape with ragged
    # edges: 128-byte DMA slabs with 8 waves on 16x16x64 MFMAs (default),
    # 64-byte DMA slabs (K % 64 == 0 shapes), register-staged (any K); every
    # output type (i32, f32 per-tensor and per-channel, bf16, f16)
    if big:
        tuning("FT_QGEMM_BIG", big)
    rng = np.random.default_rng(400 + big)
    m, n, k = 520, 777, 1280
    a, b = rand_q(rng, m, k), rand_q(rng, n, k)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    at, bt = t(a), t(b)
    acc = ft.qgemm_i32(at, bt)
    y = ft.qgemm_perchannel(at, 0.017, bt, t(sb), out_dtype=torch.bfloat16)
    yh = ft.qgemm_perchannel(at, 0.017, bt, t(sb), out_dtype=torch.float16)
    yf = ft.qgemm_perchannel(at, 0.017, bt, t(sb))
    yt = ft.qgemm(at, 0.03, bt, 0.02)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), oracle.qgemm_i32(a, b))
    pc = oracle.qgemm_perchannel(a, 0.017, b, sb)
    np.testing.assert_array_equal(yf.cpu().numpy(), pc)
    np.testing.assert_array_equal(yt.cpu().numpy(), oracle.qgemm(a, 0.03, b, 0.02))
    assert torch.equal(y.cpu(), torch.from_numpy(pc).to(torch.bfloat16))
    assert torch.equal(yh.cpu(), torch.from_numpy(pc).to(torch.float16))


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_qgemm_bit_exact(m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    a, b = rand_q(rng, m, k), rand_q(rng, n, k)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    at, bt = t(a), t(b)
    acc = ft.qgemm_i32(at, bt)
    y_pt = ft.qgemm(at, 0.03, bt, 0.02)
    y_pc = ft.qgemm_perchannel(at, 0.031, bt, t(sb))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), oracle.qgemm_i32(a, b))
    np.testing.assert_array_equal(y_pt.cpu().numpy(), oracle.qgemm(a, 0.03, b, 0.02))
    np.testing.assert_array_equal(y_pc.cpu().numpy(),
                                  oracle.qgemm_perchannel(a, 0.031, b, sb))


@pytest.mark.parametrize("m,n,k,split", [
    (20, 200, 640, 0),      # one 16-row tile, K tail inside a chunk
    (33, 300, 1040, 0),     # two tiles, ragged N, K tail
    (64, 4096, 4096, 0),    # C4 o_proj shape, auto K split
    (48, 777, 4112, 3),     # forced split, ragged everything
    (64, 1000, 2000, 5),    # split leaving an empty K range
    (17, 64, 16, 0),        # a single 16-byte K piece
    (64, 16448, 512, 0),    # 257 column workgroups: no K split
])
def test_skinny_kernel_bit_exact(m, n, k, split, tuning):
    # 16 < M <= 64 (qgemm_skinny), with and without K splits (int32 partials
    # folded by a second launch), including a split that leaves a workgroup
    # an empty K range
    if split:
        tuning("FT_QGEMM_KSPLIT", split)
    rng = np.random.default_rng(m * 7 + n + k + split)
    a, b = rand_q(rng, m, k), rand_q(rng, n, k)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    acc = ft.qgemm_i32(t(a), t(b))
    y = ft.qgemm_perchannel(t(a), 0.021, t(b), t(sb), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), oracle.qgemm_i32(a, b))
    ref = torch.from_numpy(oracle.qgemm_perchannel(a, 0.021, b, sb)).to(torch.bfloat16)
    assert torch.equal(y.cpu(), ref)


@pytest.mark.parametrize("variant", ["regs", "w4s2", "w4s3", "w8s2", "w8s3"])
@pytest.mark.parametrize("m,n,k,split", [
    (17, 200, 256, 0),      # one chunk, one 16-row tile
    (33, 300, 1280, 0),     # three tiles (MT = 4 with one row past M), ragged N
    (64, 1000, 3072, 3),    # forced split in three
    (20, 70, 2304, 2),      # split into 5 + 4 chunks; ragged N (dead waves)
    (64, 16448, 512, 0),    # 257 column workgroups, no split
    (40, 28672, 1024, 0),   # MT = 3 rows of tiles, 8 waves by default (wide N)
    (64, 6144, 4096, 2),    # C4's QKV shape with its default split
])
def test_skinny_lds_ring_bit_exact(variant, m, n, k, split, tuning):
    # the LDS-ring skinny kernel (K % 256 == 0) against the oracle in each
    # shape of workgroup (4 waves / 64 columns or 8 waves / 128 columns) and
    # ring depth (2 or 3 stages), and the register-operand kernel on the
    # same shapes (FT_QGEMM_SK_REGS=1)
    if variant == "regs":
        tuning("FT_QGEMM_SK_REGS", 1)
    else:
        tuning("FT_QGEMM_SK_WAVES", int(variant[1]))
        tuning("FT_QGEMM_SK_STAGES", int(variant[3]))
    if split:
        tuning("FT_QGEMM_KSPLIT", split)
    rng = np.random.default_rng(m * 3 + n + k + split)
    a, b = rand_q(rng, m, k), rand_q(rng, n, k)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    acc = ft.qgemm_i32(t(a), t(b))
    y = ft.qgemm_perchannel(t(a), 0.021, t(b), t(sb), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), oracle.qgemm_i32(a, b))
    ref = torch.from_numpy(oracle.qgemm_perchannel(a, 0.021, b, sb)).to(torch.bfloat16)
    assert torch.equal(y.cpu(), ref)


@pytest.mark.parametrize("kernel", [1, 2, 3, 4, 5, 6])
def test_every_gemm_kernel_bit_exact(kernel, tuning):
    tuning("FT_QGEMM_KERNEL", kernel)
    rng = np.random.default_rng(kernel)
    m = {1: 48, 5: 7, 6: 13}.get(kernel, 80)
    a, b = rand_q(rng, m, 640), rand_q(rng, 200, 640)
    sb = rng.uniform(1e-3, 1e-2, 200).astype(np.float32)
    y = ft.qgemm_perchannel(t(a), 0.5, t(b), t(sb))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), oracle.qgemm_perchannel(a, 0.5, b, sb))


@pytest.mark.parametrize("kw", [1, 2, 4])
@pytest.mark.parametrize("m,n,k", [(1, 200, 640), (5, 33, 4096), (16, 200, 640),
                                   (3, 16, 80), (16, 40, 16), (8, 1000, 14336)])
def test_decode_gemm_kernel_bit_exact(kw, m, n, k, tuning):
    # the K-split-in-workgroup decode kernel: ragged chunks (K % 512 != 0),
    # K below one MFMA step, waves with no chunk, N % 16 != 0
    tuning("FT_QGEMM_KERNEL", 6)
    tuning("FT_QGEMM_DEC_KW", kw)
    rng = np.random.default_rng(m * 100 + n + k + kw)
    a, b = rand_q(rng, m, k), rand_q(rng, n, k)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    acc = ft.qgemm_i32(t(a), t(b))
    y = ft.qgemm_perchannel(t(a), 0.021, t(b), t(sb), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), oracle.qgemm_i32(a, b))
    ref = torch.from_numpy(oracle.qgemm_perchannel(a, 0.021, b, sb)).to(torch.bfloat16)
    assert torch.equal(y.cpu(), ref)


def test_decode_gemm_lds_ring_bit_exact(tuning):
    # the LDS-staged decode kernel (K % 512 == 0, one wave per 16 columns):
    # one chunk, fewer chunks than ring stages, ragged N, odd M; the C2 shape
    # against the register-operand kernel (FT_QGEMM_DEC_REGS=1)
    tuning("FT_QGEMM_KERNEL", 6)
    tuning("FT_QGEMM_DEC_KW", 1)
    for m, n, k in [(2, 40, 512), (7, 1000, 1024), (16, 333, 2560), (9, 17, 4608)]:
        rng = np.random.default_rng(m * 10 + n + k)
        a, b = rand_q(rng, m, k), rand_q(rng, n, k)
        sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        acc = ft.qgemm_i32(t(a), t(b))
        y = ft.qgemm_perchannel(t(a), 0.021, t(b), t(sb), out_dtype=torch.float16)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(acc.cpu().numpy(), oracle.qgemm_i32(a, b))
        ref = torch.from_numpy(oracle.qgemm_perchannel(a, 0.021, b, sb)).to(torch.float16)
        assert torch.equal(y.cpu(), ref)
    for m, n, k in [(16, 11008, 4096), (13, 5000, 14336)]:
        rng = np.random.default_rng(m + n + k)
        at, bt = t(rand_q(rng, m, k)), t(rand_q(rng, n, k))
        acc = ft.qgemm_i32(at, bt)
        tuning("FT_QGEMM_DEC_REGS", 1)
        acc0 = ft.qgemm_i32(at, bt)
        tuning.clear("FT_QGEMM_DEC_REGS")
        assert torch.equal(acc, acc0)


@pytest.mark.parametrize("ksplit", [1, 2, 4, 7])
def test_skinny_k_split_bit_exact_on_repeats(ksplit, tuning):
    # forced K splits of the skinny kernel; repeated calls reuse the partials
    # buffer, whose previous contents must not leak into the fold
    tuning("FT_QGEMM_KSPLIT", ksplit)
    rng = np.random.default_rng(ksplit + 50)
    a, b = rand_q(rng, 48, 4096), rand_q(rng, 700, 4096)
    for rep in range(3):
        acc = ft.qgemm_i32(t(a), t(b))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(acc.cpu().numpy(), oracle.qgemm_i32(a, b))


@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n", [(16, 384), (256, 384), (300, 384), (300, 260)])
def test_half_outputs_are_rounded_f32(odt, m, n):
    # (300, 260): ragged tile edges and N % 8 != 0 (element-wise stores)
    rng = np.random.default_rng(m + n + 9)
    a, b = rand_q(rng, m, 2048), rand_q(rng, n, 2048)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    y = ft.qgemm_perchannel(t(a), 0.013, t(b), t(sb), out_dtype=odt)
    torch.cuda.synchronize()
    ref = torch.from_numpy(oracle.qgemm_perchannel(a, 0.013, b, sb)).to(odt)
    assert y.dtype == odt
    assert torch.equal(y.cpu(), ref)


@pytest.mark.parametrize("m,n", [(8, 256), (8, 5120), (40, 700)])
def test_device_scale_operand_matches_host_scale(m, n):
    # decode kernel (8 x 256), its LDS-ring variant (320 column tiles), skinny
    rng = np.random.default_rng(10 + n)
    x = rng.standard_normal((m, 1024)).astype(np.float32)
    b = rand_q(rng, n, 1024)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    qx, sd = ft.quantize_int8(t(x), device_scale=True)
    y_dev = ft.qgemm_perchannel(qx, sd, t(b), t(sb))
    y_host = ft.qgemm_perchannel(qx, float(sd), t(b), t(sb))
    torch.cuda.synchronize()
    assert torch.equal(y_dev, y_host)
    rq, rs = oracle.quantize_int8(x)
    np.testing.assert_array_equal(y_dev.cpu().numpy(),
                                  oracle.qgemm_perchannel(rq, rs, b, sb))


def test_k0_and_extremes_and_empty():
    y = ft.qgemm(torch.zeros((4, 0), dtype=torch.int8, device=DEV), 0.5,
                 torch.zeros((3, 0), dtype=torch.int8, device=DEV), 0.25)
    y16 = ft.qgemm(torch.zeros((4, 0), dtype=torch.int8, device=DEV), 0.5,
                   torch.zeros((3, 0), dtype=torch.int8, device=DEV), 0.25,
                   out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert (y == 0).all() and (y16 == 0).all()
    a = np.full((70, 4096), -128, np.int8)
    b = np.full((33, 4096), -128, np.int8)
    acc = ft.qgemm_i32(t(a), t(b))
    torch.cuda.synchronize()
    assert (acc.cpu().numpy() == 128 * 128 * 4096).all()
    e = ft.qgemm(torch.zeros((0, 16), dtype=torch.int8, device=DEV), 1.0,
                 torch.zeros((5, 16), dtype=torch.int8, device=DEV), 1.0)
    assert e.shape == (0, 5)


def test_staged_host_gemm():
    rng = np.random.default_rng(12)
    a, b = rand_q(rng, 20, 256), rand_q(rng, 30, 256)
    sb = rng.uniform(1e-3, 1e-2, 30).astype(np.float32)
    y = ft.qgemm_perchannel(a, 0.1, b, sb, cuda=True)
    np.testing.assert_array_equal(y, refs.ref_qgemm_pc(a, 0.1, b, sb))
