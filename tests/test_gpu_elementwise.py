"""GPU parity: kv_append (bit-exact copies), RMSNorm (+residual), RoPE
(interleaved / NeoX, position offsets, per-row positions) and SwiGLU against
the CPU oracle on the same seeded inputs."""

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


def host_view(x):
    """A GPU tensor's raw elements as a numpy array of the same width (bytes
    compared exactly)."""
    if x.dtype is torch.float32:
        return x.cpu().numpy()
    return x.cpu().view(torch.int16).numpy()


# ---------------------------------------------------------------------------
# kv append
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dt", ALL)
def test_kv_append_contiguous_exact(dt):
    rng = np.random.default_rng(1)
    b, hkv, tt, d = 5, 8, 64, 128
    kc = t(rng.standard_normal((b, hkv, tt, d)).astype(np.float32), dt)
    vc = t(rng.standard_normal((b, hkv, tt, d)).astype(np.float32), dt)
    kn = t(rng.standard_normal((b, hkv, d)).astype(np.float32), dt)
    vn = t(rng.standard_normal((b, hkv, d)).astype(np.float32), dt)
    lens = np.array([0, 1, 31, 62, 63], np.int32)
    ek, ev = host_view(kc).copy(), host_view(vc).copy()
    oracle.kv_append(ek, ev, host_view(kn), host_view(vn), lens)
    ft.kv_append(kc, vc, kn, vn, t(lens))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host_view(kc), ek)
    np.testing.assert_array_equal(host_view(vc), ev)


@pytest.mark.parametrize("dt", ALL)
@pytest.mark.parametrize("page", [16, 5])
def test_kv_append_paged_exact(dt, page):
    rng = np.random.default_rng(2 + page)
    b, hkv, d, nb, width = 6, 8, 128, 40, 5
    kp = t(rng.standard_normal((nb, hkv, page, d)).astype(np.float32), dt)
    vp = t(rng.standard_normal((nb, hkv, page, d)).astype(np.float32), dt)
    tbl = rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32)
    kn = t(rng.standard_normal((b, hkv, d)).astype(np.float32), dt)
    vn = t(rng.standard_normal((b, hkv, d)).astype(np.float32), dt)
    lens = rng.integers(0, width * page, size=b).astype(np.int32)
    ek, ev = host_view(kp).copy(), host_view(vp).copy()
    oracle.kv_append_paged(ek, ev, tbl, host_view(kn), host_view(vn), lens)
    ft.kv_append_paged(kp, vp, t(tbl), kn, vn, t(lens))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host_view(kp), ek)
    np.testing.assert_array_equal(host_view(vp), ev)


def test_kv_append_staged_host_inplace():
    rng = np.random.default_rng(9)
    kc = rng.standard_normal((2, 2, 8, 16)).astype(np.float32)
    vc = kc.copy()
    kn = rng.standard_normal((2, 2, 16)).astype(np.float32)
    lens = np.array([3, 7], np.int32)
    ek, ev = kc.copy(), vc.copy()
    oracle.kv_append(ek, ev, kn, kn, lens)
    ft.kv_append(kc, vc, kn, kn, lens, cuda=True)
    np.testing.assert_array_equal(kc, ek)
    np.testing.assert_array_equal(vc, ev)


# ---------------------------------------------------------------------------
# rmsnorm
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("rows,cols", [(1, 4096), (16, 4096), (64, 4096), (8, 257),
                                       (3, 1), (4, 65)])
@pytest.mark.parametrize("with_r", [False, True])
def test_rmsnorm_f32(rows, cols, with_r):
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    r = rng.uniform(-1, 1, x.shape).astype(np.float32) if with_r else None
    y = ft.rmsnorm(t(x), t(w), residual=None if r is None else t(r), eps=1e-5)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), oracle.rmsnorm(x, w, r, 1e-5),
                               rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_rmsnorm_half(dt):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((64, 4096)).astype(np.float32)
    r = rng.standard_normal((64, 4096)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    xt, rt = t(x, dt), t(r, dt)
    y = ft.rmsnorm(xt, t(w), residual=rt, eps=1e-5)
    torch.cuda.synchronize()
    ref = oracle.rmsnorm(xt.float().cpu().numpy(), w, rt.float().cpu().numpy(), 1e-5)
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, rtol=1e-2, atol=2e-3)


def test_rmsnorm_known_answer_and_1d():
    y = ft.rmsnorm(t(np.array([[3.0, 4.0]], np.float32)), t(np.ones(2, np.float32)),
                   eps=1e-12)
    inv = 1.0 / np.sqrt(12.5)
    np.testing.assert_allclose(y.cpu().numpy(), [[3 * inv, 4 * inv]], atol=1e-6)
    x = np.random.default_rng(5).standard_normal(8).astype(np.float32)
    w = np.ones(8, np.float32)
    y1 = ft.rmsnorm(t(x), t(w))
    assert y1.shape == (8,)
    np.testing.assert_allclose(y1.cpu().numpy(), oracle.rmsnorm(x, w), rtol=1e-5,
                               atol=1e-6)


# ---------------------------------------------------------------------------
# rope
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("neox", [False, True])
@pytest.mark.parametrize("off", [0, 3, 8192, 131000])
def test_rope_f32(neox, off):
    rng = np.random.default_rng(off + neox)
    q = rng.standard_normal((64, 128)).astype(np.float32)
    k = rng.standard_normal((64, 128)).astype(np.float32)
    qo, ko = ft.rope(t(q), t(k), pos_offset=off, neox=neox)
    torch.cuda.synchronize()
    np.testing.assert_allclose(qo.cpu().numpy(), oracle.rope(q, 10000.0, off, neox),
                               rtol=0, atol=2e-6)
    np.testing.assert_allclose(ko.cpu().numpy(), oracle.rope(k, 10000.0, off, neox),
                               rtol=0, atol=2e-6)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("neox", [False, True])
def test_rope_half(dt, neox):
    rng = np.random.default_rng(7)
    q = t(rng.standard_normal((32, 128)).astype(np.float32), dt)
    qo, ko = ft.rope(q, None, pos_offset=8192, neox=neox, theta=500000.0)
    torch.cuda.synchronize()
    assert ko is None and qo.dtype == dt
    ref = oracle.rope(q.float().cpu().numpy(), 500000.0, 8192, neox)
    np.testing.assert_allclose(qo.float().cpu().numpy(), ref, rtol=1e-2, atol=2e-3)


def test_rope_per_row_positions():
    # q as [B*Hq, D]: every head of sequence b rotates at positions[b] + off
    rng = np.random.default_rng(8)
    bsz, hq, d = 5, 4, 64
    q = rng.standard_normal((bsz * hq, d)).astype(np.float32)
    pos = np.array([0, 17, 8191, 3, 100000], np.int32)
    qo, _ = ft.rope(t(q), None, pos_offset=1, neox=True, positions=t(pos),
                    rows_per_position=hq)
    torch.cuda.synchronize()
    got = qo.cpu().numpy()
    for bi in range(bsz):
        ref = oracle.rope(q[bi * hq:(bi + 1) * hq], 10000.0, int(pos[bi]) + 1, True)
        # oracle rows r sit at r + offset: rotate each row on its own
        for h in range(hq):
            row = oracle.rope(q[bi * hq + h:bi * hq + h + 1], 10000.0,
                              int(pos[bi]) + 1, True)
            np.testing.assert_allclose(got[bi * hq + h], row[0], atol=2e-6)
        del ref


def test_rope_staged_identity_at_zero():
    q = np.random.default_rng(0).standard_normal((3, 8)).astype(np.float32)
    q2, k2 = ft.rope(q, None, cuda=True)
    assert k2 is None
    np.testing.assert_array_equal(q2[0], q[0])


# ---------------------------------------------------------------------------
# swiglu
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("n", [1, 7, 4096, 64 * 14336 + 3])
def test_swiglu_f32(n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    y = ft.swiglu(t(g), t(u))
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), oracle.swiglu(g, u), rtol=2e-6,
                               atol=1e-7)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_swiglu_half(dt):
    rng = np.random.default_rng(3)
    g = t((rng.standard_normal((64, 14336)) * 3).astype(np.float32), dt)
    u = t(rng.standard_normal((64, 14336)).astype(np.float32), dt)
    y = ft.swiglu(g, u)
    torch.cuda.synchronize()
    ref = oracle.swiglu(g.float().cpu().numpy(), u.float().cpu().numpy())
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, rtol=1e-2, atol=2e-3)


def test_swiglu_extremes_and_misaligned():
    g = t(np.array([-100.0, 0.0, 100.0, 1.0, 2.0], np.float32))
    u = t(np.array([3.0, 5.0, 2.0, 1.0, 1.0], np.float32))
    y = ft.swiglu(g[1:], u[1:])
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(),
                               refs.ref_swiglu(g[1:].cpu().numpy(), u[1:].cpu().numpy()),
                               rtol=1e-6)
