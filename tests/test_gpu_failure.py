"""Failure handling on the GPU, forced from the host with the FT_FAIL_SCRATCH
test hook (every device-scratch request fails as an allocation failure
would; no kernel faults or waits):
  - the paged decode raises (reference attention.cu:1839-1844: its launcher
    throws when the workspace cannot be allocated) and leaves nothing
    half-written; the library works again once memory is back;
  - the contiguous decode falls back (reference attention.cu:1514-1523 runs
    its single-pass kernel instead): here the split partials go to the
    static per-device array, and the result is the same bit for bit;
  - quantize_int8 above its one-launch size raises; below it needs no
    scratch and still runs."""

import numpy as np
import pytest
import torch

import fusedtok_amd as ft
import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t(a, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return x if dtype is None else x.to(dtype)


def paged(rng, b=3, hq=16, hkv=4, d=128, lens=(40, 700, 1), page=16):
    width = max((n + page - 1) // page for n in lens)
    nb = b * width + 2
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    kp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    vp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    tbl = rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32)
    return q, kp, vp, tbl, np.asarray(lens, np.int32)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_paged_decode_raises_and_recovers(dt, tuning):
    rng = np.random.default_rng(3)
    q, kp, vp, tbl, ln = paged(rng)
    args = (t(q, dt), t(kp, dt), t(vp, dt), t(tbl), t(ln))
    tuning("FT_FAIL_SCRATCH", 1)
    with pytest.raises(RuntimeError, match="out of memory"):
        ft.attention_decode_paged(*args)
    tuning.clear("FT_FAIL_SCRATCH")
    got = ft.attention_decode_paged(*args).float().cpu().numpy()
    r = lambda a: torch.from_numpy(a).to(dt).float().numpy()  # noqa: E731
    ref = oracle.attention_decode_paged(r(q), r(kp), r(vp), tbl, ln)
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=2e-3)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("generic", [False, True])
def test_contiguous_decode_falls_back_to_the_static_array(dt, generic, tuning):
    if generic:
        tuning("FT_ATTN_FORCE_GENERIC", 1)
    rng = np.random.default_rng(4)
    b, hq, hkv, tt, d = 2, 16, 4, 3000, 128
    q = t(rng.standard_normal((b, hq, d)).astype(np.float32), dt)
    k = t(rng.standard_normal((b, hkv, tt, d)).astype(np.float32), dt)
    v = t(rng.standard_normal((b, hkv, tt, d)).astype(np.float32), dt)
    lens = t(np.array([3000, 1777], np.int32))
    want = ft.attention_decode(q, k, v, lens)
    tuning("FT_FAIL_SCRATCH", 1)
    got = ft.attention_decode(q, k, v, lens)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_quantize_raises_above_one_launch_and_runs_below(tuning):
    big = torch.randn(1 << 20, device=DEV)
    small = torch.randn(1000, device=DEV)
    q_ref, s_ref = ft.quantize_int8(small)
    tuning("FT_FAIL_SCRATCH", 1)
    with pytest.raises(RuntimeError, match="out of memory"):
        ft.quantize_int8(big)
    q, s = ft.quantize_int8(small)
    assert torch.equal(q, q_ref) and s == s_ref
    tuning.clear("FT_FAIL_SCRATCH")
    _, s2 = ft.quantize_int8(big)
    assert s2 == float(np.float32(big.abs().max().item()) / np.float32(127.0))
