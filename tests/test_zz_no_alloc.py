"""The no-allocation entry point ft_attention_decode_paged_launch_bf16_noalloc
against the existing ft_attention_decode_paged_launch_bf16, both called
through the C ABI (ctypes on libfusedtok_amd.so) on the same device buffers:
outputs must be equal bit for bit (the same kernels run; only the workspace
differs), on two calls in a row, the second with a smaller input (fewer
rows, a different GQA group), so the static array holds the first call's
partials when the second starts. Both are also checked against the oracle.
A call whose partials exceed the static array is rejected before launch. The
contiguous decode's allocation-failure fallback uses the same array: a
fallback decode and a no-allocation call in turn on one stream both give
their own results."""

import ctypes
import os

import numpy as np
import pytest
import torch

import fusedtok_amd as ft  # the same library instance as the ctypes handle
import oracle

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "fusedtok_amd", "libfusedtok_amd.so")
FT_OK, FT_EINVAL = 0, 1
DEV = "cuda"
ARGS = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 6 + [ctypes.c_size_t]


@pytest.fixture(scope="module")
def lib():
    # torch (imported above) owns the HIP runtime this library binds to
    lib = ctypes.CDLL(LIB)
    lib.ft_last_error.restype = ctypes.c_char_p
    for name in ("ft_attention_decode_paged_launch_bf16",
                 "ft_attention_decode_paged_launch_bf16_noalloc"):
        getattr(lib, name).argtypes = ARGS
        getattr(lib, name).restype = ctypes.c_int
    return lib


def paged_case(seed, b, hq, hkv, d, lens, page=16):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    width = int(((lens + page - 1) // page).max())
    nb = b * width + 3
    table = rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32)
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    kp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    vp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    return q, kp, vp, table, lens


def run(lib, name, q, kp, vp, table, lens, out):
    b, hq, d = q.shape
    _, hkv, page, _ = kp.shape
    rc = getattr(lib, name)(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), table.data_ptr(),
                            lens.data_ptr(), out.data_ptr(), b, hq, hkv, page,
                            table.shape[1], d, torch.cuda.current_stream().cuda_stream)
    assert rc == FT_OK, lib.ft_last_error()


@pytest.mark.parametrize("case", [
    # (seed, batch, q heads, kv heads, dim, lengths): the second call is smaller
    [(1, 24, 32, 8, 128, [4000, 1, 0, 17, 2048, 3333, 512, 4097] * 3),
     (2, 5, 16, 8, 128, [300, 77, 1, 1024, 33])],
    # D = 64 takes the generic kernel, whose partials are laid out per chunk
    [(3, 6, 8, 2, 64, [700, 0, 64, 1500, 5, 999]),
     (4, 2, 4, 4, 64, [129, 3])],
])
def test_noalloc_equals_the_allocating_entry_point(lib, case):
    bf = torch.bfloat16
    for seed, b, hq, hkv, d, lens in case:
        q, kp, vp, table, ln = paged_case(seed, b, hq, hkv, d, lens)
        qt, kpt, vpt = (torch.from_numpy(a).to(DEV, bf) for a in (q, kp, vp))
        tt, lt = torch.from_numpy(table).to(DEV), torch.from_numpy(ln).to(DEV)
        want = torch.full((b, hq, d), float("nan"), dtype=bf, device=DEV)
        got = torch.full((b, hq, d), float("nan"), dtype=bf, device=DEV)
        run(lib, "ft_attention_decode_paged_launch_bf16", qt, kpt, vpt, tt, lt, want)
        run(lib, "ft_attention_decode_paged_launch_bf16_noalloc", qt, kpt, vpt, tt, lt, got)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"seed {seed}: outputs differ"
        ref = oracle.attention_decode_paged(qt.float().cpu().numpy(), kpt.float().cpu().numpy(),
                                            vpt.float().cpu().numpy(), table, ln)
        err = np.abs(got.float().cpu().numpy() - ref) - (2e-3 + 1e-2 * np.abs(ref))
        assert err.max() <= 0, f"seed {seed}: outside 2e-3 + 1e-2|ref| of the oracle"


def test_noalloc_rejects_a_call_beyond_the_static_workspace(lib):
    # 2048 rows x 16 kv heads x G 16 need ~280 MB of partials: refused with a
    # message before any launch (the device buffers are never touched, so
    # small real tensors stand in for the pools and the table)
    bf = torch.bfloat16
    small = torch.zeros(4096, dtype=bf, device=DEV)
    idx = torch.zeros(4096, dtype=torch.int32, device=DEV)
    fn = lib.ft_attention_decode_paged_launch_bf16_noalloc
    rc = fn(small.data_ptr(), small.data_ptr(), small.data_ptr(), idx.data_ptr(),
            idx.data_ptr(), small.data_ptr(), 2048, 256, 16, 16, 1, 128,
            torch.cuda.current_stream().cuda_stream)
    assert rc == FT_EINVAL
    assert b"static workspace" in lib.ft_last_error()


def test_fallback_decode_and_noalloc_calls_share_the_static_array(lib, tuning):
    # The contiguous decode's allocation-failure fallback (FT_FAIL_SCRATCH
    # forces it) and the no-allocation entry point both keep their split
    # partials in the one static array of the device. Called one after the
    # other on one stream, with no host sync between, each must still give
    # its own result: the second call overwrites the array only after the
    # first call's combine has read it.
    bf = torch.bfloat16
    rng = np.random.default_rng(61)
    b, hq, hkv, tt, d = 2, 16, 4, 3000, 128
    qc = torch.from_numpy(rng.standard_normal((b, hq, d)).astype(np.float32)).to(DEV, bf)
    kc = torch.from_numpy(rng.standard_normal((b, hkv, tt, d)).astype(np.float32)).to(DEV, bf)
    vc = torch.from_numpy(rng.standard_normal((b, hkv, tt, d)).astype(np.float32)).to(DEV, bf)
    lc = torch.from_numpy(np.array([3000, 1777], np.int32)).to(DEV)
    q, kp, vp, table, ln = paged_case(62, 6, 32, 8, 128, [4000, 17, 2048, 0, 999, 3333])
    qt, kpt, vpt = (torch.from_numpy(a).to(DEV, bf) for a in (q, kp, vp))
    tbl_t, ln_t = torch.from_numpy(table).to(DEV), torch.from_numpy(ln).to(DEV)
    want_c = ft.attention_decode(qc, kc, vc, lc)
    want_p = torch.empty((6, 32, d), dtype=bf, device=DEV)
    run(lib, "ft_attention_decode_paged_launch_bf16", qt, kpt, vpt, tbl_t, ln_t, want_p)
    torch.cuda.synchronize()
    tuning("FT_FAIL_SCRATCH", 1)
    for rep in range(2):
        got_c = ft.attention_decode(qc, kc, vc, lc)  # partials in the static array
        got_p = torch.full((6, 32, d), float("nan"), dtype=bf, device=DEV)
        run(lib, "ft_attention_decode_paged_launch_bf16_noalloc", qt, kpt, vpt, tbl_t, ln_t,
            got_p)
        got_c2 = ft.attention_decode(qc, kc, vc, lc)
        torch.cuda.synchronize()
        assert torch.equal(got_c, want_c), f"rep {rep}: fallback decode differs"
        assert torch.equal(got_p, want_p), f"rep {rep}: no-allocation decode differs"
        assert torch.equal(got_c2, want_c), f"rep {rep}: second fallback decode differs"
    tuning.clear("FT_FAIL_SCRATCH")
    ref = oracle.attention_decode(qc.float().cpu().numpy(), kc.float().cpu().numpy(),
                                  vc.float().cpu().numpy(), lc.cpu().numpy())
    err = np.abs(want_c.float().cpu().numpy() - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert err.max() <= 0
