"""The C-ABI library (include/fusedtok_amd.h) loads, exports every declared
entry point, and reports invalid arguments (FT_EINVAL + message) from host
validation alone - these paths run before any HIP call, so no GPU is needed.
No compute call is made here."""

import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (HIP runtime first: the library binds to it)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fusedtok_amd.h")
LIB = os.path.join(ROOT, "fusedtok_amd", "libfusedtok_amd.so")

FT_OK, FT_EINVAL, FT_EHIP = 0, 1, 2


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ft_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    assert os.path.exists(LIB), "libfusedtok_amd.so not built"
    lib = ctypes.CDLL(LIB)
    lib.ft_last_error.restype = ctypes.c_char_p
    lib.ft_version.restype = ctypes.c_char_p
    return lib


def test_header_declares_the_hot_path():
    syms = declared_symbols()
    for name in ["ft_attention_decode_launch", "ft_attention_decode_paged_launch_bf16",
                 "ft_kv_append_paged_launch", "ft_kv_append_launch_fp16",
                 "ft_quantize_int8_launch", "ft_qgemm_launch",
                 "ft_qgemm_perchannel_launch", "ft_rmsnorm_launch_bf16",
                 "ft_rope_neox_launch", "ft_swiglu_launch_bf16",
                 "ft_dequantize_int8_launch", "ft_qadd_int8_launch"]:
        assert name in syms
    assert len(syms) >= 30


def test_every_declared_symbol_is_exported(lib):
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"not exported: {missing}"


def test_version_and_clean_error(lib):
    assert lib.ft_version().decode().count(".") == 2
    assert isinstance(lib.ft_last_error(), bytes)


def _v(x=0):
    return ctypes.c_void_p(x)


U = ctypes.c_size_t


def test_attention_invalid_arguments(lib):
    f = lib.ft_attention_decode_launch
    # dim not a multiple of 4
    st = f(_v(), _v(), _v(), _v(), _v(), 1, 2, 1, 4, 30, U(0))
    assert st == FT_EINVAL
    assert b"multiple of 4" in lib.ft_last_error()
    # Hq not a multiple of Hkv
    assert f(_v(), _v(), _v(), _v(), _v(), 1, 5, 2, 4, 32, U(0)) == FT_EINVAL
    # dim > 512
    assert f(_v(), _v(), _v(), _v(), _v(), 1, 2, 1, 4, 516, U(0)) == FT_EINVAL
    # batch 0 is a valid no-op (no device work at all)
    assert f(_v(), _v(), _v(), _v(), _v(), 0, 2, 1, 4, 32, U(0)) == FT_OK
    p = lib.ft_attention_decode_paged_launch
    # unsupported GQA group on the paged path (reference attention.cu:1806-1811)
    st = p(_v(), _v(), _v(), _v(), _v(), _v(), 1, 6, 2, 16, 4, 32, U(0))
    assert st == FT_EINVAL and b"group" in lib.ft_last_error()
    # page < 1
    assert p(_v(), _v(), _v(), _v(), _v(), _v(), 1, 2, 2, 0, 4, 32, U(0)) == FT_EINVAL
    # absurd table capacity
    assert p(_v(), _v(), _v(), _v(), _v(), _v(), 1, 2, 2, 1 << 16, 1 << 16, 32,
             U(0)) == FT_EINVAL


def test_kv_append_invalid_arguments(lib):
    f = lib.ft_kv_append_launch
    assert f(_v(), _v(), _v(), _v(), _v(), 2, 2, 30, 8, U(0)) == FT_EINVAL
    assert f(_v(), _v(), _v(), _v(), _v(), 0, 2, 30, 8, U(0)) == FT_OK   # batch 0
    g = lib.ft_kv_append_paged_launch
    assert g(_v(), _v(), _v(), _v(), _v(), _v(), 2, 2, 32, 0, 4, U(0)) == FT_EINVAL


def test_qgemm_invalid_arguments(lib):
    f = lib.ft_qgemm_launch
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                  ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                  ctypes.c_size_t]
    assert f(None, None, None, -1, 4, 4, 1.0, 1.0, 0) == FT_EINVAL
    assert f(None, None, None, 4, 4, 200000, 1.0, 1.0, 0) == FT_EINVAL
    assert f(None, None, None, 0, 4, 4, 1.0, 1.0, 0) == FT_OK      # empty
    g = lib.ft_qgemm_perchannel_launch
    g.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 3 + [ctypes.c_float,
                                                             ctypes.c_size_t]
    st = g(None, None, None, None, 4, 4, 4, 1.0, 0)
    assert st == FT_EINVAL and b"per-channel" in lib.ft_last_error()
    h = lib.ft_qgemm_launch_ex
    h.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
                  ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                  ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_size_t]
    assert h(None, None, None, 1.0, 1.0, None, None, 7, 4, 4, 4, 0) == FT_EINVAL


def test_dequantize_qadd_invalid_arguments(lib):
    d = lib.ft_dequantize_int8_launch
    d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_longlong,
                  ctypes.c_size_t]
    assert d(None, None, 1.0, -1, 0) == FT_EINVAL
    assert d(None, None, 1.0, 8, 0) == FT_EINVAL and b"null" in lib.ft_last_error()
    assert d(None, None, 1.0, 0, 0) == FT_OK                      # empty
    dx = lib.ft_dequantize_int8_launch_ex
    dx.argtypes = [ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p,
                   ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t]
    assert dx(None, 1.0, None, None, 9, 8, 0) == FT_EINVAL       # dtype code
    q = lib.ft_qadd_int8_launch
    q.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_float,
                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_size_t]
    assert q(None, None, 1.0, 1.0, None, None, -2, 0) == FT_EINVAL
    assert q(None, None, 1.0, 1.0, None, None, 16, 0) == FT_EINVAL
    assert q(None, None, 1.0, 1.0, None, None, 0, 0) == FT_OK


def test_prefill_and_sampling_invalid_arguments(lib):
    f = lib.ft_attention_prefill_launch_bf16
    f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 6 + [ctypes.c_size_t]
    assert f(None, None, None, None, 1, 5, 2, 8, 64, 1, 0) == FT_EINVAL     # GQA
    assert f(None, None, None, None, 1, 4, 2, 8, 30, 1, 0) == FT_EINVAL     # dim % 4
    assert f(None, None, None, None, 1, 4, 2, 8, 516, 1, 0) == FT_EINVAL    # dim > 512
    assert f(None, None, None, None, 1, 4, 2, 8, 64, 1, 0) == FT_EINVAL     # null
    assert f(None, None, None, None, 0, 4, 2, 8, 64, 1, 0) == FT_OK         # empty
    s = lib.ft_sample_topp_launch
    s.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                  ctypes.c_ulonglong, ctypes.c_void_p, ctypes.c_size_t]
    assert s(None, 8, 0.0, 1.0, 0, None, 0) == FT_EINVAL                   # p
    assert s(None, 8, 0.9, 0.0, 0, None, 0) == FT_EINVAL                   # temperature
    assert s(None, 0, 0.9, 1.0, 0, None, 0) == FT_EINVAL                   # empty
    d = lib.ft_decode_step_launch
    d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                  ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_ulonglong,
                  ctypes.c_void_p, ctypes.c_size_t]
    assert d(None, None, 8, 1, 0.0, 0.9, 1.0, 0, None, 0) == FT_EINVAL     # penalty
    assert d(None, None, 1 << 20, 1, 1.5, 0.9, 1.0, 0, None, 0) == FT_EINVAL  # bitmap cap
    a = lib.ft_argmax_batched_launch
    a.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                  ctypes.c_size_t]
    assert a(None, 2, 0, None, 0) == FT_EINVAL
    assert a(None, 0, 4, None, 0) == FT_OK


def test_norm_rope_swiglu_invalid_arguments(lib):
    r = lib.ft_rmsnorm_launch
    r.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                          ctypes.c_size_t]
    assert r(None, None, None, None, 2, 0, 1e-6, 0) == FT_EINVAL
    assert r(None, None, None, None, 0, 8, 1e-6, 0) == FT_OK           # no rows
    ro = lib.ft_rope_launch
    ro.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                   ctypes.c_float, ctypes.c_int, ctypes.c_size_t]
    assert ro(None, None, 2, 7, 10000.0, 0, 0) == FT_EINVAL            # odd dim
    assert ro(None, None, 2, 8, 10000.0, -1, 0) == FT_EINVAL           # offset < 0
    s = lib.ft_swiglu_launch
    s.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_longlong, ctypes.c_size_t]
    assert s(None, None, None, -1, 0) == FT_EINVAL
    qz = lib.ft_quantize_int8_launch_ex
    qz.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                   ctypes.c_longlong, ctypes.c_size_t]
    assert qz(None, 9, None, None, 4, 0) == FT_EINVAL                  # bad dtype


def test_fused_invalid_arguments(lib):
    rq = lib.ft_rmsnorm_quant_launch
    rq.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                   ctypes.c_float, ctypes.c_size_t]
    assert rq(None, 0, None, None, None, None, 2, 6, 1e-6, 0) == FT_EINVAL  # cols % 4
    assert rq(None, 0, None, None, None, None, 2, 0, 1e-6, 0) == FT_EINVAL
    assert rq(None, 9, None, None, None, None, 2, 8, 1e-6, 0) == FT_EINVAL  # dtype
    assert rq(None, 1, None, None, None, None, 0, 8, 1e-6, 0) == FT_OK      # no rows
    rg = lib.ft_rmsnorm_qgemm_launch
    rg.argtypes = ([ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                    ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
                    ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p] +
                   [ctypes.c_int] * 3 + [ctypes.c_size_t])
    assert rg(None, 2, None, None, 1e-5, None, None, 0.0, None, 9, None, None,
              1, 8, 16, 0) == FT_EINVAL                                    # out dtype
    assert rg(None, 2, None, None, 1e-5, None, None, 0.0, None, 2, None, None,
              1, 8, 0, 0) == FT_EINVAL                                     # k == 0
    assert rg(None, 2, None, None, 1e-5, None, None, 0.0, None, 2, None, None,
              1, 8, 16, 0) == FT_EINVAL                                    # null operands
    assert rg(None, 2, None, None, 1e-5, None, None, 0.0, None, 2, None, None,
              0, 8, 16, 0) == FT_OK                                        # no rows
    # no output columns (b_q [0, K]) with rows: the codes and the scale are
    # still owed, so the call proceeds to the operand checks (not FT_OK)
    assert rg(None, 2, None, None, 1e-5, None, None, 0.0, None, 2, None, None,
              1, 0, 16, 0) == FT_EINVAL
    assert b"null operand" in lib.ft_last_error()
    # the GEMM's K limit is checked before anything is launched
    assert rg(None, 2, None, None, 1e-5, None, None, 0.0, None, 2, None, None,
              1, 8, 131072, 0) == FT_EINVAL
    assert b"K too large" in lib.ft_last_error()
    sq = lib.ft_swiglu_quant_launch
    sq.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_longlong,
                   ctypes.c_size_t]
    assert sq(None, None, 0, None, None, 2, 8, 4, 0) == FT_EINVAL          # ld < cols
    assert sq(None, None, 0, None, None, -1, 8, 8, 0) == FT_EINVAL
    assert sq(None, None, 2, None, None, 0, 8, 16, 0) == FT_OK
    rk = lib.ft_rope_kv_append_paged_launch
    rk.argtypes = ([ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong] +
                   [ctypes.c_void_p] * 5 + [ctypes.c_int] * 6 +
                   [ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_size_t])
    ok = dict(batch=2, hq=4, hkv=2, dim=8, page=16, width=3)

    def call(ld=64, batch=2, hq=4, hkv=2, dim=8, page=16, width=3, off=0):
        return rk(None, 1, ld, None, None, None, None, None, batch, hq, hkv, dim,
                  page, width, 10000.0, off, 0, 0)
    assert call(dim=7) == FT_EINVAL
    assert call(ld=63) == FT_EINVAL              # (4 + 2*2) * 8 = 64
    assert call(page=0) == FT_EINVAL
    assert call(off=-1) == FT_EINVAL
    assert call(batch=0) == FT_OK
    assert call(**ok) == FT_EINVAL               # null operands


def test_tuning_switches_by_name(lib):
    # the FT_* switches are read once per process; the ABI overrides them
    # by name and restores them (no device involved)
    lib.ft_set_tuning.argtypes = [ctypes.c_char_p, ctypes.c_int]
    lib.ft_clear_tuning.argtypes = [ctypes.c_char_p]
    assert lib.ft_set_tuning(b"FT_QGEMM_BAND", 8) == FT_OK
    assert lib.ft_clear_tuning(b"FT_QGEMM_BAND") == FT_OK
    assert lib.ft_set_tuning(b"FT_NO_SUCH_SWITCH", 1) == FT_EINVAL
    assert b"unknown tuning switch" in lib.ft_last_error()
    assert lib.ft_clear_tuning(None) == FT_EINVAL


def test_scratch_allocation_failure_is_reported(lib):
    # FT_FAIL_SCRATCH (test hook) fails every device-scratch request the way
    # an allocation failure does. A quantize of 2^20 elements asks for its
    # partial-maximum scratch before any launch, so the error path is reached
    # (and the pointers never touched) without a device.
    lib.ft_set_tuning.argtypes = [ctypes.c_char_p, ctypes.c_int]
    lib.ft_clear_tuning.argtypes = [ctypes.c_char_p]
    assert lib.ft_set_tuning(b"FT_FAIL_SCRATCH", 1) == FT_OK
    try:
        rc = lib.ft_quantize_int8_launch(_v(256), _v(256), _v(256), ctypes.c_longlong(1 << 20),
                                         ctypes.c_uint64(0))
        assert rc == FT_EHIP
        assert b"FT_FAIL_SCRATCH" in lib.ft_last_error()
        import fusedtok_amd as ft
        with pytest.raises(RuntimeError, match="out of memory"):
            ft._fusedtok.quantize_launch(256, 256, 256, 1 << 20, 0)
    finally:
        assert lib.ft_clear_tuning(b"FT_FAIL_SCRATCH") == FT_OK


def test_decode_layer_and_stack_invalid_arguments(lib):
    # every check here runs before the entry point's first HIP call
    P, I, U = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    out = ctypes.c_void_p(1)
    cr = lib.ft_decode_layer_create
    cr.argtypes = [P, P]
    assert cr(None, ctypes.byref(out)) == FT_EINVAL
    desc = (ctypes.c_char * 512)()  # zeroed: hidden 0 fails the shape checks
    assert cr(desc, ctypes.byref(out)) == FT_EINVAL
    assert out.value is None  # *out cleared before validation
    assert b"hidden" in lib.ft_last_error()
    fw = lib.ft_decode_layer_forward
    fw.argtypes = [P, P, P, P, P, P, P, I, I, U]
    assert fw(None, None, None, None, None, None, None, 1, 1, 0) == FT_EINVAL
    cp = lib.ft_decode_layer_capture
    cp.argtypes = [P, P, P, P, P, P, P, I, I, U]
    assert cp(None, None, None, None, None, None, None, 1, 1, 0) == FT_EINVAL
    rp = lib.ft_decode_layer_replay
    rp.argtypes = [P, U]
    assert rp(None, 0) == FT_EINVAL
    lib.ft_decode_layer_destroy.argtypes = [P]
    assert lib.ft_decode_layer_destroy(None) == FT_OK

    sc = lib.ft_decode_stack_create
    sc.argtypes = [P, I, P]
    out = ctypes.c_void_p(1)
    assert sc(None, 1, ctypes.byref(out)) == FT_EINVAL and out.value is None
    nulls = (ctypes.c_void_p * 2)(None, None)
    assert sc(nulls, 2, ctypes.byref(out)) == FT_EINVAL
    assert b"null layer" in lib.ft_last_error()
    assert sc(nulls, 0, ctypes.byref(out)) == FT_EINVAL
    assert sc(nulls, 2, None) == FT_EINVAL
    sf = lib.ft_decode_stack_forward
    sf.argtypes = [P, P, P, P, P, P, P, I, I, U]
    assert sf(None, None, None, None, None, None, None, 1, 1, 0) == FT_EINVAL
    sp = lib.ft_decode_stack_capture
    sp.argtypes = [P, P, P, P, P, P, P, I, I, U]
    assert sp(None, None, None, None, None, None, None, 1, 1, 0) == FT_EINVAL
    sr = lib.ft_decode_stack_replay
    sr.argtypes = [P, U]
    assert sr(None, 0) == FT_EINVAL
    lib.ft_decode_stack_destroy.argtypes = [P]
    assert lib.ft_decode_stack_destroy(None) == FT_OK


def test_host_device_address_null_arguments(lib):
    f = lib.ft_host_device_address
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    dev = ctypes.c_void_p(1)
    assert f(None, ctypes.byref(dev)) == FT_EINVAL
    assert f(ctypes.byref(dev), None) == FT_EINVAL
