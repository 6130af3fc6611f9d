"""Python API surface and error contract (reference tests/test_api.py,
tests/test_validation.py): ValueError for shapes / values, TypeError for
dtypes / device families. Host-origin inputs are validated before any device
work, so these run without a GPU. Without a device, valid host inputs raise
RuntimeError (no CPU fallback)."""

import numpy as np
import pytest

import fusedtok_amd as ft

HOT_PATH = ["cuda_available", "rmsnorm", "rope", "swiglu", "quantize_int8", "qgemm",
            "qgemm_perchannel", "attention_decode", "attention_decode_paged",
            "kv_append", "kv_append_paged"]


def test_reference_hot_path_names_present():
    for name in HOT_PATH:
        assert name in ft.__all__ and callable(getattr(ft, name))
        assert getattr(ft, name).__doc__


def test_attention_shape_errors():
    q = np.zeros((1, 6, 32), np.float32)
    k = np.zeros((1, 2, 8, 32), np.float32)
    with pytest.raises(ValueError):
        ft.attention_decode(np.zeros((1, 5, 32), np.float32), k, k)     # Hq % Hkv
    with pytest.raises(ValueError):
        ft.attention_decode(q, k, np.zeros((1, 2, 7, 32), np.float32))  # v shape
    with pytest.raises(ValueError):
        ft.attention_decode(np.zeros((1, 2, 30), np.float32),
                            np.zeros((1, 1, 4, 30), np.float32),
                            np.zeros((1, 1, 4, 30), np.float32))        # D % 4
    with pytest.raises(ValueError):
        ft.attention_decode(np.zeros((1, 2, 516), np.float32),
                            np.zeros((1, 1, 4, 516), np.float32),
                            np.zeros((1, 1, 4, 516), np.float32))       # D > 512
    for bad in ([9], [-1], [1, 2]):
        with pytest.raises(ValueError):
            ft.attention_decode(q, k, k, np.array(bad, np.int32))
    with pytest.raises(TypeError):
        ft.attention_decode(q, k, k, np.array([1.5]))                    # float lens


def test_paged_shape_and_table_errors():
    q = np.zeros((2, 8, 32), np.float32)
    kp = np.zeros((4, 2, 16, 32), np.float32)
    tbl = np.zeros((2, 2), np.int32)
    with pytest.raises(ValueError):
        ft.attention_decode_paged(np.zeros((2, 6, 32), np.float32),
                                  np.zeros((4, 2, 16, 32), np.float32),
                                  np.zeros((4, 2, 16, 32), np.float32),
                                  tbl)                                   # group 3
    with pytest.raises(ValueError):
        ft.attention_decode_paged(q, kp, kp, np.array([[0, 4], [1, 2]], np.int32))
    with pytest.raises(ValueError):
        ft.attention_decode_paged(q, kp, kp, np.zeros((3, 2), np.int32))  # rows
    with pytest.raises(ValueError):
        ft.attention_decode_paged(q, kp, kp, tbl, np.array([0, 33], np.int32))


def test_kv_append_errors():
    kc = np.zeros((2, 2, 8, 16), np.float32)
    kn = np.zeros((2, 2, 16), np.float32)
    with pytest.raises(ValueError):
        ft.kv_append(kc, kc.copy(), kn, kn, np.array([0, 8], np.int32))  # == T
    with pytest.raises(TypeError):
        ft.kv_append(kc.astype(np.float64), kc, kn, kn, np.array([0, 1], np.int32))
    kp = np.zeros((4, 2, 4, 16), np.float32)
    with pytest.raises(ValueError):
        ft.kv_append_paged(kp, kp.copy(), np.zeros((2, 2), np.int32), kn, kn,
                           np.array([0, 8], np.int32))                   # == S*P
    with pytest.raises(ValueError):
        ft.kv_append_paged(kp, kp.copy(), np.full((2, 2), 4, np.int32), kn, kn,
                           np.array([0, 1], np.int32))                   # block id


def test_int8_errors():
    a = np.zeros((4, 8), np.int8)
    with pytest.raises(ValueError):
        ft.qgemm(a, 1.0, np.zeros((2, 7), np.int8), 1.0)
    with pytest.raises(ValueError):
        ft.qgemm(np.zeros((4,), np.int8), 1.0, np.zeros((2, 8), np.int8), 1.0)
    with pytest.raises(ValueError):
        ft.qgemm_perchannel(a, 1.0, np.zeros((2, 8), np.int8), np.ones(3, np.float32))
    with pytest.raises(TypeError):
        ft.qgemm(np.ones((4, 8), np.float32), 0.5, a, 0.5)


def test_norm_rope_swiglu_errors():
    x = np.zeros((1, 4), np.float32)
    with pytest.raises(ValueError):
        ft.rmsnorm(x, np.ones(3, np.float32))
    with pytest.raises(ValueError):
        ft.rmsnorm(x, np.ones(4, np.float32), residual=np.zeros(5, np.float32))
    with pytest.raises(ValueError):
        ft.rmsnorm(np.zeros((2, 2, 2), np.float32), np.ones(2, np.float32))
    with pytest.raises(ValueError):
        ft.rope(np.zeros((2, 7), np.float32), None)
    with pytest.raises(ValueError):
        ft.rope(np.zeros((2, 8), np.float32), None, pos_offset=-1)
    with pytest.raises(ValueError):
        ft.swiglu(np.zeros(4, np.float32), np.zeros(5, np.float32))


def test_no_cpu_fallback_without_device():
    if ft.cuda_available():
        pytest.skip("a HIP device is present")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ft.swiglu(np.zeros(4, np.float32), np.zeros(4, np.float32))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ft.quantize_int8(np.ones(4, np.float32))


def test_stub_and_marker_cover_the_public_surface():
    # the package ships a PEP 561 marker and a stub naming every public
    # function, with the runtime __all__ in the same order (reference
    # tests/test_api.py:110-150 checks its own package the same way)
    import pathlib
    import re
    pkg = pathlib.Path(ft.__file__).parent
    assert (pkg / "py.typed").is_file()
    text = (pkg / "__init__.pyi").read_text()
    import ast
    ast.parse(text)  # a stub type checkers can read
    for name in ft.__all__:
        assert f"def {name}(" in text or f"class {name}:" in text, name
    listed = re.findall(r'"(\w+)"', re.search(r"__all__ = \[(.*?)\]", text, re.S).group(1))
    assert listed == list(ft.__all__)


def test_no_public_callables_beyond_all():
    public = {n for n, v in vars(ft).items() if not n.startswith("_") and callable(v)}
    assert public <= set(ft.__all__), sorted(public - set(ft.__all__))
