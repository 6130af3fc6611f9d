"""The declarative argument contracts (fusedtok_amd/_contract.py) and the
sampling-argument normalisation (fusedtok_amd/_sampling_args.py), on the
host: shape binding, messages, error classes, in-place staging rules and
the three history forms. No device is needed."""

import numpy as np
import pytest
import torch

import fusedtok_amd as ft
from fusedtok_amd import _sampling_args as sa
from fusedtok_amd._contract import Arr, Contract, Idx, Rule


def test_symbols_bind_across_operands():
    c = Contract(Arr("q", "B Hq D"), Arr("k", "B Hkv T D", mismatch="k must match q"),
                 Idx("lens", "B", lambda c: c.T, optional=True, what="lens shape"))
    call = c.bind(q=np.zeros((2, 8, 16), np.float32), k=np.zeros((2, 4, 5, 16), np.float32),
                  lens=np.array([5, 0], np.int32))
    assert (call.B, call.Hq, call.Hkv, call.T, call.D) == (2, 8, 4, 5, 16)
    assert not call.on_gpu
    with pytest.raises(ValueError, match="k must match q"):
        c.bind(q=np.zeros((2, 8, 16), np.float32), k=np.zeros((2, 4, 5, 8), np.float32),
               lens=None)
    with pytest.raises(ValueError, match=r"lens entries must be in \[0, 5\]"):
        c.bind(q=np.zeros((2, 8, 16), np.float32), k=np.zeros((2, 4, 5, 16), np.float32),
               lens=np.array([6, 0]))
    with pytest.raises(ValueError, match="lens shape"):
        c.bind(q=np.zeros((2, 8, 16), np.float32), k=np.zeros((2, 4, 5, 16), np.float32),
               lens=np.array([1, 2, 3]))


def test_optional_leading_dim_and_same_shape():
    c = Contract(Arr("x", "rows? cols"), Arr("r", "=x", optional=True, mismatch="r vs x"))
    assert c.bind(x=np.zeros(7, np.float32), r=None).rows == 1
    assert c.bind(x=np.zeros((3, 7), np.float32), r=None).rows == 3
    with pytest.raises(ValueError, match="r vs x"):
        c.bind(x=np.zeros((3, 7), np.float32), r=np.zeros((7,), np.float32))


def test_open_bound_and_rules():
    c = Contract(Arr("cache", "B T"), Idx("lens", "B", lambda c: c.T, open_bound=True,
                                          what="w"),
                 rules=(Rule(lambda c: c.T % 2 == 0, "T must be even"),))
    with pytest.raises(ValueError, match=r"\[0, 4\)"):
        c.bind(cache=np.zeros((1, 4), np.float32), lens=[4])
    with pytest.raises(ValueError, match="T must be even"):
        c.bind(cache=np.zeros((1, 3), np.float32), lens=[0])
    with pytest.raises(TypeError, match="integer values"):
        c.bind(cache=np.zeros((1, 4), np.float32), lens=[0.5])


def test_inplace_host_operands_must_be_writable_float32():
    with pytest.raises(TypeError, match="in-place"):
        ft.kv_append(np.zeros((1, 1, 4, 4), np.float64), np.zeros((1, 1, 4, 4), np.float32),
                     np.zeros((1, 1, 4), np.float32), np.zeros((1, 1, 4), np.float32), [0])
    strided = np.zeros((1, 1, 4, 8), np.float32)[..., ::2]
    with pytest.raises(TypeError, match="in-place"):
        ft.kv_append(strided, strided.copy(), np.zeros((1, 1, 4), np.float32),
                     np.zeros((1, 1, 4), np.float32), [0])


def test_host_messages_of_the_public_ops():
    q = np.zeros((1, 4, 8), np.float32)
    k = np.zeros((1, 2, 6, 8), np.float32)
    with pytest.raises(ValueError, match="head counts"):
        ft.attention_decode(np.zeros((1, 0, 8), np.float32), k, k)
    with pytest.raises(ValueError, match="multiple of kv heads"):
        ft.attention_decode(np.zeros((1, 3, 8), np.float32), k, k)
    with pytest.raises(ValueError, match=r"q must be \[B, Hq, D\]"):
        ft.attention_decode(np.zeros((4, 8), np.float32), k, k)
    with pytest.raises(ValueError, match="multiple of 4 and at most 512"):
        ft.attention_decode(np.zeros((1, 2, 6), np.float32), np.zeros((1, 1, 3, 6), np.float32),
                            np.zeros((1, 1, 3, 6), np.float32))
    with pytest.raises(ValueError, match="block_table must be"):
        ft.attention_decode_paged(q, np.zeros((3, 2, 4, 8), np.float32),
                                  np.zeros((3, 2, 4, 8), np.float32), np.zeros((2, 1), np.int32))
    with pytest.raises(ValueError, match=r"block_table entries must be in \[0, 3\)"):
        ft.attention_decode_paged(q, np.zeros((3, 2, 4, 8), np.float32),
                                  np.zeros((3, 2, 4, 8), np.float32), np.array([[3]]))
    with pytest.raises(ValueError, match="even"):
        ft.rope(np.zeros((2, 5), np.float32))
    with pytest.raises(ValueError, match="pos_offset"):
        ft.rope(np.zeros((2, 4), np.float32), pos_offset=-2)
    with pytest.raises(TypeError, match="a_q"):
        ft.qgemm(np.ones((2, 4), np.float32), 0.5, np.ones((3, 4), np.int8), 0.5)
    with pytest.raises(TypeError, match="b_q"):
        ft.qgemm(np.ones((2, 4), np.int8), 0.5, np.ones((3, 4), np.float32), 0.5)
    with pytest.raises(TypeError, match="int8"):
        ft.dequantize_int8(np.ones(4, np.float32), 0.5)
    with pytest.raises(TypeError, match="GPU int8"):
        ft.qadd_int8(np.ones(4, np.int8), 0.5, np.ones(4, np.int8), 0.5)
    with pytest.raises(TypeError, match="no host path"):
        ft.rmsnorm_quant(np.ones((2, 4), np.float32), np.ones(4, np.float32))


def test_sampling_params_and_seeds():
    with pytest.raises(ValueError, match="p must be"):
        ft.sample_topp(np.zeros(4, np.float32), 0.0)
    with pytest.raises(ValueError, match="temperature"):
        ft.sample_topp(np.zeros(4, np.float32), 0.5, temperature=0.0)
    with pytest.raises(ValueError, match="penalty"):
        ft.decode_step(np.zeros(4, np.float32), [0], 0.0)
    with pytest.raises(ValueError, match="empty logits"):
        ft.sample_topp(np.zeros(0, np.float32), 0.5)
    np.testing.assert_array_equal(sa.seed_vector(None, 3), [0, 1, 2])
    np.testing.assert_array_equal(sa.seed_vector(np.array([2 ** 63 - 1], np.uint64), 1),
                                  [2 ** 63 - 1])
    with pytest.raises(ValueError, match=r"2\*\*63"):
        sa.seed_vector(np.array([2 ** 63], np.uint64), 1)
    with pytest.raises(ValueError, match=r"2\*\*63"):
        sa.seed_vector([-1], 1)
    with pytest.raises(TypeError, match="integers"):
        sa.seed_vector([0.5], 1)
    with pytest.raises(ValueError, match="one entry per row"):
        sa.seed_vector([1, 2], 3)
    with pytest.raises(ValueError, match="1-D"):
        sa.seed_vector([[1]], 1)


def test_history_forms_give_one_csr_layout():
    ragged = [[3, 1], [], [4, 4, 0]]
    flat, offs = sa.histories_csr(ragged, None, 3, 8)
    np.testing.assert_array_equal(flat, [3, 1, 4, 4, 0])
    np.testing.assert_array_equal(offs, [0, 2, 2, 5])
    f2, o2 = sa.histories_csr(np.array([3, 1, 4, 4, 0]), np.array([0, 2, 2, 5]), 3, 8)
    np.testing.assert_array_equal(f2, flat)
    np.testing.assert_array_equal(o2, offs)
    f3, o3 = sa.histories_csr(torch.tensor([[1, 2], [3, 4]]), None, 2, 8)
    np.testing.assert_array_equal(f3, [1, 2, 3, 4])
    np.testing.assert_array_equal(o3, [0, 2, 4])
    with pytest.raises(ValueError, match=r"\[0, 8\)"):
        sa.histories_csr([[8]], None, 1, 8)
    with pytest.raises(ValueError, match="non-decreasing"):
        sa.histories_csr(np.array([1, 2]), np.array([0, 2, 1]), 2, 8)
    with pytest.raises(TypeError, match="ids_offsets"):
        sa.histories_csr(np.array([1, 2]), np.array([0.0, 1.5, 2.0]), 2, 8)
    with pytest.raises(ValueError, match="one entry per row"):
        sa.histories_csr([[1]], None, 2, 8)
    np.testing.assert_array_equal(sa.history_1d([5, 0], 6, None), [5, 0])
    with pytest.raises(ValueError, match=r"\[0, 6\)"):
        sa.history_1d([6], 6, None)
