"""GPU parity for attention_prefill (reference tests/test_attention.py:150-240,
632-730) against the CPU oracle (attention_prefill_cpu restatement) run on
the same storage-rounded inputs.

Bars: half storage |err| <= 2e-3 + 1e-2 |ref| (the north-star attention
tolerance; the reference's own half tolerances are looser: bf16 2e-2, fp16
2e-3); float32 rtol 1e-4 / atol 1e-5 (test_attention.py:196-197). Paths:
the MFMA kernel (bf16 / fp16, D in {64, 128}) with ragged S over its
128-row query tiles and 64-row key tiles, causal and bidirectional, GQA;
the generic kernel (float32, other D, forced)."""

import numpy as np
import pytest
import torch

import fusedtok_amd as ft
import oracle
from tests import refs

pytestmark = pytest.mark.gpu
DEV = "cuda"
HALF = [torch.bfloat16, torch.float16]


def _inputs(rng, b, hq, hkv, s, d, dt):
    q = torch.from_numpy(rng.standard_normal((b, hq, s, d)).astype(np.float32)).to(DEV, dt)
    k = torch.from_numpy(rng.standard_normal((b, hkv, s, d)).astype(np.float32)).to(DEV, dt)
    v = torch.from_numpy(rng.standard_normal((b, hkv, s, d)).astype(np.float32)).to(DEV, dt)
    return q, k, v


def _check_half(out, q, k, v, causal):
    ref = oracle.attention_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                   v.float().cpu().numpy(), causal)
    got = out.float().cpu().numpy()
    excess = np.abs(got - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert excess.max() <= 0, f"max excess {excess.max()}"


@pytest.mark.parametrize("dt", HALF)
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("s", [1, 63, 65, 128, 200, 300])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_mfma_matches_oracle(dt, d, s, causal):
    rng = np.random.default_rng(s * 10 + d + int(causal))
    q, k, v = _inputs(rng, 2, 4, 2, s, d, dt)
    out = ft.attention_prefill(q, k, v, causal=causal)
    assert out.dtype is dt and out.shape == q.shape
    _check_half(out, q, k, v, causal)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_bf16_large_v_tiles_take_the_split_path(d, causal):
    # bf16 inputs: a key tile whose V values all stay below 2^16 runs the PV
    # product in fp16 (exact V, P rounded to 11 bits); from the first tile
    # holding a larger value on, the workgroup uses bf16 P split hi + lo.
    # Here keys 130..199 carry V around 7e4 (tiles 2 and 3), so both paths
    # and the hand-over run; the oracle sees the same rounded inputs. (Large
    # values of mixed sign would cancel to outputs of order 1 whose error
    # follows the large terms, for any finite precision of P.)
    rng = np.random.default_rng(d + int(causal))
    dt = torch.bfloat16
    q, k, v = _inputs(rng, 1, 4, 2, 300, d, dt)
    v2 = v.clone()
    big = 7.0e4 + 1.0e3 * rng.standard_normal((1, 2, 70, d)).astype(np.float32)
    v[:, :, 130:200] = torch.from_numpy(big).to(DEV, dt)
    assert v.float().abs().max().item() >= 65536.0
    out = ft.attention_prefill(q, k, v, causal=causal)
    _check_half(out, q, k, v, causal)
    # and every value in range: the fp16 path alone
    _check_half(ft.attention_prefill(q, k, v2, causal=causal), q, k, v2, causal)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("prepass", [0, 2])
def test_prefill_bf16_tiny_v_tiles_take_the_split_path(d, causal, prepass, tuning):
    # fp16 holds a bf16 value exactly only for 2^-17 <= |v| < 2^16 (or 0):
    # below, fp16 subnormals drop significant bits. A tile whose values are
    # all small (largest |v| < 2^-8) takes the bf16 split path. With every V
    # around 1e-7 the output is of that order too, so it is checked at 1e-2
    # relative (the fp16 product would be off by up to ~30% there). Keys
    # 130-199 tiny (tiles 2 and 3 keep larger values: the fp16 product,
    # tiny values off by at most 2^-25) and tile 2 wholly tiny (the
    # hand-over) at the usual bar. Pre-pass and in-kernel vote.
    tuning("FT_PREFILL_PREPASS", prepass)
    rng = np.random.default_rng(60 + d + 2 * causal)
    dt = torch.bfloat16
    q, k, v = _inputs(rng, 1, 4, 2, 300, d, dt)
    tiny = (v.float() * 1e-7).to(dt)
    assert 0 < tiny.float().abs().max().item() < 2.0 ** -17
    out = ft.attention_prefill(q, k, tiny, causal=causal)
    ref = oracle.attention_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                   tiny.float().cpu().numpy(), causal)
    got = out.float().cpu().numpy()
    excess = np.abs(got - ref) - (1e-12 + 1e-2 * np.abs(ref))
    assert excess.max() <= 0, f"max excess {excess.max()}"
    mixed = v.clone()
    mixed[:, :, 130:200] = tiny[:, :, 130:200]
    _check_half(ft.attention_prefill(q, k, mixed, causal=causal), q, k, mixed, causal)
    whole = v.clone()
    whole[:, :, 128:192] = tiny[:, :, 128:192]
    _check_half(ft.attention_prefill(q, k, whole, causal=causal), q, k, whole, causal)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("big", [False, True])
def test_prefill_bf16_v_prepass_equals_in_kernel_conversion(d, causal, big, tuning):
    # bf16 inputs: V converted to fp16 by a pre-pass (with a per-tile range
    # flag) or by every workgroup as it stages the tile (with a vote): the
    # same tiles take the fp16 PV product, so the outputs are the same bits.
    # S = 300 leaves a partial last tile; `big` puts values >= 2^16 in tiles
    # 2 and 3 (the hand-over to the bf16 split path).
    rng = np.random.default_rng(40 + d + 2 * causal + big)
    dt = torch.bfloat16
    q, k, v = _inputs(rng, 2, 8, 2, 300, d, dt)
    if big:
        v[:, :, 130:200] = torch.from_numpy(
            7.0e4 + 1.0e3 * rng.standard_normal((2, 2, 70, d)).astype(np.float32)).to(DEV, dt)
    tuning("FT_PREFILL_PREPASS", 0)
    inkernel = ft.attention_prefill(q, k, v, causal=causal)
    tuning("FT_PREFILL_PREPASS", 2)
    pre = ft.attention_prefill(q, k, v, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(pre, inkernel)
    _check_half(pre, q, k, v, causal)


@pytest.mark.parametrize("dt", HALF)
def test_prefill_mfma_first_row_is_v0_and_s1_is_decode(dt):
    rng = np.random.default_rng(5)
    q, k, v = _inputs(rng, 2, 8, 2, 130, 128, dt)
    out = ft.attention_prefill(q, k, v, causal=True)
    # causal row 0 attends to key 0 only: exactly v[0] (weight 1.0, exact)
    for h in range(8):
        assert torch.equal(out[:, h, 0], v[:, h // 4, 0])
    # S = 1 prefill is the decode step over one key
    q1, k1, v1 = q[:, :, :1].contiguous(), k[:, :, :1].contiguous(), v[:, :, :1].contiguous()
    pre = ft.attention_prefill(q1, k1, v1, causal=True)
    dec = ft.attention_decode(q1.reshape(2, 8, 128).contiguous(), k1, v1)
    assert torch.equal(pre.reshape(2, 8, 128), dec)


@pytest.mark.parametrize("dt", HALF)
def test_prefill_mfma_long_sequence_sampled_rows(dt):
    # S = 2048, GQA 4: 16 query tiles x 32 key tiles per head; rows near tile
    # edges against float64 on the rounded inputs
    rng = np.random.default_rng(7)
    b, hq, hkv, s, d = 1, 8, 2, 2048, 128
    q, k, v = _inputs(rng, b, hq, hkv, s, d, dt)
    rows = [0, 1, 63, 64, 127, 128, 1000, 2046, 2047]
    qn, kn, vn = (x.float().cpu().numpy() for x in (q, k, v))
    for causal in (True, False):
        out = ft.attention_prefill(q, k, v, causal=causal).float().cpu().numpy()
        ref = refs.ref_prefill(qn, kn, vn, causal, rows=rows)
        for i in rows:
            excess = np.abs(out[:, :, i] - ref[:, :, i]) - (2e-3 + 1e-2 * np.abs(ref[:, :, i]))
            assert excess.max() <= 0, f"row {i} causal={causal}: {excess.max()}"


@pytest.mark.parametrize("b,hq,hkv,s,d", [(1, 4, 2, 1, 32), (1, 8, 8, 5, 64),
                                          (2, 6, 3, 17, 16), (1, 32, 8, 40, 128),
                                          (1, 4, 1, 33, 8), (1, 8, 2, 64, 256),
                                          (1, 4, 2, 9, 512)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_f32_generic(b, hq, hkv, s, d, causal):
    rng = np.random.default_rng(b * 100 + hq * 17 + s * 3 + d + causal)
    q = rng.standard_normal((b, hq, s, d)).astype(np.float32)
    k = rng.standard_normal((b, hkv, s, d)).astype(np.float32)
    v = rng.standard_normal((b, hkv, s, d)).astype(np.float32)
    out = ft.attention_prefill(torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV),
                               torch.from_numpy(v).to(DEV), causal=causal)
    np.testing.assert_allclose(out.cpu().numpy(), oracle.attention_prefill(q, k, v, causal),
                               rtol=1e-4, atol=1e-5)
    # host inputs are staged through the device, same result
    staged = ft.attention_prefill(q, k, v, causal=causal)
    np.testing.assert_allclose(staged, out.cpu().numpy(), rtol=0, atol=0)


@pytest.mark.parametrize("dt", HALF)
@pytest.mark.parametrize("d", [36, 48, 96, 112])
def test_prefill_half_generic_dims(dt, d):
    # dims outside {64, 128} take the generic kernel (the reference's 2.4.1
    # regression: such dims must not reach the tiled MFMA template)
    rng = np.random.default_rng(d)
    q, k, v = _inputs(rng, 1, 4, 2, 70, d, dt)
    for causal in (True, False):
        _check_half(ft.attention_prefill(q, k, v, causal=causal), q, k, v, causal)


@pytest.mark.parametrize("dt", HALF)
def test_prefill_mfma_and_generic_agree(dt, tuning):
    rng = np.random.default_rng(9)
    q, k, v = _inputs(rng, 1, 4, 2, 150, 128, dt)
    a = ft.attention_prefill(q, k, v).float()
    tuning("FT_PREFILL_FORCE_GENERIC", 1)
    g = ft.attention_prefill(q, k, v).float()
    _check_half(g.to(dt), q, k, v, True)
    assert (a - g).abs().max().item() <= 2e-3 + 1e-2 * g.abs().max().item()


def test_prefill_contract():
    q = torch.zeros((1, 4, 8, 32), device=DEV)
    k = torch.zeros((1, 2, 8, 32), device=DEV)
    with pytest.raises(ValueError):
        ft.attention_prefill(torch.zeros((1, 5, 8, 32), device=DEV), k, k)
    with pytest.raises(ValueError):
        ft.attention_prefill(q, k, torch.zeros((1, 2, 7, 32), device=DEV))
    with pytest.raises(ValueError):
        ft.attention_prefill(torch.zeros((1, 4, 8, 30), device=DEV),
                             torch.zeros((1, 2, 8, 30), device=DEV),
                             torch.zeros((1, 2, 8, 30), device=DEV))
    with pytest.raises(TypeError):
        ft.attention_prefill(q, k.to(torch.bfloat16), k)
    assert ft.attention_prefill(q[:, :, :0], k[:, :, :0], k[:, :, :0]).shape == (1, 4, 0, 32)


def test_prefill_graph_capture_replays():
    # no workspace: capturable as is; replays with eager work between them
    rng = np.random.default_rng(3)
    q, k, v = _inputs(rng, 1, 8, 2, 256, 128, torch.bfloat16)
    ref = ft.attention_prefill(q, k, v)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ft.attention_prefill(q, k, v)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        _ = ft.attention_prefill(q, k, v, causal=False)   # eager work between
