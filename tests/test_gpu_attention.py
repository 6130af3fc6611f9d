"""GPU parity: flash-decoding attention (contiguous and paged) through the
public API and its _launch entry points, against the CPU oracle on the same
seeded inputs.

Tolerances:
  f32 storage        rtol 1e-4 / atol 1e-5 (reference test_attention.py:71-79)
  bf16 / fp16        |err| <= 2e-3 + 1e-2 * |ref| against the oracle run on the
                     half-rounded inputs (the float32 reference of what the
                     kernel sees; BASELINE.json north_star tolerance)
Both kernels are covered: the MFMA kernel (bf16/fp16, D == 128, G <= 16)
and the generic one (everything else; forced with FT_ATTN_FORCE_GENERIC).
"""

import os

import numpy as np
import pytest
import torch

import fusedtok_amd as ft
import oracle
from tests import refs

pytestmark = pytest.mark.gpu

DEV = "cuda"
HALF = [torch.bfloat16, torch.float16]


def t(a, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return x if dtype is None else x.to(dtype)


def rounded(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dtype).float().numpy()


def assert_half_close(got, ref, what=""):
    err = np.abs(got - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert err.max(initial=-1) <= 0, (
        f"{what}: max |err| {np.abs(got - ref).max():.3e} exceeds 2e-3 + 1e-2|ref|")


def make_case(rng, b, hq, hkv, t_, d, with_lens):
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    k = rng.standard_normal((b, hkv, t_, d)).astype(np.float32)
    v = rng.standard_normal((b, hkv, t_, d)).astype(np.float32)
    lens = rng.integers(0, t_ + 1, size=b).astype(np.int32) if with_lens else None
    return q, k, v, lens


SHAPES = [  # reference test_attention.py:57-67
    (1, 8, 2, 1, 64, False),
    (1, 32, 8, 517, 128, False),
    (1, 32, 32, 100, 64, False),
    (3, 12, 4, 64, 32, True),
    (2, 6, 3, 33, 8, True),
    (1, 4, 1, 16, 4, True),
    (1, 8, 8, 0, 64, False),
    (2, 4, 4, 0, 32, True),
    (1, 2, 2, 4096, 256, False),
    (1, 2, 2, 300, 512, True),
]


@pytest.mark.parametrize("b,hq,hkv,tt,d,with_lens", SHAPES)
def test_decode_f32_matches_oracle(b, hq, hkv, tt, d, with_lens):
    rng = np.random.default_rng(b * 1000 + hq * 31 + hkv * 7 + tt + d)
    q, k, v, lens = make_case(rng, b, hq, hkv, tt, d, with_lens)
    y = ft.attention_decode(t(q), t(k), t(v), None if lens is None else t(lens))
    torch.cuda.synchronize()
    assert y.shape == (b, hq, d) and y.dtype == torch.float32
    np.testing.assert_allclose(y.cpu().numpy(), oracle.attention_decode(q, k, v, lens),
                               rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("dt", HALF)
@pytest.mark.parametrize("group", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("tt", [2048, 5000])
def test_decode_half_every_group(dt, group, tt):
    rng = np.random.default_rng(group * 977 + tt)
    hkv, d = 2, 128
    q, k, v, _ = make_case(rng, 1, hkv * group, hkv, tt, d, False)
    y = ft.attention_decode(t(q, dt), t(k, dt), t(v, dt))
    torch.cuda.synchronize()
    assert y.dtype == dt
    ref = oracle.attention_decode(rounded(q, dt), rounded(k, dt), rounded(v, dt))
    assert_half_close(y.float().cpu().numpy(), ref, f"{dt} G={group} T={tt}")


@pytest.mark.parametrize("group", [1, 2, 4, 8, 16])
def test_decode_f32_split_every_group(group):
    rng = np.random.default_rng(group * 31 + 7)
    hkv, d, tt = 2, 128, 3000
    q, k, v, _ = make_case(rng, 1, hkv * group, hkv, tt, d, False)
    lens = np.array([2711], np.int32)
    y = ft.attention_decode(t(q), t(k), t(v), t(lens))
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), oracle.attention_decode(q, k, v, lens),
                               rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("dt", HALF)
def test_generic_kernel_on_half_storage(dt, tuning):
    tuning("FT_ATTN_FORCE_GENERIC", 1)
    rng = np.random.default_rng(5)
    q, k, v, lens = make_case(rng, 3, 16, 4, 700, 128, True)
    y = ft.attention_decode(t(q, dt), t(k, dt), t(v, dt), t(lens))
    torch.cuda.synchronize()
    ref = oracle.attention_decode(rounded(q, dt), rounded(k, dt), rounded(v, dt), lens)
    assert_half_close(y.float().cpu().numpy(), ref, "generic")


@pytest.mark.parametrize("dt", HALF)
@pytest.mark.parametrize("first_len", [0, 1, 31, 32, 33, 127, 128, 129, 1000])
def test_decode_lens_across_chunk_and_step_boundaries(dt, first_len):
    rng = np.random.default_rng(4000 + first_len)
    q, k, v, _ = make_case(rng, 2, 32, 8, 1100, 128, False)
    lens = np.array([first_len, 1100], np.int32)
    y = ft.attention_decode(t(q, dt), t(k, dt), t(v, dt), t(lens))
    torch.cuda.synchronize()
    ref = oracle.attention_decode(rounded(q, dt), rounded(k, dt), rounded(v, dt), lens)
    got = y.float().cpu().numpy()
    assert_half_close(got, ref)
    if first_len == 0:
        assert (got[0] == 0).all()


@pytest.mark.parametrize("dt", [torch.float32] + HALF)
def test_decode_gqa_constant_v_and_poisoned_padding(dt):
    # reference test_attention.py:591-629
    b, hq, hkv, tt, d = 2, 8, 2, 300, 128
    gen = torch.Generator(device="cpu").manual_seed(3)
    q = torch.randn(b, hq, d, generator=gen).to(DEV, dt)
    k = torch.randn(b, hkv, tt, d, generator=gen).to(DEV, dt)
    v0 = torch.randn(hkv, d, generator=gen).to(DEV, dt)
    v = v0[None, :, None, :].expand(b, hkv, tt, d).contiguous()
    lens = torch.tensor([300, 100], dtype=torch.int32, device=DEV)
    k[1, :, 100:] = 30000.0           # poison the padding of row 1
    v[1, :, 100:] = 30000.0
    out = ft.attention_decode(q, k, v, lens)
    torch.cuda.synchronize()
    for bi in range(b):
        for h in range(hq):
            np.testing.assert_allclose(out[bi, h].float().cpu().numpy(),
                                       v0[h // 4].float().cpu().numpy(),
                                       rtol=1e-2, atol=2e-3)
    lens0 = torch.tensor([0, 100], dtype=torch.int32, device=DEV)
    out0 = ft.attention_decode(q, k, v, lens0)
    torch.cuda.synchronize()
    assert (out0[0].float() == 0).all()


def test_decode_repeatable():
    rng = np.random.default_rng(22)
    q, k, v, lens = make_case(rng, 2, 8, 2, 900, 128, True)
    args = [t(q, torch.bfloat16), t(k, torch.bfloat16), t(v, torch.bfloat16), t(lens)]
    first = ft.attention_decode(*args)
    for _ in range(3):
        assert torch.equal(ft.attention_decode(*args), first)


def test_decode_staged_host_inputs():
    rng = np.random.default_rng(31)
    q, k, v, lens = make_case(rng, 3, 16, 4, 333, 128, True)
    y = ft.attention_decode(q, k, v, lens, cuda=True)
    assert isinstance(y, np.ndarray) and y.dtype == np.float32
    np.testing.assert_allclose(y, refs.ref_decode(q, k, v, lens), rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------
# paged
# ---------------------------------------------------------------------------


def paged_case(rng, b, hq, hkv, d, lens, page=16, extra_pages=3, perm=True):
    width = max(1, max((l + page - 1) // page for l in lens))
    nb = b * width + extra_pages
    kp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    vp = rng.standard_normal((nb, hkv, page, d)).astype(np.float32)
    if perm:
        tbl = rng.permutation(nb)[: b * width].reshape(b, width).astype(np.int32)
    else:
        tbl = rng.integers(0, nb, (b, width)).astype(np.int32)
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    return q, kp, vp, tbl, np.asarray(lens, np.int32)


@pytest.mark.parametrize("dt", [torch.float32] + HALF)
@pytest.mark.parametrize("group", [1, 2, 4, 8, 16])
def test_paged_matches_oracle(dt, group):
    rng = np.random.default_rng(100 + group)
    hkv, d = 2, 128
    lens = [1, 16, 37, 300, 1024, 2049, 0, 33]
    q, kp, vp, tbl, ln = paged_case(rng, len(lens), hkv * group, hkv, d, lens,
                                    perm=False)
    out = ft.attention_decode_paged(t(q, dt), t(kp, dt), t(vp, dt), t(tbl), t(ln))
    torch.cuda.synchronize()
    if dt is torch.float32:
        ref = oracle.attention_decode_paged(q, kp, vp, tbl, ln)
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-4, atol=1e-5)
    else:
        ref = oracle.attention_decode_paged(rounded(q, dt), rounded(kp, dt),
                                            rounded(vp, dt), tbl, ln)
        assert_half_close(out.float().cpu().numpy(), ref, f"paged {dt} G={group}")
    assert (out[6].float() == 0).all()


@pytest.mark.parametrize("page", [1, 5, 16, 32])
def test_paged_odd_page_sizes(page):
    rng = np.random.default_rng(page)
    q, kp, vp, tbl, ln = paged_case(rng, 3, 8, 2, 128, [40, 77, 3], page=page)
    dt = torch.bfloat16
    out = ft.attention_decode_paged(t(q, dt), t(kp, dt), t(vp, dt), t(tbl), t(ln))
    torch.cuda.synchronize()
    ref = oracle.attention_decode_paged(rounded(q, dt), rounded(kp, dt), rounded(vp, dt),
                                        tbl, ln)
    assert_half_close(out.float().cpu().numpy(), ref, f"page={page}")


@pytest.mark.parametrize("dt", HALF)
def test_stream_lds_staging_matches_oracle_and_repeats(dt):
    # The MFMA kernel reads K / V as whole rows per load (128-byte lines) and
    # moves them through a per-wave LDS staging into the MFMA layout, lanes
    # reading what other lanes wrote. Three layouts (contiguous, paged with a
    # power-of-two page, paged with page 5) against the oracle; a second call
    # must reproduce every output bit for bit.
    rng = np.random.default_rng(77)
    q, k, v, _ = make_case(rng, 3, 32, 8, 700, 128, False)
    lens = np.array([700, 33, 451], np.int32)
    pq, kp, vp, tbl, ln = paged_case(rng, 4, 16, 4, 128, [1, 300, 77, 1024])
    oq, okp, ovp, otbl, oln = paged_case(rng, 3, 8, 2, 128, [40, 77, 3], page=5)
    outs = []
    for _ in range(2):
        outs.append((
            ft.attention_decode(t(q, dt), t(k, dt), t(v, dt), t(lens)),
            ft.attention_decode_paged(t(pq, dt), t(kp, dt), t(vp, dt), t(tbl), t(ln)),
            ft.attention_decode_paged(t(oq, dt), t(okp, dt), t(ovp, dt), t(otbl), t(oln))))
    torch.cuda.synchronize()
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
    assert_half_close(outs[0][0].float().cpu().numpy(),
                      oracle.attention_decode(rounded(q, dt), rounded(k, dt), rounded(v, dt),
                                              lens), "contiguous")
    assert_half_close(outs[0][1].float().cpu().numpy(),
                      oracle.attention_decode_paged(rounded(pq, dt), rounded(kp, dt),
                                                    rounded(vp, dt), tbl, ln), "paged")
    assert_half_close(outs[0][2].float().cpu().numpy(),
                      oracle.attention_decode_paged(rounded(oq, dt), rounded(okp, dt),
                                                    rounded(ovp, dt), otbl, oln), "page 5")


@pytest.mark.parametrize("dt", [torch.float32] + HALF)
@pytest.mark.parametrize("group,page", [(1, 16), (4, 16), (8, 5), (16, 16)])
@pytest.mark.parametrize("min_seg", [32, 512])
def test_paged_append_decode_equals_the_two_ops(dt, group, page, min_seg, tuning):
    # attention_decode_paged_append == kv_append_paged, then
    # attention_decode_paged(lens + 1): the pools bit for bit; the output
    # within the attention tolerance (the fresh token is merged in float32
    # by the stream kernel; f32 storage runs the two ops: bit for bit),
    # also against the oracle on the appended pools. Rows: empty (the fresh
    # token alone), one token, page - 1, page, full (no room: nothing
    # appended), one short of full, negative (nothing appended, zeros),
    # longer ones; small segments split the rows into many pieces. Three
    # steps in a row, lens + 1 each time.
    tuning("FT_ATTN_MIN_SEG", min_seg)
    rng = np.random.default_rng(group * 100 + page + min_seg + (0 if dt is torch.float32 else
                                                                7 if dt is torch.float16 else 11))
    hkv, d = 2, 128
    hq = hkv * group
    lens0 = [0, 1, page - 1, page, 0, 0, -1, 37, 300, 1027]
    width = (1027 + 3 + page - 1) // page + 1
    cap = width * page
    lens0[4], lens0[5] = cap, cap - 1
    b = len(lens0)
    q, kp, vp, tbl, _ = paged_case(rng, b, hq, hkv, d, [cap] * b, page=page)
    kp1, vp1 = t(kp, dt), t(vp, dt)
    kp2, vp2 = kp1.clone(), vp1.clone()
    qt, tblt = t(q, dt), t(tbl)
    lens = np.array(lens0, np.int32)
    for step in range(3):
        kn = t(rng.standard_normal((b, hkv, d)).astype(np.float32), dt)
        vn = t(rng.standard_normal((b, hkv, d)).astype(np.float32), dt)
        lt = t(lens)
        out1 = ft.attention_decode_paged_append(qt, kp1, vp1, tblt, kn, vn, lt)
        ft.kv_append_paged(kp2, vp2, tblt, kn, vn, lt)
        out2 = ft.attention_decode_paged(qt, kp2, vp2, tblt, t(lens + 1))
        torch.cuda.synchronize()
        assert torch.equal(kp1, kp2) and torch.equal(vp1, vp2), f"step {step}: pools differ"
        assert torch.equal(t(lens), lt), "lens modified"
        if dt is torch.float32:
            assert torch.equal(out1, out2), f"step {step}"
        else:
            got = out1.float().cpu().numpy()
            assert_half_close(got, out2.float().cpu().numpy(), f"step {step} vs two ops")
            ref = oracle.attention_decode_paged(rounded(q, dt), kp1.float().cpu().numpy(),
                                                vp1.float().cpu().numpy(), tbl,
                                                np.clip(lens + 1, 0, cap).astype(np.int32))
            assert_half_close(got, ref, f"step {step} vs oracle")
            # the empty row: the fresh token's V exactly; the negative one: zeros
            if step == 0:
                assert torch.equal(out1[0].view(hkv, group, d),
                                   vn[0].unsqueeze(1).expand(hkv, group, d))
                assert (out1[6].float() == 0).all()
        lens = lens + 1


@pytest.mark.parametrize("dt", HALF)
def test_long_equal_rows_take_one_segment_per_cu(dt, tuning):
    # Rows of equal length >= 4096 run on one segment per CU instead of the
    # default two (the decode kernel halves its own grid and tells the
    # combine kernels the count); shorter or ragged rows keep two. The
    # default call must equal the call with FT_ATTN_SEGS forced to the count
    # the kernel picks, bit for bit, in every combine form (plain, with the
    # quantize fold, the appending step), and the oracle.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tuning("FT_ATTN_SEGS", 0)  # the library's own choice, whatever the environment sets
    rng = np.random.default_rng(4242)
    cases = [([5000] * 4, cus), ([4095] * 4, 2 * cus), ([5000, 4999, 5000, 5000], 2 * cus),
             ([9000] * 2, cus)]
    for lens, picked in cases:
        q, kp, vp, tbl, ln = paged_case(rng, len(lens), 32, 8, 128, lens)
        qd, kd, vd, td, lt = t(q, dt), t(kp, dt), t(vp, dt), t(tbl), t(ln)
        kn = t(rng.standard_normal((len(lens), 8, 128)).astype(np.float32), dt)
        vn = t(rng.standard_normal((len(lens), 8, 128)).astype(np.float32), dt)
        cap = tbl.shape[1] * 16
        ln_app = t(np.minimum(ln, cap - 1).astype(np.int32))

        def run():
            out = ft.attention_decode_paged(qd, kd, vd, td, lt)
            qout, codes, scale = ft.attention_decode_paged_quant(qd, kd, vd, td, lt,
                                                                  device_scale=True)
            ka, va = kd.clone(), vd.clone()
            app = ft.attention_decode_paged_append(qd, ka, va, td, kn, vn, ln_app)
            torch.cuda.synchronize()
            return out, qout, codes, scale, app, ka, va

        got = run()
        tuning("FT_ATTN_SEGS", picked)
        ref = run()
        tuning("FT_ATTN_SEGS", 0)
        for i, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), f"lens {lens[:2]}..: output {i} differs from {picked} segments"
        assert_half_close(got[0].float().cpu().numpy(),
                          oracle.attention_decode_paged(rounded(q, dt), rounded(kp, dt),
                                                        rounded(vp, dt), tbl, ln),
                          f"lens {lens[:2]}..")


def test_paged_equals_contiguous_materialisation():
    rng = np.random.default_rng(41)
    q, kp, vp, tbl, ln = paged_case(rng, 3, 8, 2, 64, [37, 16, 48])
    out_p = ft.attention_decode_paged(t(q), t(kp), t(vp), t(tbl), t(ln))
    kc, vc = refs.materialize_paged(kp, tbl), refs.materialize_paged(vp, tbl)
    out_c = ft.attention_decode(t(q), t(kc), t(vc), t(ln))
    torch.cuda.synchronize()
    np.testing.assert_allclose(out_p.cpu().numpy(), out_c.cpu().numpy(),
                               rtol=1e-5, atol=1e-6)


def test_paged_no_lens_uses_full_width_and_host_table():
    rng = np.random.default_rng(12)
    q, kp, vp, tbl, _ = paged_case(rng, 2, 4, 4, 128, [64, 64])
    out = ft.attention_decode_paged(t(q, torch.float16), t(kp, torch.float16),
                                    t(vp, torch.float16), tbl)  # host table
    torch.cuda.synchronize()
    dt = torch.float16
    ref = oracle.attention_decode_paged(rounded(q, dt), rounded(kp, dt), rounded(vp, dt),
                                        tbl)
    assert_half_close(out.float().cpu().numpy(), ref)


def test_paged_c3_shape_every_row():
    """BASELINE config 3 at full size (B=32, Hq=32, Hkv=8, D=128, P=16, bf16,
    lens ~ U[512, 32768], permuted page pool) with a kv_append of one token
    per row first; every row is checked against the oracle over its own
    pages (reference tests/test_attention_paged.py:62-94 check paged rows
    against the materialised cache the same way), and every appended K/V row
    sits at slot lens[b] bit for bit."""
    rng = np.random.default_rng(2026)
    b, hq, hkv, d, page = 32, 32, 8, 128, 16
    lens = rng.integers(512, 32769, size=b).astype(np.int32)
    width = int(((lens + 1 + page - 1) // page).max())
    pages = int(((lens + 1 + page - 1) // page).sum())
    nb = pages + 64
    bf = torch.bfloat16
    gen = torch.Generator(device=DEV).manual_seed(5)
    kp = torch.randn(nb, hkv, page, d, device=DEV, generator=gen).to(bf)
    vp = torch.randn(nb, hkv, page, d, device=DEV, generator=gen).to(bf)
    perm = rng.permutation(nb).astype(np.int32)
    tbl = np.zeros((b, width), np.int32)
    off = 0
    for bi in range(b):
        npg = (lens[bi] + 1 + page - 1) // page
        tbl[bi, :npg] = perm[off:off + npg]
        off += npg
    q = torch.randn(b, hq, d, device=DEV, generator=gen).to(bf)
    kn = torch.randn(b, hkv, d, device=DEV, generator=gen).to(bf)
    vn = torch.randn(b, hkv, d, device=DEV, generator=gen).to(bf)
    tbl_t, lens_t = t(tbl), t(lens)
    ft.kv_append_paged(kp, vp, tbl_t, kn, vn, lens_t)
    out = ft.attention_decode_paged(q, kp, vp, tbl_t, lens_t + 1)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    kn_h, vn_h = kn.cpu(), vn.cpu()
    for bi in range(b):
        npg = (lens[bi] + 1 + page - 1) // page
        blocks = tbl[bi, :npg]
        slot_pg, slot_in = int(tbl[bi, lens[bi] // page]), int(lens[bi] % page)
        assert torch.equal(kp[slot_pg, :, slot_in].cpu(), kn_h[bi]), f"C3 row {bi}: k append"
        assert torch.equal(vp[slot_pg, :, slot_in].cpu(), vn_h[bi]), f"C3 row {bi}: v append"
        kp_b = kp[torch.from_numpy(blocks).long().to(DEV)].float().cpu().numpy()
        vp_b = vp[torch.from_numpy(blocks).long().to(DEV)].float().cpu().numpy()
        sub_tbl = np.arange(npg, dtype=np.int32)[None, :]
        ref = oracle.attention_decode_paged(q[bi:bi + 1].float().cpu().numpy(), kp_b,
                                            vp_b, sub_tbl, lens[bi:bi + 1] + 1)
        assert_half_close(got[bi:bi + 1], ref, f"C3 row {bi} len {lens[bi] + 1}")


def test_paged_graph_capture_replay():
    """Warm up, capture kv_append_paged + paged decode into a HIP graph,
    mutate the inputs, replay several times with eager work in between; every
    replay must equal the eager result (reference test_attention_paged.py:
    232-267)."""
    rng = np.random.default_rng(77)
    dt = torch.bfloat16
    # the table covers lens + 1 rows: the appended token lands at lens[b]
    # (1200 fills page 75 exactly, so the append needs a 76th page)
    q, kp, vp, tbl, ln1 = paged_case(rng, 4, 32, 8, 128, [501, 901, 34, 1201])
    ln = ln1 - 1
    assert (ln < tbl.shape[1] * 16).all()
    qt, kpt, vpt, tblt, lnt = t(q, dt), t(kp, dt), t(vp, dt), t(tbl), t(ln)
    kn = t(rng.standard_normal((4, 8, 128)).astype(np.float32), dt)
    vn = t(rng.standard_normal((4, 8, 128)).astype(np.float32), dt)
    out = torch.empty_like(qt)

    def step():
        ft._fusedtok.kv_append_paged_launch_bf16(
            kn.data_ptr(), vn.data_ptr(), tblt.data_ptr(), lnt.data_ptr(),
            kpt.data_ptr(), vpt.data_ptr(), 4, 8, 128, 16, tbl.shape[1],
            torch.cuda.current_stream().cuda_stream)
        ft._fusedtok.attention_decode_paged_launch_bf16(
            qt.data_ptr(), kpt.data_ptr(), vpt.data_ptr(), tblt.data_ptr(),
            lnt.data_ptr(), out.data_ptr(), 4, 32, 8, 16, tbl.shape[1], 128,
            torch.cuda.current_stream().cuda_stream)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for it in range(3):
        qt.mul_(1.25)
        kn.mul_(-1.0)
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = ft.attention_decode_paged(qt, kpt, vpt, tblt, lnt)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay {it} differs from eager"


@pytest.mark.parametrize("layout", ["page5", "contiguous"])
def test_long_equal_rows_other_layouts(layout, tuning):
    # the segment choice in the other two row modes: paged with a page size
    # that is not a power of two, and the contiguous cache (without lens:
    # every row holds the cache's capacity). 8 x 8 rows of ~4200 tokens
    # exceed 512 segments of the 512-token minimum, so the two counts cut
    # the rows differently.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tuning("FT_ATTN_SEGS", 0)
    rng = np.random.default_rng(515)
    dt = torch.float16
    for lens, picked in [([4200] * 8, cus), ([4200, 4100] * 4, 2 * cus)]:
        if layout == "page5":
            q, kp, vp, tbl, ln = paged_case(rng, len(lens), 32, 8, 128, lens, page=5)
            args = (t(q, dt), t(kp, dt), t(vp, dt), t(tbl), t(ln))
            call = ft.attention_decode_paged
            ref_fn = lambda: oracle.attention_decode_paged(rounded(q, dt), rounded(kp, dt),
                                                           rounded(vp, dt), tbl, ln)
        else:
            q, k, v, _ = make_case(rng, len(lens), 32, 8, max(lens), 128, False)
            ln = np.asarray(lens, np.int32)
            use_lens = len(set(lens)) > 1  # equal rows: no lens, the capacity is the length
            args = (t(q, dt), t(k, dt), t(v, dt)) + ((t(ln),) if use_lens else ())
            call = ft.attention_decode
            ref_fn = lambda: oracle.attention_decode(rounded(q, dt), rounded(k, dt),
                                                     rounded(v, dt), ln if use_lens else None)
        got = call(*args)
        tuning("FT_ATTN_SEGS", picked)
        ref = call(*args)
        tuning("FT_ATTN_SEGS", 3 * cus - picked)  # the count not picked
        other = call(*args)
        tuning("FT_ATTN_SEGS", 0)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"{layout} lens {lens}: differs from {picked} segments"
        # the rows are cut differently under the other count: the float32
        # merges of 4 and 8 pieces round differently
        assert not torch.equal(got, other), f"{layout} lens {lens}: the count made no difference"
        assert_half_close(got.float().cpu().numpy(), ref_fn(), f"{layout} lens {lens}")


def test_graph_replay_follows_the_lengths_segment_choice():
    # The segment count for equal long rows is chosen on the device from the
    # lengths, so one captured graph must follow lens that change between
    # replays: equal (one segment per CU), ragged (two), equal again. Every
    # replay equals an eager call on the same lens, bit for bit, for the
    # plain and the quantizing decode.
    rng = np.random.default_rng(91)
    dt = torch.bfloat16
    q, kp, vp, tbl, _ = paged_case(rng, 4, 32, 8, 128, [5000] * 4)
    qt, kpt, vpt, tblt = t(q, dt), t(kp, dt), t(vp, dt), t(tbl)
    lnt = t(np.full(4, 5000, np.int32))
    out = torch.empty_like(qt)
    qout = torch.empty_like(qt)
    codes = torch.empty(qt.shape, dtype=torch.int8, device=DEV)
    scale = torch.empty(1, dtype=torch.float32, device=DEV)

    def step():
        s_ = torch.cuda.current_stream().cuda_stream
        ft._fusedtok.attention_decode_paged_launch_bf16(
            qt.data_ptr(), kpt.data_ptr(), vpt.data_ptr(), tblt.data_ptr(), lnt.data_ptr(),
            out.data_ptr(), 4, 32, 8, 16, tbl.shape[1], 128, s_)
        ft._fusedtok.attention_decode_paged_quant_launch(
            qt.data_ptr(), kpt.data_ptr(), vpt.data_ptr(), tblt.data_ptr(), lnt.data_ptr(),
            qout.data_ptr(), 1, codes.data_ptr(), scale.data_ptr(), 4, 32, 8, 16,
            tbl.shape[1], 128, s_)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for it, lens in enumerate([[5000] * 4, [5000, 4100, 5000, 1], [4096] * 4, [5000] * 4]):
        lnt.copy_(torch.tensor(lens, dtype=torch.int32))
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = (out.clone(), qout.clone(), codes.clone(), scale.clone())
        e_out = ft.attention_decode_paged(qt, kpt, vpt, tblt, lnt)
        e_q, e_codes, e_scale = ft.attention_decode_paged_quant(qt, kpt, vpt, tblt, lnt,
                                                               device_scale=True)
        torch.cuda.synchronize()
        assert torch.equal(got[0], e_out), f"replay {it} ({lens}): output"
        assert torch.equal(got[1], e_q) and torch.equal(got[2], e_codes), f"replay {it}: codes"
        assert torch.equal(got[3], e_scale.reshape(1)), f"replay {it}: scale"


def test_paged_staged_host_inputs():
    rng = np.random.default_rng(43)
    q, kp, vp, tbl, ln = paged_case(rng, 2, 2, 2, 128, [1, 16])
    out = ft.attention_decode_paged(q, kp, vp, tbl, ln, cuda=True)
    np.testing.assert_allclose(out, oracle.attention_decode_paged(q, kp, vp, tbl, ln),
                               rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(out[0, 0], vp[tbl[0, 0], 0, 0], atol=1e-6)
