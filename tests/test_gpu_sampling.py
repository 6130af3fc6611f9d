"""GPU parity for the post-logits step: argmax / argmax_batched (bit-exact
against the oracle), sample_topp / decode_step (single and batched) against
the CPU oracle (sample_topp_cpu / repetition_penalty_cpu restatement) and a
float64 restatement of the same rule.

The GPU sums masses exactly (fixed point) and the oracle in float32 in
sorted order, so a token may differ only where a threshold sits within
rounding of a prefix boundary: every mismatch must show a float64 margin
below 1e-4 of the total mass (the reference states the same limit for its
own GPU path, test_sample_topp.py:115-123)."""

import numpy as np
import pytest
import torch

import fusedtok_amd as ft
import oracle
from tests import refs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _agree(got, logits, p, temp, seed, pen_ids=None, pen=1.0):
    x = logits if pen_ids is None else oracle.repetition_penalty(logits, pen_ids, pen)
    want = oracle.sample_topp(x, p, temp, seed)
    if got == want:
        return True
    _, margin = refs.ref_topp(x, p, temp, seed)
    return margin < 1e-4


def test_argmax_and_batched_bit_exact():
    x = np.array([[1, 3, 3, 2], [5, 5, 1, 0], [-np.inf] * 4, [np.nan, 9, 1, 2],
                  [1, np.nan, 7, 7]], np.float32)
    got = ft.argmax_batched(t(x))
    assert got.dtype == torch.int64 and got.is_cuda
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.argmax_batched(x))
    rng = np.random.default_rng(0)
    for rows, n in [(1, 1), (3, 777), (64, 128256), (7, 5000)]:
        y = rng.integers(-50, 50, (rows, n)).astype(np.float32)   # ties everywhere
        np.testing.assert_array_equal(ft.argmax_batched(t(y)).cpu().numpy(),
                                      oracle.argmax_batched(y))
        assert ft.argmax(t(y[0])) == int(oracle.argmax_batched(y[:1])[0])
    assert ft.argmax([3.0, 1.0, 3.0]) == 0                      # host input, staged
    with pytest.raises(ValueError):
        ft.argmax(torch.zeros(0, device=DEV))
    with pytest.raises(TypeError):
        ft.argmax_batched(torch.zeros((2, 3), dtype=torch.float64, device=DEV))


@pytest.mark.parametrize("slices", [0, 1, 2, 3, 64])
def test_argmax_sliced_rows_bit_exact(slices, tuning):
    # rows split across workgroups (fewer rows than CUs), folded by one wave
    # per row: ties across slice boundaries, NaN at index 0, all-NaN and
    # all -inf rows, the maximum in the last token, misaligned rows (odd n)
    tuning("FT_ARG_SLICES", slices)
    rng = np.random.default_rng(slices + 7)
    n = 128256
    x = rng.integers(-1000, 1000, (8, n)).astype(np.float32)
    x[0, 20000] = x[0, 100000] = x[0, 127000] = 5000.0
    x[1, 0] = np.nan
    x[1, 9] = 7000.0
    x[2, :] = np.nan
    x[3, :] = -np.inf
    x[4, -1] = 9000.0
    x[5, ::3] = np.nan
    x[6, 64000:64004] = 3000.0
    x[7, :] = 0.0
    x[7, 1::2] = -0.0
    np.testing.assert_array_equal(ft.argmax_batched(t(x)).cpu().numpy(),
                                  oracle.argmax_batched(x))
    for rows, m in [(5, 40001), (1, 1_000_003), (3, 4097)]:
        y = rng.integers(-30, 30, (rows, m)).astype(np.float32)
        np.testing.assert_array_equal(ft.argmax_batched(t(y)).cpu().numpy(),
                                      oracle.argmax_batched(y))
        assert ft.argmax(t(y[-1])) == int(oracle.argmax_batched(y[-1:])[0])


@pytest.mark.parametrize("n,scale", [(100, 3.0), (2000, 2.0), (32000, 1.5), (128256, 2.0)])
@pytest.mark.parametrize("p,temp", [(0.9, 1.0), (0.5, 0.7), (1.0, 1.3), (0.95, 0.1)])
def test_sample_topp_matches_oracle(n, scale, p, temp):
    rng = np.random.default_rng(n + int(p * 100))
    logits = (rng.standard_normal(n) * scale).astype(np.float32)
    lt = t(logits)
    seeds = [0, 1, 7, 42, 12345, 2**40 + 9]
    for seed in seeds:
        tok = ft.sample_topp(lt, p, temperature=temp, seed=seed)
        assert 0 <= tok < n
        assert _agree(tok, logits, p, temp, seed), (n, p, temp, seed, tok)
    # batched rows are the single-row pipeline, one workgroup each
    rows = np.repeat(logits[None], len(seeds), 0)
    bt = ft.sample_topp_batched(t(rows), p, temperature=temp, seeds=seeds)
    assert bt.dtype == torch.int64 and not bt.is_cuda
    singles = [ft.sample_topp(lt, p, temperature=temp, seed=s) for s in seeds]
    assert bt.tolist() == singles


def test_sample_topp_known_answers_and_determinism():
    peak = np.array([10.0] + [0.0] * 49, np.float32)
    assert {ft.sample_topp(t(peak), 0.9, temperature=0.1, seed=s) for s in range(16)} == {0}
    assert len({ft.sample_topp(t(peak), 1.0, temperature=1e4, seed=s) for s in range(64)}) > 10
    # flat logits: token = ceil(u n) - 1 (index order, equal masses)
    flat = t(np.zeros(32, np.float32))
    for s in range(40):
        assert ft.sample_topp(flat, 1.0, seed=s) == max(0, int(np.ceil(refs.splitmix_uniform(s) * 32)) - 1)
    rng = np.random.default_rng(6)
    x = t((rng.standard_normal(1000) * 2).astype(np.float32))
    first = ft.sample_topp(x, 0.9, seed=9)
    assert all(ft.sample_topp(x, 0.9, seed=9) == first for _ in range(5))
    # host input is staged through the device
    assert ft.sample_topp(x.cpu().numpy(), 0.9, seed=9) == first


def test_sample_topp_large_flat_bin_radix_path():
    # 8192 equal logits fall in one distance bin (> the 4096-entry exact
    # sort): the radix passes over the exact key resolve the index order
    n = 8192
    flat = t(np.zeros(n, np.float32))
    for s in range(20):
        u = refs.splitmix_uniform(s)
        want = max(0, int(np.ceil(u * n)) - 1)
        got = ft.sample_topp(flat, 1.0, seed=s)
        assert got == want or abs(u * n - round(u * n)) < 1e-3
    # near-flat: two values interleaved, p cuts inside the top group
    rng = np.random.default_rng(1)
    x = np.where(rng.random(20000) < 0.5, 0.0, 0.001).astype(np.float32)
    for s in range(10):
        assert _agree(ft.sample_topp(t(x), 0.3, seed=s), x, 0.3, 1.0, s)


@pytest.mark.parametrize("pen", [1.0, 1.3, 0.7, 100.0])
def test_decode_step_matches_oracle(pen):
    rng = np.random.default_rng(37)
    n = 3000
    logits = (rng.standard_normal(n) * 2).astype(np.float32)
    ids = rng.integers(0, n, size=50)
    for seed in (0, 11, 99):
        tok = ft.decode_step(t(logits), t(ids), pen, p=0.9, temperature=0.7, seed=seed)
        assert _agree(tok, logits, 0.9, 0.7, seed, ids, pen), (pen, seed, tok)
        # host ids are range-checked and give the same token
        assert ft.decode_step(t(logits), ids.tolist(), pen, p=0.9, temperature=0.7,
                              seed=seed) == tok


def test_decode_step_batched_matches_rows_and_oracle():
    rng = np.random.default_rng(41)
    rows, n = 16, 32000
    logits = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
    hist = [rng.integers(0, n, size=int(rng.integers(0, 60))).tolist() for _ in range(rows)]
    seeds = list(range(100, 100 + rows))
    got = ft.decode_step_batched(t(logits), hist, 1.25, p=0.9, temperature=0.8, seeds=seeds)
    assert got.shape == (rows,) and got.dtype == torch.int64
    for r in range(rows):
        assert _agree(int(got[r]), logits[r], 0.9, 0.8, seeds[r], np.array(hist[r], np.int64),
                      1.25), r
        assert int(got[r]) == ft.decode_step(t(logits[r]), hist[r], 1.25, p=0.9,
                                             temperature=0.8, seed=seeds[r])
    # flat ids + offsets and device output give the same tokens
    flat = np.concatenate([np.array(h, np.int64) for h in hist])
    offs = np.cumsum([0] + [len(h) for h in hist])
    dev = ft.decode_step_batched(t(logits), flat, 1.25, p=0.9, temperature=0.8, seeds=seeds,
                                 ids_offsets=offs, device_out=True)
    assert dev.is_cuda and dev.cpu().tolist() == got.tolist()


def test_decode_step_device_ids_out_of_range_are_dropped():
    # device ids are trusted (no sync); entries outside [0, n) are dropped
    rng = np.random.default_rng(38)
    logits = (rng.standard_normal(3000) * 2).astype(np.float32)
    good = rng.integers(0, 3000, size=50).tolist()
    bad = [3000, -7, 2**31 - 1]
    a = ft.decode_step(t(logits), t(np.array(good + bad, np.int64)), 1.5, p=0.9, seed=4)
    b = ft.decode_step(t(logits), t(np.array(good, np.int64)), 1.5, p=0.9, seed=4)
    assert a == b
    with pytest.raises(ValueError):                       # host ids are checked
        ft.decode_step(t(logits), good + bad, 1.5, p=0.9, seed=4)


def test_sampling_contract():
    x = t(np.ones(4, np.float32))
    for kw in [dict(p=0.0), dict(p=1.5), dict(p=0.9, temperature=0.0)]:
        pp = kw.pop("p")
        with pytest.raises(ValueError):
            ft.sample_topp(x, pp, **kw)
    with pytest.raises(ValueError):
        ft.sample_topp(t(np.ones((2, 2), np.float32)), 0.9)
    with pytest.raises(ValueError):
        ft.decode_step(x, [1], 0.0)
    with pytest.raises(TypeError):
        ft.sample_topp(torch.ones(4, dtype=torch.float64, device=DEV), 0.9)
    with pytest.raises(ValueError):
        ft.sample_topp_batched(t(np.ones((3, 4), np.float32)), 0.9, seeds=[1, 2])
    assert ft.sample_topp_batched(t(np.ones((0, 4), np.float32)), 0.9).numel() == 0


@pytest.mark.parametrize("rows,n", [(1, 128256), (3, 50000), (16, 32000), (64, 128256),
                                    (2, 16417), (5, 20000)])
def test_sliced_pipeline_matches_single_workgroup(rows, n, tuning):
    # Fewer rows than CUs: each row is split over several workgroups (slice
    # maxima, slice histograms, a per-row plan, a gather of the bins the two
    # queries can cross, the exact select). Masses are integers, so the
    # tokens equal those of the one-workgroup-per-row kernel (FT_SMP_SINGLE)
    # bit for bit, including rows that fall back to full scans.
    rng = np.random.default_rng(rows * 1000 + n)
    logits = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
    if rows >= 3:
        logits[1] = 0.0                               # flat: the plan overflows
        logits[2, :] = -np.inf                        # no finite value
    if rows >= 5:
        logits[3, rng.integers(0, n, 50)] = np.nan    # NaNs count as mass 0
        logits[4, :] = -30.0
        logits[4, n // 3] = 5.0                       # one dominant token
    seeds = list(range(11, 11 + rows))
    hist = [rng.integers(0, n, size=int(rng.integers(0, 80))).tolist() for _ in range(rows)]
    lt = t(logits)
    for p, temp in [(0.9, 0.8), (0.5, 1.3), (1.0, 1.0), (0.05, 0.3)]:
        got = {}
        for mode in (0, 1):
            tuning("FT_SMP_SINGLE", mode)
            got[mode] = (ft.decode_step_batched(lt, hist, 1.3, p=p, temperature=temp,
                                                seeds=seeds).tolist(),
                         ft.sample_topp_batched(lt, p, temperature=temp, seeds=seeds).tolist(),
                         ft.sample_topp(lt[0], p, temperature=temp, seed=seeds[0]))
        assert got[0] == got[1], (p, temp)


@pytest.mark.parametrize("slices", [2, 3, 12, 64])
def test_sliced_pipeline_any_slice_count(slices, tuning):
    # forced slice counts (FT_SMP_SLICES): odd splits, slices of a few
    # hundred tokens, the maximum count; same tokens as one workgroup per row
    rng = np.random.default_rng(slices + 90)
    rows, n = 6, 40001
    logits = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
    logits[1] = 0.0
    logits[2, rng.integers(0, n, 30)] = np.nan
    logits[3, :] = -20.0
    logits[3, n - 1] = 4.0
    seeds = list(range(3, 3 + rows))
    hist = [rng.integers(0, n, size=int(rng.integers(0, 40))).tolist() for _ in range(rows)]
    lt = t(logits)
    for p, temp in [(0.9, 0.8), (0.3, 1.2)]:
        tuning("FT_SMP_SLICES", slices)
        a = ft.decode_step_batched(lt, hist, 1.2, p=p, temperature=temp, seeds=seeds).tolist()
        tuning("FT_SMP_SINGLE", 1)
        b = ft.decode_step_batched(lt, hist, 1.2, p=p, temperature=temp, seeds=seeds).tolist()
        tuning.clear("FT_SMP_SINGLE")
        assert a == b, (p, temp)


def test_staged_vectors_read_in_place_or_through_a_copy(monkeypatch):
    # The batched samplers' histories, offsets and seeds are staged in
    # pinned host memory and read in place through its device address; where
    # the runtime reports none, one copy takes them up. Both give the same
    # tokens, call after call (the ring's slots are reused after their
    # events).
    from fusedtok_amd import _sampling_args as sargs
    lib = ft._fusedtok
    pinned = torch.empty(64, dtype=torch.int64, pin_memory=True)
    addr = lib.host_device_address(pinned.data_ptr())
    assert addr != 0
    assert lib.host_device_address(pinned.data_ptr() + 8) == addr + 8
    assert lib.host_device_address(torch.empty(8, device=DEV).data_ptr()) == 0
    pageable = np.zeros(64, np.int64)
    assert lib.host_device_address(pageable.ctypes.data) == 0

    rng = np.random.default_rng(77)
    rows, n = 12, 50000
    logits = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
    lt = t(logits)
    seeds = list(range(40, 40 + rows))
    hist = [rng.integers(0, n, size=int(rng.integers(0, 50))).tolist() for _ in range(rows)]
    first = ft.decode_step_batched(lt, hist, 1.2, p=0.9, temperature=0.8, seeds=seeds).tolist()
    first_s = ft.sample_topp_batched(lt, 0.9, temperature=0.8, seeds=seeds).tolist()
    for _ in range(9):  # more calls than ring slots
        assert ft.decode_step_batched(lt, hist, 1.2, p=0.9, temperature=0.8,
                                      seeds=seeds, device_out=True).tolist() == first
    for r in range(rows):
        assert _agree(first[r], logits[r], 0.9, 0.8, seeds[r], np.array(hist[r], np.int64), 1.2)
    monkeypatch.setattr(sargs, "_RING", sargs._PinnedRing())
    monkeypatch.setattr(lib, "host_device_address", lambda ptr: 0)
    for _ in range(6):
        assert ft.decode_step_batched(lt, hist, 1.2, p=0.9, temperature=0.8,
                                      seeds=seeds).tolist() == first
        assert ft.sample_topp_batched(lt, 0.9, temperature=0.8, seeds=seeds).tolist() == first_s


def test_staged_vectors_change_every_call_with_no_sync(monkeypatch):
    # Twelve calls queued back to back with device_out=True (no host sync),
    # alternating decode_step_batched and sample_topp_batched (whose ring
    # slots hold different layouts), each with its own seeds, histories and
    # (p, T): a slot read stale, or refilled before the work that read it
    # completed, would give another call's tokens. Every call is compared
    # with the same call through the upload path afterwards. Two of the
    # calls carry histories long enough (> IN_PLACE_MAX ids) to be uploaded.
    from fusedtok_amd import _sampling_args as sargs
    lib = ft._fusedtok
    rng = np.random.default_rng(78)
    rows, n = 12, 50000
    lt = t((rng.standard_normal((rows, n)) * 2).astype(np.float32))
    calls = []
    for i in range(12):
        seeds = [int(x) for x in rng.integers(0, 2 ** 40, rows)]
        top = 2000 if i in (4, 9) else 60
        hist = [rng.integers(0, n, size=int(rng.integers(0, top))).tolist() for _ in range(rows)]
        pt = [(0.9, 0.8), (0.5, 1.1), (0.95, 0.6)][i % 3]
        calls.append((i % 2, seeds, hist, pt))
    assert sum(len(h) for h in calls[4][2]) > sargs.IN_PLACE_MAX

    def run(call, device_out):
        kind, seeds, hist, (p, temp) = call
        if kind == 0:
            return ft.decode_step_batched(lt, hist, 1.3, p=p, temperature=temp, seeds=seeds,
                                          device_out=device_out)
        return ft.sample_topp_batched(lt, p, temperature=temp, seeds=seeds,
                                      device_out=device_out)
    outs = [run(c, True) for c in calls]
    torch.cuda.synchronize()
    got = [o.tolist() for o in outs]
    assert len({tuple(g) for g in got}) == len(got)  # the calls really differ
    monkeypatch.setattr(sargs, "_RING", sargs._PinnedRing())
    monkeypatch.setattr(lib, "host_device_address", lambda ptr: 0)
    for i, c in enumerate(calls):
        assert run(c, False).tolist() == got[i], f"call {i}"
