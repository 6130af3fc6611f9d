#!/usr/bin/env python3
"""Benchmark of the decode hot path on one MI355X.

Headline workload: paged flash-decoding with GQA, bf16,
batch 32, 32 query heads, 8 KV heads, head_dim 128, page size 16, per-row
context lengths uniform in [512, 32768], block table a seeded random
permutation of a page pool four times larger than the pages in use. One
"step" is what a decode loop does per token: kv_append_paged of one new
token per row at position lens[b], then attention_decode_paged over
lens[b] + 1 tokens - one call of attention_decode_paged_append, whose
combine kernel folds the fresh token in and appends it to the pools.

  value     = algorithmic bytes per step / measured step time   (GB/s)
              bytes: K+V rows read (sum_b (lens_b+1) * Hkv * D * 2 * 2 B),
              q, out, the block-table entries of the pages in use, and the
              kv_append copy (read + write of the new K/V rows). This is the
              reference's counting (benchmarks/bench.py:480,496) plus the
              table and the append.
  roofline  = the step's kernels (attn_decode_stream in its appending form
              + attn_combine_stream, timed together with HIP events
              recorded on the stream they are launched on): step bytes /
              their time, against 8 TB/s.
  secondary = BASELINE config 5a: W8A8 GEMM M=4096 K=8192 N=28672, int8
              uniform in [-127, 127], per-channel scales, bf16 output;
              TOPS = 2*M*N*K / t (reference benchmarks/bench.py:451), against
              the 5.0 POP/s dense int8 MFMA peak.
  chains    = BASELINE config 2 (RMSNorm -> int8 quantize -> W8A8 GEMM,
              M in {1, 8, 16}, K=4096, N=11008, fp16 in/out) and config 4
              (one Llama-3-8B W8A8 decode layer at batch 64, context 8192;
              also per layer of a 4-layer DecodeStack),
              each replayed as a captured HIP graph (the launch sequence of
              a decode loop without per-call Python cost); weights are
              cycled over enough copies to exceed the 256 MB last-level
              cache, as a model's successive layers would.
  more      = BASELINE config 1 (contiguous fp16 decode, B=1 H=32 T=4096,
              eight caches cycled in one HIP graph so the 67 MB working set
              is not served by the last-level cache) and config 5b
              (long-context paged decode, B=8 Hq=64 Hkv=8, 131072 tokens per
              row), each as K+V+q+out bytes per call over its time; and
              the int8 storage ops dequantize_int8 / qadd_int8 over 2^28
              elements; and attention_prefill (bf16, 32 / 8 heads, D=128,
              S=4096, causal and bidirectional) in TFLOP/s against the
              2.5 PFLOP/s dense bf16 MFMA peak; and the post-logits step
              (decode_step_batched, argmax_batched) at 64 rows x 128256.
  cpu_baseline = the C++ restatement of the reference's single-threaded
              attention_decode_paged_cpu / kv_append_paged_cpu (oracle/),
              on a bounded sample of the same rows, one core.

`traffic` (HBM bytes per launch, from rocprofv3 FETCH_SIZE / WRITE_SIZE
counters scaled by a copy-kernel calibration) is read from
profiles/hbm_traffic.json when that file holds an entry for the kernel.
`roofline.copy_gbs` is a plain 1 GiB device copy measured in the same run
(read + write bytes per second), and `frac_of_copy` the attention rate
against it.

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 10]
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0

C3 = dict(batch=32, hq=32, hkv=8, dim=128, page=16, len_lo=512, len_hi=32768,
          pool_factor=4, seed=2026)
C5A = dict(m=4096, k=8192, n=28672, seed=5)
C2 = dict(ms=(1, 8, 16), k=4096, n=11008, seed=2, copies=8, reps=20)
C4 = dict(batch=64, ctx=8192, hidden=4096, hq=32, hkv=8, dim=128, inter=14336,
          page=16, eps=1e-5, theta=500000.0, layers=2, stack_depth=4, seed=4, reps=10)
C1 = dict(batch=1, hq=32, hkv=32, t=4096, dim=128, copies=8, seed=1, reps=20)
C5B = dict(batch=8, hq=64, hkv=8, ctx=131072, dim=128, page=16, seed=51)


# C5a launches timed (after 300 untimed ones): fixed, not scaled with
# --steps; the power manager settles the clock lower over longer runs, so
# the line also carries `sustained_ms`, the mean over C5A_SUSTAINED further
# back-to-back launches (~4 s)
C5A_LAUNCHES = 100
C5A_SUSTAINED = 6000


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    # 100 timed steps: the loop's fixed start and end cost (~0.1 ms) is then
    # ~0.25% of the timed region at config 3
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu", action="store_true",
                   help="skip the CPU baseline leg")
    p.add_argument("--no-gemm", action="store_true",
                   help="skip the secondary W8A8 GEMM measurement")
    p.add_argument("--no-chains", action="store_true",
                   help="skip the config 2 / config 4 chain measurements")
    p.add_argument("--only", choices=["decode", "gemm", "copy", "c1", "c2", "c4", "c5b",
                            "int8", "prefill", "sampling", "cpu"],
                   default=None,
                   help="run one workload only (profiling runs); 'copy' is "
                        "the HBM-counter calibration: a plain 1 GiB "
                        "device-to-device tensor copy")
    return p.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# config 3 workload
# ---------------------------------------------------------------------------
def make_c3(torch, np, dev):
    c = C3
    rng = np.random.default_rng(c["seed"])
    b, hq, hkv, d, page = c["batch"], c["hq"], c["hkv"], c["dim"], c["page"]
    lens = rng.integers(c["len_lo"], c["len_hi"] + 1, size=b).astype(np.int32)
    npg = (lens + 1 + page - 1) // page           # pages after the append
    width = int(npg.max())
    used = int(npg.sum())
    pool = used * c["pool_factor"]
    perm = rng.permutation(pool).astype(np.int32)
    table = np.zeros((b, width), np.int32)
    off = 0
    for i in range(b):
        table[i, :npg[i]] = perm[off:off + npg[i]]
        off += npg[i]
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    bf = torch.bfloat16
    kp = torch.empty((pool, hkv, page, d), dtype=bf, device=dev)
    vp = torch.empty((pool, hkv, page, d), dtype=bf, device=dev)
    for t in (kp, vp):  # N(0,1), generated in slabs to bound the f32 temp
        flat = t.view(pool, -1)
        for s in range(0, pool, 8192):
            e = min(pool, s + 8192)
            flat[s:e].copy_(torch.randn((e - s, flat.shape[1]), device=dev,
                                        generator=gen))
    q = torch.randn((b, hq, d), device=dev, generator=gen).to(bf)
    kn = torch.randn((b, hkv, d), device=dev, generator=gen).to(bf)
    vn = torch.randn((b, hkv, d), device=dev, generator=gen).to(bf)
    w = dict(lens=lens, table=table, kp=kp, vp=vp, q=q, kn=kn, vn=vn,
             lens_t=torch.from_numpy(lens).to(dev),
             lens1_t=torch.from_numpy(lens + 1).to(dev),
             table_t=torch.from_numpy(table).to(dev),
             pool_pages=pool, used_pages=used)
    tokens = int((lens + 1).sum())
    w["attn_bytes"] = (tokens * hkv * d * 2 * 2      # K + V rows
                       + 2 * b * hq * d * 2          # q + out
                       + used * 4 + b * 4)           # table entries + lens
    w["append_bytes"] = 2 * (2 * b * hkv * d * 2) + b * 4 + b * 4
    w["tokens"] = tokens
    return w


def c3_step(ft, w):
    # kv_append_paged(..., lens) + attention_decode_paged(..., lens + 1) in
    # one call: the combine kernel folds the fresh token in and appends it
    ft.attention_decode_paged_append(w["q"], w["kp"], w["vp"], w["table_t"], w["kn"],
                                     w["vn"], w["lens_t"])


def bench_c3(torch, np, ft, dev, steps, warmup):
    w = make_c3(torch, np, dev)
    torch.cuda.synchronize()
    for _ in range(warmup):
        c3_step(ft, w)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()   # the stream ft launches on
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record(stream)
        c3_step(ft, w)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    attn_ms = sum(a.elapsed_time(b) for a, b in ev) / steps
    return w, wall, attn_ms


# ---------------------------------------------------------------------------
# config 5a workload (secondary)
# ---------------------------------------------------------------------------
def bench_c5a(torch, ft, dev, steps, warmup, sustained=0):
    c = C5A
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    m, k, n = c["m"], c["k"], c["n"]
    a = torch.randint(-127, 128, (m, k), device=dev, generator=gen,
                      dtype=torch.int32).to(torch.int8)
    bq = torch.randint(-127, 128, (n, k), device=dev, generator=gen,
                       dtype=torch.int32).to(torch.int8)
    sb = (torch.rand((n,), device=dev, generator=gen) * 9e-3 + 1e-3).float()
    sa = 0.0123
    for _ in range(warmup):
        ft.qgemm_perchannel(a, sa, bq, sb, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        ft.qgemm_perchannel(a, sa, bq, sb, out_dtype=torch.bfloat16)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    ops = 2.0 * m * n * k
    tops = ops / (ms * 1e-3) / 1e12
    sustained_ms = None
    if sustained:
        # the same launches kept up for seconds: the clock the power manager
        # holds under sustained load
        e0.record(stream)
        for _ in range(sustained):
            ft.qgemm_perchannel(a, sa, bq, sb, out_dtype=torch.bfloat16)
        e1.record(stream)
        torch.cuda.synchronize()
        sustained_ms = round(e0.elapsed_time(e1) / sustained, 4)
    return dict(metric="W8A8 GEMM TOPS (BASELINE config 5a)", value=round(tops, 2),
                unit="TOPS", ms_per_launch=round(ms, 4), dtype="int8",
                sustained_ms=sustained_ms, sustained_launches=sustained or None,
                sustained_frac=(round(ops / (sustained_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4)
                                if sustained_ms else None),
                config={"workload": "qgemm_perchannel M=4096 K=8192 N=28672, bf16 out",
                        "seed": c["seed"]},
                roofline={"bound": "mfma", "achieved": round(tops, 2),
                          "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                          "frac": round(tops / INT8_PEAK_TOPS, 4),
                          "traffic": traffic_for("qgemm_c5a"),
                          "kernel": "qgemm_big_w16"})


# ---------------------------------------------------------------------------
# chains: config 2 and config 4, timed as HIP graph replays
# ---------------------------------------------------------------------------
def sustain(torch, fn, seconds):
    """Untimed back-to-back fn() launches for about `seconds`, so that the
    clock has settled where sustained work holds it before the timed calls
    (the first hundred-odd launches after idle run at a lower, still moving
    clock)."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()


def graph_time_us(torch, fn, per_graph, reps, warmup=2):
    """Capture `per_graph` calls of fn() into one HIP graph; replay it `reps`
    times; return microseconds per fn() call."""
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(per_graph):
            fn(i)
    sustain(torch, g.replay, 0.2)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * per_graph)
    del g
    return us


def bench_c2(torch, ft, dev):
    c = C2
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    k, n = c["k"], c["n"]
    ws = [torch.randint(-127, 128, (n, k), device=dev, generator=gen,
                        dtype=torch.int32).to(torch.int8) for _ in range(c["copies"])]
    sb = (torch.rand((n,), device=dev, generator=gen) * 9e-3 + 1e-3).float()
    wn = (torch.rand((k,), device=dev, generator=gen) + 0.5).float()
    out = []
    for m in c["ms"]:
        x = torch.randn((m, k), device=dev, generator=gen).to(torch.float16)

        def chain(i):
            # one launch for M = 1; rmsnorm_quant + the GEMM otherwise
            return ft.rmsnorm_qgemm(x, wn, ws[i % len(ws)], sb, eps=1e-5,
                                    out_dtype=torch.float16)[0]
        us = graph_time_us(torch, chain, 2 * len(ws), c["reps"])
        nbytes = n * k + n * 4 + k * 4 + m * k * (2 + 1) + m * n * 2
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append({"m": m, "us_per_chain": round(us, 2), "GB/s": round(gbs, 1),
                    "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
    del ws
    return {"metric": "fused RMSNorm -> quantize -> W8A8 GEMM (BASELINE config 2)",
            "unit": "us per chain", "dtype": "int8 GEMM, fp16 in/out",
            "config": {"workload": "rmsnorm_qgemm (rmsnorm_quant + qgemm_perchannel), "
                                   "K=4096 N=11008, per-channel scales, fp16 out",
                       "seed": c["seed"], "weight_copies": c["copies"]},
            "bytes": "W (N*K) + scales + x, q, y", "results": out}


def bench_c4(torch, np, ft, dev):
    c = C4
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    b, hq, hkv, d, hid, inter = c["batch"], c["hq"], c["hkv"], c["dim"], c["hidden"], c["inter"]
    page = c["page"]
    bf = torch.bfloat16

    def wq(rows, cols):
        return (torch.randint(-127, 128, (rows, cols), device=dev, generator=gen,
                              dtype=torch.int32).to(torch.int8),
                (torch.rand((rows,), device=dev, generator=gen) * 9e-3 + 1e-3).float())
    layers = []
    for _ in range(c["layers"]):
        layers.append(dict(wn1=(torch.rand((hid,), device=dev, generator=gen) + 0.5).float(),
                           wn2=(torch.rand((hid,), device=dev, generator=gen) + 0.5).float(),
                           qkv=wq((hq + 2 * hkv) * d, hid), o=wq(hid, hq * d),
                           gu=wq(2 * inter, hid), down=wq(hid, inter)))
    # paged KV: every row holds ctx tokens; the new token goes to slot ctx
    npg = (c["ctx"] + 1 + page - 1) // page
    pool = b * npg + 64
    rng = np.random.default_rng(c["seed"])
    table = torch.from_numpy(rng.permutation(pool)[: b * npg].reshape(b, npg)
                             .astype(np.int32)).to(dev)
    kp = torch.randn((pool, hkv, page, d), device=dev, generator=gen, dtype=bf)
    vp = torch.randn((pool, hkv, page, d), device=dev, generator=gen, dtype=bf)
    lens = torch.full((b,), c["ctx"], dtype=torch.int32, device=dev)
    x = torch.randn((b, hid), device=dev, generator=gen).to(bf)

    # the layer object runs the fused chain: rmsnorm_quant -> QKV GEMM with
    # RoPE + paged append -> decode attention + quantize -> o_proj GEMM with
    # residual RMSNorm + quantize -> gate/up GEMM -> swiglu_quant -> down
    objs = [ft.DecodeLayer(norm1=L["wn1"], norm2=L["wn2"], w_qkv=L["qkv"][0],
                           s_qkv=L["qkv"][1], w_o=L["o"][0], s_o=L["o"][1],
                           w_gu=L["gu"][0], s_gu=L["gu"][1], w_down=L["down"][0],
                           s_down=L["down"][1], q_heads=hq, kv_heads=hkv, page=page,
                           max_batch=b, dtype=bf, eps=c["eps"], theta=c["theta"], neox=True,
                           pos_offset=0)
            for L in layers]
    y = torch.empty_like(x)

    def layer(i):
        # position ctx = lens[b] + pos_offset 0; attention over lens + 1
        return objs[i % len(objs)].forward(x, kp, vp, table, lens, out=y)
    us = graph_time_us(torch, layer, 2 * len(layers), c["reps"])
    # the same layers chained as a model runs them: a DecodeStack of
    # stack_depth layers (the weight sets cycled), where each layer's first
    # RMSNorm folds the previous down GEMM's K-split partials
    chain = [objs[i % len(objs)] for i in range(c["stack_depth"])]
    stack = ft.DecodeStack(chain)
    kps, vps = [kp] * len(chain), [vp] * len(chain)

    def stacked(i):
        return stack.forward(x, kps, vps, table, lens, out=y)
    us_stack = graph_time_us(torch, stacked, 2, c["reps"]) / len(chain)
    stack.close()
    wbytes = sum(int(w[0].numel()) + 4 * int(w[1].numel())
                 for w in (layers[0]["qkv"], layers[0]["o"], layers[0]["gu"], layers[0]["down"]))
    kvbytes = b * (c["ctx"] + 1) * hkv * d * 2 * 2
    nbytes = wbytes + kvbytes
    gbs = nbytes / (us * 1e-6) / 1e9
    for o in objs:
        o.close()
    del kp, vp, layers, objs
    return {"metric": "Llama-3-8B W8A8 decode layer (BASELINE config 4)",
            "value": round(us, 2), "unit": "us per layer",
            "tokens_per_s": round(b / (us * 1e-6), 1),
            "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "stacked_us_per_layer": round(us_stack, 2),
            "stacked_frac_of_hbm_peak": round(nbytes / (us_stack * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "bytes_per_layer": nbytes, "dtype": "bf16 activations / KV, int8 GEMMs",
            "kernels_per_layer": 10, "kernels_per_chained_layer": 9,
            "config": {"workload": "DecodeLayer (Llama block with both residual adds): "
                                   "rmsnorm_quant -> QKV qgemm + RoPE "
                                   "(NeoX, position 8192) + paged append -> "
                                   "attention_decode_paged + quantize -> o_proj qgemm + "
                                   "rmsnorm_quant(+residual) -> gate/up qgemm + "
                                   "swiglu_quant -> down qgemm + residual",
                       "batch": b, "context": c["ctx"], "layers_cycled": c["layers"],
                       "stack_depth": c["stack_depth"],
                       "seed": c["seed"]}}


# ---------------------------------------------------------------------------
# config 1 (contiguous fp16 decode) and config 5b (long-context paged decode)
# ---------------------------------------------------------------------------
def bench_c1(torch, ft, dev):
    """Contiguous decode, fp16, B=1 H=32 D=128 T=4096: 67 MB per call, small
    enough for the 256 MB last-level cache, so `copies` caches are cycled
    (537 MB) inside one captured HIP graph."""
    c = C1
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    b, hq, hkv, t, d = c["batch"], c["hq"], c["hkv"], c["t"], c["dim"]
    f16 = torch.float16
    caches = [(torch.randn((b, hkv, t, d), device=dev, generator=gen).to(f16),
               torch.randn((b, hkv, t, d), device=dev, generator=gen).to(f16))
              for _ in range(c["copies"])]
    q = torch.randn((b, hq, d), device=dev, generator=gen).to(f16)

    def call(i):
        kc, vc = caches[i % len(caches)]
        return ft.attention_decode(q, kc, vc)
    us = graph_time_us(torch, call, 2 * len(caches), c["reps"])
    nbytes = 2 * b * hkv * t * d * 2 + 2 * b * hq * d * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    del caches
    return {"metric": "contiguous flash-decode KV GB/s (BASELINE config 1)",
            "value": round(gbs, 1), "unit": "GB/s", "us_per_call": round(us, 2),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_call": nbytes,
            "dtype": "fp16",
            "config": {"workload": "attention_decode fp16 B=1 Hq=Hkv=32 D=128 T=4096, "
                                   f"{c['copies']} caches cycled in one HIP graph",
                       "seed": c["seed"]}}


def bench_c5b(torch, np, ft, dev, steps):
    """Long-context paged decode, bf16, B=8 Hq=64 Hkv=8 D=128, 131072 tokens
    per row (4.3 GB of K/V per call), random page permutation."""
    c = C5B
    b, hq, hkv, d, page, ctx = c["batch"], c["hq"], c["hkv"], c["dim"], c["page"], c["ctx"]
    rng = np.random.default_rng(c["seed"])
    npg = ctx // page
    pool = b * npg + 64
    table = torch.from_numpy(rng.permutation(pool)[: b * npg].reshape(b, npg)
                             .astype(np.int32)).to(dev)
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    bf = torch.bfloat16
    kp = torch.empty((pool, hkv, page, d), dtype=bf, device=dev)
    vp = torch.empty((pool, hkv, page, d), dtype=bf, device=dev)
    for t in (kp, vp):
        flat = t.view(pool, -1)
        for s in range(0, pool, 8192):
            e = min(pool, s + 8192)
            flat[s:e].copy_(torch.randn((e - s, flat.shape[1]), device=dev, generator=gen))
    q = torch.randn((b, hq, d), device=dev, generator=gen).to(bf)
    lens = torch.full((b,), ctx, dtype=torch.int32, device=dev)
    for _ in range(3):
        ft.attention_decode_paged(q, kp, vp, table, lens)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        ft.attention_decode_paged(q, kp, vp, table, lens)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    nbytes = 2 * b * hkv * ctx * d * 2 + 2 * b * hq * d * 2 + b * npg * 4 + b * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    del kp, vp
    return {"metric": "long-context paged flash-decode KV GB/s (BASELINE config 5b)",
            "value": round(gbs, 1), "unit": "GB/s", "us_per_call": round(us, 2),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_call": nbytes,
            "dtype": "bf16",
            "config": {"workload": "attention_decode_paged bf16 B=8 Hq=64 Hkv=8 D=128 "
                                   "P=16, 131072 tokens per row", "seed": c["seed"],
                       "pool_pages": pool}}


# ---------------------------------------------------------------------------
# int8 storage neighbours: dequantize_int8 and qadd_int8 (HBM-bound)
# ---------------------------------------------------------------------------
INT8 = dict(n=1 << 28, seed=8, steps=10)


def bench_int8(torch, ft, dev):
    """dequantize (n int8 -> n float32) and qadd (two n-element int8 inputs,
    device scales, device out scale) over n = 2^28 elements. Algorithmic
    bytes: dequantize n + 4n; qadd 2n read per pass (absmax, then quantize)
    + n written = 5n."""
    c = INT8
    n = c["n"]
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    qa = torch.randint(-127, 128, (n,), device=dev, generator=gen,
                       dtype=torch.int32).to(torch.int8)
    qb = torch.randint(-127, 128, (n,), device=dev, generator=gen,
                       dtype=torch.int32).to(torch.int8)
    sa = torch.full((1,), 0.013, device=dev)
    sb = torch.full((1,), 0.021, device=dev)
    x = ft.dequantize_int8(qa, sa)          # allocate once, warm up
    ft.qadd_int8(qa, sa, qb, sb, device_scale=True)
    stream = torch.cuda.current_stream()
    res = {}
    for name, fn, nbytes in (
            ("dequantize_int8 (f32 out)", lambda: ft.dequantize_int8(qa, sa), 5 * n),
            ("qadd_int8 (device scales)",
             lambda: ft.qadd_int8(qa, sa, qb, sb, device_scale=True), 5 * n)):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(c["steps"]):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / c["steps"]
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = {"us_per_call": round(us, 1), "GB/s": round(gbs, 1),
                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                     "bytes_per_call": nbytes}
    del qa, qb, x
    return {"metric": "int8 storage ops GB/s", "unit": "GB/s", "dtype": "int8",
            "config": {"workload": f"n = 2^28 elements, seed {c['seed']}"},
            "results": res}


# ---------------------------------------------------------------------------
# prefill attention (the step before decode)
# ---------------------------------------------------------------------------
PREFILL = dict(batch=1, hq=32, hkv=8, seq=4096, dim=128, seed=12, steps=20)
BF16_PEAK_TFLOPS = 2500.0


def bench_prefill(torch, ft, dev):
    """attention_prefill, bf16, Llama-3-8B heads (32 q / 8 kv, D=128) over a
    4096-token prompt, causal and bidirectional. FLOPs: 4·S_eff·D per
    (query row, head) with S_eff the keys it attends to (QK^T and PV, 2
    flops per multiply-add): causal sum_i (i+1) = S(S+1)/2 keys per head."""
    c = PREFILL
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    b, hq, hkv, s, d = c["batch"], c["hq"], c["hkv"], c["seq"], c["dim"]
    bf = torch.bfloat16
    q = torch.randn((b, hq, s, d), device=dev, generator=gen).to(bf)
    k = torch.randn((b, hkv, s, d), device=dev, generator=gen).to(bf)
    v = torch.randn((b, hkv, s, d), device=dev, generator=gen).to(bf)
    stream = torch.cuda.current_stream()
    res = {}
    for causal in (True, False):
        sustain(torch, lambda: ft.attention_prefill(q, k, v, causal=causal), 0.3)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(c["steps"]):
            ft.attention_prefill(q, k, v, causal=causal)
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / c["steps"]
        keys = s * (s + 1) // 2 if causal else s * s
        flops = 4.0 * b * hq * keys * d
        tf = flops / (us * 1e-6) / 1e12
        res["causal" if causal else "bidirectional"] = {
            "us_per_call": round(us, 1), "TFLOP/s": round(tf, 1),
            "frac_of_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), "flops": flops}
    del q, k, v
    return {"metric": "prefill attention TFLOP/s", "unit": "TFLOP/s", "dtype": "bf16",
            "config": {"workload": "attention_prefill bf16 B=1 Hq=32 Hkv=8 S=4096 D=128",
                       "seed": c["seed"]},
            "roofline": {"bound": "mfma", "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "kernel": "attn_prefill_mfma<bf16, 128>"},
            "results": res}


# ---------------------------------------------------------------------------
# post-logits step: decode_step_batched and argmax_batched
# ---------------------------------------------------------------------------
SAMPLE = dict(rows=64, vocab=128256, hist=64, seed=13, steps=20)


def bench_sampling(torch, ft, dev):
    """The step after the LM head at config 4's batch: 64 rows of Llama-3's
    128256-entry vocabulary (float32 logits, N(0, 2^2)), repetition penalty
    over a 64-token history per row, temperature 0.8, nucleus p = 0.9, tokens
    left on the device; and greedy argmax_batched. Bytes: the logits read
    once (rows x vocab x 4)."""
    import numpy as np
    c = SAMPLE
    rows, n = c["rows"], c["vocab"]
    gen = torch.Generator(device=dev).manual_seed(c["seed"])
    logits = torch.randn((rows, n), device=dev, generator=gen) * 2.0
    rng = np.random.default_rng(c["seed"])
    hist = rng.integers(0, n, size=(rows, c["hist"]))
    stream = torch.cuda.current_stream()
    res = {}
    calls = {
        "decode_step_batched": lambda: ft.decode_step_batched(
            logits, hist, 1.2, p=0.9, temperature=0.8, device_out=True),
        "argmax_batched": lambda: ft.argmax_batched(logits),
    }
    for name, fn in calls.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(c["steps"]):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / c["steps"]
        gbs = rows * n * 4 / (us * 1e-6) / 1e9
        res[name] = {"us_per_call": round(us, 1), "GB/s": round(gbs, 1),
                     "us_per_row": round(us / rows, 3)}
    del logits
    return {"metric": "post-logits step, us per call", "unit": "us", "dtype": "f32",
            "config": {"workload": f"decode_step_batched / argmax_batched, {rows} rows x "
                                   f"{n} vocab, penalty 1.2 over {c['hist']} ids, T=0.8, "
                                   "p=0.9", "seed": c["seed"]},
            "results": res}


# ---------------------------------------------------------------------------
# CPU baselines, timed on this host after the GPU legs. The reference CPU
# path (its single-threaded *_cpu functions, unbuildable here) runs as the
# oracle's C++ restatement on ONE pinned core ("port"); a torch-CPU float32
# composite of the same math runs on every core the process may use.
# Bounded samples, stated in each entry; about 20-30 s of CPU work in all.
# ---------------------------------------------------------------------------
def host_facts():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0))}


class one_core:
    """Pin this process to one of its allowed cores for the block (the
    oracle is single-threaded; this keeps it from migrating)."""
    def __enter__(self):
        self.saved = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {min(self.saved)})

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.saved)


def timed(fn, reps=3):
    """Median wall time of `reps` runs of fn()."""
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline_c3(torch, np, w, budget_s=8.0):
    """Oracle on config 3 rows (kv_append_paged + attention_decode_paged),
    one core, rows taken in order until the budget is spent."""
    import oracle
    c = C3
    page, hkv, d = c["page"], c["hkv"], c["dim"]
    lens, table = w["lens"], w["table"]
    done_rows, done_bytes, spent = 0, 0, 0.0
    for i in range(len(lens)):
        npg = (int(lens[i]) + 1 + page - 1) // page
        blocks = torch.from_numpy(table[i, :npg].astype(np.int64)).to(w["kp"].device)
        # the row's pages as the oracle sees them (bf16 values widened to f32),
        # taken BEFORE the append so the CPU leg does the same work
        kp = w["kp"][blocks].float().cpu().numpy()
        vp = w["vp"][blocks].float().cpu().numpy()
        q = w["q"][i:i + 1].float().cpu().numpy()
        kn = w["kn"][i:i + 1].float().cpu().numpy()
        vn = w["vn"][i:i + 1].float().cpu().numpy()
        sub = np.arange(npg, dtype=np.int32)[None, :]
        ln = lens[i:i + 1].astype(np.int32)
        with one_core():
            t0 = time.perf_counter()
            oracle.kv_append_paged(kp, vp, sub, kn, vn, ln)
            oracle.attention_decode_paged(q, kp, vp, sub, ln + 1)
            spent += time.perf_counter() - t0
        done_rows += 1
        done_bytes += ((int(lens[i]) + 1) * hkv * d * 2 * 2 + 2 * c["hq"] * d * 2
                       + npg * 4 + 4 + 2 * 2 * hkv * d * 2)
        if spent >= budget_s:
            break
    gbs = done_bytes / spent / 1e9
    return {"config": "C3", "value": round(gbs, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{done_rows} of {len(lens)} config-3 rows "
                      f"(kv_append_paged + attention_decode_paged, "
                      f"{int(lens[:done_rows].sum()) + done_rows} tokens), "
                      f"oracle/oracle.cpp restatement of the reference *_cpu "
                      f"functions, g++ -O2, one pinned core, {spent:.2f} s; "
                      f"bytes counted as on the GPU (bf16 K/V)"}


def cpu_baselines_more(torch, np):
    """C1, C2 and C5a on the oracle (one core), and a torch-CPU f32
    composite of C1, C3-like rows and C5a on all allowed cores."""
    import oracle
    rng = np.random.default_rng(17)
    out = []
    # C1: contiguous decode, B=1, Hq=Hkv=32, T=4096 (fp16 bytes counted)
    c = C1
    q = rng.standard_normal((1, c["hq"], c["dim"])).astype(np.float32)
    k = rng.standard_normal((1, c["hkv"], c["t"], c["dim"])).astype(np.float32)
    v = rng.standard_normal((1, c["hkv"], c["t"], c["dim"])).astype(np.float32)
    c1_bytes = 2 * c["hkv"] * c["t"] * c["dim"] * 2 + 2 * c["hq"] * c["dim"] * 2
    with one_core():
        t = timed(lambda: oracle.attention_decode(q, k, v))
    out.append({"config": "C1", "value": round(c1_bytes / t / 1e9, 4), "unit": "GB/s",
                "cores": 1, "kind": "port", "sample": f"the whole call, median of 3: "
                f"{t * 1e3:.2f} ms (fp16 bytes counted)"})
    qt, kt, vt = (torch.from_numpy(a) for a in (q, k, v))

    def torch_attn():
        s = torch.matmul(kt[0], qt[0].unsqueeze(-1)).squeeze(-1) / c["dim"] ** 0.5
        return torch.matmul(torch.softmax(s, -1).unsqueeze(1), vt[0])
    t = timed(torch_attn)
    out.append({"config": "C1", "value": round(c1_bytes / t / 1e9, 4), "unit": "GB/s",
                "cores": torch.get_num_threads(), "kind": "torch-cpu",
                "sample": f"float32 softmax(qK^T/sqrt(D))V, whole call, median of 3: "
                          f"{t * 1e3:.2f} ms"})
    # C2: RMSNorm -> quantize -> W8A8 GEMM, N=11008, K=4096, per M
    c = C2
    wt = rng.integers(-127, 128, (c["n"], c["k"])).astype(np.int8)
    sb = rng.uniform(1e-3, 1e-2, c["n"]).astype(np.float32)
    wn = (rng.random(c["k"]) + 0.5).astype(np.float32)
    res = []
    for m in c["ms"]:
        x = rng.standard_normal((m, c["k"])).astype(np.float32)

        def chain():
            qx, sx = oracle.quantize_int8(oracle.rmsnorm(x, wn, eps=1e-5))
            return oracle.qgemm_perchannel(qx, sx, wt, sb)
        with one_core():
            t = timed(chain)
        res.append({"m": m, "us_per_chain": round(t * 1e6, 1)})
    out.append({"config": "C2", "value": res, "unit": "us per chain", "cores": 1,
                "kind": "port", "sample": "rmsnorm -> quantize_int8 -> qgemm_perchannel "
                "(oracle), each M, median of 3"})
    # C5a: 4096 x 8192 x 28672 on a 64-row subset, extrapolated linearly
    c = C5A
    rows = 64
    a = rng.integers(-127, 128, (rows, c["k"])).astype(np.int8)
    b = rng.integers(-127, 128, (c["n"], c["k"])).astype(np.int8)
    sb = rng.uniform(1e-3, 1e-2, c["n"]).astype(np.float32)
    with one_core():
        t0 = time.perf_counter()
        oracle.qgemm_perchannel(a, 0.01, b, sb)
        t = time.perf_counter() - t0
    full = t * c["m"] / rows
    out.append({"config": "C5a", "value": round(2.0 * c["m"] * c["n"] * c["k"] / full / 1e12, 5),
                "unit": "TOPS", "cores": 1, "kind": "port",
                "sample": f"{rows} of {c['m']} rows ({t:.2f} s), extrapolated linearly "
                          f"to {full:.0f} s for the whole GEMM"})
    af, bf_ = torch.from_numpy(a.astype(np.float32)), torch.from_numpy(b.astype(np.float32))
    t = timed(lambda: torch.matmul(af, bf_.t()))
    full = t * c["m"] / rows
    out.append({"config": "C5a", "value": round(2.0 * c["m"] * c["n"] * c["k"] / full / 1e12, 4),
                "unit": "TOPS", "cores": torch.get_num_threads(), "kind": "torch-cpu",
                "sample": f"float32 matmul of the int8 values (not bit-exact past 2^24), "
                          f"{rows} rows, median of 3 ({t * 1e3:.1f} ms), extrapolated to "
                          f"{c['m']} rows"})
    # C3-like rows on torch-CPU: 4 sequences of 8192 tokens, 32/8 heads
    b4, hq, hkv, d, tt = 4, C3["hq"], C3["hkv"], C3["dim"], 8192
    qq = torch.randn(b4, hkv, hq // hkv, d)
    kk = torch.randn(b4, hkv, tt, d)
    vv = torch.randn(b4, hkv, tt, d)

    def torch_gqa():
        s = torch.matmul(qq, kk.transpose(-1, -2)) / d ** 0.5
        return torch.matmul(torch.softmax(s, -1), vv)
    t = timed(torch_gqa)
    c3b = 2 * b4 * hkv * tt * d * 2 + 2 * b4 * hq * d * 2
    out.append({"config": "C3", "value": round(c3b / t / 1e9, 4), "unit": "GB/s",
                "cores": torch.get_num_threads(), "kind": "torch-cpu",
                "sample": f"float32 GQA decode over 4 rows of 8192 tokens (bf16 bytes "
                          f"counted), median of 3: {t * 1e3:.2f} ms"})
    return out


def traffic_for(key):
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def measured_copy_gbs(torch, dev):
    """Bandwidth of a plain 1 GiB device-to-device copy (torch's copy kernel),
    counted as bytes read + bytes written per second: the practical HBM
    figure the decode fractions are also quoted against."""
    src = torch.ones((1 << 29,), dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(10):
        dst.copy_(src)
    e1.record(stream)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / 10
    del src, dst
    torch.cuda.empty_cache()
    return 2 * (1 << 30) / sec / 1e9


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this "
              "build's decode path is single-GPU; run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import fusedtok_amd as ft
    if not ft.cuda_available():
        print("no HIP device visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    if args.only == "copy":
        src = torch.ones((1 << 29,), dtype=torch.bfloat16, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy: {args.warmup + args.steps} x 1 GiB read + 1 GiB written")
        return
    if args.only == "gemm":
        # the main run's C5a leg: ~0.25 s of warm-up launches, then timed
        log("gemm", json.dumps(bench_c5a(torch, ft, dev, C5A_LAUNCHES, max(300, args.warmup),
                                         C5A_SUSTAINED)))
        return
    if args.only == "c2":
        log("c2", json.dumps(bench_c2(torch, ft, dev)))
        return
    if args.only == "c4":
        log("c4", json.dumps(bench_c4(torch, np, ft, dev)))
        return
    if args.only == "c1":
        log("c1", json.dumps(bench_c1(torch, ft, dev)))
        return
    if args.only == "c5b":
        log("c5b", json.dumps(bench_c5b(torch, np, ft, dev, args.steps)))
        return
    if args.only == "int8":
        log("int8", json.dumps(bench_int8(torch, ft, dev)))
        return
    if args.only == "prefill":
        log("prefill", json.dumps(bench_prefill(torch, ft, dev)))
        return
    if args.only == "sampling":
        log("sampling", json.dumps(bench_sampling(torch, ft, dev)))
        return

    copy_gbs = measured_copy_gbs(torch, dev) if args.only is None else None
    if copy_gbs:
        log(f"device copy: {copy_gbs:.1f} GB/s (read + write)")
    log(f"config 3: building workload (seed {C3['seed']})")
    w, wall, attn_ms = bench_c3(torch, np, ft, dev, args.steps, args.warmup)
    step_bytes = w["attn_bytes"] + w["append_bytes"]
    ms_step = wall / args.steps * 1e3
    value = step_bytes / (wall / args.steps) / 1e9
    attn_gbs = step_bytes / (attn_ms * 1e-3) / 1e9
    log(f"config 3: {ms_step:.4f} ms/step, {value:.1f} GB/s; attention + append "
        f"{attn_ms * 1e3:.1f} us, {attn_gbs:.1f} GB/s")
    if args.only == "decode":
        return

    secondary = None
    if not args.no_gemm and args.only is None:
        del w["kp"], w["vp"]
        torch.cuda.empty_cache()
        # sustained rate: ~0.25 s of launches first, so the power manager
        # has settled at the board limit (measured: socket power 1400 W, the
        # clock falls from 2.4 GHz to ~1.8 GHz, with a deeper dip during the
        # first ~100 launches)
        secondary = bench_c5a(torch, ft, dev, C5A_LAUNCHES, 300, C5A_SUSTAINED)
        log(f"config 5a: {secondary['value']} TOPS ({secondary['ms_per_launch']} ms); "
            f"sustained over {C5A_SUSTAINED} launches: {secondary['sustained_ms']} ms")

    chains = None
    if not args.no_chains and args.only is None:
        torch.cuda.empty_cache()
        chains = [bench_c2(torch, ft, dev)]
        log("config 2:", json.dumps(chains[0]["results"]))
        torch.cuda.empty_cache()
        chains.append(bench_c4(torch, np, ft, dev))
        log(f"config 4: {chains[1]['value']} us per layer, "
            f"{chains[1]['stacked_us_per_layer']} us per layer chained in a DecodeStack")
        torch.cuda.empty_cache()

    decode_more = None
    if not args.no_chains and args.only is None:
        decode_more = [bench_c1(torch, ft, dev)]
        log(f"config 1: {decode_more[0]['value']} GB/s")
        torch.cuda.empty_cache()
        decode_more.append(bench_c5b(torch, np, ft, dev, max(5, args.steps // 2)))
        log(f"config 5b: {decode_more[1]['value']} GB/s")
        torch.cuda.empty_cache()
        decode_more.append(bench_int8(torch, ft, dev))
        log("int8 storage:", json.dumps(decode_more[2]["results"]))
        torch.cuda.empty_cache()
        decode_more.append(bench_prefill(torch, ft, dev))
        log("prefill:", json.dumps(decode_more[3]["results"]))
        torch.cuda.empty_cache()
        decode_more.append(bench_sampling(torch, ft, dev))
        log("sampling:", json.dumps(decode_more[4]["results"]))
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu and args.only in (None, "cpu"):
        w2 = make_c3(torch, np, dev)  # pools were released for the GEMM leg
        c3 = cpu_baseline_c3(torch, np, w2)
        del w2
        torch.cuda.empty_cache()
        log(f"cpu baseline: {c3['value']} GB/s over {c3['sample']}")
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        more = cpu_baselines_more(torch, np)
        for e in more:
            log(f"cpu {e['config']} {e['kind']}: {e['value']} {e['unit']} ({e['cores']} cores)")
        cpu = dict(c3)
        cpu.pop("config")
        cpu["host"] = dict(host_facts(), torch_threads=torch.get_num_threads())
        cpu["configs"] = [c3] + more

    line = {
        "metric": "flash-decode KV GB/s (% HBM peak); W8A8 GEMM TOPS (% int8 MFMA peak)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V/q, lens ~ U[512,32768], permuted page pool)",
        "config": {"workload": "BASELINE config 3: kv_append_paged + "
                               "attention_decode_paged (one call: "
                               "attention_decode_paged_append), bf16, B=32 Hq=32 "
                               "Hkv=8 D=128 P=16",
                   "seed": C3["seed"], "tokens": w["tokens"],
                   "pool_pages": w["pool_pages"], "used_pages": w["used_pages"],
                   "bytes_per_step": step_bytes, "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(attn_gbs, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for("attention_c3"),
                     "kernel": "attention_decode_paged_append = attn_decode_stream "
                               "(appending form) + attn_combine_append",
                     "avg_us": round(attn_ms * 1e3, 2),
                     "bytes_per_launch": step_bytes,
                     "copy_gbs": round(copy_gbs, 1) if copy_gbs else None,
                     "frac_of_copy": round(attn_gbs / copy_gbs, 4) if copy_gbs else None},
        "cpu_baseline": cpu,
        "secondary": secondary,
        "chains": chains,
        "more": decode_more,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
