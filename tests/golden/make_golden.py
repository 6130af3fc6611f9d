"""Writes tests/golden/golden.npz: seeded inputs and expected outputs for
the decode hot path, computed with numpy only (float64 closed forms and
exact integer arithmetic from tests/refs.py) - independent of both the C++
oracle and the HIP kernels. Re-run to regenerate:

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests import refs  # noqa: E402


def main():
    rng = np.random.default_rng(20261201)
    g = {}
    # contiguous decode: B=2, Hq=8, Hkv=2, T=40, D=32, ragged lens
    q = rng.standard_normal((2, 8, 32)).astype(np.float32)
    k = rng.standard_normal((2, 2, 40, 32)).astype(np.float32)
    v = rng.standard_normal((2, 2, 40, 32)).astype(np.float32)
    lens = np.array([40, 23], np.int32)
    g.update(dec_q=q, dec_k=k, dec_v=v, dec_lens=lens,
             dec_out=refs.ref_decode(q, k, v, lens).astype(np.float32))
    # paged decode: B=3, Hq=8, Hkv=2, P=16, D=32, non-monotonic table
    nb, page = 12, 16
    kp = rng.standard_normal((nb, 2, page, 32)).astype(np.float32)
    vp = rng.standard_normal((nb, 2, page, 32)).astype(np.float32)
    tbl = rng.permutation(nb)[:9].reshape(3, 3).astype(np.int32)
    plens = np.array([37, 16, 48], np.int32)
    pq = rng.standard_normal((3, 8, 32)).astype(np.float32)
    g.update(pg_q=pq, pg_kp=kp, pg_vp=vp, pg_tbl=tbl, pg_lens=plens,
             pg_out=refs.ref_decode_paged(pq, kp, vp, tbl, plens).astype(np.float32))
    # quantize
    x = (rng.standard_normal(777) * 3).astype(np.float32)
    qq, s = refs.ref_quantize(x)
    g.update(qz_x=x, qz_q=qq, qz_scale=np.float32(s))
    # W8A8 per-channel GEMM
    a = rng.integers(-127, 128, (5, 96)).astype(np.int8)
    b = rng.integers(-127, 128, (40, 96)).astype(np.int8)
    sb = rng.uniform(1e-3, 1e-2, 40).astype(np.float32)
    g.update(gm_a=a, gm_b=b, gm_sa=np.float32(0.037), gm_sb=sb,
             gm_acc=refs.ref_qgemm_i32(a, b).astype(np.int32),
             gm_y=refs.ref_qgemm_pc(a, np.float32(0.037), b, sb))
    # rmsnorm + residual
    rx = rng.standard_normal((4, 96)).astype(np.float32)
    rr = rng.uniform(-1, 1, (4, 96)).astype(np.float32)
    rw = rng.uniform(0.5, 1.5, 96).astype(np.float32)
    g.update(rn_x=rx, rn_r=rr, rn_w=rw,
             rn_y=refs.ref_rmsnorm(rx, rw, 1e-5, rr).astype(np.float32))
    # rope neox at position 8192 (float64 angles)
    px = rng.standard_normal((3, 32)).astype(np.float32)
    g.update(rp_x=px, rp_y=refs.ref_rope(px, 10000.0, 8192, True).astype(np.float32))
    # swiglu
    sg = (rng.standard_normal(300) * 4).astype(np.float32)
    su = rng.standard_normal(300).astype(np.float32)
    g.update(sw_g=sg, sw_u=su, sw_y=refs.ref_swiglu(sg, su).astype(np.float32))
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **g)
    print("wrote", os.path.join(HERE, "golden.npz"))


if __name__ == "__main__":
    main()
