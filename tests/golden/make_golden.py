"""Write the golden vectors of the routed-MoE CPU path from the reference's own code.

The reference holds no kernel-level golden vectors for this path, so this script makes them: it runs
track2_opt/solar_engine/csrc/cpu_kern.c — compiled from the reference's source by oracle/Makefile into
oracle/_ref/libcpu_kern.so — on small seeded inputs and stores inputs and outputs in golden_cpu_kern.npz.
The weights are described by their synthetic-generator keys (regenerated bit-for-bit by the test), x / gates / the
starting `out` are stored explicitly.  Run:  make -C oracle && python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libcpu_kern.so missing (or no AVX-512 BF16 on this host)")
    R = O.Ref()
    R.set_threads(4)
    rng = np.random.default_rng(20261201)
    H, F, E = 256, 128, 3
    c = np.float32(0.02 / np.sqrt(8 * (65536.0 ** 2 - 1) / 12))
    keys = np.array([[O.synth_key(77, 10 * e + m) for m in range(3)] for e in range(E)], np.uint64)
    gs = [O.synth_bf16(int(keys[e, 0]), F * H, c).reshape(F, H) for e in range(E)]
    us = [O.synth_bf16(int(keys[e, 1]), F * H, c).reshape(F, H) for e in range(E)]
    ds = [O.synth_bf16(int(keys[e, 2]), H * F, c).reshape(H, F) for e in range(E)]
    x = O.f2bf(rng.normal(0, 1, H).astype(np.float32))
    w = np.array([0.5, 0.3125, 0.1875], np.float32)
    out0 = rng.normal(0, 1, H).astype(np.float32)

    # ck_gemv with a length that exercises dot_bf16's 32-element tail (1056 = 16*64 + 32)
    Wg = O.f2bf(rng.normal(0, 0.02, (24, 1056)).astype(np.float32))
    xg = O.f2bf(rng.normal(0, 1, 1056).astype(np.float32))
    y_gemv = R.gemv(Wg, xg)

    o1 = np.zeros(H, np.float32); R.moe1(gs, us, ds, w, x, o1, H, F)                  # ck_moe1 (== cpu_moe per token)
    o2 = out0.copy(); R.moe1(gs, us, ds, w, x, o2, H, F, fn="ck_moe2")               # ck_moe2, accumulating
    bases = [R.place_expert(g, u, d) for g, u, d in zip(gs, us, ds)]
    o3 = out0.copy(); R.moe3(bases, w, x, o3, H, F)                                   # ck_moe3, accumulating
    q, sc, rs = R.place_expert_q8(gs[0], us[0], ds[0])                                # quant_row via ck_place_expert_q8
    qs, scs = [], []
    for g, u, d in zip(gs, us, ds):
        qq, ss, _ = R.place_expert_q8(g, u, d); qs.append(qq); scs.append(ss)
    oq = out0.copy(); R.moe_q8w(qs, scs, w, x, oq, H, F)                              # ck_moe_q8w, accumulating

    np.savez_compressed(os.path.join(HERE, "golden_cpu_kern.npz"), H=H, F=F, E=E, c=c, keys=keys, x=x, w=w,
                        out0=out0, Wg=Wg, xg=xg, y_gemv=y_gemv, out_moe1=o1, out_moe2=o2, out_moe3=o3, q0=q, sc0=sc,
                        rs0=rs, out_q8w=oq)
    print("wrote", os.path.join(HERE, "golden_cpu_kern.npz"))


if __name__ == "__main__":
    main()
