"""libck_gpu.so: the reference engine's CPU-kernel boundary (track2_opt/solar_engine/src/host.rs:18-37, implemented by
csrc/cpu_kern.c) served by the GPU tier.  The export check runs without a GPU; the parity checks call the shim's ck_*
through ctypes exactly as the engine's FFI would, against the oracle's restatement of cpu_kern.c (bit-exact to the
reference's own build, tests/test_oracle.py):
  * ck_gemv: bit-identical y (moe_gemv_f32_dev runs ck_gemv's summation order);
  * ck_place_expert_q8: bit-identical q, sc and rs;
  * ck_moe3 / ck_moe2 / ck_moe_q8w: out += sum_e w_e expert_e(x) within the layer bars (max-abs 2e-2, rel-L2 5e-3),
    including a call of 10 experts (split into runs of 8 by the shim, in list order) and accumulation into a
    non-zero out.
"""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from moe_ref import assert_layer_close

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "npu-offload_amd", "lib", "libck_gpu.so")
# the engine's extern "C" block (host.rs:18-37)
ENGINE_SYMBOLS = ["ck_set_threads", "ck_mmio_read", "ck_mmio_set_threads", "ck_gemv", "ck_moe2", "ck_place_expert",
                  "ck_moe3", "ck_read_bw", "ck_place_expert_q8", "ck_moe_q8", "ck_moe_q8w", "ck_moe_q8x",
                  "ck_touch_experts", "ck_moe1"]


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.strip()}


def test_shim_exports_the_engine_boundary():
    names = exported(LIB)
    missing = [n for n in ENGINE_SYMBOLS if n not in names]
    assert not missing, missing
    ref = os.path.join(os.path.dirname(O.__file__), "_ref", "libcpu_kern.so")
    if os.path.exists(ref):  # and every ck_* the reference's own library exports
        ref_ck = {n for n in exported(ref) if n.startswith("ck_")}
        assert ref_ck <= names, sorted(ref_ck - names)


def load_shim():
    import moe_gpu
    moe_gpu.load_library()  # binds the process's HIP runtime first
    L = C.CDLL(LIB)
    vp, i, f = C.c_void_p, C.c_int, C.c_float
    L.ck_gemv.argtypes = [vp, vp, vp, i, i]
    L.ck_place_expert.argtypes = [vp, vp, vp, vp, i, i]
    L.ck_moe3.argtypes = [i, vp, vp, vp, vp, i, i]
    L.ck_moe2.argtypes = [i, vp, vp, vp, vp, vp, vp, i, i]
    L.ck_place_expert_q8.argtypes = [vp, vp, vp, vp, vp, vp, i, i]
    L.ck_moe_q8w.argtypes = [i, vp, vp, vp, vp, vp, i, i]
    L.ck_gpu_last_error.restype = C.c_char_p
    return L


def ptrs(arrs):
    a = (C.c_void_p * len(arrs))()
    for k, x in enumerate(arrs):
        a[k] = x.ctypes.data
    return a


def bf(rng, shape, sd):
    return O.f2bf((sd * rng.standard_normal(shape)).astype(np.float32))


@pytest.mark.gpu
def test_shim_gemv_bit_identical_to_ck_gemv():
    L = load_shim()
    rng = np.random.default_rng(60)
    for M, K in ((1000, 1024), (128, 4096), (7, 512)):
        W = bf(rng, (M, K), 0.02); x = bf(rng, K, 1.0)
        y = np.zeros(M, np.float32)
        L.ck_gemv(W.ctypes.data, x.ctypes.data, y.ctypes.data, M, K)
        assert L.ck_gpu_last_error() == b"no error", L.ck_gpu_last_error()
        np.testing.assert_array_equal(y.view(np.uint32), O.gemv(W, x).view(np.uint32))


@pytest.mark.gpu
def test_shim_experts_match_cpu_kern():
    L = load_shim()
    rng = np.random.default_rng(61)
    H, F, n = 1024, 512, 10
    ex = [(bf(rng, (F, H), 0.02), bf(rng, (F, H), 0.02), bf(rng, (H, F), 0.02)) for _ in range(n)]
    bases = []
    for g, u, d in ex:
        dst = np.zeros(3 * F * H, np.uint16)
        L.ck_place_expert(g.ctypes.data, u.ctypes.data, d.ctypes.data, dst.ctypes.data, H, F)
        np.testing.assert_array_equal(dst, np.concatenate([g.ravel(), u.ravel(), d.ravel()]))
        bases.append(dst)
    x = bf(rng, H, 1.0)
    w = rng.uniform(0.05, 0.3, n).astype(np.float32)
    out0 = rng.normal(0, 1, H).astype(np.float32)
    for E in (3, 8, 10):  # 10: two runs of the tier's top-8 call, summed in list order
        got = out0.copy()
        L.ck_moe3(E, ptrs(bases[:E]), w.ctypes.data, x.ctypes.data, got.ctypes.data, H, F)
        assert L.ck_gpu_last_error() == b"no error", L.ck_gpu_last_error()
        exp = out0.copy()
        O.ck_moe3(bases[:E], w[:E], x, exp, H, F)
        assert_layer_close(got, exp)
    got = np.zeros(H, np.float32)  # ck_moe2: (g, u, d) pointers, uploaded on first use
    gs, us, ds = zip(*ex[:5])
    L.ck_moe2(5, ptrs(gs), ptrs(us), ptrs(ds), w.ctypes.data, x.ctypes.data, got.ctypes.data, H, F)
    exp = np.zeros(H, np.float32)
    O.ck_moe3([np.concatenate([a.ravel() for a in e]) for e in ex[:5]], w[:5], x, exp, H, F)
    assert_layer_close(got, exp)


@pytest.mark.gpu
def test_shim_int8_matches_cpu_kern():
    L = load_shim()
    rng = np.random.default_rng(62)
    H, F, n = 1024, 512, 4
    qs, scs = [], []
    g, u, d = np.empty((F, H), np.uint16), np.empty((F, H), np.uint16), np.empty((H, F), np.uint16)
    for _ in range(n):
        # the same g / u / d buffers for every expert, refilled in place: each placed expert must still get its own
        # slot (placements are keyed by the caller's q buffer, not by the source addresses)
        g[:], u[:], d[:] = bf(rng, (F, H), 0.02), bf(rng, (F, H), 0.02), bf(rng, (H, F), 0.02)
        q = np.zeros(3 * F * H, np.int8); sc = np.zeros(2 * F + H, np.float32); rs = np.zeros(2 * F + H, np.int32)
        L.ck_place_expert_q8(g.ctypes.data, u.ctypes.data, d.ctypes.data, q.ctypes.data, sc.ctypes.data, rs.ctypes.data,
                              H, F)
        q2, sc2, rs2 = O.quant_expert(g, u, d)
        np.testing.assert_array_equal(q, q2)
        np.testing.assert_array_equal(sc.view(np.uint32), sc2.view(np.uint32))
        np.testing.assert_array_equal(rs, rs2)
        qs.append(q); scs.append(sc)
    x = bf(rng, H, 1.0)
    w = rng.uniform(0.1, 0.4, n).astype(np.float32)
    got = np.zeros(H, np.float32)
    L.ck_moe_q8w(n, ptrs(qs), ptrs(scs), w.ctypes.data, x.ctypes.data, got.ctypes.data, H, F)
    assert L.ck_gpu_last_error() == b"no error", L.ck_gpu_last_error()
    exp = np.zeros(H, np.float32)
    O.moe_q8w(qs, scs, w, x, exp, H, F)
    assert_layer_close(got, exp)
