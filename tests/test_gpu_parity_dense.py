"""GPU parity of the attention block's dense steps (moe_gemv_dev, moe_gemv_norm_dev, moe_gemv_f32_dev, moe_rope_dev,
moe_rope_append_dev through the C ABI) against the oracle: gemv (cpu_kern.c:32) + round_bf for the projections
(main.rs:109-111, :119), rmsnorm (host.rs:71-76), rope and the KV append (main.rs:65-77, :112-118).

Bars:
  * gemv: bit-identical where the products and sums are exact in any order (small-integer multiples), else within one
    bf16 ulp of round_bf(ck_gemv) on at most 2 % of the rows (the fp32 sums run in the GPU's order);
  * rope: bit-identical (elementwise, the same fp32 operations and roundings).
"""
import numpy as np
import pytest

import oracle as O
from moe_gpu import gemv_dev, rope_dev

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-dense] {msg}", flush=True)


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to("cuda:0")


def host(t):
    return t.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("M,K", [(4096, 4096), (1024, 4096), (1000, 4096), (37, 2048), (3, 1024)])
def test_gemv_projection(M, K):
    import torch

    say(f"gemv M={M} K={K}")
    rng = np.random.default_rng(M + K)
    W = O.f2bf((0.02 * rng.standard_normal((M, K))).astype(np.float32))
    x = O.f2bf(rng.standard_normal(K).astype(np.float32))
    Wi = O.f2bf((rng.integers(-8, 9, size=(M, K)) / 8.0).astype(np.float32))  # exact sums in any order
    xi = O.f2bf((rng.integers(-8, 9, size=K) / 8.0).astype(np.float32))
    for Wm, xv, exact in ((Wi, xi, True), (W, x, False)):
        Wd, xd = dev(Wm), dev(xv)
        yd = torch.zeros(M, dtype=torch.int16, device="cuda:0")
        torch.cuda.synchronize()
        gemv_dev(Wd, xd, yd)
        torch.cuda.synchronize()
        got, ref = host(yd), O.f2bf(O.gemv(Wm, xv))
        if exact:
            np.testing.assert_array_equal(got, ref)
        else:
            ulps = np.abs(got.astype(np.int32) - ref.astype(np.int32))
            assert ulps.max() <= 1 and (ulps > 0).mean() <= 0.02, (ulps.max(), (ulps > 0).mean())


@pytest.mark.parametrize("n_heads", [32, 8])
def test_rope_bitexact(n_heads):
    import torch

    say(f"rope heads={n_heads}")
    rng = np.random.default_rng(n_heads)
    D = 128
    x = O.f2bf(rng.standard_normal((n_heads, D)).astype(np.float32))
    th = rng.uniform(0, 200, D // 2)
    c = O.f2bf(np.cos(np.concatenate([th, th])).astype(np.float32))
    s = O.f2bf(np.sin(np.concatenate([th, th])).astype(np.float32))
    xd, cd, sd = dev(x), dev(c), dev(s)
    torch.cuda.synchronize()
    rope_dev(xd, cd, sd)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(xd), O.rope(x, c, s))


@pytest.mark.parametrize("M,K", [(6144, 4096), (1024, 4096)])
def test_gemv_norm_projection(M, K):
    """moe_gemv_norm_dev: the input RMSNorm folded into the projection.  Bit-identical to round_bf(gemv(W,
    rmsnorm(x, w))) where every sum is exact in any order; else within one bf16 ulp on at most 2 % of the rows."""
    import torch

    from moe_gpu import gemv_norm_dev

    say(f"gemv+norm M={M} K={K}")
    rng = np.random.default_rng(M + 7)
    W = O.f2bf((0.02 * rng.standard_normal((M, K))).astype(np.float32))
    x = O.f2bf(rng.standard_normal(K).astype(np.float32))
    w = O.f2bf((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    # exact: x = 1 everywhere (sum of squares exact, r = 1/sqrt(1 + eps), bf16(x r) = 1), w and W small integers / 8
    xi = O.f2bf(np.ones(K, np.float32))
    wi = O.f2bf((rng.integers(1, 9, size=K) / 8.0).astype(np.float32))
    Wi = O.f2bf((rng.integers(-8, 9, size=(M, K)) / 8.0).astype(np.float32))
    for Wm, xv, wv, exact in ((Wi, xi, wi, True), (W, x, w, False)):
        yd = torch.zeros(M, dtype=torch.int16, device="cuda:0")
        Wd, xd, wd = dev(Wm), dev(xv), dev(wv)
        torch.cuda.synchronize()
        gemv_norm_dev(Wd, xd, wd, yd)
        torch.cuda.synchronize()
        got, ref = host(yd), O.f2bf(O.gemv(Wm, O.rmsnorm(xv, wv)))
        if exact:
            np.testing.assert_array_equal(got, ref)
        else:
            ulps = np.abs(got.astype(np.int32) - ref.astype(np.int32))
            assert ulps.max() <= 1 and (ulps > 0).mean() <= 0.02, (ulps.max(), (ulps > 0).mean())


def test_rope_append_bitexact():
    """moe_rope_append_dev: q roped in place, k roped into the key cache row of pos, v copied into the value cache row
    (main.rs:112-118); every other cache row untouched."""
    import torch

    from moe_gpu import rope_append_dev

    NQ, NKV, D, CTX, pos = 32, 8, 128, 64, 37
    rng = np.random.default_rng(5)
    qkv = O.f2bf(rng.standard_normal((NQ + 2 * NKV) * D).astype(np.float32))
    th = rng.uniform(0, 200, D // 2)
    c = O.f2bf(np.cos(np.concatenate([th, th])).astype(np.float32))
    s = O.f2bf(np.sin(np.concatenate([th, th])).astype(np.float32))
    kc = O.f2bf(rng.standard_normal((CTX, NKV, D)).astype(np.float32))
    vc = O.f2bf(rng.standard_normal((CTX, NKV, D)).astype(np.float32))
    qd, cd, sd, kd, vd = dev(qkv), dev(c), dev(s), dev(kc), dev(vc)
    say("rope + kv append")
    torch.cuda.synchronize()
    rope_append_dev(qd, cd, sd, kd, vd, pos, NQ, NKV)
    torch.cuda.synchronize()
    q = qkv[:NQ * D].reshape(NQ, D); k = qkv[NQ * D:(NQ + NKV) * D].reshape(NKV, D); v = qkv[(NQ + NKV) * D:].reshape(NKV, D)
    got = host(qd)
    np.testing.assert_array_equal(got[:NQ * D].reshape(NQ, D), O.rope(q, c, s))
    np.testing.assert_array_equal(got[NQ * D:], qkv[NQ * D:])  # k and v rows of the buffer unchanged
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[pos] = O.rope(k, c, s); vc2[pos] = v
    np.testing.assert_array_equal(host(kd).reshape(CTX, NKV, D), kc2)
    np.testing.assert_array_equal(host(vd).reshape(CTX, NKV, D), vc2)


@pytest.mark.parametrize("with_norm", [True, False])
def test_qkv_rope_append_equals_the_two_launches(with_norm):
    """moe_qkv_rope_append_dev (the q|k|v GEMV with RoPE and the cache append in its epilogue) gives the bits of
    moe_gemv_norm_dev / moe_gemv_dev followed by moe_rope_append_dev; no other cache row changes."""
    import torch

    from moe_gpu import gemv_dev, gemv_norm_dev, qkv_rope_append_dev, rope_append_dev

    NQ, NKV, D, H, CTX, pos = 32, 8, 128, 4096, 16, 11
    M = (NQ + 2 * NKV) * D
    rng = np.random.default_rng(77)
    W = dev(O.f2bf((0.02 * rng.standard_normal((M, H))).astype(np.float32))).view(M, H)
    x = dev(O.f2bf(rng.standard_normal(H).astype(np.float32)))
    nw = dev(O.f2bf(rng.uniform(0.5, 1.5, H).astype(np.float32))) if with_norm else None
    th = rng.uniform(0, 200, D // 2)
    c = dev(O.f2bf(np.cos(np.concatenate([th, th])).astype(np.float32)))
    s = dev(O.f2bf(np.sin(np.concatenate([th, th])).astype(np.float32)))
    kc0 = O.f2bf(rng.standard_normal((CTX, NKV, D)).astype(np.float32))
    vc0 = O.f2bf(rng.standard_normal((CTX, NKV, D)).astype(np.float32))
    k1, v1, k2, v2 = dev(kc0), dev(vc0), dev(kc0), dev(vc0)
    qkv = torch.zeros(M, dtype=torch.int16, device="cuda:0")
    q2 = torch.zeros(NQ * D, dtype=torch.int16, device="cuda:0")
    say(f"qkv + rope + append, norm={with_norm}")
    torch.cuda.synchronize()
    if with_norm:
        gemv_norm_dev(W, x, nw, qkv)
    else:
        gemv_dev(W, x, qkv)
    rope_append_dev(qkv, c, s, k1, v1, pos, NQ, NKV)
    qkv_rope_append_dev(W, x, nw, c, s, q2, k2, v2, pos, NQ, NKV)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(q2), host(qkv)[:NQ * D])
    np.testing.assert_array_equal(host(k2), host(k1))
    np.testing.assert_array_equal(host(v2), host(v1))
    kd = host(k2).reshape(CTX, NKV, D)
    np.testing.assert_array_equal(np.delete(kd, pos, axis=0), np.delete(kc0, pos, axis=0))


def test_gemv_f32_bit_identical_to_ck_gemv():
    """moe_gemv_f32_dev runs ck_gemv's own summation order (two 16-lane vdpbf16ps accumulators, GCC's reduce tree)."""
    import torch

    from moe_gpu import load_library

    L = load_library()
    rng = np.random.default_rng(9)
    for M, K in ((128, 4096), (1000, 1024), (5, 512), (77, 8192)):
        say(f"gemv f32 M={M} K={K}")
        W = O.f2bf((0.02 * rng.standard_normal((M, K))).astype(np.float32))
        x = O.f2bf(rng.standard_normal(K).astype(np.float32))
        y = torch.zeros(M, dtype=torch.float32, device="cuda:0")
        Wd, xd = dev(W), dev(x)
        torch.cuda.synchronize()
        assert L.moe_gemv_f32_dev(M, K, Wd.data_ptr(), xd.data_ptr(), y.data_ptr(), None) == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), O.gemv(W, x).view(np.uint32))
