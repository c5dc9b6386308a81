"""GPU parity of the attention block's dense steps (moe_gemv_dev, moe_rope_dev through the C ABI) against the oracle:
gemv (cpu_kern.c:32) + round_bf for the projections (main.rs:109-111, :119), rope (main.rs:65-77).

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
