"""GPU parity of the decode step's tail (final RMSNorm + LM-head GEMV + greedy argmax, moe_head_* through the C ABI)
against the oracle (rmsnorm: host.rs:71-76; gemv: cpu_kern.c:32; argmax rules: main.rs:384-385, chip.rs:183-194).

Bars:
  * logits: max-abs <= 2e-3 against gemv(W, rmsnorm(x)) of the oracle.  The normalised token may differ from the
    oracle's by one bf16 ulp in a few elements (the GPU sums x^2 in a tree, the host left to right, so x * r can land
    on the other side of a bf16 rounding boundary); fp32 accumulation order differs as well;
  * ids / best: exactly the rule's pick over the GPU's own logits (bit-exact), and the oracle's pick wherever the
    oracle's top-2 gap exceeds twice the logit bar (else the GPU's row is within that bar of the oracle's maximum);
  * constructed ties and near-ties (exact in any summation order): bit-exact rows and values under both rules.
"""
import numpy as np
import pytest

import oracle as O
from moe_gpu import ARGMAX_BF16, ARGMAX_FP32, EINVAL, ESTATE, LmHead, MoeGpuError

pytestmark = pytest.mark.gpu
TOL = 2e-3


def say(msg):
    print(f"[gpu-head] {msg}", flush=True)


def ref_logits(W, wf, x, eps=1e-5):
    hn = [O.rmsnorm(x[t], wf, eps) for t in range(x.shape[0])]
    return np.stack([O.gemv(W, h) for h in hn])


def check(ids, best, lg, ref, rule):
    assert np.abs(lg - ref).max() <= TOL, np.abs(lg - ref).max()
    for t in range(lg.shape[0]):
        i_self, v_self = O.lm_head_argmax(lg[t], rule)
        assert (int(ids[t]), float(best[t])) == (i_self, v_self)
        i_ref, v_ref = O.lm_head_argmax(ref[t], rule)
        vals = ref[t] if rule == ARGMAX_FP32 else O.bf2f(O.f2bf(ref[t]))
        gap = v_ref - np.max(np.delete(vals, i_ref))
        if gap > 2 * TOL:
            assert int(ids[t]) == i_ref
        else:
            assert vals[int(ids[t])] >= v_ref - 2 * TOL


def bf(v: float) -> int:
    return int(O.f2bf(np.array([v], np.float32))[0])


def bf16_normal(rng, shape, sd, mean=0.0):
    return O.f2bf((mean + sd * rng.standard_normal(shape)).astype(np.float32))


@pytest.fixture(scope="module")
def small():
    H, V = 1024, 4999  # V odd: the last row step is partial
    rng = np.random.default_rng(40)
    W = bf16_normal(rng, (V, H), 0.02)
    wf = bf16_normal(rng, H, 0.1, 1.0)
    say(f"small head H={H} V={V}: create + upload")
    head = LmHead(H, V)
    head.load(W, wf)
    yield head, W, wf
    head.close()


@pytest.mark.parametrize("T", [1, 3, 6])
def test_small_head_both_rules(small, T):
    head, W, wf = small
    rng = np.random.default_rng(41 + T)
    x = bf16_normal(rng, (T, head.H), 1.0)
    ref = ref_logits(W, wf, x)
    for rule in (ARGMAX_FP32, ARGMAX_BF16):
        say(f"small head T={T} rule={rule}")
        ids, best, lg = head.argmax(x, rule=rule, want_logits=True)
        check(ids, best, lg, ref, rule)
        ids2, best2 = head.argmax(x, rule=rule)  # without the logits output: same picks
        np.testing.assert_array_equal(ids2, ids)
        np.testing.assert_array_equal(best2.view(np.uint32), best.view(np.uint32))


def test_constructed_ties_and_rules():
    # x = 1 gives r = 1/sqrt(1 + 1e-5) and bf16(x * r) = 1, so the normalised token is w_final exactly;
    # w_final = e0 + 2^-10 e1 makes logit[v] = W[v,0] + 2^-10 W[v,1], exact in any order.
    H, V = 1024, 4999
    rng = np.random.default_rng(42)
    W = bf16_normal(rng, (V, H), 0.02)
    wf = np.zeros(H, np.uint16)
    wf[:2] = O.f2bf(np.array([1.0, 2.0 ** -10], np.float32))
    one = bf(1.0)
    W[1000, :2] = [one, 0]      # 1.0
    W[3000, :2] = [one, one]    # 1 + 2^-10 (bf16: 1.0)
    W[V - 1, :2] = [one, one]   # duplicate of row 3000 in the last, partial step
    x = np.full((2, H), one, np.uint16)
    ref = ref_logits(W, wf, x)  # the oracle agrees with the construction
    assert ref[0, 1000] == 1.0 and ref[0, 3000] == ref[1, V - 1] == 1.0009765625
    assert O.lm_head_argmax(ref[0], 0) == (3000, 1.0009765625) and O.lm_head_argmax(ref[0], 1) == (1000, 1.0)
    say("constructed ties")
    head = LmHead(H, V)
    try:
        head.load(W, wf)
        ids, best, lg = head.argmax(x, rule=ARGMAX_FP32, want_logits=True)
        assert ids.tolist() == [3000, 3000] and best.tolist() == [1.0009765625] * 2
        assert lg[0, 1000] == 1.0 and lg[1, V - 1] == 1.0009765625
        ids, best = head.argmax(x, rule=ARGMAX_BF16)
        assert ids.tolist() == [1000, 1000] and best.tolist() == [1.0, 1.0]
        # a unique maximum in the last row
        W[V - 1, :2] = [bf(2.0), 0]
        head.load(W, wf)
        for rule in (ARGMAX_FP32, ARGMAX_BF16):
            ids, best = head.argmax(x, rule=rule)
            assert ids.tolist() == [V - 1, V - 1] and best.tolist() == [2.0, 2.0]
    finally:
        head.close()


def test_signed_zero_and_nan_rules():
    """Mixed-sign zeros tie (the lower row wins) and a NaN is never picked, except a NaN at row 0 under the fp32 rule,
    which the reference's first-maximum loop (main.rs:384-385: `lg[i] > lg[best]` from best = 0) never leaves.
    w_final = 2^-70 e0 makes logit[v] = W[v, 0] * 2^-70: W[5, 0] = -2^-70 gives -2^-140, which rounds to bf16 -0;
    W[9, 0] = +2^-70 gives bf16 +0; every other row is -2^-70 (bf16-exact), so under the bf16 rule rows 5 and 9 tie at
    zero (chip.rs:183-194: equal values -> lower row)."""
    H, V = 1024, 64
    W = np.zeros((V, H), np.uint16)
    W[:, 0] = bf(-1.0)
    W[5, 0] = bf(-(2.0 ** -70))
    W[9, 0] = bf(2.0 ** -70)
    wf = np.zeros(H, np.uint16)
    wf[0] = bf(2.0 ** -70)
    x = np.full((1, H), bf(1.0), np.uint16)
    head = LmHead(H, V)
    try:
        say("signed zeros: bf16 rule ties -0 and +0")
        head.load(W, wf)
        ids, best = head.argmax(x, rule=ARGMAX_BF16)
        assert ids.tolist() == [5] and best.tolist() == [0.0]
        say("NaN rows: never picked, except row 0 under the fp32 rule")
        W[3, 0] = 0x7FC0  # NaN
        head.load(W, wf)
        for rule in (ARGMAX_FP32, ARGMAX_BF16):
            ids, _ = head.argmax(x, rule=rule)
            assert int(ids[0]) in (5, 9) and (rule == ARGMAX_FP32 or int(ids[0]) == 5)
        W[0, 0] = 0x7FC0
        head.load(W, wf)
        ids, best = head.argmax(x, rule=ARGMAX_FP32)
        assert ids.tolist() == [0] and np.isnan(best[0])
        ids, _ = head.argmax(x, rule=ARGMAX_BF16)
        assert ids.tolist() == [5]
    finally:
        head.close()


def test_head_errors():
    head = LmHead(1024, 64)
    try:
        with pytest.raises(MoeGpuError) as e:
            head.argmax(np.zeros((1, 1024), np.uint16))
        assert e.value.code == ESTATE
        head.load(np.zeros((64, 1024), np.uint16), np.zeros(1024, np.uint16))
        for T, rule in ((0, 0), (65, 0), (1, 2)):
            with pytest.raises(MoeGpuError) as e:
                head._chk(head.L.moe_head_argmax(head.h, T, np.zeros((1, 1024), np.uint16).ctypes.data,
                                                            rule, np.zeros(1, np.int32).ctypes.data,
                                                            np.zeros(1, np.float32).ctypes.data, None))
            assert e.value.code == EINVAL
        # all-zero weights: every logit 0, the lowest row wins under both rules
        for rule in (ARGMAX_FP32, ARGMAX_BF16):
            ids, best = head.argmax(np.full((1, 1024), bf(1.0), np.uint16), rule=rule)
            assert ids.tolist() == [0] and best.tolist() == [0.0]
    finally:
        head.close()


def test_solar_head_full_size_and_device_path():
    """V = 196608, H = 4096 (the 1.61 GB table of a Solar decode step), weights drawn on the device."""
    import torch

    H, V = 4096, 196608
    say("solar head: draw weights on the device")
    g = torch.Generator(device="cuda:0").manual_seed(43)
    Wd = (torch.randn(V, H, device="cuda:0", generator=g) * 0.02).to(torch.bfloat16)
    wfd = (1 + 0.1 * torch.randn(H, device="cuda:0", generator=g)).to(torch.bfloat16)
    head = LmHead(H, V)
    try:
        torch.cuda.synchronize()  # the head copies on its own stream
        head.load_dev(Wd.view(torch.int16), wfd.view(torch.int16))
        W = Wd.view(torch.int16).cpu().numpy().view(np.uint16)
        wf = wfd.view(torch.int16).cpu().numpy().view(np.uint16)
        del Wd
        rng = np.random.default_rng(44)
        x = bf16_normal(rng, (2, H), 1.0)
        say("solar head: oracle logits")
        ref = ref_logits(W, wf, x)
        for rule in (ARGMAX_FP32, ARGMAX_BF16):
            say(f"solar head rule={rule}")
            ids, best, lg = head.argmax(x, rule=rule, want_logits=True)
            check(ids, best, lg, ref, rule)
            # the device entry point on torch buffers gives the same bits
            xd = torch.from_numpy(x.view(np.int16)).to("cuda:0")
            idd = torch.zeros(2, dtype=torch.int32, device="cuda:0")
            bd = torch.zeros(2, dtype=torch.float32, device="cuda:0")
            torch.cuda.synchronize()
            head.argmax_dev(2, xd, idd, bd, rule=rule)
            head.synchronize()
            np.testing.assert_array_equal(idd.cpu().numpy(), ids)
            np.testing.assert_array_equal(bd.cpu().numpy().view(np.uint32), best.view(np.uint32))
    finally:
        head.close()


@pytest.mark.parametrize("T,H", [(1, 4096), (5, 4096), (3, 1000)])
def test_per_layer_rmsnorm(T, H):
    """moe_rmsnorm_dev against the oracle's rmsnorm (host.rs:71-76).  With x in multiples of 1/4 up to 4 the sum of
    squares is exact in any order, so the outputs are bit-identical; with random x the GPU's tree sum may move a few
    elements by one bf16 ulp."""
    import torch

    from moe_gpu import rmsnorm_dev

    say(f"rmsnorm T={T} H={H}")
    rng = np.random.default_rng(T * H)
    w = bf16_normal(rng, H, 0.1, 1.0)
    x_exact = O.f2bf((rng.integers(-16, 17, size=(T, H)) / 4.0).astype(np.float32))
    x_rand = bf16_normal(rng, (T, H), 3.0)
    wd = torch.from_numpy(w.view(np.int16)).to("cuda:0")
    for x, exact in ((x_exact, True), (x_rand, False)):
        xd = torch.from_numpy(x.view(np.int16)).to("cuda:0")
        od = torch.zeros_like(xd)
        torch.cuda.synchronize()
        rmsnorm_dev(xd, wd, od)
        torch.cuda.synchronize()
        got = od.cpu().numpy().view(np.uint16)
        ref = np.stack([O.rmsnorm(x[t], w) for t in range(T)])
        if exact:
            np.testing.assert_array_equal(got, ref)
        else:
            ulps = np.abs(got.astype(np.int32) - ref.astype(np.int32))
            assert ulps.max() <= 1 and (ulps > 0).mean() <= 1e-2
