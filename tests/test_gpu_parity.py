"""GPU parity: libmoe_gpu (through its C ABI) against the CPU oracle on identical seeded inputs.

Bars (from the task's definition of done):
  * router logits: bit-identical to the reference's ck_gemv (cpu_kern.c:9-19, :31-35; its restatement O.gemv, and at
    scale the reference's own build);
  * top-k expert ids: bit-exact (the oracle selects on the same logits, ties to the lower index);
  * gates: softmax restricted to the kept ranks, relative error <= 1e-6; Solar's sigmoid rule likewise;
  * layer outputs (bf16 weights, fp32 accumulation): max-abs <= 2e-2 and rel-L2 <= 5e-3 against cpu_moe semantics;
    int8 weight-only outputs against the reference's own int8 dequantisation (ck_moe_q8w semantics), same bars;
  * the device quantiser: bit-identical int8 codes and scales to quant_row.
"""
import numpy as np
import pytest

import oracle as O
from moe_gpu import (ACCUMULATE, EINVAL, ESTATE, INT8, OPT_FUSED, OPT_GRID, OPT_ROUTE_RULE, OPT_ROUTER_POLL,
                     ROUTE_SIGMOID, ROUTE_SOFTMAX, MoeGpu, MoeGpuError, gpu_moe, synth_c)
from moe_gpu.workloads import SOLAR, SOLAR_INT8, TINY, Workload, solar_batch
from moe_ref import HostLayer, assert_layer_close, oracle_layer, random_layer, random_x, upload

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-parity] {msg}", flush=True)


def check_route(gpu_ids, gpu_gates, ref, keep):
    np.testing.assert_array_equal(gpu_ids, ref["ids"])
    g, r = gpu_gates[:, :keep].astype(np.float64), ref["gates"][:, :keep].astype(np.float64)
    assert np.all(np.abs(g - r) <= 1e-6 * np.abs(r) + 1e-12), (g, r)
    assert np.all(gpu_gates[:, keep:] == 0)


# ------------------------------------------------------------------------------------------------ tiny (config 1)
@pytest.fixture(scope="module")
def tiny():
    say("tiny: create tier H=1024 F=512 E=16 k=2 and upload numpy-normal weights")
    rng = np.random.default_rng(0)
    hl = random_layer(TINY, rng)
    tier = MoeGpu(TINY.H, TINY.F, TINY.E, TINY.k, TINY.n_shared, n_layers=1, max_tokens=16)
    upload(tier, hl)
    yield tier, hl
    tier.close()


def test_tiny_route_bitexact(tiny):
    tier, hl = tiny
    rng = np.random.default_rng(1)
    for T in (1, 3, 16):
        say(f"tiny route T={T}")
        x = random_x(T, TINY.H, rng)
        ids, gates, lg = tier.route(0, x, want_logits=True)
        ref = oracle_layer(hl, x)
        np.testing.assert_array_equal(lg.view(np.uint32), ref["logits"].view(np.uint32))
        check_route(ids, gates, ref, TINY.k)


# ------------------------------------------------------------------------- several-token routing, wide expert counts
# The several-token selection has three layouts (E <= 128: up to 8 keys per lane of a token's 16-lane row; E <= 256: up
# to 16; above: rank counting, several passes of 1024 keys), and the grouping counts first occurrences over two
# 64-entry ballots (T * keep up to 128 entries).  Batch 16 runs the standalone routing kernel, batch 5 the fused
# kernel's per-workgroup routing.
WIDE = [Workload("wide: H=1024 E=200+1 shared top-8 F=256", 1024, 256, 200, 8, 1, zipf_s=1.1, seed=31),
        Workload("wide: H=1024 E=300 top-6 F=256", 1024, 256, 300, 6, 0, zipf_s=1.1, seed=32)]


@pytest.mark.parametrize("wi", [0, 1])
def test_route_and_layer_many_tokens_wide_experts(wi):
    w = WIDE[wi]
    say(f"{w.name}: upload numpy-normal weights")
    rng = np.random.default_rng(40 + wi)
    hl = random_layer(w, rng)
    tier = MoeGpu(w.H, w.F, w.E, w.k, w.n_shared, n_layers=1, max_tokens=16)
    try:
        upload(tier, hl)
        for T in (16, 5):
            x = random_x(T, w.H, rng)
            for keep in (w.k, w.k // 2):
                say(f"  T={T} keep={keep}: route, then the layer")
                ids, gates, lg = tier.route(0, x, keep=keep, want_logits=True)
                ref = oracle_layer(hl, x, keep=keep)
                np.testing.assert_array_equal(lg.view(np.uint32), ref["logits"].view(np.uint32))
                check_route(ids, gates, ref, keep)
                out, ids2, gates2 = tier.layer(0, x, keep=keep)
                np.testing.assert_array_equal(ids2, ids)
                np.testing.assert_array_equal(gates2.view(np.uint32), gates.view(np.uint32))
                assert_layer_close(out, ref["out"])
    finally:
        tier.close()


def test_tiny_layer(tiny):
    tier, hl = tiny
    rng = np.random.default_rng(2)
    for T in (1, 2, 5):
        say(f"tiny layer T={T}")
        x = random_x(T, TINY.H, rng)
        out, ids, gates = tier.layer(0, x)
        ref = oracle_layer(hl, x)
        check_route(ids, gates, ref, TINY.k)
        r = assert_layer_close(out, ref["out"])
        assert r["rel_l2"] < 1e-4, r  # far inside the bar: only fp32 summation order and rare bf16 act flips differ


def test_tiny_batch_invariance_bitwise(tiny):
    """Below 8 tokens a token's bits do not depend on its batch.  From 8 tokens on (the grouped MFMA path for units of
    more than 4 tokens) each token stays within the bars of itself alone and of the oracle."""
    tier, hl = tiny
    x = random_x(8, TINY.H, np.random.default_rng(3))
    say("tiny batch invariance T=7 vs T=1")
    out7, _, _ = tier.layer(0, x[:7])
    for t in range(7):
        o1, _, _ = tier.layer(0, x[t:t + 1])
        np.testing.assert_array_equal(o1[0].view(np.uint32), out7[t].view(np.uint32))
    say("tiny T=8 (MFMA for large units) vs T=1 and the oracle")
    out8, _, _ = tier.layer(0, x)
    ref = oracle_layer(hl, x)
    assert_layer_close(out8, ref["out"])
    for t in range(8):
        o1, _, _ = tier.layer(0, x[t:t + 1])
        assert_layer_close(out8[t:t + 1], o1)


def test_tiny_moe_given_ids_keep_and_empty_ranks(tiny):
    tier, hl = tiny
    rng = np.random.default_rng(4)
    x = random_x(4, TINY.H, rng)
    ids = np.array([[3, 7], [7, 3], [0, -1], [15, 1]], np.int32)
    gates = np.array([[0.6, 0.4], [0.25, 0.75], [1.0, 0.9], [0.5, 0.5]], np.float32)
    say("tiny moe with caller ids (incl. an empty rank)")
    out = tier.moe(0, x, ids, gates)
    ref = oracle_layer(hl, x, ids=ids, gates=gates)
    assert_layer_close(out, ref["out"])
    say("tiny moe keep=1")
    out1 = tier.moe(0, x, ids, gates, keep=1)
    ref1 = oracle_layer(hl, x, keep=1, ids=ids, gates=gates)
    assert_layer_close(out1, ref1["out"])


def test_tiny_ck_moe3_semantics_accumulate(tiny):
    """moe_placed == ck_moe3 (cpu_kern.c:141-172): out[H] += sum_e w[e] * expert_e(x), caller's out kept."""
    tier, hl = tiny
    rng = np.random.default_rng(5)
    x = random_x(1, TINY.H, rng)[0]
    ids, w = [5, 2], np.array([0.7, 0.3], np.float32)
    out0 = rng.normal(0, 1, TINY.H).astype(np.float32)
    got = out0.copy()
    say("tiny moe_placed (accumulate)")
    tier.moe_placed(0, ids, w, x, got)
    exp = out0.copy()
    bases = [np.concatenate([*hl.expert(e)[:2], hl.expert(e)[2]], axis=None) for e in ids]
    O.ck_moe3(bases, w, x, exp, TINY.H, TINY.F)
    assert_layer_close(got, exp)


def test_tiny_gpu_moe_matches_cpu_moe_interface(tiny):
    """gpu_moe(x, experts, toks, ws) == cpu_moe(x, gus, ds, toks, ws) (cpu_moe.cpp:38-96) on a grouped batch."""
    tier, hl = tiny
    rng = np.random.default_rng(6)
    x = random_x(3, TINY.H, rng)
    experts = [4, 9, 1]
    toks = [np.array([0, 2]), np.array([1]), np.array([0, 1, 2])]
    ws = [np.array([0.5, 0.25], np.float32), np.array([1.0], np.float32), np.array([0.5, 0.125, 0.75], np.float32)]
    say("tiny gpu_moe vs cpu_moe")
    got = gpu_moe(tier, 0, x, experts, toks, ws)
    gus = [np.concatenate(hl.expert(e)[:2]) for e in experts]
    ds = [hl.expert(e)[2] for e in experts]
    exp = O.cpu_moe(x, gus, ds, toks, ws)
    assert_layer_close(got, exp)


def test_tiny_int8_only_layer_and_stale_copies():
    """A layer whose routed experts are loaded only as int8 (no bf16 routed tables are allocated) serves int8 calls
    and refuses bf16 ones; reloading one expert in bf16 makes its int8 copy stale, which the device-id entry points
    refuse (they cannot check ids) while the host entry point refuses only calls that select it."""
    rng = np.random.default_rng(3)
    hl = random_layer(TINY, rng)
    tier = MoeGpu(TINY.H, TINY.F, TINY.E, TINY.k, 0, n_layers=1, max_tokens=4)
    try:
        say("tiny int8-only layer")
        tier.place_router(0, hl.router(), hl.bias)
        for e in range(TINY.E):
            q, sc = hl.expert_q8(e)
            tier.place_expert_q8(0, e, q, sc)
        x = random_x(3, TINY.H, rng)
        out, ids, gates = tier.layer(0, x, flags=INT8)
        ref = oracle_layer(hl, x, int8=True)
        check_route(ids, gates, ref, TINY.k)
        assert_layer_close(out, ref["out"])
        with pytest.raises(MoeGpuError) as ei:
            tier.layer(0, x)
        assert ei.value.code == ESTATE
        say("tiny stale int8 copy")
        tier.place_expert(0, 5, *hl.expert(5))  # bf16 reload: expert 5's int8 copy is stale now
        with pytest.raises(MoeGpuError) as ei:
            tier.layer(0, x, flags=INT8)
        assert ei.value.code == ESTATE
        ids_ok = np.array([[1, 2]], np.int32); g = np.array([[0.5, 0.5]], np.float32)
        o2 = tier.moe(0, x[:1], ids_ok, g, flags=INT8)  # experts 1 and 2 are current
        assert np.isfinite(o2).all()
        with pytest.raises(MoeGpuError) as ei:
            tier.moe(0, x[:1], np.array([[5, 2]], np.int32), g, flags=INT8)
        assert ei.value.code == ESTATE
    finally:
        tier.close()


def test_tiny_errors(tiny):
    tier, _ = tiny
    x = random_x(2, TINY.H, np.random.default_rng(7))
    say("tiny error paths")
    with pytest.raises(MoeGpuError) as ei:
        tier.moe(0, x, np.array([[16, 1], [0, 1]], np.int32), np.ones((2, 2), np.float32))
    assert ei.value.code == EINVAL
    with pytest.raises(MoeGpuError) as ei:
        tier.moe(0, x, np.array([[2, 2], [0, 1]], np.int32), np.ones((2, 2), np.float32))
    assert ei.value.code == EINVAL
    with pytest.raises(MoeGpuError) as ei:
        tier.layer(1, x)
    assert ei.value.code == EINVAL
    with pytest.raises(MoeGpuError) as ei:
        tier.layer(0, random_x(17, TINY.H, np.random.default_rng(8)))
    assert ei.value.code == EINVAL
    with pytest.raises(MoeGpuError) as ei:
        tier.layer(0, x, flags=INT8)
    assert ei.value.code == ESTATE
    # the tier still works after the errors
    out, _, _ = tier.layer(0, x)
    assert np.isfinite(out).all()


def test_unloaded_layer_is_an_error():
    tier = MoeGpu(TINY.H, TINY.F, TINY.E, TINY.k, 0, n_layers=2, max_tokens=2)
    try:
        with pytest.raises(MoeGpuError) as ei:
            tier.layer(1, random_x(1, TINY.H, np.random.default_rng(0)))
        assert ei.value.code == ESTATE
    finally:
        tier.close()


def test_synth_fill_matches_host_generator():
    import torch
    tier = MoeGpu(TINY.H, TINY.F, TINY.E, TINY.k, 0, n_layers=1, max_tokens=1)
    try:
        n, key, c = 1 << 16, O.synth_key(9, 1234), synth_c(0.02)
        buf = torch.empty(n, dtype=torch.int16, device="cuda")
        say("synth_fill vs host generator")
        tier.synth_fill(buf, n, key, c, start=4096)
        tier.synchronize()
        got = buf.cpu().numpy().view(np.uint16)
        np.testing.assert_array_equal(got, O.synth_bf16(key, n, c, start=4096))
    finally:
        tier.close()


# ------------------------------------------------------------------------------------------------ another shape
MEDIUM = Workload("medium: H=1536 E=40+2 shared top-6 F=768", 1536, 768, 40, 6, 2, zipf_s=1.1, seed=21)


def test_medium_shape_two_shared_experts():
    """A shape unlike both configs (two shared experts, top-6 of 40, H=1536, F=768, a biased router): routing
    bit-exact, bf16 and int8 (keep 3) outputs within the bars, fused == unfused bit for bit."""
    from moe_gpu import OPT_FUSED
    rng = np.random.default_rng(180)
    say("medium: upload numpy-normal weights H=1536 F=768 E=40+2 k=6")
    hl = random_layer(MEDIUM, rng)  # its router bias: log-Zipf(1.1) ranks, seed 21
    tier = MoeGpu(MEDIUM.H, MEDIUM.F, MEDIUM.E, MEDIUM.k, MEDIUM.n_shared, n_layers=1, max_tokens=8)
    try:
        upload(tier, hl)
        tier.quantize_layer(0)
        for T in (1, 3, 8):
            x = random_x(T, MEDIUM.H, rng)
            for flags, keep in ((0, 0), (INT8, 3)):
                say(f"medium T={T} flags={flags}")
                ref = oracle_layer(hl, x, keep=keep, int8=bool(flags))
                tier.set_option(OPT_FUSED, 1)
                of, idf, gf = tier.layer(0, x, keep=keep, flags=flags)
                tier.set_option(OPT_FUSED, 0)
                ou, idu, _ = tier.layer(0, x, keep=keep, flags=flags)
                check_route(idf, gf, ref, keep or MEDIUM.k)
                np.testing.assert_array_equal(idf, idu)
                np.testing.assert_array_equal(of.view(np.uint32), ou.view(np.uint32))
                assert_layer_close(of, ref["out"])
    finally:
        tier.set_option(OPT_FUSED, 1)
        tier.close()


# ------------------------------------------------------------------------------------------------ Solar (configs 2-4)
@pytest.fixture(scope="module")
def solar():
    say("solar: create tier H=4096 F=1280 E=128+1 k=8, synthesize layer 0 on the device")
    w = SOLAR
    hl = HostLayer(w, layer=0, seed=11)
    tier = MoeGpu(w.H, w.F, w.E, w.k, w.n_shared, n_layers=1, max_tokens=8)
    tier.synth_layer(0, 11, w.sigma_w, hl.bias)
    yield tier, hl
    tier.close()


def test_solar_router_weights_match_host_generator(solar):
    tier, hl = solar
    x = random_x(1, SOLAR.H, np.random.default_rng(20))
    say("solar route logits vs host-regenerated router")
    ids, gates, lg = tier.route(0, x, want_logits=True)
    ref_lg = O.router_logits(x, hl.router())
    np.testing.assert_array_equal(lg.view(np.uint32), ref_lg.view(np.uint32))


def test_solar_layer_batch1(solar):
    tier, hl = solar
    rng = np.random.default_rng(21)
    for trial in range(2):
        x = random_x(1, SOLAR.H, rng)
        say(f"solar layer T=1 trial {trial}")
        out, ids, gates = tier.layer(0, x)
        ref = oracle_layer(hl, x)
        check_route(ids, gates, ref, SOLAR.k)
        r = assert_layer_close(out, ref["out"])
        say(f"  max_abs={r['max_abs']:.3g} rel_l2={r['rel_l2']:.3g}")


@pytest.mark.parametrize("T", [2, 4, 8])
def test_solar_layer_batched(solar, T):
    tier, hl = solar
    w = solar_batch(T)
    x = random_x(T, w.H, np.random.default_rng(30 + T))
    say(f"solar layer T={T}")
    out, ids, gates = tier.layer(0, x)
    ref = oracle_layer(hl, x)
    check_route(ids, gates, ref, w.k)
    assert_layer_close(out, ref["out"])
    # batch invariance: each token alone gives the same bits below 8 tokens; at 8 (the grouped MFMA path) the bars
    for t in (0, T - 1):
        o1, _, _ = tier.layer(0, x[t:t + 1])
        if T < 8:
            np.testing.assert_array_equal(o1[0].view(np.uint32), out[t].view(np.uint32))
        else:
            assert_layer_close(out[t:t + 1], o1)


def test_solar_accumulate_flag(solar):
    """MOE_GPU_ACCUMULATE: out += layer(x), the caller's out is the combine's starting value (ck_* `out[h] +=`)."""
    tier, hl = solar
    rng = np.random.default_rng(40)
    x = random_x(2, SOLAR.H, rng)
    base = rng.normal(0, 1, (2, SOLAR.H)).astype(np.float32)
    say("solar layer accumulate")
    got, _, _ = tier.layer(0, x, flags=ACCUMULATE, out=base.copy())
    ref = oracle_layer(hl, x)
    exp = O.combine(ref["ysh"], ref["yr"], ref["ids"], ref["gates"], ref["keep"], out=base.copy())
    assert_layer_close(got, exp)


def test_solar_int8_quantiser_bitexact(solar):
    tier, hl = solar
    say("solar int8: device quantise layer 0")
    tier.quantize_layer(0)
    for e in (0, 77, 127):
        q, sc = tier.get_expert_q8(0, e)
        q_ref, sc_ref = hl.expert_q8(e)
        np.testing.assert_array_equal(q, q_ref)
        np.testing.assert_array_equal(sc.view(np.uint32), sc_ref.view(np.uint32))


def test_solar_int8_layer_keep4(solar):
    tier, hl = solar
    tier.quantize_layer(0)
    w = SOLAR_INT8
    rng = np.random.default_rng(50)
    for T in (1, 4):
        x = random_x(T, w.H, rng)
        say(f"solar int8 layer keep=4 T={T}")
        out, ids, gates = tier.layer(0, x, keep=4, flags=INT8)
        ref = oracle_layer(hl, x, keep=4, int8=True)
        check_route(ids, gates, ref, 4)
        assert abs(gates[:, :4].sum(axis=1) - 1).max() < 1e-6
        assert_layer_close(out, ref["out"])


def test_solar_int8_q8w_semantics(solar):
    """moe_q8 == ck_moe_q8w (cpu_kern.c:306-333) with the reference's own quantised weights."""
    tier, hl = solar
    tier.quantize_layer(0)
    rng = np.random.default_rng(60)
    x = random_x(1, SOLAR.H, rng)[0]
    ids, w = [9, 100, 31], np.array([0.5, 0.3, 0.2], np.float32)
    got = np.zeros(SOLAR.H, np.float32)
    say("solar moe_q8 vs ck_moe_q8w")
    tier.moe_q8(0, ids, w, x, got)
    exp = np.zeros(SOLAR.H, np.float32)
    qs = [hl.expert_q8(e)[0] for e in ids]; scs = [hl.expert_q8(e)[1] for e in ids]
    O.moe_q8w(qs, scs, w, x, exp, SOLAR.H, SOLAR.F)
    assert_layer_close(got, exp)


def test_solar_q8_upload_roundtrip(solar):
    tier, hl = solar
    q, sc = hl.expert_q8(42)
    say("solar int8 upload round trip")
    tier.place_expert_q8(0, 42, q, sc)
    q2, sc2 = tier.get_expert_q8(0, 42)
    np.testing.assert_array_equal(q2, q)
    np.testing.assert_array_equal(sc2.view(np.uint32), sc.view(np.uint32))


def test_solar_router_matches_reference_build_at_scale(solar):
    """10240 seeded Solar tokens: the GPU's router logits are bit-identical to the reference's own compiled ck_gemv
    (the oracle's restatement where that build cannot run), and the ids equal route() over those logits, for keep 8
    and keep 4."""
    tier, hl = solar
    wr = hl.router()
    n, T = 10240, 8
    rng = np.random.default_rng(2024)
    xs = random_x(n, SOLAR.H, rng)
    if O.ref_available():
        R = O.Ref()
        R.set_threads(16)
        gemv, src = R.gemv, "reference build"
    else:
        gemv, src = O.gemv, "restatement"
    say(f"solar router at scale: {n} tokens against ck_gemv ({src})")
    ref_lg = np.stack([gemv(wr, xs[i]) for i in range(n)])
    for keep in (8, 4):
        mism = 0
        for i in range(0, n, T):
            ids, gates, lg = tier.route(0, xs[i:i + T], keep=keep, want_logits=True)
            if keep == 8:
                np.testing.assert_array_equal(lg.view(np.uint32), ref_lg[i:i + T].view(np.uint32))
            rid, rg = O.route(ref_lg[i:i + T], hl.bias, SOLAR.k, keep)
            mism += int((ids != rid).any(axis=1).sum())
            assert np.all(np.abs(gates[:, :keep] - rg[:, :keep]) <= 1e-6 * np.abs(rg[:, :keep]) + 1e-12)
        say(f"  keep={keep}: {mism} tokens with differing ids")
        assert mism == 0


@pytest.fixture(scope="module")
def solar_sigmoid():
    """Solar layer routed by Solar's own rule (host.rs:119-128): sigmoid scores and a small correction bias."""
    w = SOLAR
    hl = HostLayer(w, layer=0, seed=12)
    hl.bias = np.random.default_rng(77).normal(0.0, 0.05, w.E).astype(np.float32)
    tier = MoeGpu(w.H, w.F, w.E, w.k, w.n_shared, n_layers=1, max_tokens=8)
    say("solar sigmoid: synthesize layer 0 on the device")
    tier.synth_layer(0, 12, w.sigma_w, hl.bias)
    tier.set_option(OPT_ROUTE_RULE, ROUTE_SIGMOID)
    yield tier, hl
    tier.close()


@pytest.mark.parametrize("T", [1, 4])
def test_solar_sigmoid_rule_layer(solar_sigmoid, T):
    tier, hl = solar_sigmoid
    x = random_x(T, SOLAR.H, np.random.default_rng(300 + T))
    say(f"solar sigmoid layer T={T}")
    out, ids, gates = tier.layer(0, x)
    ref = oracle_layer(hl, x, rule="sigmoid")
    np.testing.assert_array_equal(ids, ref["ids"])
    assert np.abs(gates.view(np.int32).astype(np.int64) - ref["gates"].view(np.int32).astype(np.int64)).max() <= 1
    assert_layer_close(out, ref["out"])
    tier.set_option(OPT_FUSED, 0)
    try:
        ou, idu, gu = tier.layer(0, x)
    finally:
        tier.set_option(OPT_FUSED, 1)
    np.testing.assert_array_equal(ou.view(np.uint32), out.view(np.uint32))


def test_solar_sigmoid_route_many_tokens(solar_sigmoid):
    tier, hl = solar_sigmoid
    rng = np.random.default_rng(310)
    say("solar sigmoid route: 512 tokens, ids bit-exact, gates within one ulp")
    exact = total = 0
    for _ in range(64):
        x = random_x(8, SOLAR.H, rng)
        for keep in (8, 4):
            ids, gates, lg = tier.route(0, x, keep=keep, want_logits=True)
            rid, rg = O.route(lg, hl.bias, SOLAR.k, keep, rule="sigmoid")
            np.testing.assert_array_equal(ids, rid)
            # the sigmoid's exp: the GPU rounds a double exp once to fp32, the oracle calls the C library's expf
            # (what the reference's f32::exp calls); both are within about half an ulp, so they differ by one ulp
            # where the exact value lies near a rounding boundary
            d = np.abs(gates.view(np.int32).astype(np.int64) - rg.view(np.int32).astype(np.int64))
            assert d.max() <= 1
            exact += int((d == 0).sum()); total += d.size
    say(f"  gates bit-exact: {exact} / {total}")
    assert exact >= 0.99 * total


def test_solar_block_call_matches_moe_host(solar_sigmoid):
    """moe_gpu_block_dev (residual add + post-attention norm + experts + moe_host's rounding and residual add, one
    launch) against the oracle's moe_host composition (main.rs:120-141), and fused == unfused bit for bit."""
    import torch
    from moe_ref import oracle_moe_block
    tier, hl = solar_sigmoid
    rng = np.random.default_rng(340)
    H = SOLAR.H
    resid = O.f2bf(rng.normal(0, 1, H).astype(np.float32))
    attn_o = O.f2bf(rng.normal(0, 0.3, H).astype(np.float32))
    norm_w = O.f2bf(rng.normal(1, 0.1, H).astype(np.float32))
    dev = torch.device("cuda:0")
    t = lambda a: torch.from_numpy(a.view(np.int16)).to(dev)
    d_resid, d_o, d_w = t(resid), t(attn_o), t(norm_w)
    xn = torch.zeros(H, dtype=torch.int16, device=dev)
    out = torch.zeros(H, dtype=torch.float32, device=dev)
    ids = torch.zeros(SOLAR.k, dtype=torch.int32, device=dev)
    say("solar block call (sigmoid routing)")
    tier.block_dev(0, 1, d_resid, d_o, d_w, xn, out=out, ids=ids)
    tier.synchronize()
    got = xn.cpu().numpy().view(np.uint16)
    exp_x, exp_ids, margin = oracle_moe_block(hl, O.f2bf(O.bf2f(resid) + O.bf2f(attn_o)), norm_w, "sigmoid")
    assert margin > 1e-4
    np.testing.assert_array_equal(ids.cpu().numpy(), exp_ids)
    r = assert_layer_close(O.bf2f(got), O.bf2f(exp_x))
    say(f"  x_next max_abs={r['max_abs']:.3g} rel_l2={r['rel_l2']:.3g}")
    tier.set_option(OPT_FUSED, 0)
    try:
        xu = torch.zeros_like(xn); ou = torch.zeros_like(out)
        tier.block_dev(0, 1, d_resid, d_o, d_w, xu, out=ou)
        tier.synchronize()
    finally:
        tier.set_option(OPT_FUSED, 1)
    np.testing.assert_array_equal(xu.cpu().numpy(), xn.cpu().numpy())
    np.testing.assert_array_equal(ou.cpu().numpy().view(np.uint32), out.cpu().numpy().view(np.uint32))


def test_solar_grid_not_all_resident_and_router_recompute(solar):
    """Units go to running workgroups only: a grid four times what fits at once, and workgroups computing missing
    router rows themselves (router poll 0), give the same bits as the default launch."""
    tier, hl = solar
    for T in (1, 8):
        x = random_x(T, SOLAR.H, np.random.default_rng(320 + T))
        base, bid, bg = tier.layer(0, x)
        fit = tier.get_option(3)  # MOE_GPU_OPT_LAST_GRID
        say(f"solar T={T}: grid {4 * fit} (4x resident), then router poll 0")
        tier.set_option(OPT_GRID, 4 * fit)
        try:
            o4, i4, g4 = tier.layer(0, x)
        finally:
            tier.set_option(OPT_GRID, 0)
        np.testing.assert_array_equal(o4.view(np.uint32), base.view(np.uint32))
        tier.set_option(OPT_ROUTER_POLL, 0)
        try:
            o0, i0, g0 = tier.layer(0, x)
            tier.set_option(OPT_GRID, 4 * fit)
            o5, _, _ = tier.layer(0, x)
        finally:
            tier.set_option(OPT_ROUTER_POLL, 1024)
            tier.set_option(OPT_GRID, 0)
        np.testing.assert_array_equal(i0, bid)
        np.testing.assert_array_equal(o0.view(np.uint32), base.view(np.uint32))
        np.testing.assert_array_equal(o5.view(np.uint32), base.view(np.uint32))


def test_layer_refuses_graph_capture(solar):
    import torch
    tier, hl = solar
    dev = torch.device("cuda:0")
    s = torch.cuda.Stream()
    x = torch.zeros((1, SOLAR.H), dtype=torch.int16, device=dev)
    out = torch.zeros((1, SOLAR.H), dtype=torch.float32, device=dev)
    y = torch.zeros(16, device=dev)
    torch.cuda.synchronize()
    tier.set_stream(s)
    err = None
    g = torch.cuda.CUDAGraph()
    say("layer_dev inside a graph capture")
    try:
        with torch.cuda.graph(g, stream=s):
            try:
                tier.layer_dev(0, 1, x, out)
            except MoeGpuError as e:
                err = e
            y.add_(1.0)
    finally:
        tier.set_stream(None)
    assert err is not None and err.code == ESTATE
    torch.cuda.synchronize()
    o, _, _ = tier.layer(0, random_x(1, SOLAR.H, np.random.default_rng(330)))  # the tier still works
    assert np.isfinite(o).all()


# ------------------------------------------------------------------------------------------------ fused == unfused
@pytest.mark.parametrize("T", [1, 3, 8])
def test_solar_fused_equals_unfused_bitwise(solar, T):
    """The persistent fused kernel and the one-kernel-per-phase path run the same unit functions: identical bits."""
    tier, hl = solar
    x = random_x(T, SOLAR.H, np.random.default_rng(70 + T))
    say(f"solar fused vs unfused T={T}")
    tier.set_option(OPT_FUSED, 1)
    of, idf, gf = tier.layer(0, x)
    tier.set_option(OPT_FUSED, 0)
    ou, idu, gu = tier.layer(0, x)
    tier.set_option(OPT_FUSED, 1)
    np.testing.assert_array_equal(idf, idu)
    np.testing.assert_array_equal(gf.view(np.uint32), gu.view(np.uint32))
    np.testing.assert_array_equal(of.view(np.uint32), ou.view(np.uint32))
    ids = idf.copy()
    ids[:, -1] = -1  # caller-given routing with an empty rank
    mf = tier.moe(0, x, ids, gf)
    tier.set_option(OPT_FUSED, 0)
    mu = tier.moe(0, x, ids, gf)
    tier.set_option(OPT_FUSED, 1)
    np.testing.assert_array_equal(mf.view(np.uint32), mu.view(np.uint32))


def test_solar_fused_int8_equals_unfused_bitwise(solar):
    from moe_gpu import OPT_FUSED
    tier, hl = solar
    tier.quantize_layer(0)
    x = random_x(2, SOLAR.H, np.random.default_rng(80))
    say("solar fused vs unfused int8 keep=4")
    tier.set_option(OPT_FUSED, 1)
    of, _, _ = tier.layer(0, x, keep=4, flags=INT8)
    tier.set_option(OPT_FUSED, 0)
    ou, _, _ = tier.layer(0, x, keep=4, flags=INT8)
    tier.set_option(OPT_FUSED, 1)
    np.testing.assert_array_equal(of.view(np.uint32), ou.view(np.uint32))


def test_fused_repeated_calls_stay_consistent(solar):
    """The fused kernel's counters are cleared by its last workgroup: many back-to-back calls give identical bits."""
    tier, hl = solar
    x = random_x(1, SOLAR.H, np.random.default_rng(90))
    say("solar fused repeated calls")
    first, _, _ = tier.layer(0, x)
    for _ in range(20):
        again, _, _ = tier.layer(0, x)
        np.testing.assert_array_equal(again.view(np.uint32), first.view(np.uint32))


@pytest.mark.parametrize("fused", [1, 0])
def test_solar_routed_only_ck_moe3_semantics(solar, fused):
    """moe_placed on a tier with a shared expert: routed-only sum, accumulated into the caller's out (ck_moe3)."""
    from moe_gpu import OPT_FUSED
    tier, hl = solar
    rng = np.random.default_rng(100 + fused)
    x = random_x(1, SOLAR.H, rng)[0]
    ids, w = [3, 64, 127, 0], np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    out0 = rng.normal(0, 1, SOLAR.H).astype(np.float32)
    got = out0.copy()
    say(f"solar moe_placed fused={fused}")
    tier.set_option(OPT_FUSED, fused)
    try:
        tier.moe_placed(0, ids, w, x, got)
    finally:
        tier.set_option(OPT_FUSED, 1)
    exp = out0.copy()
    bases = [np.concatenate([a.ravel() for a in hl.expert(e)]) for e in ids]
    O.ck_moe3(bases, w, x, exp, SOLAR.H, SOLAR.F)
    assert_layer_close(got, exp)


def test_fused_varied_calls_match_unfused(solar):
    """Back-to-back fused calls with changing T and inputs: every call equals the one-kernel-per-phase path, so no
    workgroup reads stale routing, act or partial outputs from an earlier call."""
    from moe_gpu import OPT_FUSED
    tier, hl = solar
    rng = np.random.default_rng(110)
    xs = [random_x(int(rng.integers(1, 9)), SOLAR.H, rng) for _ in range(12)]
    say("solar fused varied calls")
    tier.set_option(OPT_FUSED, 1)
    fused = [tier.layer(0, x)[0] for x in xs]
    tier.set_option(OPT_FUSED, 0)
    try:
        for x, f in zip(xs, fused):
            u = tier.layer(0, x)[0]
            np.testing.assert_array_equal(f.view(np.uint32), u.view(np.uint32))
    finally:
        tier.set_option(OPT_FUSED, 1)


# ------------------------------------------------------------------------------------------------ K split / queue lag
@pytest.mark.parametrize("kp", [2, 4])
def test_tiny_ksplit_matches_oracle_and_paths(tiny, kp):
    """Split gate|up tiles (K parts reduced in fixed order by the tile's last part): within the bars of the oracle,
    and the fused and one-kernel-per-phase paths give identical bits for the same K split."""
    from moe_gpu import OPT_FUSED, OPT_KSPLIT
    tier, hl = tiny
    rng = np.random.default_rng(120 + kp)
    try:
        for T in (1, 3, 16):
            say(f"tiny K split {kp} T={T}")
            x = random_x(T, TINY.H, rng)
            ref = oracle_layer(hl, x)
            tier.set_option(OPT_KSPLIT, kp)
            tier.set_option(OPT_FUSED, 1)
            of, idf, gf = tier.layer(0, x)
            tier.set_option(OPT_FUSED, 0)
            ou, idu, gu = tier.layer(0, x)
            check_route(idf, gf, ref, TINY.k)
            np.testing.assert_array_equal(idf, idu)
            np.testing.assert_array_equal(of.view(np.uint32), ou.view(np.uint32))
            r = assert_layer_close(of, ref["out"])
            assert r["rel_l2"] < 1e-4, r
    finally:
        tier.set_option(OPT_FUSED, 1)
        tier.set_option(OPT_KSPLIT, 0)


def test_solar_queue_lag_does_not_change_bits(solar):
    """The fused queue order (lag of down blocks) only reorders work: identical bits for every lag and grid size."""
    from moe_gpu import OPT_LAG, OPT_SHARED_WAITS, OPT_WG_PER_CU
    tier, hl = solar
    x = random_x(3, SOLAR.H, np.random.default_rng(130))
    say("solar queue lag / grid / shared-wait sweep T=3")
    base, _, _ = tier.layer(0, x)
    try:
        for lag in (1, 3, 7, 40):
            for wg in (1, 2):
                tier.set_option(OPT_LAG, lag)
                tier.set_option(OPT_WG_PER_CU, wg)
                tier.set_option(OPT_SHARED_WAITS, (lag + wg) % 2)
                o, _, _ = tier.layer(0, x)
                np.testing.assert_array_equal(o.view(np.uint32), base.view(np.uint32))
    finally:
        tier.set_option(OPT_LAG, 0)
        tier.set_option(OPT_WG_PER_CU, 1)
        tier.set_option(OPT_SHARED_WAITS, 0)


@pytest.mark.parametrize("kp", [1, 4])
def test_solar_ksplit_within_bars(solar, kp):
    """Solar layer with other K splits than the automatic one (2 parts at H=4096): same ids, outputs within bars."""
    from moe_gpu import OPT_KSPLIT
    tier, hl = solar
    x = random_x(1, SOLAR.H, np.random.default_rng(140 + kp))
    say(f"solar K split {kp}")
    ref = oracle_layer(hl, x)
    try:
        tier.set_option(OPT_KSPLIT, kp)
        out, ids, gates = tier.layer(0, x)
    finally:
        tier.set_option(OPT_KSPLIT, 0)
    check_route(ids, gates, ref, SOLAR.k)
    assert_layer_close(out, ref["out"])


@pytest.mark.parametrize("kp,kps", [(1, 2), (2, 1), (1, 4), (4, 1)])
def test_solar_shared_ksplit_paths_and_bars(solar, kp, kps):
    """The shared expert's gate|up K split set apart from the routed experts' (as an int8 call does: int8 routed
    parts at kp 1, the bf16 shared expert at 2): fused and unfused give identical bits, bf16 and int8 outputs stay
    within the bars of the oracle."""
    from moe_gpu import OPT_FUSED, OPT_KSPLIT, OPT_KSPLIT_SHARED
    tier, hl = solar
    tier.quantize_layer(0)
    x = random_x(2, SOLAR.H, np.random.default_rng(160 + 10 * kp + kps))
    try:
        tier.set_option(OPT_KSPLIT, kp)
        tier.set_option(OPT_KSPLIT_SHARED, kps)
        for flags, keep in ((0, 0), (INT8, 4)):
            say(f"solar K split {kp} / shared {kps}, flags {flags}")
            ref = oracle_layer(hl, x, keep=keep, int8=bool(flags))
            tier.set_option(OPT_FUSED, 1)
            of, idf, gf = tier.layer(0, x, keep=keep, flags=flags)
            tier.set_option(OPT_FUSED, 0)
            ou, idu, _ = tier.layer(0, x, keep=keep, flags=flags)
            np.testing.assert_array_equal(idf, idu)
            np.testing.assert_array_equal(of.view(np.uint32), ou.view(np.uint32))
            assert_layer_close(of, ref["out"])
    finally:
        tier.set_option(OPT_FUSED, 1)
        tier.set_option(OPT_KSPLIT, 0)
        tier.set_option(OPT_KSPLIT_SHARED, 0)


def test_solar_unit_trace(solar):
    """The fused kernel's unit trace: one record per unit of the work list, stamps in order within each unit (router
    units: operands in, then dot products done; down units: act staged, then stream done; the tile's combining unit:
    other terms in after its stream), and tracing
    leaves the output bits unchanged."""
    from moe_gpu import OPT_LAST_GRID
    tier, hl = solar
    x = random_x(1, SOLAR.H, np.random.default_rng(170))
    say("solar unit trace T=1")
    base, _, _ = tier.layer(0, x)
    try:
        tier.trace_units(True)
        out, _, _ = tier.layer(0, x)
        tr = tier.read_trace().astype(np.int64)
        grid = tier.get_option(OPT_LAST_GRID)
    finally:
        tier.trace_units(False)
    np.testing.assert_array_equal(out.view(np.uint32), base.view(np.uint32))
    nR, maxs, S, nht, ntile = (SOLAR.E + 7) // 8, SOLAR.n_shared + SOLAR.k, SOLAR.n_shared, SOLAR.H // 64, SOLAR.F // 32
    kp, kps = 1, 4  # automatic K parts at H = 4096 in a bf16 call: routed, shared
    assert tr.shape == (nR + 1 + S * ntile * kps + (maxs - S) * ntile * kp + maxs * nht, 6)
    start, ready, end, wg, aux, aux2 = tr.T
    assert np.all(start > 0) and np.all(end >= start)
    assert np.all((wg >= 0) & (wg < grid))
    router = np.arange(len(tr)) < nR
    assert np.all(start[router] <= aux[router]) and np.all(aux[router] <= aux2[router])
    assert np.all(aux2[router] <= end[router])
    down = (aux2 > 0) & ~router
    assert down.sum() == maxs * nht
    assert np.all(start[down] <= aux[down]) and np.all(aux[down] <= aux2[down]) and np.all(aux2[down] <= end[down])
    comb = down & (ready > 0)
    assert comb.sum() == nht  # one combining unit per output tile (folded at T=1)
    assert np.all(aux2[comb] <= ready[comb]) and np.all(ready[comb] <= end[comb])


def test_fused_calls_interleaved_with_route_calls(solar):
    """Route-only calls between fused layer calls (they take call tags but run no fused kernel) must not disturb the
    fused kernel's work queue: every layer call gives the first call's bits."""
    tier, hl = solar
    x = random_x(1, SOLAR.H, np.random.default_rng(150))
    say("solar fused calls interleaved with route calls")
    first, ids0, _ = tier.layer(0, x)
    for pattern in ("r", "rr", "", "r", "rrr", ""):
        for _ in pattern:
            ids, _ = tier.route(0, x)
            np.testing.assert_array_equal(ids, ids0)
        again, _, _ = tier.layer(0, x)
        np.testing.assert_array_equal(again.view(np.uint32), first.view(np.uint32))
