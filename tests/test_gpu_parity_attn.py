"""GPU parity of decode attention (moe_attn_decode_dev through the C ABI) against the oracle's restatement of
main.rs:86-104.

Bars:
  * scores: bit-identical (the GPU sums each q . k left to right in fp32, as the reference);
  * out (bf16): |gpu - ref| <= 2^-7 |ref| + 1e-3 max|ref| and rel-L2 <= 5e-3.  The softmax total and the P.V sums
    run in the GPU's order, so a probability or an output can land on the other side of a bf16 rounding boundary;
  * a one-hot softmax (exact in any order) gives out = v[t*] bit for bit, per kv head of the group mapping.
"""
import numpy as np
import pytest

import oracle as O
from moe_gpu import (EINVAL, MoeGpuError, attn_decode_dev, attn_decode_oproj_dev, attn_scores, attn_workspace_bytes,
                     gemv_dev)

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-attn] {msg}", flush=True)


def run_gpu(q, k, v, NKV, S=None):
    import torch

    NQ = q.shape[0]
    S = k.shape[0] if S is None else S
    dev = "cuda:0"
    qd = torch.from_numpy(q.view(np.int16)).to(dev)
    kd = torch.from_numpy(k.view(np.int16)).to(dev)
    vd = torch.from_numpy(v.view(np.int16)).to(dev)
    od = torch.zeros((NQ, 128), dtype=torch.int16, device=dev)
    ws = torch.zeros(attn_workspace_bytes(NQ, S) // 4, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    attn_decode_dev(qd, kd, vd, od, ws, NQ, NKV, S)  # null stream: ordered after torch's copies
    torch.cuda.synchronize()
    return od.cpu().numpy().view(np.uint16), attn_scores(ws, NQ, S).cpu().numpy()


def check_out(gpu, ref):
    g, r = O.bf2f(gpu).astype(np.float64), O.bf2f(ref).astype(np.float64)
    assert np.all(np.abs(g - r) <= 2.0 ** -7 * np.abs(r) + 1e-3 * np.abs(r).max()), np.abs(g - r).max()
    assert np.linalg.norm(g - r) <= 5e-3 * np.linalg.norm(r)


@pytest.mark.parametrize("NQ,NKV,S", [(32, 8, 4096), (32, 8, 1), (32, 8, 37), (32, 8, 300), (4, 4, 777), (16, 2, 513),
                                      (32, 8, 5000), (16, 2, 9000)])
def test_attention_matches_oracle(NQ, NKV, S):
    say(f"attention NQ={NQ} NKV={NKV} S={S}")
    rng = np.random.default_rng(S + NQ)
    q = O.f2bf(rng.standard_normal((NQ, 128)).astype(np.float32))
    k = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    v = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    ref, sc = O.attention(q, k, v, NKV)
    out, gsc = run_gpu(q, k, v, NKV)
    np.testing.assert_array_equal(gsc.view(np.uint32), sc.view(np.uint32))
    check_out(out, ref)


@pytest.mark.parametrize("NQ,NKV,S", [(32, 8, 4096), (16, 2, 1000), (8, 8, 300)])
def test_attention_fallback_paths_same_bits(NQ, NKV, S, monkeypatch):
    """MOE_ATTN_POLL=0 ends every wait for another workgroup's words at once, so workgroups compute missing chunk
    statistics and partials themselves: the output and scores must not change by a bit."""
    say(f"attention fallback NQ={NQ} NKV={NKV} S={S}")
    rng = np.random.default_rng(S + 11)
    q = O.f2bf(rng.standard_normal((NQ, 128)).astype(np.float32))
    k = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    v = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    out, sc = run_gpu(q, k, v, NKV)
    monkeypatch.setenv("MOE_ATTN_POLL", "0")
    out0, sc0 = run_gpu(q, k, v, NKV)
    monkeypatch.delenv("MOE_ATTN_POLL")
    np.testing.assert_array_equal(out0, out)
    np.testing.assert_array_equal(sc0.view(np.uint32), sc.view(np.uint32))


def test_attention_longest_context():
    """S = 65536 (the maximum): more workgroups than fit on the chip at once, so each takes several chunks."""
    NQ, NKV, S = 32, 8, 65536
    say(f"attention NQ={NQ} NKV={NKV} S={S}")
    rng = np.random.default_rng(9)
    q = O.f2bf(rng.standard_normal((NQ, 128)).astype(np.float32))
    k = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    v = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    ref, sc = O.attention(q, k, v, NKV)
    out, gsc = run_gpu(q, k, v, NKV)
    np.testing.assert_array_equal(gsc.view(np.uint32), sc.view(np.uint32))
    check_out(out, ref)


def test_attention_graph_replays():
    """One call captured in a HIP graph and replayed with new q, eager calls on the same workspace in between: the
    epochs live in the workspace, so every replay and every eager call gets a fresh one and the same bits."""
    import torch

    NQ, NKV, S = 32, 8, 1000
    say(f"attention graph replays NQ={NQ} NKV={NKV} S={S}")
    dev = "cuda:0"
    rng = np.random.default_rng(21)
    k = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    v = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    kd = torch.from_numpy(k.view(np.int16)).to(dev)
    vd = torch.from_numpy(v.view(np.int16)).to(dev)
    qd = torch.zeros((NQ, 128), dtype=torch.int16, device=dev)
    od = torch.zeros((NQ, 128), dtype=torch.int16, device=dev)
    oe = torch.zeros((NQ, 128), dtype=torch.int16, device=dev)
    ws = torch.zeros(attn_workspace_bytes(NQ, S) // 4, dtype=torch.float32, device=dev)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    attn_decode_dev(qd, kd, vd, od, ws, NQ, NKV, S, stream=s)  # first call on the workspace: outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        attn_decode_dev(qd, kd, vd, od, ws, NQ, NKV, S, stream=s)
    torch.cuda.synchronize()
    for r in range(4):
        q = O.f2bf(rng.standard_normal((NQ, 128)).astype(np.float32))
        qd.copy_(torch.from_numpy(q.view(np.int16)).to(dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = od.cpu().numpy().view(np.uint16).copy()
        attn_decode_dev(qd, kd, vd, oe, ws, NQ, NKV, S, stream=s)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got, oe.cpu().numpy().view(np.uint16))
        ref, _ = O.attention(q, k, v, NKV)
        check_out(got, ref)


def test_attention_one_hot_exact():
    say("attention one-hot")
    rng = np.random.default_rng(3)
    NQ, NKV, S = 32, 8, 600
    q = np.zeros((NQ, 128), np.uint16)
    q[:, 0] = O.f2bf(np.array([1.0], np.float32))[0]
    k = O.f2bf((0.01 * rng.standard_normal((S, NKV, 128))).astype(np.float32))
    v = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    star = [0, 255, 256, 599, 300, 1, 511, 512]  # chunk edges
    for g, t in enumerate(star):
        k[t, g, 0] = O.f2bf(np.array([2000.0], np.float32))[0]
    out, _ = run_gpu(q, k, v, NKV)
    for h in range(NQ):
        np.testing.assert_array_equal(out[h], v[star[h // 4], h // 4])


def test_attention_errors():
    import torch

    ws = torch.zeros(1024, dtype=torch.float32, device="cuda:0")
    x = torch.zeros(4096, dtype=torch.int16, device="cuda:0")
    for args in ((32, 8, 64, 16), (32, 5, 128, 16), (32, 2, 128, 16), (32, 8, 128, 0), (32, 8, 128, 4096), (32, 8, 128, 65537)):
        NQ, NKV, D, S = args
        with pytest.raises(MoeGpuError) as e:
            attn_decode_dev(x, x, x, x, ws, NQ, NKV, S, head_dim=D)
        assert e.value.code == EINVAL


@pytest.mark.parametrize("NQ,NKV,S,M", [(32, 8, 4096, 4096), (32, 8, 1, 4096), (32, 8, 300, 4096), (32, 4, 777, 4096),
                                        (32, 16, 513, 4096), (32, 8, 9000, 4096), (32, 8, 1000, 1000)])
def test_attention_oproj_matches_two_launches(NQ, NKV, S, M, monkeypatch):
    """The o projection folded into the attention launch (moe_attn_decode_oproj_dev) against attention then the
    dense GEMV (moe_attn_decode_dev + moe_gemv_dev) on the same inputs: out and o bit for bit, also with every wait
    ended at once (MOE_ATTN_POLL=0: the attention outputs recomputed by each workgroup)."""
    import torch

    say(f"attention + o projection NQ={NQ} NKV={NKV} S={S} M={M}")
    dev = "cuda:0"
    rng = np.random.default_rng(S + NKV + M)
    q = O.f2bf(rng.standard_normal((NQ, 128)).astype(np.float32))
    k = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    v = O.f2bf(rng.standard_normal((S, NKV, 128)).astype(np.float32))
    wo = O.f2bf((0.02 * rng.standard_normal((M, NQ * 128))).astype(np.float32))
    qd, kd, vd, wod = (torch.from_numpy(a.view(np.int16)).to(dev) for a in (q, k, v, wo))
    ws = torch.zeros(attn_workspace_bytes(NQ, S) // 4, dtype=torch.float32, device=dev)
    a1 = torch.zeros((NQ, 128), dtype=torch.int16, device=dev)
    o1 = torch.zeros(M, dtype=torch.int16, device=dev)
    torch.cuda.synchronize()
    attn_decode_dev(qd, kd, vd, a1, ws, NQ, NKV, S)
    gemv_dev(wod, a1.view(-1), o1)
    torch.cuda.synchronize()
    for poll in (None, "0"):
        if poll is not None:
            monkeypatch.setenv("MOE_ATTN_POLL", poll)
        a2 = torch.zeros((NQ, 128), dtype=torch.int16, device=dev)
        o2 = torch.zeros(M, dtype=torch.int16, device=dev)
        for _ in range(2):  # twice: the second call's epoch differs, no stale words are taken
            attn_decode_oproj_dev(qd, kd, vd, a2, wod, o2, ws, NQ, NKV, S)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(a2.cpu().numpy(), a1.cpu().numpy())
        np.testing.assert_array_equal(o2.cpu().numpy(), o1.cpu().numpy())
    monkeypatch.delenv("MOE_ATTN_POLL")
    ref, _ = O.attention(q, k, v, NKV)
    check_out(a1.cpu().numpy().view(np.uint16), ref)


def test_attention_oproj_errors():
    import torch

    dev = "cuda:0"
    NQ, NKV, S = 16, 4, 64  # NQ * 128 = 2048: the folded projection needs 4096 columns
    q = torch.zeros((NQ, 128), dtype=torch.int16, device=dev)
    k = torch.zeros((S, NKV, 128), dtype=torch.int16, device=dev)
    ws = torch.zeros(attn_workspace_bytes(NQ, S) // 4, dtype=torch.float32, device=dev)
    wo = torch.zeros((4096, NQ * 128), dtype=torch.int16, device=dev)
    o = torch.zeros(4096, dtype=torch.int16, device=dev)
    with pytest.raises(MoeGpuError) as ei:
        attn_decode_oproj_dev(q, k, k, q, wo, o, ws, NQ, NKV, S)
    assert ei.value.code == EINVAL
