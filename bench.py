"""Benchmark of the routed-MoE layer on one MI355X.

A step is one MoE layer call (router GEMV + softmax top-k, grouped SwiGLU experts incl. the shared expert, gated
combine) over one batch of T decode tokens whose activations are already resident in HBM.  Expert tables of
`--layers` distinct layers are resident and the steps rotate over them, so the working set (4 GB per Solar layer)
is far larger than the 256 MB Infinity Cache and every step streams its experts from HBM.

Prints one JSON line.  value = microseconds per MoE layer per token (lower is better); the line also carries the
achieved HBM bandwidth (algorithmic bytes / time) as a fraction of the 8 TB/s peak, the dominant kernel's roofline
figure measured with hipEvents on the stream it runs on, and the reference CPU path timed on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "npu-offload_amd"))

from moe_gpu import INT8, MoeGpu, synth_c, synth_key  # noqa: E402
from moe_gpu.workloads import SOLAR, SOLAR_INT8, TINY, Workload, solar_batch, zipf_bias  # noqa: E402

METRIC = "MoE layer µs/token + achieved HBM TB/s (fraction of ~8 TB/s), bf16 batch 1"
HBM_PEAK_GBPS = 8000.0
WORKLOADS = {"solar": SOLAR, "solar-int8": SOLAR_INT8, "solar-b2": solar_batch(2), "solar-b4": solar_batch(4),
             "solar-b8": solar_batch(8), "tiny": TINY}


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(w: Workload, budget_s: float = 12.0) -> dict | None:
    """The reference's CPU expert path timed on this host: ck_gemv router + host route + ck_moe3 over the shared
    expert and the routed experts (track2_opt/solar_engine/src/main.rs:128-141 `moe_host`), built from the
    reference's own cpu_kern.c; falls back to the scalar restatement when AVX-512 BF16 is unavailable."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    H, F, E, k = w.H, w.F, w.E, w.k
    cores = len(os.sched_getaffinity(0))
    cores = int(os.environ.get("OMP_NUM_THREADS", cores))
    ne = 48  # expert pool rotated beyond the LLC, as track2_opt/solar_engine/src/bin/cpu_bench.rs:15-31
    n = F * H
    src = O.f2bf((np.arange(3 * n) % 97).astype(np.float32) * 1e-4)
    g, u, d = src[:n].reshape(F, H), src[n:2 * n].reshape(F, H), src[2 * n:].reshape(H, F)
    x = O.f2bf((np.arange(H) % 13).astype(np.float32) * 0.01)
    wr = O.f2bf(np.random.default_rng(0).normal(0, 0.02, (E, H)).astype(np.float32))
    bias = zipf_bias(E, w.zipf_s, 0)
    kind = "reference" if O.ref_available() else "port"
    if kind == "reference":
        R = O.Ref()
        R.set_threads(cores)
        pool = [R.place_expert(g, u, d) for _ in range(ne)]
        gemv, moe3 = R.gemv, R.moe3
    else:
        cores = 1
        pool = [np.concatenate([g.ravel(), u.ravel(), d.ravel()]) for _ in range(4)]
        ne = len(pool)
        gemv = O.gemv
        moe3 = O.ck_moe3
    keep = w.keep_eff
    ts = []
    t_end = time.perf_counter() + budget_s
    it = 0
    while (it < 60 or time.perf_counter() < t_end) and it < 5000:
        bases = [pool[(it * (keep + w.n_shared) + j) % ne] for j in range(keep + w.n_shared)]
        t0 = time.perf_counter()
        lg = gemv(wr, x)
        ids, gates = O.route(lg, bias, k, keep)
        out = np.zeros(H, np.float32)
        if w.n_shared:
            moe3(bases[keep:], np.ones(w.n_shared, np.float32), x, out, H, F)
        moe3(bases[:keep], gates[0, :keep], x, out, H, F)
        dt = time.perf_counter() - t0
        if it >= 10:
            ts.append(dt)
        it += 1
        if kind == "port" and it >= 3:
            ts.append(dt)
            break
    med = statistics.median(ts)
    nbytes = w.router_bytes() + (keep + w.n_shared) * 3 * F * H * 2
    return {"value": round(med * 1e6, 1), "unit": "us/layer/token", "cores": cores, "kind": kind,
            "GBps": round(nbytes / med / 1e9, 1),
            "sample": f"{len(ts)} batch-1 layer calls (bf16, {keep} routed + {w.n_shared} shared experts from a "
                      f"{ne}-expert pool + router GEMV/top-k), median; {'cpu_kern.c ck_gemv+ck_moe3' if kind == 'reference' else 'scalar restatement'}"}


def cpu_baseline_batched(w: Workload, budget_s: float = 12.0) -> dict | None:
    """The reference's batched CPU path for T > 1 tokens timed on this host: per token ck_gemv router (the reference's
    own cpu_kern.c build) + host route, the tokens grouped by expert in first-seen order (runtime.py:344-347), then
    cpu_moe (solar_hybrid/cpu_moe.cpp:38-96) over the shared expert and the grouped routed experts, each weight row
    streamed once per call for all its tokens.  cpu_moe runs as the oracle's AVX-512 BF16 + OpenMP port of
    cpu_moe.cpp (its torch-extension build is not made here).  Needs an AVX-512 BF16 host."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    if not O.ref_available():
        return None
    H, F, E, k, T = w.H, w.F, w.E, w.k, w.T
    cores = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    R = O.Ref()
    R.set_threads(cores)
    ne = 48  # distinct expert weight sets rotated beyond the LLC (about 1.5 GB)
    rng = np.random.default_rng(0)
    base = O.f2bf((rng.normal(0, 0.02, 3 * F * H)).astype(np.float32))
    pool = []
    for i in range(ne):
        b = np.roll(base, i * 4099)
        pool.append((np.ascontiguousarray(b[:2 * F * H].reshape(2 * F, H)),
                     np.ascontiguousarray(b[2 * F * H:].reshape(H, F))))
    wr = O.f2bf(rng.normal(0, 0.02, (E, H)).astype(np.float32))
    bias = zipf_bias(E, w.zipf_s, 0)
    keep = w.keep_eff
    ts, distinct = [], []
    t_end = time.perf_counter() + budget_s
    it = 0
    while (it < 12 or time.perf_counter() < t_end) and it < 400:
        x = O.f2bf(rng.normal(0, 1, (T, H)).astype(np.float32))
        t0 = time.perf_counter()
        lg = np.stack([R.gemv(wr, x[t]) for t in range(T)])
        ids, gates = O.route(lg, bias, k, keep)
        groups = O.group_tokens(ids, gates, keep)
        gus, ds, toks, ws = [], [], [], []
        for s in range(w.n_shared):  # the shared expert: every token, weight 1
            g, d = pool[(it * 37 + s) % ne]
            gus.append(g); ds.append(d); toks.append(np.arange(T, dtype=np.int64)); ws.append(np.ones(T, np.float32))
        for j, (e, tk, wt) in enumerate(groups):
            g, d = pool[(it * 37 + w.n_shared + j) % ne]
            gus.append(g); ds.append(d); toks.append(tk); ws.append(wt)
        O.cpu_moe_port(x, gus, ds, toks, ws)
        dt = time.perf_counter() - t0
        if it >= 2:
            ts.append(dt)
            distinct.append(len(groups))
        it += 1
    med = statistics.median(ts)
    nbytes = w.router_bytes() + (float(np.mean(distinct)) + w.n_shared) * 3 * F * H * 2
    return {"value": round(med * 1e6 / T, 1), "unit": "us/layer/token", "cores": cores, "kind": "port",
            "GBps": round(nbytes / med / 1e9, 1), "us_per_call": round(med * 1e6, 1),
            "sample": f"{len(ts)} calls of {T} tokens: ck_gemv router per token (cpu_kern.c build) + host route + "
                      f"first-seen grouping + cpu_moe (cpu_moe.cpp:38-96, the oracle's AVX-512 BF16/OpenMP port) over "
                      f"the shared expert and {np.mean(distinct):.1f} distinct routed experts from a {ne}-set pool, "
                      f"median"}


LM_HEAD_H, LM_HEAD_V = 4096, 196608
LM_HEAD_METRIC = "LM head (final RMSNorm + GEMV over V=196608 + greedy argmax) µs/token + achieved HBM TB/s, bf16 batch 1"


def cpu_baseline_lm_head(budget_s: float = 10.0) -> dict | None:
    """The reference host step's tail timed on this host: rmsnorm (host.rs:71-76, restated) + ck_gemv over the
    [196608, 4096] table (cpu_kern.c:32, the reference's own build) + the first-maximum loop (main.rs:384-385)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    if not O.ref_available():
        return None
    H, V = LM_HEAD_H, LM_HEAD_V
    cores = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    R = O.Ref()
    R.set_threads(cores)
    blk = O.f2bf(np.random.default_rng(0).normal(0, 0.02, (64, H)).astype(np.float32))
    W = np.empty((V, H), np.uint16)
    for r in range(0, V, 64):
        W[r:r + 64] = blk
    wf = O.f2bf(np.ones(H, np.float32))
    x = O.f2bf(np.random.default_rng(1).normal(0, 1, H).astype(np.float32))
    ts = []
    t_end = time.perf_counter() + budget_s
    while (len(ts) < 5 or time.perf_counter() < t_end) and len(ts) < 200:
        t0 = time.perf_counter()
        hn = O.rmsnorm(x, wf)
        lg = R.gemv(W, hn)
        int(np.argmax(lg))
        ts.append(time.perf_counter() - t0)
    med = statistics.median(ts[1:])
    return {"value": round(med * 1e6, 1), "unit": "us/token", "cores": cores, "kind": "reference",
            "GBps": round(V * H * 2 / med / 1e9, 1),
            "sample": f"{len(ts) - 1} decode-step tails (rmsnorm + cpu_kern.c ck_gemv over the 1.61 GB table + "
                      f"argmax), median"}


def bench_lm_head(args) -> None:
    """The step's tail on the GPU: moe_head_argmax_dev on one token, the 1.61 GB table resident in HBM (no layer
    rotation is needed: the table is six times the size of the Infinity Cache)."""
    import torch

    from moe_gpu import LmHead

    H, V, K, W_ = LM_HEAD_H, LM_HEAD_V, args.steps, args.warmup
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    log("lm-head: draw the table on the device")
    g = torch.Generator(device=dev).manual_seed(0)
    Wt = (torch.randn(V, H, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    wf = (1 + 0.1 * torch.randn(H, device=dev, generator=g)).to(torch.bfloat16)
    P = 16
    xs = torch.randn(P, H, device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
    ids = torch.zeros(K + W_, dtype=torch.int32, device=dev)
    best = torch.zeros(K + W_, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    head = LmHead(H, V)
    head.load_dev(Wt.view(torch.int16), wf.view(torch.int16))
    del Wt
    torch.cuda.empty_cache()
    head.set_stream(stream)
    log(f"warmup {W_} steps")
    for i in range(W_):
        head.argmax_dev(1, xs[i % P], ids[i:i + 1], best[i:i + 1])
    torch.cuda.synchronize()
    log(f"timing {K} steps")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(K):
        head.argmax_dev(1, xs[i % P], ids[W_ + i:W_ + i + 1], best[W_ + i:W_ + i + 1])
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ev_ms = e0.elapsed_time(e1)
    nbytes = V * H * 2
    ev_us = ev_ms / K * 1e3
    achieved = nbytes / (ev_us * 1e-6) / 1e9
    if args.copy_calibration > 0:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        log(f"copy calibration: 5 x {args.copy_calibration} MiB")
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    cpu = None if args.no_cpu_baseline else cpu_baseline_lm_head()
    traffic = measured_traffic("head_kernel", "lm-head")
    line = {
        "metric": LM_HEAD_METRIC, "value": round(wall_ms * 1e3 / K, 2), "unit": "us/token", "n_gpus": 1, "steps": K,
        "warmup": W_, "ms_per_step": round(wall_ms / K, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded, weights ~N(0,0.02), x ~N(0,1))",
        "event_ms_per_step": round(ev_ms / K, 5),
        "config": {"workload": "lm-head: final RMSNorm + LM head H=4096 V=196608 + argmax, bf16, batch 1",
                   "H": H, "V": V, "tokens": 1},
        "roofline": {"kernel": "head_kernel", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "bytes_per_launch": nbytes, "avg_us": round(ev_us, 2),
                     "timing": "timed-region hipEvents on the head's stream; each step is head_kernel + a one-wave "
                               "finish kernel, so achieved slightly understates the GEMV kernel's own rate"},
        "cpu_baseline": cpu,
    }
    head.close()
    print(json.dumps(line), flush=True)


ATTN_NQ, ATTN_NKV, ATTN_D, ATTN_S = 32, 8, 128, 4096
ATTN_METRIC = "decode attention (GQA 32 q / 8 kv heads, d=128, KV 4096) µs/layer/token + achieved HBM TB/s, bf16 batch 1"


def bench_attn(args) -> None:
    """Decode attention of one token over a layer's KV cache (S = 4096), rotating over 32 distinct caches
    (537 MB, beyond the Infinity Cache)."""
    import torch

    from moe_gpu import attn_decode_dev, attn_workspace_bytes

    NQ, NKV, D, S, K, W_ = ATTN_NQ, ATTN_NKV, ATTN_D, ATTN_S, args.steps, args.warmup
    L = 32
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    g = torch.Generator(device=dev).manual_seed(0)
    log(f"attn: {L} caches of 2 x [{S}, {NKV}, {D}] bf16")
    kc = torch.randn(L, S, NKV, D, device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
    vc = torch.randn(L, S, NKV, D, device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
    qs = torch.randn(L, NQ, D, device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
    out = torch.zeros(NQ, D, dtype=torch.int16, device=dev)
    ws = torch.zeros(attn_workspace_bytes(NQ, S) // 4, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    for i in range(W_):
        attn_decode_dev(qs[i % L], kc[i % L], vc[i % L], out, ws, NQ, NKV, S, stream=stream)
    torch.cuda.synchronize()
    log(f"timing {K} steps")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(K):
        attn_decode_dev(qs[i % L], kc[i % L], vc[i % L], out, ws, NQ, NKV, S, stream=stream)
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ev_us = e0.elapsed_time(e1) / K * 1e3
    nbytes = 2 * S * NKV * D * 2
    achieved = nbytes / (ev_us * 1e-6) / 1e9
    if args.copy_calibration > 0:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        log(f"copy calibration: 5 x {args.copy_calibration} MiB")
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O

        qh, kh, vh = (t[0].cpu().numpy().view(np.uint16) for t in (qs, kc, vc))
        ts = []
        for _ in range(5):
            c0 = time.perf_counter()
            O.attention(qh, kh, vh, NKV)
            ts.append(time.perf_counter() - c0)
        med = statistics.median(ts)
        cpu = {"value": round(med * 1e6, 1), "unit": "us/layer/token", "cores": 1, "kind": "port",
               "GBps": round(nbytes / med / 1e9, 2),
               "sample": "5 calls of the oracle's numpy restatement of main.rs:86-104 (the reference's Rust host "
                         "attention cannot be built here), median"}
    line = {
        "metric": ATTN_METRIC, "value": round(wall_ms * 1e3 / K, 2), "unit": "us/layer/token", "n_gpus": 1,
        "steps": K, "warmup": W_, "ms_per_step": round(wall_ms / K, 5), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded, q/k/v ~N(0,1))",
        "event_ms_per_step": round(ev_us / 1e3, 5),
        "config": {"workload": "attn: GQA decode attention, 32 q / 8 kv heads, d=128, KV 4096, bf16, batch 1",
                   "n_q_heads": NQ, "n_kv_heads": NKV, "head_dim": D, "kv_len": S, "tokens": 1},
        "roofline": {"kernel": "attn_fused_kernel", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic("attn_fused_kernel", "attn"), "bytes_per_launch": nbytes,
                     "avg_us": round(ev_us, 2),
                     "timing": "timed-region hipEvents on the call's stream (one kernel per call)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_proj(args) -> None:
    """The attention block's projections of one token (q 4096 x 4096, k and v 1024 x 4096, o 4096 x 4096: 83.9 MB of
    bf16 weights per layer, main.rs:109-111 and :119), rotating over 8 layers (671 MB)."""
    import torch

    from moe_gpu import gemv_dev

    H, QD, KVD, L, K, W_ = 4096, 4096, 1024, 8, args.steps, args.warmup
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    g = torch.Generator(device=dev).manual_seed(0)
    log(f"proj: {L} layers of q/k/v/o weights")
    # q, k and v read the same input: the engine places them as one [QD + 2 KVD, H] table, one launch
    fused = not args.proj_separate
    shapes = [(QD + 2 * KVD, H), (H, QD)] if fused else [(QD, H), (KVD, H), (KVD, H), (H, QD)]
    ws = [[(torch.randn(m, k, device=dev, generator=g) * 0.02).to(torch.bfloat16).view(torch.int16) for m, k in shapes]
          for _ in range(L)]
    h = torch.randn(H, device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
    a_in = torch.randn(QD, device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
    outs = [torch.zeros(m, dtype=torch.int16, device=dev) for m, _ in shapes]
    torch.cuda.synchronize()

    def step(i):
        wl = ws[i % L]
        for j in range(len(shapes) - 1):
            gemv_dev(wl[j], h, outs[j], stream=stream)
        gemv_dev(wl[-1], a_in, outs[-1], stream=stream)

    for i in range(W_):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(K):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ev_us = e0.elapsed_time(e1) / K * 1e3
    nbytes = sum(m * k for m, k in shapes) * 2
    achieved = nbytes / (ev_us * 1e-6) / 1e9
    line = {
        "metric": "attention-block projections (q/k/v/o GEMV, H=4096, 32 q / 8 kv heads) µs/layer/token + achieved "
                  "HBM TB/s, bf16 batch 1",
        "value": round(wall_ms * 1e3 / K, 2), "unit": "us/layer/token", "n_gpus": 1, "steps": K, "warmup": W_,
        "ms_per_step": round(wall_ms / K, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded, weights ~N(0,0.02))", "event_ms_per_step": round(ev_us / 1e3, 5),
        "config": {"workload": "proj: q/k/v/o projections of one token, H=4096, QD=4096, KVD=1024, bf16", "tokens": 1,
                   "qkv_one_table": fused},
        "roofline": {"kernel": f"gemv_kernel x {len(shapes)}", "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_launch": nbytes, "avg_us": round(ev_us, 2),
                     "timing": "timed-region hipEvents over the GEMV launches of a step"},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


DEC_NQ, DEC_NKV, DEC_D, DEC_CTX, DEC_L, DEC_V = 32, 8, 128, 4096, 48, 196608
DECODE_METRIC = ("decode tokens/s, 48-layer Solar-scale MoE decoder (GQA 32 q / 8 kv heads, KV 4096, 128+1 experts "
                 "top-8, LM head 196608), bf16 batch 1")


def rope_rows(max_ctx: int, D: int = 128, theta: float = 1e6):
    """cos / sin [max_ctx, D] bf16 bits, HF layout (the frequencies repeated for both halves)."""
    inv = theta ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    ang = np.arange(max_ctx, dtype=np.float64)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], axis=1).astype(np.float32)
    f = lambda a: ((a.view(np.uint32).astype(np.uint64) + 0x7FFF + ((a.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    return f(np.cos(ang)), f(np.sin(ang))


def cpu_baseline_decode(budget_layers: int = 2) -> dict | None:
    """The reference host step's arithmetic for `budget_layers` layers on this host's cores, scaled to 48 layers + the
    LM head: the reference's own ck_gemv for the q|k|v, o, router and LM-head GEMVs and ck_moe3 for the 9 experts
    (cpu_kern.c, built from its source), the oracle's numpy restatement of the attention (main.rs:86-104; the Rust
    host attention cannot be built here)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    if not O.ref_available():
        return None
    H, F, E, QD, KVD = 4096, 1280, 128, DEC_NQ * DEC_D, DEC_NKV * DEC_D
    cores = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    R = O.Ref()
    R.set_threads(cores)
    rng = np.random.default_rng(0)
    bf = lambda shape, sd: O.f2bf((sd * rng.standard_normal(shape)).astype(np.float32))
    wqkv, wo, wr = bf((QD + 2 * KVD, H), 0.02), bf((H, QD), 0.02), bf((E, H), 0.02)
    kc, vc = bf((DEC_CTX, DEC_NKV, DEC_D), 1.0), bf((DEC_CTX, DEC_NKV, DEC_D), 1.0)
    n = F * H
    src = O.f2bf((np.arange(3 * n) % 97).astype(np.float32) * 1e-4)
    g, u, d = src[:n].reshape(F, H), src[n:2 * n].reshape(F, H), src[2 * n:].reshape(H, F)
    pool = [R.place_expert(g, u, d) for _ in range(18)]
    wln = np.ones(H, np.uint16) * 0x3F80
    x = bf(H, 1.0)
    t0 = time.perf_counter()
    for l in range(budget_layers):
        h = O.rmsnorm(x, wln)
        qkv = O.f2bf(R.gemv(wqkv, h))
        a, _ = O.attention(qkv[:QD].reshape(DEC_NQ, DEC_D), kc, vc, DEC_NKV)
        o = O.f2bf(R.gemv(wo, a.ravel()))
        h2 = O.rmsnorm(O.f2bf(O.bf2f(x) + O.bf2f(o)), wln)
        lg = R.gemv(wr, h2)
        ids, gates = O.route(lg[None], None, 8)
        out = np.zeros(H, np.float32)
        R.moe3(pool[9 * (l % 2):9 * (l % 2) + 1], np.ones(1, np.float32), h2, out, H, F)
        R.moe3(pool[9 * (l % 2) + 1:9 * (l % 2) + 9], gates[0], h2, out, H, F)
        x = O.f2bf(O.bf2f(x) + out)
    per_layer = (time.perf_counter() - t0) / budget_layers
    # the LM head: ck_gemv over a 1/8 slice of the table, scaled
    W = np.tile(bf((64, H), 0.02), (DEC_V // 8 // 64, 1))
    t1 = time.perf_counter()
    R.gemv(W, x)
    head = (time.perf_counter() - t1) * 8
    tok_s = 1.0 / (DEC_L * per_layer + head)
    return {"value": round(tok_s, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{budget_layers} decode layers (rmsnorm + cpu_kern.c ck_gemv q|k|v/o/router + numpy attention over "
                      f"4096 positions + ck_moe3 shared + 8 routed experts) and 1/8 of the LM-head ck_gemv, scaled to "
                      f"48 layers + the full head; {per_layer * 1e3:.1f} ms per layer, {head * 1e3:.1f} ms head"}


def bench_decode(args) -> None:
    """Greedy decode steps of a 48-layer Solar-scale MoE decoder with every weight resident (about 203 GB): per layer
    RMSNorm + q|k|v GEMV, RoPE + KV append, GQA attention over 4096 positions, o GEMV, the Solar MoE block (softmax
    top-8 with the Zipf-skewed router bias of the Solar layer workload), then the final norm, the 196608-row LM head
    and the argmax.  Each step attends over 4096 positions (the step's own row at position 4095 included); steps
    chain on the device (a step's token is the previous step's pick)."""
    import torch

    from moe_gpu import ROUTE_SOFTMAX, MoeModel

    H, F, E, k, S, L, V = 4096, 1280, 128, 8, 1, DEC_L, DEC_V
    QD, KVD = DEC_NQ * DEC_D, DEC_NKV * DEC_D
    K, W_ = args.steps, args.warmup
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    log(f"decode: create a {L}-layer model")
    m = MoeModel(H, DEC_NQ, DEC_NKV, F, E, k, S, L, V, DEC_CTX, route_rule=ROUTE_SOFTMAX)
    m.set_stream(stream)
    tier = m.experts
    c02 = synth_c(0.02)
    kv_key = lambda l, j: synth_key(9, (1 << 41) + 2 * l + j)
    buf = torch.empty((QD + 2 * KVD) * H + H * QD + 2 * H, dtype=torch.int16, device=dev)
    for l in range(L):
        tier.synth_layer(l, 2000 + l, 0.02, zipf_bias(E, 1.1, 2000 + l))
        tier.synth_fill(buf, buf.numel(), synth_key(11, (1 << 42) + l), c02)
        o0, o1, o2, o3 = QD * H, (QD + KVD) * H, (QD + 2 * KVD) * H, (QD + 2 * KVD) * H + H * QD
        norm = torch.full((H,), 0x3F80, dtype=torch.int16, device=dev)  # bf16 1.0
        m.load_layer(l, norm, buf[:o0], buf[o0:o1], buf[o1:o2], buf[o2:o3], norm)
        kd, vd = m.kv_cache(l)
        for j, p in enumerate((kd, vd)):
            tier.synth_fill(p, (DEC_CTX - 1) * KVD, kv_key(l, j), synth_c(1.0))
        if l % 8 == 7:
            log(f"  {l + 1} layers resident")
    del buf
    emb = torch.empty((V, H), dtype=torch.int16, device=dev)
    tier.synth_fill(emb, V * H, synth_key(12, 1 << 43), synth_c(1.0))
    m.load_embedding(emb)
    tier.synth_fill(emb, V * H, synth_key(13, 1 << 43), c02)
    m.head.load_dev(emb, torch.full((H,), 0x3F80, dtype=torch.int16, device=dev))
    del emb
    torch.cuda.empty_cache()
    cs, sn = rope_rows(DEC_CTX)
    m.load_rope(cs, sn)
    toks = torch.zeros(K + W_ + 1, dtype=torch.int32, device=dev)
    toks[0] = 1
    best = torch.zeros(1, dtype=torch.float32, device=dev)
    pos = DEC_CTX - 1
    torch.cuda.synchronize()
    log(f"warmup {W_} steps")
    for i in range(W_):
        m.step_dev(toks[i:i + 1], pos, toks[i + 1:i + 2], best)
    m.synchronize()
    log(f"timing {K} steps")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(W_, W_ + K):
        m.step_dev(toks[i:i + 1], pos, toks[i + 1:i + 2], best)
    e1.record(stream)
    m.synchronize()
    wall_s = time.perf_counter() - t0
    ev_s = e0.elapsed_time(e1) / 1e3
    ms_tok = wall_s / K * 1e3
    # algorithmic bytes per token: every weight byte once (attention block, router, shared + routed experts, LM head)
    # and the KV rows read; the distinct routed experts of a token are 8 at batch 1
    per_layer = (QD + 2 * KVD) * H * 2 + H * QD * 2 + 2 * DEC_CTX * KVD * 2 + E * H * 2 + (k + S) * 3 * F * H * 2
    nbytes = L * per_layer + V * H * 2 + H * 2
    achieved = nbytes / (ev_s / K) / 1e9
    cpu = None if args.no_cpu_baseline else cpu_baseline_decode()
    line = {
        "metric": DECODE_METRIC, "value": round(K / wall_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": K,
        "warmup": W_, "ms_per_step": round(ms_tok, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded device generator; weights ~0.02 sd, "
        "embeddings and KV ~1 sd, norm weights 1)", "event_ms_per_step": round(ev_s / K * 1e3, 4),
        "config": {"workload": "decode: 48 layers x (RMSNorm + GQA attention 32q/8kv d128 over KV 4096 + RMSNorm + "
                               "Solar MoE block H4096 F1280 E128+1 top-8) + LM head V196608, greedy, batch 1",
                   "layers": L, "kv_len": DEC_CTX, "vocab": V, "tokens": 1},
        "roofline": {"kernel": "whole step (3 launches per layer, 3 more per token)", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_launch": int(nbytes), "avg_us": round(ev_s / K * 1e6, 1),
                     "timing": "timed-region hipEvents on the model's stream over K chained steps"},
        "cpu_baseline": cpu,
    }
    m.close()
    print(json.dumps(line), flush=True)


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` on bench workload `workload` from the committed rocprofv3 counter summary
    (profiles/<kernel>_<workload>_traffic.txt, line `traffic_bytes_per_launch: N`), or None."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--workload", default="solar", choices=sorted(WORKLOADS) + ["lm-head", "attn", "proj", "decode"])
    ap.add_argument("--layers", type=int, default=16, help="distinct resident layers the steps rotate over")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--proj-separate", action="store_true", help="proj workload: q, k, v as three launches")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after timing, run 5 plain device copies of MIB MiB (reference kernel for rocprof "
                         "FETCH_SIZE / WRITE_SIZE scaling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this library has no multi-GPU path (the expert tier would shard by expert "
              "across GPUs, which is designed but not built); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.workload == "lm-head":
        bench_lm_head(args)
        return
    if args.workload == "attn":
        bench_attn(args)
        return
    if args.workload == "proj":
        bench_proj(args)
        return
    if args.workload == "decode":
        bench_decode(args)
        return

    import torch

    w = WORKLOADS[args.workload]
    T, L = w.T, args.layers
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"workload {w.name}: creating tier with {L} resident layers")
    tier = MoeGpu(w.H, w.F, w.E, w.k, w.n_shared, n_layers=L, max_tokens=max(8, T))
    stream = torch.cuda.Stream()  # a real stream handle (the current stream is the null stream), default priority
    torch.cuda.set_stream(stream)
    tier.set_stream(stream)
    for l in range(L):
        tier.synth_layer(l, 1000 + l, w.sigma_w, zipf_bias(w.E, w.zipf_s, 1000 + l))
        if w.int8:
            tier.quantize_layer(l)
    flags = INT8 if w.int8 else 0
    P = 64  # distinct token activations
    xs = torch.empty((P, T, w.H), dtype=torch.int16, device=dev)
    tier.synth_fill(xs, P * T * w.H, synth_key(7, 1 << 40), synth_c(1.0))
    out = torch.empty((T, w.H), dtype=torch.float32, device=dev)
    K, W = args.steps, args.warmup
    ids = torch.empty((K, T, w.k), dtype=torch.int32, device=dev)
    gates = torch.empty((K, T, w.k), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    log(f"warmup {W} steps")
    for i in range(W):
        tier.layer_dev(i % L, T, xs[i % P], out, ids[i % K], gates[i % K], keep=w.keep, flags=flags)
    torch.cuda.synchronize()
    log(f"timing {K} steps")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(K):
        tier.layer_dev(i % L, T, xs[i % P], out, ids[i], gates[i], keep=w.keep, flags=flags)
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ev_ms = e0.elapsed_time(e1)
    ms_per_step = wall_ms / K
    # algorithmic bytes: router + each distinct routed expert of the step once + shared experts
    idh = ids.cpu().numpy()
    keep = w.keep_eff
    distinct = [len(set(idh[i, :, :keep].ravel().tolist())) for i in range(K)]
    bytes_steps = [w.algorithmic_bytes(u) for u in distinct]
    avg_bytes = float(np.mean(bytes_steps))
    achieved = avg_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"{ms_per_step * 1e3:.2f} us/step (events {ev_ms / K * 1e3:.2f}), {achieved:.0f} GB/s algorithmic")

    # per-call latency distribution: one event pair around every call (hipEvents on the call's stream)
    log("per-call event pass")
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    for i in range(K):
        evs[i][0].record(stream)
        tier.layer_dev(i % L, T, xs[i % P], out, ids[i], gates[i], keep=w.keep, flags=flags)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    per_call = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
    median_us, p90_us = per_call[len(per_call) // 2], per_call[min(len(per_call) - 1, int(0.9 * len(per_call)))]

    # PCIe-inclusive rate of the host-buffer entry point (x uploaded, out/ids/gates downloaded, synchronous):
    # reported beside the device-resident value, never as it
    xh = xs[:8].cpu().numpy().view(np.uint16)
    n_host = min(K, 100)
    for i in range(5):
        tier.layer(i % L, xh[i % 8], keep=w.keep, flags=flags)
    t0 = time.perf_counter()
    for i in range(n_host):
        tier.layer(i % L, xh[i % 8], keep=w.keep, flags=flags)
    host_us = (time.perf_counter() - t0) / n_host * 1e6
    torch.cuda.set_stream(stream)

    roofline = None
    kernels = None
    if not args.no_profile:
        log("per-kernel event pass")
        tier.profile_reset()
        tier.profile_kernels(True)
        for i in range(K):
            tier.layer_dev(i % L, T, xs[i % P], out, ids[i], gates[i], keep=w.keep, flags=flags)
        torch.cuda.synchronize()
        prof = tier.profile_read()
        tier.profile_kernels(False)
        kernels = {n: {"avg_us": round(ms / max(c, 1) * 1e3, 2), "launches": c} for n, (ms, c) in prof.items() if c}
        if prof.get("fused_layer_kernel", (0, 0))[1]:
            # one fused kernel streams everything the layer reads: router, routed experts, shared expert.  It is the
            # only kernel of a step, so its average launch duration is the timed region's event time over the K
            # back-to-back launches on its stream (the per-kernel event pairs of this pass add their own overhead).
            k_name, k_ms, k_n = "fused_layer_kernel", ev_ms, K
            k_bytes = avg_bytes
        else:
            # unfused: gate|up streams 2/3 of every expert's bytes and dominates
            (k_ms, k_n), k_name = prof["gateup_kernel"], "gateup_kernel"
            per_expert_gu = 2 * w.F * w.H * (1 if w.int8 else 2)
            k_bytes = float(np.mean([u * per_expert_gu + w.n_shared * 2 * w.F * w.H * 2 for u in distinct]))
        k_avg_s = k_ms / k_n * 1e-3
        k_gbps = k_bytes / k_avg_s / 1e9
        traffic = measured_traffic(k_name, args.workload)
        roofline = {"kernel": k_name, "bound": "hbm", "achieved": round(k_gbps, 1), "peak": HBM_PEAK_GBPS,
                    "unit": "GB/s", "frac": round(k_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                    "bytes_per_launch": int(k_bytes), "avg_us": round(k_avg_s * 1e6, 2)}

    if args.copy_calibration > 0:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        log(f"copy calibration: 5 x {args.copy_calibration} MiB")
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(w) if w.T == 1 else cpu_baseline_batched(w)

    us_tok = ms_per_step * 1e3 / T
    line = {
        "metric": METRIC if args.workload == "solar" else METRIC.replace("bf16 batch 1", f"{args.workload} workload"),
        "value": round(us_tok, 2), "unit": "us/layer/token", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8w-bf16" if w.int8 else "bf16", "data": "synthetic (seeded, weights ~N(0,0.02), x ~N(0,1))",
        "achieved_TBps": round(achieved / 1e3, 3), "hbm_frac": round(achieved / HBM_PEAK_GBPS, 4),
        "median_us_per_call": round(median_us, 2), "p90_us_per_call": round(p90_us, 2),
        "host_buffer_us_per_call": round(host_us, 2),
        "algorithmic_bytes_per_step": int(avg_bytes), "event_ms_per_step": round(ev_ms / K, 5),
        "decode_layer_calls_per_s": round(1e3 / ms_per_step, 1),
        # the MoE blocks of a 48-layer Solar decode step alone (attention and LM head are not part of this path)
        "decode_tokens_per_s_moe_blocks_48_layers": round(T * 1e3 / (48 * ms_per_step), 1),
        "config": {"workload": w.name, "H": w.H, "F": w.F, "E": w.E, "topk": w.k, "n_shared": w.n_shared,
                   "tokens": T, "keep": keep, "resident_layers": L, "distinct_experts_avg": float(np.mean(distinct))},
        "roofline": roofline, "kernels": kernels, "cpu_baseline": cpu,
    }
    tier.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
