"""Test helpers: host-side weight generation and the oracle's view of one MoE layer call.

The oracle composes the restated reference kernels (oracle/moe_oracle.c): router logits by ck_gemv (cpu_kern.c:31-35,
the order the GPU router also uses), the softmax (host.rs.tpl:247-267) or sigmoid (host.rs:119-128) top-k route,
per-expert outputs with cpu_moe semantics (cpu_moe.cpp:38-96) or ck_moe_q8w semantics for int8 (cpu_kern.c:306-333),
and the fixed-order combine.
"""
from __future__ import annotations

import numpy as np

import oracle as O
from moe_gpu import synth_c, tensor_id
from moe_gpu.workloads import Workload, zipf_bias


def tolerance_report(got: np.ndarray, exp: np.ndarray) -> dict:
    got = np.asarray(got, np.float64); exp = np.asarray(exp, np.float64)
    d = got - exp
    return {
        "max_abs": float(np.abs(d).max()) if d.size else 0.0,
        "rel_l2": float(np.linalg.norm(d) / max(np.linalg.norm(exp), 1e-30)),
        "finite": bool(np.isfinite(got).all()),
    }


def assert_layer_close(got, exp, max_abs=2e-2, rel_l2=5e-3):
    """North-star tolerance for bf16 layers with fp32 accumulation: max-abs 2e-2 and rel-L2 5e-3."""
    r = tolerance_report(got, exp)
    assert r["finite"], r
    assert r["max_abs"] <= max_abs and r["rel_l2"] <= rel_l2, r
    return r


def assert_bf16_close(got: np.ndarray, exp: np.ndarray, max_ulp: int = 2, rel_l2: float = 1e-2):
    """bf16 values (bit arrays) that went through several roundings in different summation orders: each element within
    max_ulp bf16 ulps, an ulp taken at the larger of the element's magnitude and the reference's rms (a value near zero
    is the sum of terms of ordinary size, so its error is one of ordinary size), and rel-L2 within rel_l2."""
    g = O.bf2f(got).astype(np.float64); e = O.bf2f(exp).astype(np.float64)
    assert np.isfinite(g).all()
    rms = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    mag = np.maximum(np.maximum(np.abs(g), np.abs(e)), rms)
    ulp = np.exp2(np.floor(np.log2(np.maximum(mag, 2.0 ** -126))) - 7)
    d = np.abs(g - e)
    worst = float((d / ulp).max()) if d.size else 0.0
    r = {"max_ulp": worst, "rel_l2": float(np.linalg.norm(g - e) / max(np.linalg.norm(e), 1e-30)),
         "frac_diff": float((d > 0).mean())}
    assert worst <= max_ulp and r["rel_l2"] <= rel_l2, r
    return r


# ------------------------------------------------------------------------------------------ host weights
class HostLayer:
    """Weights of one layer on the host, either explicit arrays or regenerated from the synthetic generator."""

    def __init__(self, w: Workload, layer: int = 0, seed: int | None = None, arrays: dict | None = None):
        self.w, self.layer = w, layer
        self.seed = w.seed if seed is None else seed
        self.arrays = arrays
        self.c = synth_c(w.sigma_w)
        self.bias = zipf_bias(w.E, w.zipf_s, self.seed) if w.zipf_s else None
        self._cache: dict = {}

    def _synth(self, e: int, m: int, n: int) -> np.ndarray:
        return O.synth_bf16(O.synth_key(self.seed, tensor_id(self.layer, e, m)), n, self.c)

    def router(self) -> np.ndarray:
        if self.arrays is not None:
            return self.arrays["wr"]
        return self._synth(4095, 0, self.w.E * self.w.H).reshape(self.w.E, self.w.H)

    def _gud(self, e_tid: int):
        if e_tid not in self._cache:
            F, H = self.w.F, self.w.H
            g = self._synth(e_tid, 0, F * H).reshape(F, H)
            u = self._synth(e_tid, 1, F * H).reshape(F, H)
            d = self._synth(e_tid, 2, H * F).reshape(H, F)
            self._cache[e_tid] = (g, u, d)
        return self._cache[e_tid]

    def expert(self, e: int):
        """(g [F,H], u [F,H], d [H,F]) bf16 of routed expert e."""
        if self.arrays is not None:
            return self.arrays["g"][e], self.arrays["u"][e], self.arrays["d"][e]
        return self._gud(e)

    def shared(self, s: int):
        if self.arrays is not None:
            return self.arrays["sg"][s], self.arrays["su"][s], self.arrays["sd"][s]
        return self._gud(4000 + s)

    def expert_q8(self, e: int):
        key = ("q8", e)
        if key not in self._cache:
            g, u, d = self.expert(e)
            q, sc, _ = O.quant_expert(g, u, d)
            self._cache[key] = (q, sc)
        return self._cache[key]


def random_layer(w: Workload, rng: np.random.Generator) -> HostLayer:
    """Layer with true-normal random weights (N(0, sigma_w)) held as host arrays."""
    F, H, E, S = w.F, w.H, w.E, w.n_shared
    bf = lambda shape: O.f2bf(rng.normal(0.0, w.sigma_w, shape).astype(np.float32))
    arrays = {"wr": bf((E, H)), "g": bf((E, F, H)), "u": bf((E, F, H)), "d": bf((E, H, F)),
              "sg": bf((S, F, H)), "su": bf((S, F, H)), "sd": bf((S, H, F))}
    return HostLayer(w, arrays=arrays)


def upload(tier, hl: HostLayer, layer: int = 0):
    w = hl.w
    tier.place_router(layer, hl.router(), hl.bias)
    for e in range(w.E):
        tier.place_expert(layer, e, *hl.expert(e))
    for s in range(w.n_shared):
        tier.place_shared(layer, s, *hl.shared(s))


def random_x(T: int, H: int, rng: np.random.Generator) -> np.ndarray:
    return O.f2bf(rng.normal(0.0, 1.0, (T, H)).astype(np.float32))


# ------------------------------------------------------------------------------------------ oracle layer
def oracle_layer(hl: HostLayer, x: np.ndarray, keep: int | None = None, int8: bool | None = None,
                 ids: np.ndarray | None = None, gates: np.ndarray | None = None, with_shared: bool = True,
                 rule: str = "softmax"):
    """Returns dict(logits, ids, gates, out) for one layer call on x [T,H]."""
    w = hl.w
    x = np.atleast_2d(x)
    T = x.shape[0]
    keep = keep or w.keep_eff
    q8 = w.int8 if int8 is None else int8
    logits = None
    if ids is None:
        logits = O.router_logits(x, hl.router())
        ids, gates = O.route(logits, hl.bias, w.k, keep, rule=rule)
    nsh = w.n_shared if with_shared else 0
    ysh = np.zeros((T, nsh, w.H), np.float32)
    yr = np.zeros((T, w.k, w.H), np.float32)
    for t in range(T):
        for s in range(nsh):
            g, u, d = hl.shared(s)
            ysh[t, s] = O.expert_y(x[t], np.concatenate([g, u]), d)
        for r in range(keep):
            e = int(ids[t, r])
            if e < 0:
                continue
            if q8:
                q, sc = hl.expert_q8(e)
                yr[t, r] = O.expert_y_q8(x[t], q, sc, w.H, w.F)
            else:
                g, u, d = hl.expert(e)
                yr[t, r] = O.expert_y(x[t], np.concatenate([g, u]), d)
    out = O.combine(ysh, yr, ids, gates, keep)
    return {"logits": logits, "ids": ids, "gates": gates, "out": out, "ysh": ysh, "yr": yr, "keep": keep}


# ------------------------------------------------------------------------------------------ decode step oracle
def oracle_moe_block(hl: HostLayer, r: np.ndarray, post_norm: np.ndarray, rule: str = "sigmoid"):
    """A decode layer's MoE half as the reference's host layer computes it (track2_opt/solar_engine/src/main.rs:
    121-141): h2 = rmsnorm(r, post_attention_layernorm); logits = ck_gemv(router, h2); route; the shared expert(s)
    summed (gate 1.0) and rounded to bf16; the routed experts' gated sum (one fused multiply-add per rank, rank
    order) rounded to bf16; x = bf16(r + bf16(moe + shared)).  r: bf16 bits [H].  Returns (x bits, ids, score margin
    between the k-th and (k+1)-th selection key)."""
    w = hl.w
    h2 = O.rmsnorm(r, post_norm)
    lg = O.gemv(hl.router(), h2)
    ids, gates = O.route(lg[None], hl.bias, w.k, None, rule=rule)
    s = (np.float32(1) / (np.float32(1) + np.exp(-lg).astype(np.float32))) if rule == "sigmoid" else lg
    key = np.sort((s + (hl.bias if hl.bias is not None else 0)).astype(np.float32))[::-1]
    margin = float(key[w.k - 1] - key[w.k])
    shared = np.zeros(w.H, np.float32)
    for si in range(w.n_shared):
        g, u, d = hl.shared(si)
        shared = (shared + O.expert_y(h2, np.concatenate([g, u]), d)).astype(np.float32)
    yr = np.zeros((1, w.k, w.H), np.float32)
    for rk in range(w.k):
        g, u, d = hl.expert(int(ids[0, rk]))
        yr[0, rk] = O.expert_y(h2, np.concatenate([g, u]), d)
    moe = O.combine(np.zeros((1, 0, w.H), np.float32), yr, ids, gates, w.k)[0]  # fma chain from 0, rank order
    m = O.bf2f(O.f2bf(O.bf2f(O.f2bf(moe)) + O.bf2f(O.f2bf(shared))))
    x = O.f2bf(O.bf2f(r) + m)
    return x, ids[0], margin


def oracle_decode_layer(x: np.ndarray, lw: dict, kc: np.ndarray, vc: np.ndarray, pos: int, cos_row: np.ndarray,
                        sin_row: np.ndarray, hl: HostLayer, n_q: int, n_kv: int, rule: str = "sigmoid"):
    """One decoder layer of the reference's host step (main.rs:106-126): input norm, q/k/v GEMV + round_bf, RoPE,
    KV append at pos (kc / vc [max_ctx, NKV, D] updated in place), attention over 0..pos, o GEMV + round_bf, then the
    MoE half.  x: bf16 bits [H].  Returns (x bits, ids, routing margin)."""
    D = 128
    h = O.rmsnorm(x, lw["in_norm"])
    q = O.f2bf(O.gemv(lw["wq"], h)).reshape(n_q, D)
    k = O.f2bf(O.gemv(lw["wk"], h)).reshape(n_kv, D)
    v = O.f2bf(O.gemv(lw["wv"], h)).reshape(n_kv, D)
    q = O.rope(q, cos_row, sin_row)
    kc[pos] = O.rope(k, cos_row, sin_row)
    vc[pos] = v
    a, _ = O.attention(q, kc[:pos + 1], vc[:pos + 1], n_kv)
    o = O.f2bf(O.gemv(lw["wo"], a.ravel()))
    r = O.f2bf(O.bf2f(x) + O.bf2f(o))
    return oracle_moe_block(hl, r, lw["post_norm"], rule)


def rope_tables(max_ctx: int, D: int = 128, theta: float = 1e6):
    """cos / sin rows [max_ctx, D] as bf16 bits in HF layout (the D/2 frequencies repeated for both halves), the
    format of the reference's rope_cos.bin / rope_sin.bin (main.rs:4)."""
    inv = theta ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    ang = np.arange(max_ctx, dtype=np.float64)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], axis=1)
    return O.f2bf(np.cos(ang).astype(np.float32)), O.f2bf(np.sin(ang).astype(np.float32))
