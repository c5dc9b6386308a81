"""Python front-end of the CPU oracle (TEST INFRASTRUCTURE: it checks the product, it is never the product).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import this module.  It wraps
three libraries built by ``oracle/Makefile``:

* ``libmoe_oracle.so``   — scalar restatement of the reference's arithmetic (see moe_oracle.c's header for the
  file:line of every function it follows);
* ``libcpu_moe_port.so`` — AVX-512 BF16/OpenMP port of ``solar_hybrid/cpu_moe.cpp`` (CPU baseline);
* ``_ref/libcpu_kern.so`` — the reference's own ``track2_opt/solar_engine/csrc/cpu_kern.c``, compiled from its source
  (used to pin the restatement and as the "reference" CPU baseline).

Function names follow the reference: ``cpu_moe`` (cpu_moe.cpp:38), ``ck_moe3`` (cpu_kern.c:141), ``gemv``
(cpu_kern.c:32), ``quant_row``/``quant_expert`` (cpu_kern.c:218, :227), ``moe_q8w`` (cpu_kern.c:306), ``route``
(host.rs.tpl:247 softmax, host.rs:119 sigmoid), ``group_tokens`` (runtime.py:344-347), ``rmsnorm`` (host.rs:71-76), ``lm_head_argmax``
(main.rs:384-385, chip.rs:183-194), ``attention`` (main.rs:86-104), ``rope`` (main.rs:65-77).
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS: dict = {}

u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")


def _load(name: str) -> C.CDLL:
    if name not in _LIBS:
        path = os.path.join(HERE, name)
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle` (or __graft_entry__.build())")
        _LIBS[name] = C.CDLL(path)
    return _LIBS[name]


def lib() -> C.CDLL:
    L = _load("libmoe_oracle.so")
    if not getattr(L, "_typed", False):
        L.or_f2bf.restype = C.c_uint16; L.or_f2bf.argtypes = [C.c_float]
        L.or_bf2f.restype = C.c_float; L.or_bf2f.argtypes = [C.c_uint16]
        L.or_dot_bf16.restype = C.c_float; L.or_dot_bf16.argtypes = [u16p, u16p, C.c_int]
        L.or_dot_bf16_i8.restype = C.c_float; L.or_dot_bf16_i8.argtypes = [u16p, i8p, C.c_int]
        L.or_gemv.restype = None; L.or_gemv.argtypes = [u16p, u16p, f32p, C.c_int, C.c_int]
        L.or_cpu_moe.restype = None
        L.or_cpu_moe.argtypes = [C.c_int] * 4 + [u16p, C.c_void_p, C.c_void_p, C.c_void_p, i32p, C.c_void_p, f32p]
        L.or_ck_moe3.restype = None
        L.or_ck_moe3.argtypes = [C.c_int, C.c_void_p, f32p, u16p, f32p, C.c_int, C.c_int]
        L.or_quant_row.restype = None
        L.or_quant_row.argtypes = [u16p, C.c_int, i8p, C.POINTER(C.c_float), C.POINTER(C.c_int32)]
        L.or_quant_expert.restype = None
        L.or_quant_expert.argtypes = [u16p, u16p, u16p, i8p, f32p, i32p, C.c_int, C.c_int]
        L.or_moe_q8w.restype = None
        L.or_moe_q8w.argtypes = [C.c_int, C.c_void_p, C.c_void_p, f32p, u16p, f32p, C.c_int, C.c_int]
        for fn in (L.or_route_softmax, L.or_route_sigmoid):
            fn.restype = None
            fn.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, f32p, C.c_void_p, i32p, f32p]
        L.or_combine.restype = None
        L.or_combine.argtypes = [C.c_int] * 5 + [f32p, f32p, i32p, f32p, f32p, C.c_int]
        L.or_synth_key.restype = C.c_uint64; L.or_synth_key.argtypes = [C.c_uint64, C.c_uint64]
        L.or_synth_bf16.restype = None
        L.or_synth_bf16.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, u16p]
        L._typed = True
    return L


def _ptrs(arrs: Sequence[np.ndarray]):
    a = (C.c_void_p * max(1, len(arrs)))()
    for i, x in enumerate(arrs):
        a[i] = x.ctypes.data
    return a


# ----------------------------------------------------------------------------- bf16 helpers (cpu_moe.cpp:30-34)
def f2bf(x) -> np.ndarray:
    """fp32 -> bf16 bits, round-to-nearest-even by the reference's bias trick (no NaN special case)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return (u >> 16).astype(np.uint16)


def bf2f(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- restated kernels
def dot_bf16(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, np.uint16); b = np.ascontiguousarray(b, np.uint16)
    assert a.size == b.size and a.size % 32 == 0
    return float(lib().or_dot_bf16(a, b, a.size))


def gemv(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """ck_gemv (cpu_kern.c:32): y[m] = dot_bf16(W[m], x)."""
    W = np.ascontiguousarray(W, np.uint16); x = np.ascontiguousarray(x, np.uint16)
    M, K = W.shape
    y = np.zeros(M, np.float32)
    lib().or_gemv(W, x, y, M, K)
    return y


def cpu_moe(x: np.ndarray, gus: Sequence[np.ndarray], ds: Sequence[np.ndarray], toks: Sequence[np.ndarray],
            ws: Sequence[np.ndarray]) -> np.ndarray:
    """cpu_moe (cpu_moe.cpp:38-96): out[T,H] fp32 = sum over experts (list order) of w * Wd(bf16(silu(g)*u))."""
    x = np.ascontiguousarray(x, np.uint16)
    T, H = x.shape
    E = len(gus)
    out = np.zeros((T, H), np.float32)
    if E == 0:
        return out
    F = ds[0].shape[1]
    assert H % 32 == 0 and F % 32 == 0
    gus = [np.ascontiguousarray(g, np.uint16) for g in gus]
    ds = [np.ascontiguousarray(d, np.uint16) for d in ds]
    toks = [np.ascontiguousarray(t, np.int64) for t in toks]
    ws = [np.ascontiguousarray(w, np.float32) for w in ws]
    ntok = np.array([t.size for t in toks], np.int32)
    lib().or_cpu_moe(T, H, F, E, x, _ptrs(gus), _ptrs(ds), _ptrs(toks), ntok, _ptrs(ws), out)
    return out


def ck_moe3(bases: Sequence[np.ndarray], w: np.ndarray, x: np.ndarray, out: np.ndarray, H: int, F: int) -> None:
    """ck_moe3 (cpu_kern.c:141-172): out[H] += sum_e w[e] * expert_e(x), experts in ck_place_expert layout."""
    bases = [np.ascontiguousarray(b, np.uint16) for b in bases]
    lib().or_ck_moe3(len(bases), _ptrs(bases), np.ascontiguousarray(w, np.float32), np.ascontiguousarray(x, np.uint16),
                     out, H, F)


def quant_row(row: np.ndarray):
    """quant_row (cpu_kern.c:218-224) -> (q int8[n], scale fp32, rowsum int32)."""
    row = np.ascontiguousarray(row, np.uint16)
    q = np.zeros(row.size, np.int8); s = C.c_float(); r = C.c_int32()
    lib().or_quant_row(row, row.size, q, C.byref(s), C.byref(r))
    return q, np.float32(s.value), int(r.value)


def quant_expert(g: np.ndarray, u: np.ndarray, d: np.ndarray):
    """ck_place_expert_q8 layout (cpu_kern.c:226-241): q int8 [(2F+H)*len], sc fp32 [2F+H], rs int32 [2F+H]."""
    F, H = g.shape
    q = np.zeros(2 * F * H + H * F, np.int8)
    sc = np.zeros(2 * F + H, np.float32); rs = np.zeros(2 * F + H, np.int32)
    lib().or_quant_expert(np.ascontiguousarray(g, np.uint16), np.ascontiguousarray(u, np.uint16),
                          np.ascontiguousarray(d, np.uint16), q, sc, rs, H, F)
    return q, sc, rs


def moe_q8w(qs, scs, w, x, out, H, F) -> None:
    """ck_moe_q8w (cpu_kern.c:306-333): out[H] += sum_e w[e] * int8 weight-only expert_e(x)."""
    lib().or_moe_q8w(len(qs), _ptrs(qs), _ptrs(scs), np.ascontiguousarray(w, np.float32),
                     np.ascontiguousarray(x, np.uint16), out, H, F)


def router_logits(x: np.ndarray, wr: np.ndarray) -> np.ndarray:
    """Router logits [T,E] fp32: ck_gemv (cpu_kern.c:31-35) of the router weight for every token row."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.uint16)
    return np.stack([gemv(wr, x[t]) for t in range(x.shape[0])])


def route(logits: np.ndarray, bias: np.ndarray | None, k: int, keep: int | None = None, rule: str = "softmax"):
    """ids [T,k] int32, gates [T,k] fp32 (ranks >= keep: 0).  rule "softmax": host.rs.tpl:247-267 on (logits + bias);
    rule "sigmoid": Solar's route(), host.rs:119-128 (sigmoid scores, the bias selects only, gates s / (sum + 1e-20))."""
    logits = np.ascontiguousarray(np.atleast_2d(logits), np.float32)
    T, E = logits.shape
    ids = np.zeros((T, k), np.int32); gates = np.zeros((T, k), np.float32)
    b = np.ascontiguousarray(bias, np.float32) if bias is not None else None
    fn = {"softmax": lib().or_route_softmax, "sigmoid": lib().or_route_sigmoid}[rule]
    fn(T, E, k, keep or k, logits, b.ctypes.data if b is not None else None, ids, gates)
    return ids, gates


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """host.rs:71-76 (HF SolarOpenRMSNorm): ms = sum(x^2) / H summed in fp32 left to right, r = 1 / sqrt(ms + eps),
    out = bf16(bf16(x * r) * w).  x: bf16 bits [H] (the residual, bf16 values); w: bf16 bits [H] -> bf16 bits [H]."""
    xf = bf2f(x).astype(np.float32)
    ms = np.cumsum(xf * xf, dtype=np.float32)[-1] / np.float32(xf.size)
    r = np.float32(1.0) / np.sqrt(np.float32(ms + np.float32(eps)))
    return f2bf(bf2f(f2bf(xf * r)) * bf2f(w))


def lm_head_argmax(logits: np.ndarray, rule: int = 0):
    """Greedy pick over one token's logits [V]: rule 0 compares the fp32 logits and keeps the first maximum
    (main.rs:384-385); rule 1 compares them rounded to bf16, exact ties -> lowest row (chip.rs:183-194).
    Returns (row, value compared)."""
    v = np.ascontiguousarray(logits, np.float32)
    if rule:
        v = bf2f(f2bf(v))
    i = int(np.argmax(v))
    return i, float(v[i])


def rope(x: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    """main.rs:65-77 for one position: x bf16 bits [n_heads, D]; rot = (-x[D/2:], x[:D/2]);
    out = bf16(bf16(x * cos) + bf16(rot * sin)), every product and sum in fp32."""
    xf = bf2f(np.ascontiguousarray(x, np.uint16))
    D = xf.shape[-1]
    rot = np.concatenate([-xf[..., D // 2:], xf[..., :D // 2]], axis=-1)
    a = bf2f(f2bf(xf * bf2f(cos_row)))
    b = bf2f(f2bf(rot * bf2f(sin_row)))
    return f2bf(a + b).reshape(x.shape)


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, n_kv: int, scale: float | None = None):
    """Decode attention of main.rs:86-104 for one token.  q: bf16 bits [NQ, D] (after RoPE); kc, vc: bf16 bits
    [S, NKV, D].  Per q head h (kv head h // (NQ / NKV)): sc = bf16(bf16(q . k) * scale) with the dot summed left to
    right in fp32; p = bf16(exp(sc - max) / tot) with tot summed left to right; out = bf16(sum_t p v_t) summed left
    to right.  Returns (out bf16 bits [NQ, D], scores fp32 [NQ, S])."""
    q = np.ascontiguousarray(q, np.uint16); NQ, D = q.shape
    S = kc.shape[0]; G = NQ // n_kv
    sc32 = np.float32(1.0) / np.sqrt(np.float32(D)) if scale is None else np.float32(scale)
    qf, kf, vf = bf2f(q), bf2f(kc).reshape(S, n_kv, D), bf2f(vc).reshape(S, n_kv, D)
    out = np.zeros((NQ, D), np.uint16); scores = np.zeros((NQ, S), np.float32)
    for h in range(NQ):
        g = h // G
        dot = np.cumsum(qf[h][None, :] * kf[:, g, :], axis=1, dtype=np.float32)[:, -1]
        sc = bf2f(f2bf(bf2f(f2bf(dot)) * sc32))
        e = np.exp(sc - sc.max()).astype(np.float32)
        tot = np.cumsum(e, dtype=np.float32)[-1]
        p = bf2f(f2bf(e / tot))
        out[h] = f2bf(np.cumsum(p[:, None] * vf[:, g, :], axis=0, dtype=np.float32)[-1])
        scores[h] = sc
    return out, scores


def group_tokens(ids: np.ndarray, gates: np.ndarray, keep: int | None = None):
    """Per-expert token lists in first-seen order scanning tokens then ranks (runtime.py:344-347).

    Returns [(expert, toks int64[n], ws fp32[n])]."""
    T, k = ids.shape
    keep = keep or k
    per: dict = {}
    for t in range(T):
        for j in range(keep):
            per.setdefault(int(ids[t, j]), []).append((t, float(gates[t, j])))
    return [(e, np.array([r for r, _ in v], np.int64), np.array([w for _, w in v], np.float32)) for e, v in per.items()]


def combine(ysh: np.ndarray, yr: np.ndarray, ids: np.ndarray, gates: np.ndarray, keep: int,
            out: np.ndarray | None = None) -> np.ndarray:
    """Fixed-order combine: ysh [T,S,H] unweighted shared outputs, yr [T,k,H] unweighted routed outputs by rank."""
    T, k, H = yr.shape
    nsh = ysh.shape[1]
    acc = out is not None
    o = out if acc else np.zeros((T, H), np.float32)
    lib().or_combine(T, H, nsh, k, keep, np.ascontiguousarray(ysh, np.float32), np.ascontiguousarray(yr, np.float32),
                     np.ascontiguousarray(ids, np.int32), np.ascontiguousarray(gates, np.float32), o, 1 if acc else 0)
    return o


def expert_y(x_t: np.ndarray, gu: np.ndarray, d: np.ndarray) -> np.ndarray:
    """One expert's unweighted output for one token, cpu_moe semantics (fp32 [H])."""
    return cpu_moe(np.atleast_2d(x_t), [gu], [d], [np.array([0], np.int64)], [np.array([1.0], np.float32)])[0]


def expert_y_q8(x_t: np.ndarray, q: np.ndarray, sc: np.ndarray, H: int, F: int) -> np.ndarray:
    """One int8 weight-only expert's unweighted output (ck_moe_q8w with w = 1: dot * row scale)."""
    o = np.zeros(H, np.float32)
    moe_q8w([np.ascontiguousarray(q, np.int8)], [np.ascontiguousarray(sc, np.float32)], np.array([1.0], np.float32),
            np.ascontiguousarray(x_t, np.uint16), o, H, F)
    return o


# ----------------------------------------------------------------------------- synthetic generator
def synth_key(seed: int, tensor_id: int) -> int:
    return int(lib().or_synth_key(seed, tensor_id))


def synth_bf16(key: int, n: int, c: float, start: int = 0) -> np.ndarray:
    out = np.zeros(n, np.uint16)
    lib().or_synth_bf16(key, start, n, np.float32(c), out)
    return out


# ----------------------------------------------------------------------------- AVX-512 port + reference build
def port_lib():
    L = _load("libcpu_moe_port.so")
    if not getattr(L, "_typed", False):
        L.or_cpu_moe_avx512.restype = None
        L.or_cpu_moe_avx512.argtypes = [C.c_int] * 4 + [u16p, C.c_void_p, C.c_void_p, C.c_void_p, i32p, C.c_void_p, f32p]
        L.or_port_threads.restype = C.c_int
        L._typed = True
    return L


def cpu_has_avx512bf16() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    fl = line.split()
                    return all(x in fl for x in ("avx512f", "avx512bw", "avx512vl", "avx512_bf16", "avx512_vnni"))
    except OSError:
        pass
    return False


def cpu_moe_port(x, gus, ds, toks, ws) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    T, H = x.shape
    E = len(gus)
    out = np.zeros((T, H), np.float32)
    F = ds[0].shape[1]
    ntok = np.array([t.size for t in toks], np.int32)
    port_lib().or_cpu_moe_avx512(T, H, F, E, x, _ptrs(gus), _ptrs(ds), _ptrs(toks), ntok, _ptrs(ws), out)
    return out


def ref_available() -> bool:
    return os.path.exists(os.path.join(HERE, "_ref", "libcpu_kern.so")) and cpu_has_avx512bf16()


class Ref:
    """ctypes view of the reference's own cpu_kern.c (compiled by oracle/Makefile into oracle/_ref/)."""

    def __init__(self):
        L = _load(os.path.join("_ref", "libcpu_kern.so"))
        L.ck_set_threads.argtypes = [C.c_int]; L.ck_set_threads.restype = None
        L.ck_gemv.argtypes = [u16p, u16p, f32p, C.c_int, C.c_int]; L.ck_gemv.restype = None
        for n in ("ck_moe1", "ck_moe2"):
            getattr(L, n).argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, f32p, u16p, f32p, C.c_int, C.c_int]
            getattr(L, n).restype = None
        L.ck_place_expert.argtypes = [u16p, u16p, u16p, u16p, C.c_int, C.c_int]; L.ck_place_expert.restype = None
        L.ck_moe3.argtypes = [C.c_int, C.c_void_p, f32p, u16p, f32p, C.c_int, C.c_int]; L.ck_moe3.restype = None
        L.ck_place_expert_q8.argtypes = [u16p, u16p, u16p, i8p, f32p, i32p, C.c_int, C.c_int]
        L.ck_place_expert_q8.restype = None
        L.ck_moe_q8w.argtypes = [C.c_int, C.c_void_p, C.c_void_p, f32p, u16p, f32p, C.c_int, C.c_int]
        L.ck_moe_q8w.restype = None
        self.L = L

    def set_threads(self, n: int):
        self.L.ck_set_threads(n)

    def gemv(self, W, x):
        M, K = W.shape
        y = np.zeros(M, np.float32)
        self.L.ck_gemv(np.ascontiguousarray(W, np.uint16), np.ascontiguousarray(x, np.uint16), y, M, K)
        return y

    def moe1(self, gs, us, ds, w, x, out, H, F, fn="ck_moe1"):
        getattr(self.L, fn)(len(gs), _ptrs(gs), _ptrs(us), _ptrs(ds), np.ascontiguousarray(w, np.float32),
                            np.ascontiguousarray(x, np.uint16), out, H, F)

    def place_expert(self, g, u, d):
        F, H = g.shape
        dst = np.zeros(3 * F * H, np.uint16)
        self.L.ck_place_expert(g, u, d, dst, H, F)
        return dst

    def moe3(self, bases, w, x, out, H, F):
        self.L.ck_moe3(len(bases), _ptrs(bases), np.ascontiguousarray(w, np.float32), np.ascontiguousarray(x, np.uint16),
                       out, H, F)

    def place_expert_q8(self, g, u, d):
        F, H = g.shape
        q = np.zeros(3 * F * H, np.int8); sc = np.zeros(2 * F + H, np.float32); rs = np.zeros(2 * F + H, np.int32)
        self.L.ck_place_expert_q8(g, u, d, q, sc, rs, H, F)
        return q, sc, rs

    def moe_q8w(self, qs, scs, w, x, out, H, F):
        self.L.ck_moe_q8w(len(qs), _ptrs(qs), _ptrs(scs), np.ascontiguousarray(w, np.float32),
                          np.ascontiguousarray(x, np.uint16), out, H, F)
