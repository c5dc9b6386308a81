"""Python view of libmoe_gpu (the MI355X routed-MoE expert tier) through its C ABI (include/moe_gpu.h).

Mirrors the reference's host-side interface for this path:

* ``MoeGpu`` — one GPU tier holding every expert in HBM (the chip thread of track2_opt/solar_engine/src/chip.rs:96-143
  with the NPU tables replaced by HIP tables).  Methods keep the reference's names and argument meaning:
  ``place_expert`` / ``place_expert_q8`` (host.rs:145, :168), ``moe_placed`` (``moe_cpu_placed``, host.rs:156:
  ``out += sum_e w_e * expert_e(x)``), ``moe_q8`` (``moe_cpu_q8`` with Q8_MODE=w, host.rs:181-188), ``route``
  (router GEMV + softmax top-k, host.rs.tpl:247-267) and ``layer`` (route + experts + shared + combine).
* ``gpu_moe`` — the ``cpu_moe(x, gus, ds, toks, ws)`` operator of solar_hybrid/cpu_moe.cpp:38-96 (called from
  runtime.py:325-328), with experts named by id on a ``MoeGpu`` instead of passed as host tensors.

Errors surface as ``MoeGpuError`` carrying the library's code and message (the engine's eyre::Result replies).
There is no CPU fallback: if libmoe_gpu.so is missing or has no code object for the GPU, construction raises.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Sequence

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("MOE_GPU_LIB") or os.path.join(PKG, "lib", "libmoe_gpu.so")

OK, EINVAL, EHIP, ENOMEM, ESTATE, ENOKERNEL = 0, -1, -2, -3, -4, -5
ACCUMULATE, INT8 = 1, 2

# exported symbols, in include/moe_gpu.h order
SYMBOLS = (
    "moe_gpu_create", "moe_gpu_destroy", "moe_gpu_last_error", "moe_gpu_set_stream", "moe_gpu_synchronize",
    "moe_gpu_load_expert", "moe_gpu_load_shared", "moe_gpu_load_router", "moe_gpu_load_expert_dev",
    "moe_gpu_load_shared_dev", "moe_gpu_load_expert_q8", "moe_gpu_quantize_experts", "moe_gpu_get_expert_q8",
    "moe_gpu_route", "moe_gpu_moe", "moe_gpu_layer", "moe_gpu_route_dev", "moe_gpu_moe_dev", "moe_gpu_layer_dev",
    "moe_gpu_synth_layer", "moe_gpu_synth_fill", "moe_gpu_synth_key", "moe_gpu_enable_timing", "moe_gpu_last_time_ms",
    "moe_gpu_set_option", "moe_gpu_get_option", "moe_gpu_trace_units", "moe_gpu_read_trace",
    "moe_gpu_profile_kernels", "moe_gpu_profile_slots", "moe_gpu_profile_read", "moe_gpu_profile_reset",
    "moe_head_create", "moe_head_destroy", "moe_head_last_error", "moe_head_set_stream", "moe_head_synchronize",
    "moe_head_load", "moe_head_load_dev", "moe_head_argmax", "moe_head_argmax_dev",
    "moe_rmsnorm_dev", "moe_gemv_dev", "moe_gemv_f32_dev", "moe_gemv_norm_dev", "moe_rope_dev", "moe_rope_append_dev",
    "moe_qkv_rope_append_dev",
    "moe_attn_workspace_bytes", "moe_attn_decode_dev", "moe_attn_last_error", "moe_attn_noalloc_max_bytes",
    "moe_attn_decode_noalloc_dev", "moe_attn_decode_oproj_dev",
    "moe_gpu_block_dev",
    "moe_model_create", "moe_model_destroy", "moe_model_last_error", "moe_model_experts", "moe_model_head",
    "moe_model_set_stream", "moe_model_synchronize", "moe_model_load_layer", "moe_model_load_embedding",
    "moe_model_load_rope", "moe_model_set_layers", "moe_model_kv_cache", "moe_model_step_dev", "moe_model_step", "moe_model_residual",
    "moe_model_get_config", "moe_gpu_get_shape",
    "moe_st_open", "moe_st_close", "moe_st_last_error", "moe_st_count", "moe_st_tensor", "moe_st_load_moe_layer",
    "moe_st_load_model", "moe_placement_read",
)
ARGMAX_FP32, ARGMAX_BF16 = 0, 1
OPT_FUSED, OPT_WG_PER_CU, OPT_LAST_GRID, OPT_KSPLIT, OPT_LAG, OPT_SHARED_WAITS, OPT_KSPLIT_SHARED = 1, 2, 3, 4, 5, 6, 7
OPT_GRID, OPT_ROUTER_POLL, OPT_ROUTE_RULE = 8, 9, 10
ROUTE_SOFTMAX, ROUTE_SIGMOID = 0, 1

_lib = None


class ModelConfig(C.Structure):
    """moe_model_config of include/moe_gpu.h."""
    _fields_ = [(n, C.c_int) for n in ("H", "n_q_heads", "n_kv_heads", "head_dim", "F", "E", "topk", "n_shared",
                                        "n_layers", "vocab", "max_ctx")] + \
               [("eps", C.c_float), ("route_rule", C.c_int), ("argmax_rule", C.c_int)]


class MoeGpuError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"moe_gpu error {code}: {msg}")
        self.code = code


def _bind_hip_runtime() -> None:
    """A process must hold exactly one HIP runtime.  PyTorch wheels bundle their own libamdhip64 (same SONAME
    libamdhip64.so.7, loaded by file name from torch/lib); if libmoe_gpu bound /opt/rocm's copy first, a later
    `import torch` would load a second runtime that sees no GPU.  When torch is installed, load its copy first so
    libmoe_gpu's libamdhip64.so.7 dependency resolves to it and both share devices, streams and memory."""
    import importlib.util

    try:
        spec = importlib.util.find_spec("torch")
    except (ImportError, ValueError):
        spec = None
    if spec is not None and spec.origin:
        p = os.path.join(os.path.dirname(spec.origin), "lib", "libamdhip64.so")
        if os.path.exists(p):
            C.CDLL(p, mode=C.RTLD_GLOBAL)


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Load libmoe_gpu.so (no compute happens here; safe without a GPU)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is missing: build it with `python npu-offload_amd/build.py`")
    _bind_hip_runtime()
    L = C.CDLL(path)
    vp, i, u, f = C.c_void_p, C.c_int, C.c_uint, C.c_float
    sig = {
        "moe_gpu_create": (i, [i, i, i, i, i, i, i, i, C.POINTER(vp)]),
        "moe_gpu_destroy": (None, [vp]),
        "moe_gpu_last_error": (C.c_char_p, [vp]),
        "moe_gpu_set_stream": (i, [vp, vp]),
        "moe_gpu_synchronize": (i, [vp]),
        "moe_gpu_load_expert": (i, [vp, i, i, vp, vp, vp]),
        "moe_gpu_load_shared": (i, [vp, i, i, vp, vp, vp]),
        "moe_gpu_load_router": (i, [vp, i, vp, vp]),
        "moe_gpu_load_expert_dev": (i, [vp, i, i, vp, vp, vp]),
        "moe_gpu_load_shared_dev": (i, [vp, i, i, vp, vp, vp]),
        "moe_gpu_load_expert_q8": (i, [vp, i, i, vp, vp]),
        "moe_gpu_quantize_experts": (i, [vp, i, i, i]),
        "moe_gpu_get_expert_q8": (i, [vp, i, i, vp, vp]),
        "moe_gpu_route": (i, [vp, i, i, vp, i, vp, vp, vp]),
        "moe_gpu_moe": (i, [vp, i, i, vp, vp, vp, i, i, u, vp]),
        "moe_gpu_layer": (i, [vp, i, i, vp, i, u, vp, vp, vp]),
        "moe_gpu_route_dev": (i, [vp, i, i, vp, i, vp, vp, vp]),
        "moe_gpu_moe_dev": (i, [vp, i, i, vp, vp, vp, i, i, u, vp]),
        "moe_gpu_layer_dev": (i, [vp, i, i, vp, i, u, vp, vp, vp]),
        "moe_gpu_synth_layer": (i, [vp, i, C.c_uint64, f, vp]),
        "moe_gpu_synth_fill": (i, [vp, vp, C.c_uint64, C.c_uint64, C.c_uint64, f]),
        "moe_gpu_synth_key": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "moe_gpu_enable_timing": (i, [vp, i]),
        "moe_gpu_last_time_ms": (i, [vp, C.POINTER(f)]),
        "moe_gpu_set_option": (i, [vp, i, i]),
        "moe_gpu_trace_units": (i, [vp, i]),
        "moe_gpu_read_trace": (i, [vp, vp, i, C.POINTER(i)]),
        "moe_gpu_get_option": (i, [vp, i, C.POINTER(i)]),
        "moe_gpu_profile_kernels": (i, [vp, i]),
        "moe_gpu_profile_slots": (i, []),
        "moe_gpu_profile_read": (i, [vp, i, C.POINTER(C.c_double), C.POINTER(i), C.POINTER(C.c_char_p)]),
        "moe_gpu_profile_reset": (i, [vp]),
        "moe_head_create": (i, [i, i, i, f, C.POINTER(vp)]),
        "moe_head_destroy": (None, [vp]),
        "moe_head_last_error": (C.c_char_p, [vp]),
        "moe_head_set_stream": (i, [vp, vp]),
        "moe_head_synchronize": (i, [vp]),
        "moe_head_load": (i, [vp, vp, vp]),
        "moe_head_load_dev": (i, [vp, vp, vp]),
        "moe_head_argmax": (i, [vp, i, vp, i, vp, vp, vp]),
        "moe_head_argmax_dev": (i, [vp, i, vp, i, vp, vp, vp]),
        "moe_rmsnorm_dev": (i, [i, i, vp, vp, f, vp, vp]),
        "moe_gemv_dev": (i, [i, i, vp, vp, vp, vp]),
        "moe_rope_dev": (i, [i, i, vp, vp, vp, vp]),
        "moe_attn_workspace_bytes": (C.c_size_t, [i, i, i]),
        "moe_attn_decode_dev": (i, [i, i, i, i, f, vp, vp, vp, vp, vp, C.c_size_t, vp]),
        "moe_attn_last_error": (C.c_char_p, []),
        "moe_attn_noalloc_max_bytes": (C.c_size_t, []),
        "moe_attn_decode_noalloc_dev": (i, [i, i, i, i, f, vp, vp, vp, vp, vp]),
        "moe_attn_decode_oproj_dev": (i, [i, i, i, i, f, vp, vp, vp, vp, vp, i, vp, vp, C.c_size_t, vp]),
        "moe_gemv_norm_dev": (i, [i, i, vp, vp, vp, f, vp, vp]),
        "moe_gemv_f32_dev": (i, [i, i, vp, vp, vp, vp]),
        "moe_rope_append_dev": (i, [i, i, i, vp, vp, vp, vp, vp, i, vp]),
        "moe_qkv_rope_append_dev": (i, [i, i, i, i, vp, vp, vp, f, vp, vp, vp, vp, vp, i, vp]),
        "moe_gpu_block_dev": (i, [vp, i, i, vp, vp, vp, f, i, u, vp, vp, vp, vp]),
        "moe_model_create": (i, [i, C.POINTER(ModelConfig), C.POINTER(vp)]),
        "moe_model_destroy": (None, [vp]),
        "moe_model_last_error": (C.c_char_p, [vp]),
        "moe_model_experts": (vp, [vp]),
        "moe_model_head": (vp, [vp]),
        "moe_model_set_stream": (i, [vp, vp]),
        "moe_model_synchronize": (i, [vp]),
        "moe_model_load_layer": (i, [vp, i, vp, vp, vp, vp, vp, vp]),
        "moe_model_load_embedding": (i, [vp, vp]),
        "moe_model_load_rope": (i, [vp, vp, vp]),
        "moe_model_kv_cache": (i, [vp, i, C.POINTER(vp), C.POINTER(vp)]),
        "moe_model_set_layers": (i, [vp, i]),
        "moe_model_step_dev": (i, [vp, vp, i, vp, vp]),
        "moe_model_step": (i, [vp, i, i, C.POINTER(C.c_int32), C.POINTER(f)]),
        "moe_model_residual": (i, [vp, vp]),
        "moe_model_get_config": (i, [vp, vp]),
        "moe_gpu_get_shape": (i, [vp, vp, vp, vp, vp, vp, vp]),
        "moe_st_open": (i, [C.c_char_p, C.POINTER(vp)]),
        "moe_st_close": (None, [vp]),
        "moe_st_last_error": (C.c_char_p, [vp]),
        "moe_st_count": (i, [vp]),
        "moe_st_tensor": (i, [vp, C.c_char_p, C.POINTER(vp), C.POINTER(C.c_size_t), C.POINTER(i),
                              C.POINTER(C.c_int64), C.POINTER(i)]),
        "moe_st_load_moe_layer": (i, [vp, vp, i, i, vp, i]),
        "moe_st_load_model": (i, [vp, vp]),
        "moe_placement_read": (i, [C.c_char_p, i, i, vp, i, C.POINTER(i)]),
    }
    for name in SYMBOLS:
        fn = getattr(L, name)
        fn.restype, fn.argtypes = sig[name]
    _lib = L
    return L


def _p(a) -> int | None:
    """Pointer of a numpy array, a torch tensor or an int address."""
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if isinstance(a, np.ndarray):
        assert a.flags.c_contiguous
        return a.ctypes.data
    if hasattr(a, "data_ptr"):
        assert a.is_contiguous()
        return a.data_ptr()
    raise TypeError(type(a))


def _u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16, a.dtype
    return a


def synth_key(seed: int, tensor_id: int) -> int:
    return int(load_library().moe_gpu_synth_key(seed, tensor_id))


def tensor_id(layer: int, e: int, m: int) -> int:
    """Synthetic tensor ids: routed e, shared s -> e = 4000 + s, router -> e = 4095 (m = 0 gate, 1 up, 2 down)."""
    return (layer * 4096 + e) * 4 + m


SYNTH_SD = float(np.sqrt(8 * (65536.0 ** 2 - 1) / 12))  # sd of the Irwin-Hall(8) integer sum


def synth_c(sigma: float) -> float:
    return float(np.float32(sigma / SYNTH_SD))


class MoeGpu:
    """One MI355X expert tier: every routed and shared expert of `n_layers` layers resident in HBM."""

    def __init__(self, H: int, F: int, E: int, topk: int, n_shared: int = 0, n_layers: int = 1, max_tokens: int = 8,
                 device: int = 0):
        self.L = load_library()
        h = C.c_void_p()
        rc = self.L.moe_gpu_create(device, H, F, E, topk, n_shared, n_layers, max_tokens, C.byref(h))
        if rc != OK:
            raise MoeGpuError(rc, self.L.moe_gpu_last_error(None).decode())
        self.h = h
        self.H, self.F, self.E, self.k, self.n_shared, self.n_layers, self.max_tokens = (
            H, F, E, topk, n_shared, n_layers, max_tokens)

    # -------------------------------------------------------------------------------------------------- plumbing
    def _chk(self, rc: int):
        if rc != OK:
            raise MoeGpuError(rc, self.L.moe_gpu_last_error(self.h).decode())

    def close(self):
        if getattr(self, "h", None):
            self.L.moe_gpu_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream) -> None:
        """stream: a torch.cuda.Stream, a raw hipStream_t address or None (the context's own stream).
        A handle of 0 (the legacy null stream) also selects the context's own stream."""
        s = getattr(stream, "cuda_stream", stream)
        self._chk(self.L.moe_gpu_set_stream(self.h, s))

    def synchronize(self):
        self._chk(self.L.moe_gpu_synchronize(self.h))

    def enable_timing(self, on: bool = True):
        self._chk(self.L.moe_gpu_enable_timing(self.h, 1 if on else 0))

    def last_time_ms(self) -> float:
        v = C.c_float()
        self._chk(self.L.moe_gpu_last_time_ms(self.h, C.byref(v)))
        return float(v.value)

    def set_option(self, opt: int, value: int):
        self._chk(self.L.moe_gpu_set_option(self.h, opt, int(value)))

    def get_option(self, opt: int) -> int:
        v = C.c_int()
        self._chk(self.L.moe_gpu_get_option(self.h, opt, C.byref(v)))
        return int(v.value)

    def trace_units(self, on: bool = True):
        self._chk(self.L.moe_gpu_trace_units(self.h, 1 if on else 0))

    def read_trace(self) -> np.ndarray:
        """[units, 6] uint64 of the last fused launch, in its unit order: start, inputs ready, end (100 MHz ticks),
        workgroup, aux, aux2 (see moe_gpu_trace_units in include/moe_gpu.h)."""
        cap = 1 << 16
        buf = np.zeros((cap, 6), np.uint64); n = C.c_int()
        self._chk(self.L.moe_gpu_read_trace(self.h, _p(buf), cap, C.byref(n)))
        return buf[: n.value].copy()

    def profile_kernels(self, on: bool = True):
        self._chk(self.L.moe_gpu_profile_kernels(self.h, 1 if on else 0))

    def profile_reset(self):
        self._chk(self.L.moe_gpu_profile_reset(self.h))

    def profile_read(self) -> dict:
        """{kernel name: (total ms, launches)} since the last reset (synchronises)."""
        res = {}
        for k in range(self.L.moe_gpu_profile_slots()):
            ms, n, nm = C.c_double(), C.c_int(), C.c_char_p()
            self._chk(self.L.moe_gpu_profile_read(self.h, k, C.byref(ms), C.byref(n), C.byref(nm)))
            res[nm.value.decode()] = (float(ms.value), int(n.value))
        return res

    # -------------------------------------------------------------------------------------------------- weights
    def place_expert(self, layer: int, e: int, g, u, d):
        """host.rs:145 place_expert / chip.rs:208-233 table upload: bf16 g,u [F,H], d [H,F] -> HBM tables."""
        g, u, d = _u16(g), _u16(u), _u16(d)
        assert g.shape == (self.F, self.H) and u.shape == (self.F, self.H) and d.shape == (self.H, self.F)
        self._chk(self.L.moe_gpu_load_expert(self.h, layer, e, _p(g), _p(u), _p(d)))

    def place_shared(self, layer: int, s: int, g, u, d):
        g, u, d = _u16(g), _u16(u), _u16(d)
        assert g.shape == (self.F, self.H) and u.shape == (self.F, self.H) and d.shape == (self.H, self.F)
        self._chk(self.L.moe_gpu_load_shared(self.h, layer, s, _p(g), _p(u), _p(d)))

    def place_router(self, layer: int, wr, bias=None):
        wr = _u16(wr)
        assert wr.shape == (self.E, self.H)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self._chk(self.L.moe_gpu_load_router(self.h, layer, _p(wr), _p(b)))

    def place_expert_q8(self, layer: int, e: int, q=None, sc=None):
        """host.rs:168 place_expert_q8: with q/sc (ck_place_expert_q8 layout) upload them, else quantise the
        resident bf16 copy on the device (same quant_row bits)."""
        if q is None:
            self._chk(self.L.moe_gpu_quantize_experts(self.h, layer, e, e + 1))
        else:
            q = np.ascontiguousarray(q, np.int8); sc = np.ascontiguousarray(sc, np.float32)
            assert q.size == 3 * self.F * self.H and sc.size == 2 * self.F + self.H
            self._chk(self.L.moe_gpu_load_expert_q8(self.h, layer, e, _p(q), _p(sc)))

    def quantize_layer(self, layer: int, e0: int = 0, e1: int | None = None):
        self._chk(self.L.moe_gpu_quantize_experts(self.h, layer, e0, self.E if e1 is None else e1))

    def get_expert_q8(self, layer: int, e: int):
        q = np.zeros(3 * self.F * self.H, np.int8); sc = np.zeros(2 * self.F + self.H, np.float32)
        self._chk(self.L.moe_gpu_get_expert_q8(self.h, layer, e, _p(q), _p(sc)))
        return q, sc

    def synth_layer(self, layer: int, seed: int, sigma: float = 0.02, bias=None):
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self._chk(self.L.moe_gpu_synth_layer(self.h, layer, seed, synth_c(sigma), _p(b)))

    def synth_fill(self, dst, n: int, key: int, c: float, start: int = 0):
        self._chk(self.L.moe_gpu_synth_fill(self.h, _p(dst), n, key, start, c))

    # -------------------------------------------------------------------------------------------------- compute (host)
    def route(self, layer: int, x, keep: int = 0, want_logits: bool = False):
        x = _u16(np.atleast_2d(x)); T = x.shape[0]
        ids = np.zeros((T, self.k), np.int32); gates = np.zeros((T, self.k), np.float32)
        lg = np.zeros((T, self.E), np.float32) if want_logits else None
        self._chk(self.L.moe_gpu_route(self.h, layer, T, _p(x), keep, _p(ids), _p(gates), _p(lg)))
        return (ids, gates, lg) if want_logits else (ids, gates)

    def moe(self, layer: int, x, ids, gates, keep: int = 0, with_shared: bool = True, flags: int = 0, out=None):
        x = _u16(np.atleast_2d(x)); T = x.shape[0]
        ids = np.ascontiguousarray(np.atleast_2d(ids), np.int32); gates = np.ascontiguousarray(np.atleast_2d(gates), np.float32)
        assert ids.shape == (T, self.k) and gates.shape == (T, self.k)
        if out is None:
            out = np.zeros((T, self.H), np.float32)
        self._chk(self.L.moe_gpu_moe(self.h, layer, T, _p(x), _p(ids), _p(gates), keep, 1 if with_shared else 0, flags,
                                     _p(out)))
        return out

    def layer(self, layer: int, x, keep: int = 0, flags: int = 0, out=None):
        x = _u16(np.atleast_2d(x)); T = x.shape[0]
        if out is None:
            out = np.zeros((T, self.H), np.float32)
        ids = np.zeros((T, self.k), np.int32); gates = np.zeros((T, self.k), np.float32)
        self._chk(self.L.moe_gpu_layer(self.h, layer, T, _p(x), keep, flags, _p(out), _p(ids), _p(gates)))
        return out, ids, gates

    def moe_placed(self, layer: int, ids: Sequence[int], w, x, out: np.ndarray):
        """moe_cpu_placed (host.rs:156 -> ck_moe3): out[H] += sum_e w[e] * expert_{ids[e]}(x), routed only."""
        self._placed(layer, ids, w, x, out, 0)

    def moe_q8(self, layer: int, ids: Sequence[int], w, x, out: np.ndarray):
        """moe_cpu_q8 with Q8_MODE=w (host.rs:181-188 -> ck_moe_q8w): int8 weight-only routed experts, out +=."""
        self._placed(layer, ids, w, x, out, INT8)

    def _placed(self, layer, ids, w, x, out, flags):
        n = len(ids)
        if n == 0:
            return
        assert n <= self.k and out.dtype == np.float32 and out.size == self.H
        idv = np.zeros((1, self.k), np.int32); gv = np.zeros((1, self.k), np.float32)
        idv[0, :n] = ids; gv[0, :n] = w
        o = out.reshape(1, self.H)
        self._chk(self.L.moe_gpu_moe(self.h, layer, 1, _p(_u16(np.atleast_2d(x))), _p(idv), _p(gv), n, 0,
                                     flags | ACCUMULATE, _p(o)))

    # -------------------------------------------------------------------------------------------------- compute (device)
    def layer_dev(self, layer: int, T: int, x, out, ids=None, gates=None, keep: int = 0, flags: int = 0):
        self._chk(self.L.moe_gpu_layer_dev(self.h, layer, T, _p(x), keep, flags, _p(out), _p(ids), _p(gates)))

    def moe_dev(self, layer: int, T: int, x, ids, gates, out, keep: int = 0, with_shared: bool = True, flags: int = 0):
        self._chk(self.L.moe_gpu_moe_dev(self.h, layer, T, _p(x), _p(ids), _p(gates), keep, 1 if with_shared else 0,
                                         flags, _p(out)))

    def route_dev(self, layer: int, T: int, x, ids, gates, logits=None, keep: int = 0):
        self._chk(self.L.moe_gpu_route_dev(self.h, layer, T, _p(x), keep, _p(ids), _p(gates), _p(logits)))

    def block_dev(self, layer: int, T: int, resid, attn_o, norm_w, x_next, eps: float = 1e-5, out=None, ids=None,
                  gates=None, keep: int = 0, flags: int = 0):
        """A decode layer's second half (main.rs:120-141): x_next = bf16(r + bf16(bf16(routed) + bf16(shared))) with
        r = bf16(resid + attn_o) and the experts run on rmsnorm(r, norm_w).  Device tensors."""
        self._chk(self.L.moe_gpu_block_dev(self.h, layer, T, _p(resid), _p(attn_o), _p(norm_w), eps, keep, flags,
                                           _p(x_next), _p(out), _p(ids), _p(gates)))


class LmHead:
    """The decode step's tail on the GPU: final RMSNorm, LM-head GEMV, greedy argmax (main.rs:381-386; the chip's
    lm_head_am + best_key, dense/lm_head.rs:174-181 and chip.rs:183-194).  ``argmax`` returns (ids, best values)
    and, with ``want_logits``, the fp32 logits [T, V]."""

    def __init__(self, H: int, V: int, eps: float = 1e-5, device: int = 0):
        self.L = load_library()
        h = C.c_void_p()
        rc = self.L.moe_head_create(device, H, V, eps, C.byref(h))
        if rc != OK:
            raise MoeGpuError(rc, self.L.moe_head_last_error(None).decode())
        self.h, self.H, self.V = h, H, V

    def _chk(self, rc: int):
        if rc != OK:
            raise MoeGpuError(rc, self.L.moe_head_last_error(self.h).decode())

    def close(self):
        if getattr(self, "h", None):
            self.L.moe_head_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream) -> None:
        self._chk(self.L.moe_head_set_stream(self.h, getattr(stream, "cuda_stream", stream)))

    def synchronize(self):
        self._chk(self.L.moe_head_synchronize(self.h))

    def load(self, w_lm, w_final):
        """Host arrays: w_lm uint16 [V, H] (lm_head.weight bf16 bits), w_final uint16 [H] (model.norm.weight)."""
        w_lm, w_final = _u16(w_lm), _u16(w_final)
        assert w_lm.shape == (self.V, self.H) and w_final.shape == (self.H,)
        self._chk(self.L.moe_head_load(self.h, _p(w_lm), _p(w_final)))

    def load_dev(self, w_lm, w_final):
        """Device tensors (bf16 or int16 views of bf16 bits) of the same shapes."""
        assert tuple(w_lm.shape) == (self.V, self.H) and tuple(w_final.shape) == (self.H,)
        self._chk(self.L.moe_head_load_dev(self.h, _p(w_lm), _p(w_final)))

    def argmax(self, x, rule: int = ARGMAX_FP32, want_logits: bool = False):
        x = _u16(x).reshape(-1, self.H)
        T = x.shape[0]
        ids = np.zeros(T, np.int32)
        best = np.zeros(T, np.float32)
        lg = np.zeros((T, self.V), np.float32) if want_logits else None
        self._chk(self.L.moe_head_argmax(self.h, T, _p(x), rule, _p(ids), _p(best), _p(lg)))
        return (ids, best, lg) if want_logits else (ids, best)

    def argmax_dev(self, T: int, x, ids, best, logits=None, rule: int = ARGMAX_FP32):
        """Device pointers; enqueued on the head's stream, not synchronised."""
        self._chk(self.L.moe_head_argmax_dev(self.h, T, _p(x), rule, _p(ids), _p(best), _p(logits)))


def rmsnorm_dev(x, w, out, eps: float = 1e-5, stream=None) -> None:
    """Per-layer RMSNorm (host.rs:71-76) on device tensors: x, out [T, H] and w [H], bf16 bits."""
    T, H = x.shape
    assert tuple(out.shape) == (T, H) and tuple(w.shape) == (H,)
    rc = load_library().moe_rmsnorm_dev(T, H, _p(x), _p(w), eps, _p(out), getattr(stream, "cuda_stream", stream))
    if rc != OK:
        raise MoeGpuError(rc, f"moe_rmsnorm_dev(T={T}, H={H}) failed")


def gemv_dev(W, x, y, stream=None) -> None:
    """Projection GEMV with round_bf (main.rs:109-111): W [M, K], x [K], y [M], bf16 bits on the device."""
    M, K = W.shape
    rc = load_library().moe_gemv_dev(M, K, _p(W), _p(x), _p(y), getattr(stream, "cuda_stream", stream))
    if rc != OK:
        raise MoeGpuError(rc, f"moe_gemv_dev(M={M}, K={K}) failed")


def rope_dev(x, cos_row, sin_row, stream=None) -> None:
    """Rotary embedding in place (main.rs:65-77): x [n_heads, D] bf16 bits on the device, cos/sin rows [D]."""
    n, D = x.shape
    rc = load_library().moe_rope_dev(n, D, _p(x), _p(cos_row), _p(sin_row), getattr(stream, "cuda_stream", stream))
    if rc != OK:
        raise MoeGpuError(rc, f"moe_rope_dev(n={n}, D={D}) failed")


def attn_decode_dev(q, k_cache, v_cache, out, workspace, n_q_heads: int, n_kv_heads: int, S: int,
                    scale: float | None = None, head_dim: int = 128, stream=None) -> None:
    """GQA decode attention over a KV cache (main.rs:86-104) on device tensors: q [NQ, D], caches [>= S, NKV, D],
    out [NQ, D] (bf16 bits as int16 or bfloat16), workspace a device buffer of attn_workspace_bytes().  Enqueued on
    `stream` (a torch stream or raw handle; None: the null stream)."""
    L = load_library()
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
    ws_bytes = workspace.numel() * workspace.element_size()
    rc = L.moe_attn_decode_dev(n_q_heads, n_kv_heads, head_dim, S, scale, _p(q), _p(k_cache), _p(v_cache), _p(out),
                               _p(workspace), ws_bytes, getattr(stream, "cuda_stream", stream))
    if rc != OK:
        raise MoeGpuError(rc, L.moe_attn_last_error().decode())


def attn_decode_oproj_dev(q, k_cache, v_cache, out, w_o, o_out, workspace, n_q_heads: int, n_kv_heads: int, S: int,
                          scale: float | None = None, head_dim: int = 128, stream=None) -> None:
    """attn_decode_dev with the o projection in the same launch (main.rs:86-104, :119): out as attn_decode_dev and
    o_out [M] = bf16(w_o . out), w_o [M, NQ * D] bf16 bits (NQ * D = 4096), bit-identical to gemv_dev(w_o, out)."""
    L = load_library()
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
    ws_bytes = workspace.numel() * workspace.element_size()
    rc = L.moe_attn_decode_oproj_dev(n_q_heads, n_kv_heads, head_dim, S, scale, _p(q), _p(k_cache), _p(v_cache),
                                     _p(out), _p(w_o), int(w_o.shape[0]), _p(o_out), _p(workspace), ws_bytes,
                                     getattr(stream, "cuda_stream", stream))
    if rc != OK:
        raise MoeGpuError(rc, L.moe_attn_last_error().decode())


def attn_workspace_bytes(n_q_heads: int, S: int, head_dim: int = 128) -> int:
    return int(load_library().moe_attn_workspace_bytes(n_q_heads, head_dim, S))


ATTN_SCORES_OFFSET = 256  # bytes: the workspace's header, then the last call's scores [NQ, S] fp32


def attn_scores(workspace, n_q_heads: int, S: int):
    """The scores [NQ, S] (fp32) of the last attn_decode_dev call on `workspace`, as a view of it."""
    f = workspace.view(-1).view(dtype=__import__("torch").float32)
    o = ATTN_SCORES_OFFSET // 4
    return f[o:o + n_q_heads * S].view(n_q_heads, S)


def gemv_norm_dev(W, x, norm_w, y, eps: float = 1e-5, stream=None) -> None:
    """y = bf16(W . rmsnorm(x, norm_w)) on device tensors (the input norm folded into the q|k|v projection)."""
    M, K = W.shape
    rc = load_library().moe_gemv_norm_dev(M, K, _p(W), _p(x), _p(norm_w), eps, _p(y),
                                          getattr(stream, "cuda_stream", stream))
    if rc != OK:
        raise MoeGpuError(rc, f"moe_gemv_norm_dev(M={M}, K={K}) failed")


def rope_append_dev(qkv, cos_row, sin_row, k_cache, v_cache, pos: int, n_q_heads: int, n_kv_heads: int,
                    head_dim: int = 128, stream=None) -> None:
    rc = load_library().moe_rope_append_dev(n_q_heads, n_kv_heads, head_dim, _p(qkv), _p(cos_row), _p(sin_row),
                                            _p(k_cache), _p(v_cache), pos, getattr(stream, "cuda_stream", stream))
    if rc != OK:
        raise MoeGpuError(rc, "moe_rope_append_dev failed")


def qkv_rope_append_dev(W, x, norm_w, cos_row, sin_row, q, k_cache, v_cache, pos: int, n_q_heads: int,
                        n_kv_heads: int, eps: float = 1e-5, stream=None) -> None:
    """The q|k|v projection (rmsnorm folded in when norm_w is given), RoPE and the KV-cache append in one launch:
    q [NQ * 128] receives roped q, the caches' row pos the roped k and the v (main.rs:109-118)."""
    M, K = W.shape
    rc = load_library().moe_qkv_rope_append_dev(K, n_q_heads, n_kv_heads, 128, _p(W), _p(x),
                                                _p(norm_w) if norm_w is not None else None, eps, _p(cos_row),
                                                _p(sin_row), _p(q), _p(k_cache), _p(v_cache), pos,
                                                getattr(stream, "cuda_stream", stream))
    if rc != OK:
        raise MoeGpuError(rc, f"moe_qkv_rope_append_dev(H={K}, NQ={n_q_heads}, NKV={n_kv_heads}) failed")


class MoeModel:
    """A whole MoE decoder's greedy decode step on one GPU (the engine's host step, main.rs:372-387).  The experts and
    routers are loaded through ``experts`` (a MoeGpu view of the model's context), the LM head through ``head``."""

    def __init__(self, H: int, n_q_heads: int, n_kv_heads: int, F: int, E: int, topk: int, n_shared: int,
                 n_layers: int, vocab: int, max_ctx: int, eps: float = 1e-5, route_rule: int = ROUTE_SIGMOID,
                 argmax_rule: int = ARGMAX_FP32, head_dim: int = 128, device: int = 0):
        self.L = load_library()
        cfg = ModelConfig(H, n_q_heads, n_kv_heads, head_dim, F, E, topk, n_shared, n_layers, vocab, max_ctx, eps,
                          route_rule, argmax_rule)
        h = C.c_void_p()
        rc = self.L.moe_model_create(device, C.byref(cfg), C.byref(h))
        if rc != OK:
            raise MoeGpuError(rc, self.L.moe_model_last_error(None).decode())
        self.h, self.cfg = h, cfg
        self.experts = MoeGpu.__new__(MoeGpu)  # a view: the model owns and destroys the context
        self.experts.L, self.experts.h = self.L, C.c_void_p(self.L.moe_model_experts(h))
        self.experts.H, self.experts.F, self.experts.E, self.experts.k = H, F, E, topk
        self.experts.n_shared, self.experts.n_layers, self.experts.max_tokens = n_shared, n_layers, 1
        self.experts.close = lambda: None
        self.head = LmHead.__new__(LmHead)
        self.head.L, self.head.h, self.head.H, self.head.V = self.L, C.c_void_p(self.L.moe_model_head(h)), H, vocab
        self.head.close = lambda: None

    def _chk(self, rc: int):
        if rc != OK:
            raise MoeGpuError(rc, self.L.moe_model_last_error(self.h).decode())

    def close(self):
        if getattr(self, "h", None):
            self.L.moe_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream) -> None:
        self._chk(self.L.moe_model_set_stream(self.h, getattr(stream, "cuda_stream", stream)))

    def synchronize(self):
        self._chk(self.L.moe_model_synchronize(self.h))

    def load_layer(self, layer: int, in_norm, wq, wk, wv, wo, post_norm):
        """Host arrays (uint16 bf16 bits) or device tensors."""
        arrs = [a if hasattr(a, "data_ptr") else _u16(a) for a in (in_norm, wq, wk, wv, wo, post_norm)]
        self._chk(self.L.moe_model_load_layer(self.h, layer, *[_p(a) for a in arrs]))

    def load_embedding(self, emb):
        emb = emb if hasattr(emb, "data_ptr") else _u16(emb)
        self._chk(self.L.moe_model_load_embedding(self.h, _p(emb)))

    def load_rope(self, cos_tab, sin_tab):
        c = cos_tab if hasattr(cos_tab, "data_ptr") else _u16(cos_tab)
        s_ = sin_tab if hasattr(sin_tab, "data_ptr") else _u16(sin_tab)
        self._chk(self.L.moe_model_load_rope(self.h, _p(c), _p(s_)))

    def set_layers(self, n: int):
        """Steps run the first n layers, then the head."""
        self._chk(self.L.moe_model_set_layers(self.h, n))

    def kv_cache(self, layer: int):
        """(k, v) device addresses of the layer's caches [max_ctx, NKV, D] bf16."""
        k, v = C.c_void_p(), C.c_void_p()
        self._chk(self.L.moe_model_kv_cache(self.h, layer, C.byref(k), C.byref(v)))
        return k.value, v.value

    def step(self, token: int, pos: int):
        nxt, best = C.c_int32(), C.c_float()
        self._chk(self.L.moe_model_step(self.h, token, pos, C.byref(nxt), C.byref(best)))
        return int(nxt.value), float(best.value)

    def step_dev(self, token, pos: int, nxt, best=None):
        self._chk(self.L.moe_model_step_dev(self.h, _p(token), pos, _p(nxt), _p(best)))

    def residual(self) -> np.ndarray:
        x = np.zeros(self.cfg.H, np.uint16)
        self._chk(self.L.moe_model_residual(self.h, _p(x)))
        return x


ST_BF16, ST_F32, ST_F16, ST_I8, ST_I32, ST_I64, ST_U8 = 0, 1, 2, 3, 4, 5, 6


class SafeTensors:
    """A model directory of safetensors files, memory-mapped by the library (moe_st_*, the engine's Weights,
    track2_opt/solar_engine/src/host.rs:78-117): tensors by HF name, and loads into a tier or a decode model."""

    def __init__(self, directory: str):
        self.L = load_library()
        h = C.c_void_p()
        rc = self.L.moe_st_open(directory.encode(), C.byref(h))
        if rc != OK:
            raise MoeGpuError(rc, self.L.moe_st_last_error(None).decode())
        self.h = h

    def _chk(self, rc: int):
        if rc != OK:
            raise MoeGpuError(rc, self.L.moe_st_last_error(self.h).decode())

    def __len__(self) -> int:
        return self.L.moe_st_count(self.h)

    def tensor(self, name: str):
        """(dtype code, shape, bytes) of a tensor (the bytes copied out of the mapping)."""
        data, nb, dt = C.c_void_p(), C.c_size_t(), C.c_int()
        shape = (C.c_int64 * 8)(); nd = C.c_int(8)
        self._chk(self.L.moe_st_tensor(self.h, name.encode(), C.byref(data), C.byref(nb), C.byref(dt), shape,
                                       C.byref(nd)))
        return dt.value, tuple(shape[:nd.value]), C.string_at(data, nb.value)

    def load_moe_layer(self, tier: "MoeGpu", model_layer: int, tier_layer: int, experts=None):
        ids = None if experts is None else np.ascontiguousarray(experts, np.int32)
        self._chk(self.L.moe_st_load_moe_layer(self.h, tier.h, model_layer, tier_layer, _p(ids),
                                                -1 if ids is None else len(ids)))

    def load_model(self, m: "MoeModel"):
        self._chk(self.L.moe_st_load_model(self.h, m.h))

    def close(self):
        if getattr(self, "h", None):
            self.L.moe_st_close(self.h)
            self.h = None

    def __del__(self):
        self.close()


def placement_read(path: str, layer: int, tier: int) -> np.ndarray:
    """Expert ids of (layer, tier) from the engine's placement.json (main.rs:455; moe_offload/placement.py:3)."""
    L = load_library()
    n = C.c_int()
    rc = L.moe_placement_read(path.encode(), layer, tier, None, 0, C.byref(n))
    if rc != OK:
        raise MoeGpuError(rc, L.moe_st_last_error(None).decode())
    ids = np.zeros(n.value, np.int32)
    rc = L.moe_placement_read(path.encode(), layer, tier, _p(ids), n.value, C.byref(n))
    if rc != OK:
        raise MoeGpuError(rc, L.moe_st_last_error(None).decode())
    return ids


def gpu_moe(tier: MoeGpu, layer: int, x, experts: Sequence[int], toks: Sequence, ws: Sequence) -> np.ndarray:
    """cpu_moe (solar_hybrid/cpu_moe.cpp:38-96) on the GPU tier: experts by id, per-expert token rows and weights.

    Returns out [T,H] fp32 = sum over experts (in list order, per token) of w * expert(x[tok]); no shared expert."""
    x = _u16(np.atleast_2d(x)); T = x.shape[0]
    per_tok: list[list] = [[] for _ in range(T)]
    for e, tk, w in zip(experts, toks, ws):
        for t, wt in zip(np.asarray(tk).tolist(), np.asarray(w, np.float32).tolist()):
            per_tok[t].append((int(e), wt))
    kmax = max((len(p) for p in per_tok), default=0)
    if kmax > tier.k:
        raise MoeGpuError(EINVAL, f"a token is routed to {kmax} experts > topk={tier.k}")
    out = np.zeros((T, tier.H), np.float32)
    if kmax == 0:
        return out
    # tokens with fewer experts leave their remaining ranks empty (id -1)
    ids = np.full((T, tier.k), -1, np.int32); gates = np.zeros((T, tier.k), np.float32)
    for t, p in enumerate(per_tok):
        for r, (e, w) in enumerate(p):
            ids[t, r], gates[t, r] = e, w
    return tier.moe(layer, x, ids, gates, keep=kmax, with_shared=False)
