"""The C ABI library, host side only (no GPU, no compute): it loads, exports every function include/moe_gpu.h
declares, and its pure-host helpers agree with the oracle."""
import os
import re
import subprocess
import sys

import numpy as np

import moe_gpu
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moe_gpu.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_(?:gpu|head|attn|rmsnorm|gemv|rope|qkv|model|st|placement)_?\w+)\s*\(", text)))


def test_header_declares_the_wrapped_symbols():
    decl = declared_functions()
    assert decl == sorted(moe_gpu.SYMBOLS), set(decl) ^ set(moe_gpu.SYMBOLS)


def test_library_exports_every_declared_symbol():
    L = moe_gpu.load_library()
    for name in declared_functions():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", moe_gpu.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (moe_(?:gpu|head|attn|rmsnorm|gemv|rope|qkv|model|st|placement)_?\w+)", out))
    assert set(declared_functions()) <= exported


def test_host_helpers_match_oracle():
    L = moe_gpu.load_library()
    assert L.moe_gpu_last_error(None) is not None
    assert L.moe_head_last_error(None) is not None
    assert L.moe_gpu_profile_slots() >= 5
    for seed, tid in [(0, 0), (11, 12345), (2 ** 40, 7)]:
        assert moe_gpu.synth_key(seed, tid) == O.synth_key(seed, tid)
    assert moe_gpu.tensor_id(2, 4000, 1) == (2 * 4096 + 4000) * 4 + 1
    assert abs(moe_gpu.synth_c(0.02) * moe_gpu.SYNTH_SD - 0.02) < 1e-8


def test_gpu_moe_builds_rank_tables(monkeypatch):
    """gpu_moe maps cpu_moe's per-expert token lists to per-token rank tables (expert-list order, -1 padding)."""
    seen = {}

    class FakeTier:
        H, k, E = 64, 4, 16

        def moe(self, layer, x, ids, gates, keep=0, with_shared=True):
            seen.update(ids=ids.copy(), gates=gates.copy(), keep=keep, with_shared=with_shared)
            return np.zeros((x.shape[0], self.H), np.float32)

    x = np.zeros((3, 64), np.uint16)
    moe_gpu.gpu_moe(FakeTier(), 0, x, [5, 2, 9], [np.array([0, 2]), np.array([2]), np.array([0])],
                    [np.array([0.5, 0.25], np.float32), np.array([1.0], np.float32), np.array([0.125], np.float32)])
    assert seen["ids"].tolist() == [[5, 9, -1, -1], [-1, -1, -1, -1], [5, 2, -1, -1]]
    assert seen["gates"][2, :2].tolist() == [0.25, 1.0] and seen["keep"] == 2 and not seen["with_shared"]


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "8"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr
