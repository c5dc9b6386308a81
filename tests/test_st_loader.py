"""The model's weights on disk (moe_st_*, moe_placement_read): safetensors files written by the `safetensors` package
(the format the engine's Weights reads, track2_opt/solar_engine/src/host.rs:78-117), tensors looked up by their HF
names, loaded into the GPU tier and checked against the oracle layer on the same arrays; the engine's placement.json
(main.rs:455, moe_offload/placement.py:3).

CPU tests: header parsing, lookup, the later-file-wins rule, malformed files rejected as errors, placement reads.
GPU test: a layer loaded from disk gives the oracle's routing and output within the layer bars."""
import json
import os
import struct

import numpy as np
import pytest

import oracle as O
from moe_gpu import ST_BF16, ST_F32, MoeGpuError, SafeTensors, placement_read

torch = pytest.importorskip("torch")
st_torch = pytest.importorskip("safetensors.torch")


def bf16_tensor(a: np.ndarray):
    """bf16 bits (uint16) -> torch.bfloat16 tensor with the same bits."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def bf(rng, shape, sd=0.02):
    return O.f2bf(rng.normal(0.0, sd, shape).astype(np.float32))


def test_open_lookup_and_later_file_wins(tmp_path):
    rng = np.random.default_rng(1)
    a, b, c = bf(rng, (8, 16)), bf(rng, (3,)), rng.normal(size=5).astype(np.float32)
    st_torch.save_file({"x.weight": bf16_tensor(a), "y": bf16_tensor(b)}, str(tmp_path / "model-00001.safetensors"))
    st_torch.save_file({"y": bf16_tensor(b[::-1].copy()), "z.bias": torch.from_numpy(c)},
                       str(tmp_path / "model-00002.safetensors"), metadata={"format": "pt"})
    (tmp_path / "config.json").write_text("{}")  # other files are ignored
    st = SafeTensors(str(tmp_path))
    try:
        assert len(st) == 3
        dt, shape, raw = st.tensor("x.weight")
        assert (dt, shape) == (ST_BF16, (8, 16))
        np.testing.assert_array_equal(np.frombuffer(raw, np.uint16).reshape(8, 16), a)
        dt, shape, raw = st.tensor("y")  # in both files: the later file's (files in name order, host.rs:86)
        np.testing.assert_array_equal(np.frombuffer(raw, np.uint16), b[::-1])
        dt, shape, raw = st.tensor("z.bias")
        assert (dt, shape) == (ST_F32, (5,))
        np.testing.assert_array_equal(np.frombuffer(raw, np.float32), c)
        with pytest.raises(MoeGpuError, match="missing tensor"):
            st.tensor("nope")
    finally:
        st.close()


def _write_raw(path, header: dict, data: bytes, hlen_extra: int = 0):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h) + hlen_extra) + h + data)


@pytest.mark.parametrize("case", ["offsets_past_end", "size_mismatch", "no_dtype", "bad_json", "header_too_long",
                                  "bad_dtype", "empty_dir"])
def test_malformed_files_are_errors(tmp_path, case):
    good = {"t": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [0, 8]}}
    if case == "offsets_past_end":
        _write_raw(tmp_path / "a.safetensors", {"t": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [8, 16]}}, b"\0" * 8)
    elif case == "size_mismatch":
        _write_raw(tmp_path / "a.safetensors", {"t": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 8]}}, b"\0" * 8)
    elif case == "no_dtype":
        _write_raw(tmp_path / "a.safetensors", {"t": {"shape": [2, 2], "data_offsets": [0, 8]}}, b"\0" * 8)
    elif case == "bad_json":
        (tmp_path / "a.safetensors").write_bytes(struct.pack("<Q", 5) + b'{"t":' + b"\0" * 8)
    elif case == "header_too_long":
        _write_raw(tmp_path / "a.safetensors", good, b"\0" * 8, hlen_extra=100)
    elif case == "bad_dtype":
        _write_raw(tmp_path / "a.safetensors", {"t": {"dtype": "C64", "shape": [1], "data_offsets": [0, 8]}}, b"\0" * 8)
    with pytest.raises(MoeGpuError):
        SafeTensors(str(tmp_path))


def test_placement_json(tmp_path):
    p = tmp_path / "placement.json"
    p.write_text(json.dumps([[[5, 1, 9], [2, 3]], [[7], []]]))
    np.testing.assert_array_equal(placement_read(str(p), 0, 0), [5, 1, 9])
    np.testing.assert_array_equal(placement_read(str(p), 0, 1), [2, 3])
    np.testing.assert_array_equal(placement_read(str(p), 1, 0), [7])
    assert placement_read(str(p), 1, 1).size == 0
    with pytest.raises(MoeGpuError, match="no tier"):
        placement_read(str(p), 2, 0)
    p.write_text("[[[1, 2], [3")
    with pytest.raises(MoeGpuError):
        placement_read(str(p), 0, 1)


def write_moe_layer(path, l: int, hl, bias: np.ndarray):
    """One layer's MoE tensors under the engine's names (main.rs:466-468, :519; host.rs:111-116)."""
    w = hl.w
    t = {f"model.layers.{l}.mlp.gate.weight": bf16_tensor(hl.router()),
         f"model.layers.{l}.mlp.gate.e_score_correction_bias": torch.from_numpy(bias)}
    for e in range(w.E):
        g, u, d = hl.expert(e)
        p = f"model.layers.{l}.mlp.experts.{e}."
        t[p + "gate_proj.weight"], t[p + "up_proj.weight"], t[p + "down_proj.weight"] = map(bf16_tensor, (g, u, d))
    for s in range(w.n_shared):
        g, u, d = hl.shared(s)
        p = f"model.layers.{l}.mlp.shared_experts." if w.n_shared == 1 else f"model.layers.{l}.mlp.shared_experts.{s}."
        t[p + "gate_proj.weight"], t[p + "up_proj.weight"], t[p + "down_proj.weight"] = map(bf16_tensor, (g, u, d))
    st_torch.save_file(t, str(path))


@pytest.mark.gpu
def test_layer_loaded_from_disk_matches_oracle(tmp_path):
    from dataclasses import replace

    from moe_gpu import MoeGpu
    from moe_gpu.workloads import TINY
    from moe_ref import assert_layer_close, oracle_layer, random_layer, random_x

    w = replace(TINY, n_shared=1)
    rng = np.random.default_rng(5)
    hl = random_layer(w, rng)
    hl.bias = rng.normal(0.0, 0.01, w.E).astype(np.float32)
    other = random_layer(w, np.random.default_rng(6))
    write_moe_layer(tmp_path / "model-00001.safetensors", 0, other, np.zeros(w.E, np.float32))
    write_moe_layer(tmp_path / "model-00002.safetensors", 3, hl, hl.bias)
    st = SafeTensors(str(tmp_path))
    tier = MoeGpu(w.H, w.F, w.E, w.k, w.n_shared, n_layers=2, max_tokens=4)
    try:
        print("[gpu-st] load model layer 3 into tier layer 1", flush=True)
        st.load_moe_layer(tier, 3, 1)
        with pytest.raises(MoeGpuError, match="missing tensor"):
            st.load_moe_layer(tier, 7, 0)
        x = random_x(2, w.H, np.random.default_rng(7))
        out, ids, gates = tier.layer(1, x)
        ref = oracle_layer(hl, x)
        np.testing.assert_array_equal(ids, ref["ids"])
        np.testing.assert_allclose(gates, ref["gates"], rtol=0, atol=1e-6)
        assert_layer_close(out, ref["out"])
    finally:
        tier.close()
        st.close()
