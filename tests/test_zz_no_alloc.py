"""The allocation-free decode-attention entry point (moe_attn_decode_noalloc_dev) against the workspace entry point
(moe_attn_decode_dev), through the C ABI: bit-identical outputs on two calls in a row, the second smaller, so the
shared device scratch holds the first call's contents when the second runs; sizes beyond the scratch are refused
before any work is enqueued."""
import numpy as np
import pytest

from moe_gpu import EINVAL, load_library

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-noalloc] {msg}", flush=True)


def test_noalloc_matches_workspace_entry_point():
    import torch

    from moe_gpu import attn_decode_dev, attn_workspace_bytes

    L = load_library()
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    g = torch.Generator(device=dev).manual_seed(5)
    NQ, NKV, D = 32, 8, 128
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    Smax = 4096
    kc = torch.randn(Smax, NKV, D, device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
    vc = torch.randn(Smax, NKV, D, device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
    for S in (4096, 777):  # the second call is smaller: it must not depend on what the first left in the scratch
        q = torch.randn(NQ, D, device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
        ws = torch.zeros(attn_workspace_bytes(NQ, S) // 4, dtype=torch.float32, device=dev)
        ref = torch.zeros(NQ, D, dtype=torch.int16, device=dev)
        got = torch.full((NQ, D), -1, dtype=torch.int16, device=dev)
        torch.cuda.synchronize()
        say(f"noalloc attention S={S}, NQ={NQ}, NKV={NKV}")
        attn_decode_dev(q, kc, vc, ref, ws, NQ, NKV, S, stream=stream)
        rc = L.moe_attn_decode_noalloc_dev(NQ, NKV, D, S, scale, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                           got.data_ptr(), stream.cuda_stream)
        assert rc == 0, L.moe_attn_last_error().decode()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())


def test_noalloc_refuses_sizes_beyond_its_scratch():
    L = load_library()
    cap = L.moe_attn_noalloc_max_bytes()
    assert cap > 0
    S_big = 1 << 16  # the longest context: 64 heads x 65536 positions need 84 MB, beyond the scratch
    say("noalloc attention refuses an oversize call")
    rc = L.moe_attn_decode_noalloc_dev(64, 8, 128, S_big, 0.088, 16, 16, 16, 16, None)
    assert rc == EINVAL
    assert b"scratch" in L.moe_attn_last_error()
