"""The HIP library on the committed golden fixtures (expected outputs from the float64
numpy reference; expected 8-bit codes from the brute-force / closed-form encoders)."""
import os

import numpy as np
import pytest

from kvcases import HS, assert_close

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _dev_tensor(a, dev):
    import torch
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(a).to(dev)


@pytest.mark.parametrize("name,dtype", [("g_f32", "f32"), ("g_bf16", "bf16")])
@pytest.mark.parametrize("strategy", ["fused_single", "split_merge", "lastblock", "designated", "graph", "coop"])
def test_golden_attention(dev, name, dtype, strategy):
    import torch
    from cuda_gpt2_inference_amd import kvattn
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    B, NH, maxT = int(g["B"]), int(g["NH"]), int(g["maxT"])
    qkv, cache = _dev_tensor(g["qkv"], dev), _dev_tensor(g["cache"], dev)
    cur = torch.from_numpy(g["totals"] - 1).to(dev)
    out = torch.empty(B * NH * HS, dtype=torch.float32 if dtype == "f32" else torch.bfloat16, device=dev)
    S = 0 if strategy in ("fused_single", "split_merge", "lastblock", "designated") else 5
    ws = kvattn.Workspace(B, NH, maxT, S)
    kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, cur_len=cur, lens_per_seq=True, S=S,
                  strategy=strategy, **ws.kwargs())
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), g["out"], dtype, f"{name} {strategy}")


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_golden_w8_append_and_attention(dev, fmt):
    import torch
    from cuda_gpt2_inference_amd import kvattn
    g = np.load(os.path.join(GOLDEN, f"g_{fmt}.npz"))
    B, NH, maxT = int(g["B"]), int(g["NH"]), int(g["maxT"])
    src = g["src"].reshape(maxT, -1)
    codes = torch.zeros(2 * B * NH * maxT * HS, dtype=torch.uint8, device=dev)
    scales = torch.zeros(2 * B * NH * maxT, dtype=torch.float32, device=dev)
    cur = torch.zeros(1, dtype=torch.int32, device=dev)
    for j in range(maxT):
        cur.fill_(j)
        kvattn.kv_cache_write(codes, _dev_tensor(np.ascontiguousarray(src[j]), dev), B, NH, HS, maxT,
                              kv_dtype=fmt, kv_scale=scales, cur_len=cur)
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy(), g["codes"])
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), g["scales"].view(np.uint32))
    qkv = _dev_tensor(np.ascontiguousarray(src[maxT - 1]), dev)
    for strategy, S in (("fused_single", 0), ("split_merge", 4), ("lastblock", 0), ("designated", 0),
                        ("designated", 3), ("coop", 3)):
        out = torch.empty(B * NH * HS, dtype=torch.bfloat16, device=dev)
        ws = kvattn.Workspace(B, NH, maxT, S)
        kvattn.decode(out, qkv, codes, B, NH, HS, maxT, kv_dtype=fmt, kv_scale=scales, cur_len=cur, S=S,
                      strategy=strategy, **ws.kwargs())
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), g["out"], fmt, f"{fmt} {strategy}")
