"""Attention from the packed QKV layout (the split-transpose fused into the attention
kernels): bitwise equal to split-transpose + the tiled entry points + split-back."""
import numpy as np
import pytest
import torch

from gpu_util import default_scale

pytestmark = pytest.mark.gpu


def unfused(lib, qkv, do, B, H, T, d, scale):
    dt = qkv.dtype
    q, k, v = (torch.empty((B, H, T, d), device="cuda:0", dtype=dt) for _ in range(3))
    lib.qkv_split_transpose_forward(qkv, q, k, v, B, T, H, d)
    o, m, l = lib.attention_forward(q, k, v, scale)
    dq, dk, dv, ws = lib.attention_backward(q, k, v, o, do, m, l, scale)
    dqkv = torch.empty_like(qkv)
    lib.qkv_split_transpose_backward(dq, dk, dv, dqkv, B, T, H, d)
    return o, m, l, dqkv, ws


def packed(lib, qkv, do, B, H, T, d, scale):
    dt = qkv.dtype
    o = torch.full((B, H, T, d), float("nan"), device="cuda:0", dtype=dt)
    m = torch.full((B, H, T), float("nan"), device="cuda:0")
    l = torch.full_like(m, float("nan"))
    lib.packed_causal_attention_forward(qkv, o, B, H, T, d, scale, m, l)
    dqkv = torch.full_like(qkv, float("nan"))
    ws = torch.full_like(m, float("nan"))
    lib.packed_causal_attention_backward(qkv, o, do, m, l, dqkv, ws, B, H, T, d, scale)
    return o, m, l, dqkv, ws


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,T,d", [(1, 1, 1, 64), (2, 3, 17, 32), (1, 2, 100, 64),
                                     (2, 2, 257, 128), (2, 4, 640, 64), (16, 16, 2048, 64)])
def test_packed_bitwise_equals_split_then_tiled(lib, dtype, B, H, T, d):
    g = torch.Generator(device="cpu").manual_seed(T * 7 + d)
    qkv = torch.randn((B, T, 3 * H * d), generator=g).to("cuda:0", dtype)
    do = torch.randn((B, H, T, d), generator=g).to("cuda:0", dtype)
    scale = default_scale(d)
    want = unfused(lib, qkv, do, B, H, T, d, scale)
    got = packed(lib, qkv, do, B, H, T, d, scale)
    torch.cuda.synchronize()
    for name, w, x in zip(("o", "m", "l", "dqkv", "D"), want, got):
        assert torch.equal(w, x), f"{name}: packed differs from split + tiled"
