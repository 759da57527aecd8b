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


def fused(lib, qkv, do_merged, B, H, T, d, scale, stages=False):
    dt = qkv.dtype
    o = torch.full((B, T, H * d), float("nan"), device="cuda:0", dtype=dt)
    m = torch.full((B, H, T), float("nan"), device="cuda:0")
    l = torch.full_like(m, float("nan"))
    lib.fused_causal_attention_forward(qkv, o, B, H, T, d, scale, m, l)
    dqkv = torch.full_like(qkv, float("nan"))
    ws = torch.full_like(m, float("nan"))
    if stages:
        lib.fused_causal_attention_backward_dq(qkv, o, do_merged, m, l, dqkv, ws, B, H, T, d,
                                               scale)
        lib.fused_causal_attention_backward_dkdv(qkv, do_merged, m, l, ws, dqkv, B, H, T, d,
                                                 scale)
    else:
        lib.fused_causal_attention_backward(qkv, o, do_merged, m, l, dqkv, ws, B, H, T, d,
                                            scale)
    return o, m, l, dqkv, ws


@pytest.mark.parametrize("stages", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,T,d", [(1, 1, 1, 64), (2, 3, 17, 32), (2, 2, 257, 128),
                                     (2, 4, 640, 64), (8, 12, 1024, 64)])
def test_fused_bitwise_equals_packed_with_head_merge(lib, dtype, stages, B, H, T, d):
    """Output in the merged-heads layout (B, T, H*d) and gradient read from it: bitwise the
    packed path with the head merge (a permutation) applied to O and undone on dO."""
    g = torch.Generator(device="cpu").manual_seed(T * 11 + d + H)
    qkv = torch.randn((B, T, 3 * H * d), generator=g).to("cuda:0", dtype)
    do_merged = torch.randn((B, T, H * d), generator=g).to("cuda:0", dtype)
    do_heads = do_merged.view(B, T, H, d).permute(0, 2, 1, 3).contiguous()
    scale = default_scale(d)
    o_p, m_p, l_p, dqkv_p, ws_p = packed(lib, qkv, do_heads, B, H, T, d, scale)
    o_f, m_f, l_f, dqkv_f, ws_f = fused(lib, qkv, do_merged, B, H, T, d, scale, stages)
    torch.cuda.synchronize()
    assert torch.equal(o_f, o_p.permute(0, 2, 1, 3).reshape(B, T, H * d)), "O (merged)"
    for name, w, x in (("m", m_p, m_f), ("l", l_p, l_f), ("dqkv", dqkv_p, dqkv_f),
                       ("D", ws_p, ws_f)):
        assert torch.equal(w, x), f"{name}: fused differs from packed + head merge"


def test_fused_matches_reference_head_merge_launcher(lib):
    """fp32: the fused forward's output equals head_merge_transpose_forward applied to the
    packed output (the reference's model.cu:336 step) bitwise."""
    B, H, T, d = 2, 3, 70, 64
    g = torch.Generator(device="cpu").manual_seed(5)
    qkv = torch.randn((B, T, 3 * H * d), generator=g).to("cuda:0")
    scale = default_scale(d)
    o = torch.empty((B, H, T, d), device="cuda:0")
    lib.packed_causal_attention_forward(qkv, o, B, H, T, d, scale)
    merged = torch.full((B, T, H * d), float("nan"), device="cuda:0")
    lib.head_merge_transpose_forward(o, merged, B, H, T, d)
    o_f = torch.full_like(merged, float("nan"))
    lib.fused_causal_attention_forward(qkv, o_f, B, H, T, d, scale)
    torch.cuda.synchronize()
    assert torch.equal(o_f, merged)
