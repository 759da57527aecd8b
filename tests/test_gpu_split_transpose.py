"""QKV split-transpose and head merge on the GPU: bit-exact against the C oracle / numpy
permutation (index work), round trips, casts against torch's round-to-nearest-even."""
import numpy as np
import pytest
import torch

from gpu_util import to_dev
from oracle import c_oracle as co

pytestmark = pytest.mark.gpu

SHAPES = [  # (B, T, H, d): vector paths, element path (d=3, d=6), T=1, config sizes
    (2, 37, 3, 64), (1, 1, 1, 32), (3, 5, 2, 3), (2, 9, 4, 6), (1, 17, 2, 128),
    (8, 1024, 12, 64),
]


def _split_np(qkv, B, T, H, d):
    return qkv.reshape(B, T, 3, H, d).transpose(2, 0, 3, 1, 4)


@pytest.mark.parametrize("B,T,H,d", SHAPES)
def test_split_f32_bit_exact(lib, B, T, H, d):
    rng = np.random.default_rng(B * 1000 + T)
    qkv = rng.standard_normal((B, T, 3 * H * d)).astype(np.float32)
    g = to_dev(qkv)
    q, k, v = (torch.empty((B, H, T, d), device="cuda:0") for _ in range(3))
    lib.qkv_split_transpose_forward(g, q, k, v, B, T, H, d)
    back = torch.empty_like(g)
    lib.qkv_split_transpose_backward(q, k, v, back, B, T, H, d)
    torch.cuda.synchronize()
    want = _split_np(qkv, B, T, H, d)
    for got, w in zip((q, k, v), want):
        np.testing.assert_array_equal(got.cpu().numpy(), w)
    np.testing.assert_array_equal(back.cpu().numpy(), qkv)
    if B * T * H * d <= 1 << 16:
        cq, ck, cv = co.qkv_split_fwd(qkv, B, T, H, d)
        np.testing.assert_array_equal(q.cpu().numpy(), cq)


def test_split_misaligned_views_take_element_path(lib):
    B, T, H, d = 2, 11, 3, 64
    n = B * T * H * d
    base = torch.randn(3 * n + 1, device="cuda:0")
    qkv = base[1:]  # 4-byte offset: not 16-byte aligned
    outs = torch.empty(3 * n + 1, device="cuda:0")
    q = outs[1:n + 1]
    k = torch.empty(n, device="cuda:0")
    v = torch.empty(n, device="cuda:0")
    lib.qkv_split_transpose_forward(qkv, q, k, v, B, T, H, d)
    torch.cuda.synchronize()
    want = _split_np(qkv.cpu().numpy(), B, T, H, d)
    np.testing.assert_array_equal(q.cpu().numpy().reshape(B, H, T, d), want[0])
    np.testing.assert_array_equal(v.cpu().numpy().reshape(B, H, T, d), want[2])


@pytest.mark.parametrize("B,T,H,d", [(2, 37, 3, 64), (16, 2048, 16, 64), (1, 9, 2, 128), (2, 5, 3, 6)])
def test_split_bf16_and_casts(lib, B, T, H, d):
    rng = np.random.default_rng(7)
    qkv32 = rng.standard_normal((B, T, 3 * H * d)).astype(np.float32)
    g32 = to_dev(qkv32)
    g16 = g32.to(torch.bfloat16)
    want16 = [torch.from_numpy(np.ascontiguousarray(x)) for x in _split_np(qkv32, B, T, H, d)]
    want16 = [x.to(torch.bfloat16) for x in want16]  # torch RNE cast, then permutation
    # bf16 -> bf16
    outs = [torch.empty((B, H, T, d), device="cuda:0", dtype=torch.bfloat16) for _ in range(3)]
    lib.qkv_split_transpose_forward(g16, *outs, B, T, H, d)
    # f32 -> bf16 (fused RNE cast)
    outs_c = [torch.empty((B, H, T, d), device="cuda:0", dtype=torch.bfloat16) for _ in range(3)]
    lib.qkv_split_transpose_forward(g32, *outs_c, B, T, H, d)
    # bf16 -> bf16 backward and bf16 -> f32 backward
    back16 = torch.empty_like(g16)
    lib.qkv_split_transpose_backward(*outs, back16, B, T, H, d)
    back32 = torch.empty_like(g32)
    lib.qkv_split_transpose_backward(*outs, back32, B, T, H, d)
    torch.cuda.synchronize()
    for a, b, w in zip(outs, outs_c, want16):
        assert torch.equal(a.cpu().view(torch.int16), w.view(torch.int16))
        assert torch.equal(b.cpu().view(torch.int16), w.view(torch.int16))
    assert torch.equal(back16.cpu().view(torch.int16), g16.cpu().view(torch.int16))
    assert torch.equal(back32.cpu(), g16.float().cpu())


@pytest.mark.parametrize("B,H,T,d", [(2, 3, 37, 64), (1, 2, 5, 3), (8, 12, 1024, 64)])
def test_head_merge_bit_exact(lib, B, H, T, d):
    x = np.random.default_rng(3).standard_normal((B, H, T, d)).astype(np.float32)
    g = to_dev(x)
    merged = torch.empty((B, T, H * d), device="cuda:0")
    lib.head_merge_transpose_forward(g, merged, B, H, T, d)
    back = torch.empty_like(g)
    lib.head_merge_transpose_backward(merged, back, B, H, T, d)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(merged.cpu().numpy(), x.transpose(0, 2, 1, 3).reshape(B, T, H * d))
    np.testing.assert_array_equal(back.cpu().numpy(), x)
