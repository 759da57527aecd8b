"""Pins the plain-C restatement of the reference kernels (oracle/tiled_ref.c) against the
torch/numpy oracle and against index maps written independently with numpy reshapes."""
import math

import numpy as np
import pytest
import torch

from oracle import attention_ref as ref
from oracle import c_oracle as co


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("B,T,H,d", [(2, 5, 3, 4), (1, 1, 1, 1), (3, 17, 2, 7)])
def test_split_transpose_index_map(B, T, H, d):
    qkv = _rand((B, T, 3 * H * d), 1)
    q, k, v = co.qkv_split_fwd(qkv, B, T, H, d)
    # model.py:35-41: qkv.chunk(3, -1) then view(B, T, H, d).transpose(1, 2)
    want = qkv.reshape(B, T, 3, H, d).transpose(2, 0, 3, 1, 4)
    np.testing.assert_array_equal(q, want[0])
    np.testing.assert_array_equal(k, want[1])
    np.testing.assert_array_equal(v, want[2])
    np.testing.assert_array_equal(co.qkv_split_bwd(q, k, v, B, T, H, d), qkv)


def test_head_merge_index_map():
    B, H, T, d = 2, 3, 5, 4
    x = _rand((B, H, T, d), 2)
    merged = co.head_merge_fwd(x, B, H, T, d)
    np.testing.assert_array_equal(merged, x.transpose(0, 2, 1, 3).reshape(B, T, H * d))
    np.testing.assert_array_equal(co.head_merge_bwd(merged, B, H, T, d), x)


def test_causal_softmax_kat_and_torch():
    p = co.causal_softmax_fwd(np.ones((4, 4), np.float32), 1, 1, 4, 1.0)
    assert abs(p[0, 0] - 1) < 1e-5 and abs(p[1, 0] - 0.5) < 1e-4 and p[1, 2] == 0
    B, H, T = 2, 2, 33
    s = _rand((B, H, T, T), 3)
    p = co.causal_softmax_fwd(s, B, H, T, 0.3)
    att = torch.from_numpy(s) * 0.3
    att = att.masked_fill(ref.causal_mask(T) == 0, float("-inf"))
    np.testing.assert_allclose(p, torch.softmax(att, -1).numpy(), atol=2e-7)
    dp = _rand((B, H, T, T), 4)
    ds = co.causal_softmax_bwd(dp, p, B, H, T, 0.3)
    p64, dp64 = p.astype(np.float64), dp.astype(np.float64)
    dp64 = np.where(np.tril(np.ones((T, T))) > 0, dp64, 0)
    want = 0.3 * p64 * (dp64 - (dp64 * p64).sum(-1, keepdims=True))
    np.testing.assert_allclose(ds, want, atol=1e-6)


@pytest.mark.parametrize("T,d", [(1, 32), (7, 32), (40, 64), (70, 128)])
def test_tiled_matches_torch_oracle(T, d):
    B, H = 2, 2
    q, k, v, do = (_rand((B, H, T, d), s) for s in range(4))
    scale = 1 / math.sqrt(d)
    o, m, l = co.tiled_fwd(q, k, v, scale)
    r = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float32)
    np.testing.assert_allclose(o, r.o.numpy(), atol=2e-6)
    np.testing.assert_allclose(m, r.m.numpy(), atol=1e-6)
    np.testing.assert_allclose(l, r.l.numpy(), rtol=1e-5)
    dq, dk, dv, D = co.tiled_bwd(q, k, v, o, do, m, l, scale)
    np.testing.assert_allclose(D, (r.o.numpy() * do).sum(-1), atol=1e-5)
    np.testing.assert_allclose(dq, r.dq.numpy(), atol=1e-5)
    np.testing.assert_allclose(dk, r.dk.numpy(), atol=1e-5)
    np.testing.assert_allclose(dv, r.dv.numpy(), atol=1e-5)


def test_tiled_reference_kat():
    T, d = 8, 32
    q = np.full((1, 1, T, d), 0.1, np.float32)
    v = np.ones_like(q)
    do = np.full_like(q, 0.5)
    o, m, l = co.tiled_fwd(q, q, v, 1 / math.sqrt(d))
    np.testing.assert_allclose(o, 1.0, atol=1e-6)
    dq, dk, dv, _ = co.tiled_bwd(q, q, v, o, do, m, l, 1 / math.sqrt(d))
    np.testing.assert_allclose(dq, 0, atol=1e-6)
    np.testing.assert_allclose(dk, 0, atol=1e-6)
    want = np.array([sum(0.5 / (i + 1) for i in range(j, T)) for j in range(T)])
    np.testing.assert_allclose(dv[0, 0], np.repeat(want[:, None], d, 1), rtol=1e-6)
