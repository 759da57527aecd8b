"""Materialised fused causal softmax forward/backward on the GPU vs the C restatement of
the reference kernel and torch (register path T <= 2048, streaming path above)."""
import numpy as np
import pytest
import torch

from gpu_util import to_dev
from oracle import attention_ref as ref
from oracle import c_oracle as co

pytestmark = pytest.mark.gpu


def test_reference_kat(lib):
    """tests/test_kernels.cu:91-120: all scores 1, scale 1, T = 4."""
    s = torch.ones(16, device="cuda:0")
    p = torch.empty_like(s)
    lib.causal_softmax_forward(s, p, 1, 1, 4, 1.0)
    torch.cuda.synchronize()
    p = p.cpu().numpy().reshape(4, 4)
    want = np.tril(np.ones((4, 4))) / np.arange(1, 5)[:, None]
    np.testing.assert_allclose(p, want, atol=1e-7)


@pytest.mark.parametrize("B,H,T", [(1, 1, 1), (2, 3, 7), (1, 2, 64), (2, 2, 301), (1, 1, 1024),
                                   (1, 1, 2052), (1, 1, 4100), (1, 1, 2050)])
def test_forward_backward_vs_oracle(lib, B, H, T):
    rng = np.random.default_rng(T)
    s = (rng.standard_normal((B, H, T, T)) * 3).astype(np.float32)
    dp = rng.standard_normal((B, H, T, T)).astype(np.float32)
    scale = 0.37
    sg, dpg = to_dev(s), to_dev(dp)
    pg = torch.full_like(sg, float("nan"))  # every element must be written
    lib.causal_softmax_forward(sg, pg, B, H, T, scale)
    dsg = torch.full_like(sg, float("nan"))
    lib.causal_softmax_backward(dpg, pg, dsg, B, H, T, scale)
    torch.cuda.synchronize()
    p = pg.cpu().numpy()
    ds = dsg.cpu().numpy()
    att = torch.from_numpy(s) * scale
    att = att.masked_fill(ref.causal_mask(T) == 0, float("-inf"))
    np.testing.assert_allclose(p, torch.softmax(att, -1).numpy(), atol=1e-6)
    upper = np.triu(np.ones((T, T), bool), 1)
    assert np.all(p[..., upper] == 0) and np.all(ds[..., upper] == 0)
    if T <= 301:
        np.testing.assert_allclose(p, co.causal_softmax_fwd(s, B, H, T, scale), atol=2e-7)
        np.testing.assert_allclose(ds, co.causal_softmax_bwd(dp, p, B, H, T, scale), atol=2e-6)
    else:
        p64 = p.astype(np.float64)
        dpm = np.where(upper, 0.0, dp.astype(np.float64))
        want = scale * p64 * (dpm - (dpm * p64).sum(-1, keepdims=True))
        np.testing.assert_allclose(ds, want, atol=2e-6)


def test_odd_T_scalar_path_and_offset_pointer(lib):
    B, H, T = 1, 2, 13
    s = np.random.default_rng(1).standard_normal((B * H * T * T,)).astype(np.float32)
    base = torch.zeros(s.size + 1, device="cuda:0")
    base[1:] = to_dev(s)
    out = torch.zeros(s.size + 1, device="cuda:0")
    lib.causal_softmax_forward(base[1:], out[1:], B, H, T, 1.0)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out[1:].cpu().numpy(), co.causal_softmax_fwd(s, B, H, T, 1.0),
                               atol=2e-7)


@pytest.mark.parametrize("T,zb", [(300, 128), (1024, 128), (2052, 128), (13, 4), (64, 8)])
def test_blocked_zeros(lib, T, zb):
    """zero_block: the written part of every row equals the full-suffix pass bitwise, the
    zeros stop at the end of the zero_block-column block holding the diagonal, and the rest of
    the row keeps what was there (register and streaming paths, vector and scalar rows)."""
    B, H = 1, 2
    rng = np.random.default_rng(T + zb)
    sg = to_dev((rng.standard_normal((B, H, T, T)) * 3).astype(np.float32))
    dpg = to_dev(rng.standard_normal((B, H, T, T)).astype(np.float32))
    scale = 0.37
    p_full, ds_full = torch.empty_like(sg), torch.empty_like(sg)
    lib.causal_softmax_forward(sg, p_full, B, H, T, scale)
    lib.causal_softmax_backward(dpg, p_full, ds_full, B, H, T, scale)
    p_blk = torch.full_like(sg, float("nan"))
    ds_blk = torch.full_like(sg, float("nan"))
    lib.causal_softmax_forward(sg, p_blk, B, H, T, scale, zero_block=zb)
    lib.causal_softmax_backward(dpg, p_full, ds_blk, B, H, T, scale, zero_block=zb)
    torch.cuda.synchronize()
    i = torch.arange(T, device="cuda:0")
    written = i[None, :] < torch.clamp((i[:, None] // zb + 1) * zb, max=T)
    for full, blk in ((p_full, p_blk), (ds_full, ds_blk)):
        assert torch.equal(blk[..., written], full[..., written])
        assert torch.isnan(blk[..., ~written]).all()
