"""The fp32 MFMA backward in the dS-first order (attn_*_causal_backward_ds_f32 and its three
stages): dK/dV write dS, dQ is computed from it.  Against the two-stage order (the same D, dK
and dV bitwise, dQ within fp32 rounding), the CPU oracle, and fp64 at config 2."""
import numpy as np
import pytest
import torch

from gpu_util import default_scale, max_abs
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

TOL = 1e-5  # the fp32 gate (max-abs against the torch-fp32 restatement)


def heads(qkv, B, H, T, d):
    x = qkv.reshape(B, T, 3, H, d).permute(2, 0, 3, 1, 4)
    return x[0].contiguous(), x[1].contiguous(), x[2].contiguous()


def forward(lib, qkv, B, H, T, d, scale, merged):
    shape = (B, T, H * d) if merged else (B, H, T, d)
    o = torch.full(shape, float("nan"), device="cuda:0")
    m = torch.full((B, H, T), float("nan"), device="cuda:0")
    l = torch.full_like(m, float("nan"))
    fwd = lib.fused_causal_attention_forward if merged else lib.packed_causal_attention_forward
    fwd(qkv, o, B, H, T, d, scale, m, l)
    return o, m, l


def ds_area(lib, B, H, T, d):
    """The dS workspace, filled with NaNs: every element the dQ stage reads is written first."""
    n = lib.f32_ds_workspace_bytes(B, H, T, d)
    assert n == B * H * ((T + 31) // 32 * 32) ** 2 * 4
    return torch.full((n // 4,), float("nan"), device="cuda:0")


def both_orders(lib, qkv, do, B, H, T, d, scale, merged):
    fam = "fused" if merged else "packed"
    o, m, l = forward(lib, qkv, B, H, T, d, scale, merged)
    if merged:
        do = do.permute(0, 2, 1, 3).reshape(B, T, H * d).contiguous()
    two, D2 = torch.full_like(qkv, float("nan")), torch.full_like(m, float("nan"))
    getattr(lib, f"{fam}_causal_attention_backward")(qkv, o, do, m, l, two, D2, B, H, T, d,
                                                     scale)
    one, D1 = torch.full_like(qkv, float("nan")), torch.full_like(m, float("nan"))
    getattr(lib, f"{fam}_causal_attention_backward_ds")(qkv, o, do, m, l, one, D1,
                                                        ds_area(lib, B, H, T, d), B, H, T, d,
                                                        scale)
    torch.cuda.synchronize()
    return o, two, D2, one, D1


# (1, 2, 2048, 64) and (1, 2, 2080, 64): either side of the length where the d = 64 kernels
# change from the shared-tile to the per-wave form
SHAPES = [(1, 1, 1, 64), (2, 3, 17, 32), (1, 2, 100, 64), (2, 2, 257, 128), (2, 4, 640, 64),
          (1, 1, 1000, 32), (2, 3, 300, 128), (1, 2, 2048, 64), (1, 2, 2080, 64)]


@pytest.mark.parametrize("B,H,T,d", SHAPES)
@pytest.mark.parametrize("merged", [False, True])
def test_ds_order_against_two_stage_and_oracle(lib, B, H, T, d, merged):
    g = torch.Generator(device="cpu").manual_seed(T * 11 + d)
    qkv = torch.randn((B, T, 3 * H * d), generator=g)
    do = torch.randn((B, H, T, d), generator=g)
    scale = default_scale(d)
    o, two, D2, one, D1 = both_orders(lib, qkv.to("cuda:0"), do.to("cuda:0"), B, H, T, d,
                                      scale, merged)
    C = H * d
    assert torch.equal(D1, D2), "D differs from the two-stage order's"
    assert torch.equal(one[..., C:], two[..., C:]), "dK/dV differ from the two-stage order's"
    dq1, dq2 = one[..., :C], two[..., :C]
    assert torch.isfinite(dq1).all()
    assert (dq1 - dq2).abs().max().item() <= 2e-6 * max(dq2.abs().max().item(), 1.0)
    q, k, v = heads(qkv, B, H, T, d)
    want = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float32)
    got = dict(zip(("dq", "dk", "dv"), heads(one.cpu(), B, H, T, d)))
    for n in ("dq", "dk", "dv"):
        e = max_abs(got[n].numpy(), getattr(want, n).numpy())
        assert e <= TOL, f"{n}: max-abs {e:.3e}"


@pytest.mark.parametrize("merged", [False, True])
def test_three_stages_equal_one_call(lib, merged):
    B, H, T, d = 2, 3, 333, 64
    g = torch.Generator(device="cpu").manual_seed(23)
    qkv = torch.randn((B, T, 3 * H * d), generator=g).to("cuda:0")
    do = torch.randn((B, H, T, d), generator=g).to("cuda:0")
    scale = 0.125
    fam = "fused" if merged else "packed"
    o, m, l = forward(lib, qkv, B, H, T, d, scale, merged)
    if merged:
        do = do.permute(0, 2, 1, 3).reshape(B, T, H * d).contiguous()
    one, D1 = torch.full_like(qkv, float("nan")), torch.full_like(m, float("nan"))
    getattr(lib, f"{fam}_causal_attention_backward_ds")(qkv, o, do, m, l, one, D1,
                                                        ds_area(lib, B, H, T, d), B, H, T, d,
                                                        scale)
    three, D3 = torch.full_like(qkv, float("nan")), torch.full_like(m, float("nan"))
    ds = ds_area(lib, B, H, T, d)
    getattr(lib, f"{fam}_causal_attention_backward_prep")(o, do, D3, B, H, T, d)
    getattr(lib, f"{fam}_causal_attention_backward_dkdv_ds")(qkv, do, m, l, D3, three, ds, B, H,
                                                             T, d, scale)
    lib.causal_attention_backward_dq_ds(qkv, three, ds, B, H, T, d, scale)
    torch.cuda.synchronize()
    assert torch.isfinite(one).all()
    assert torch.equal(one, three) and torch.equal(D1, D3)


def test_config2_against_fp64(lib):
    """BASELINE config 2 (B8 H12 T1024 d64): within the gate of torch fp32, and dQ as close to
    fp64 as the two-stage order's (max-abs within 1.5x, rms within 1.1x)."""
    B, H, T, d = 8, 12, 1024, 64
    g = torch.Generator(device="cpu").manual_seed(42)
    qkv = torch.randn((B, T, 3 * H * d), generator=g)
    do = torch.randn((B, H, T, d), generator=g)
    o, two, D2, one, D1 = both_orders(lib, qkv.to("cuda:0"), do.to("cuda:0"), B, H, T, d, 0.125,
                                      False)
    q, k, v = heads(qkv, B, H, T, d)
    want = ref.attention_fwd_bwd(q, k, v, do, 0.125, dtype=torch.float32)
    w64 = ref.attention_fwd_bwd(q, k, v, do, 0.125, dtype=torch.float64)
    got = dict(zip(("dq", "dk", "dv"), heads(one.cpu(), B, H, T, d)))
    old = dict(zip(("dq", "dk", "dv"), heads(two.cpu(), B, H, T, d)))
    rms = lambda a, b: float(np.sqrt(np.mean((a.astype(np.float64) - b) ** 2)))
    for n in ("dq", "dk", "dv"):
        assert max_abs(got[n].numpy(), getattr(want, n).numpy()) <= TOL
    w = w64.dq.numpy()
    e = (max_abs(got["dq"].numpy(), w), max_abs(old["dq"].numpy(), w))
    r = (rms(got["dq"].numpy(), w), rms(old["dq"].numpy(), w))
    print(f"config2 dq to fp64 (dS-first, two-stage): max-abs {e[0]:.2e} {e[1]:.2e}, "
          f"rms {r[0]:.2e} {r[1]:.2e}")
    assert e[0] <= 1.5 * e[1] and r[0] <= 1.1 * r[1]
