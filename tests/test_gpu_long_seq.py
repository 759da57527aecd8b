"""The fp32 paths at long sequences (d = 64, T = 4096 and 8192): the fp32 MFMA path (its
two-stage and dS-first backwards) and the three-plane path (dS-first at d = 64) against the
fp64 restatement of the reference.  fp32 summation noise grows with T in any fp32
implementation, so each result's max-abs distance to fp64 is bounded by torch fp32's own
distance at the same shape: within 2x for the fp32 MFMA path (measured 0.7-1.2x: its
compensated tile sums) and within 3x for the three-plane path (measured: O 0.5-1.1x, dQ
1.6-2.5x, dK and dV 0.7-1.1x: they sum the whole query range in the MFMA accumulator, the
smaller terms of the last queries first), with no floor: a summation order that let the error
grow with T (the ascending walk measured 2.9-3.3x for dK and dV) fails here.  And bf16 at
T = 16384."""
import numpy as np
import pytest
import torch

from gpu_util import gpu_fwd_bwd, max_abs, rel_l2
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def heads(qkv, B, H, T, d):
    x = qkv.reshape(B, T, 3, H, d).permute(2, 0, 3, 1, 4)
    return x[0].contiguous(), x[1].contiguous(), x[2].contiguous()


def run_paths(lib, qkv, do, B, H, T, d, scale):
    """(o, dq, dk, dv) as CPU tensors of: the fp32 MFMA path with the two-stage and the
    dS-first backward, and the three-plane path."""
    dev = qkv.device
    o = torch.empty((B, H, T, d), device=dev)
    m = torch.empty((B, H, T), device=dev)
    l = torch.empty_like(m)
    lib.packed_causal_attention_forward(qkv, o, B, H, T, d, scale, m, l)
    out = {}
    two, D = torch.empty_like(qkv), torch.empty_like(m)
    lib.packed_causal_attention_backward(qkv, o, do, m, l, two, D, B, H, T, d, scale)
    ds = torch.empty(lib.f32_ds_workspace_bytes(B, H, T, d) // 4, device=dev)
    first, D1 = torch.empty_like(qkv), torch.empty_like(m)
    lib.packed_causal_attention_backward_ds(qkv, o, do, m, l, first, D1, ds, B, H, T, d, scale)
    torch.cuda.synchronize()
    del ds
    out["fp32 mfma"] = (o.cpu(),) + heads(two.cpu(), B, H, T, d)
    out["fp32 mfma, dS-first"] = (o.cpu(),) + heads(first.cpu(), B, H, T, d)
    planes = torch.empty(lib.f32x3_workspace_bytes(B, H, T, d), dtype=torch.uint8, device=dev)
    o3, m3, l3 = torch.empty_like(o), torch.empty_like(m), torch.empty_like(m)
    lib.packed_causal_attention_forward_f32x3(qkv, o3, B, H, T, d, scale, planes, m3, l3)
    x3, D3 = torch.empty_like(qkv), torch.empty_like(m)
    lib.packed_causal_attention_backward_f32x3(qkv, o3, do, m3, l3, x3, D3, B, H, T, d, scale,
                                               planes, True)
    torch.cuda.synchronize()
    out["three-plane"] = (o3.cpu(),) + heads(x3.cpu(), B, H, T, d)
    return out


@pytest.mark.parametrize("B,H,T", [(1, 2, 4096), (1, 1, 8192)])
def test_long_sequences_against_fp64(lib, B, H, T):
    d, scale = 64, 0.125
    g = torch.Generator(device="cpu").manual_seed(T + H)
    qkv = torch.randn((B, T, 3 * H * d), generator=g)
    do = torch.randn((B, H, T, d), generator=g)
    got = run_paths(lib, qkv.to("cuda:0"), do.to("cuda:0"), B, H, T, d, scale)
    q, k, v = heads(qkv, B, H, T, d)
    w32 = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float32)
    w64 = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float64)
    factor = {"fp32 mfma": 2.0, "fp32 mfma, dS-first": 2.0, "three-plane": 3.0}
    for path, res in got.items():
        for n, x in zip(("o", "dq", "dk", "dv"), res):
            w = getattr(w64, n).numpy()
            ours, theirs = max_abs(x.numpy(), w), max_abs(getattr(w32, n).numpy(), w)
            print(f"T={T} {path} {n}: |gpu-fp64| {ours:.2e}  |torch32-fp64| {theirs:.2e}")
            assert np.isfinite(x.numpy()).all(), f"{path} {n}"
            assert ours <= factor[path] * theirs, f"{path} {n}: {ours:.3e}"


def test_bf16_long_sequence_against_oracle(lib):
    """bf16 at B1 H2 T16384 d64 (two heads: the block mapping without XCD grouping, 128 query
    blocks per head), head (0, 1) against the fp32 restatement on the same bf16-rounded
    inputs at the bf16 gate (rel-L2 <= 2e-2, scripts/compare_parity.py:17)."""
    B, H, T, d = 1, 2, 16384, 64
    q, k, v, do = (ref.bf16_round(x) for x in ref.seeded_inputs(B, H, T, d, seed=16))
    scale = 0.125
    got = gpu_fwd_bwd(lib, q, k, v, do, scale, dtype=torch.bfloat16)
    for n in ("o", "dq", "dk", "dv"):
        assert np.isfinite(got[n]).all(), n
    sl = lambda x: x[:, 1:2]
    want = ref.attention_fwd_bwd(sl(q), sl(k), sl(v), sl(do), scale, dtype=torch.float32)
    for n in ("o", "dq", "dk", "dv"):
        e = rel_l2(sl(got[n]), getattr(want, n).numpy())
        print(f"bf16 T={T} head (0,1) {n}: rel-L2 {e:.2e}")
        assert e <= 2e-2, f"{n}: rel-L2 {e:.3e}"
