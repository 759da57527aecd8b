"""attn_tiled_causal_backward_f32_noalloc (D in the library's fixed device scratch, nothing
allocated) against attn_tiled_causal_backward_f32 (D in a caller workspace): bitwise equal
dq, dk, dv, on two calls in a row, the second with a smaller problem, so that a stale D
from the first call in the shared scratch would show."""
import pytest
import torch

from oracle import attention_ref as ref
from gpu_util import default_scale, to_dev

# Problems beyond the scratch are rejected before any launch; that validation is checked
# on the CPU (tests/test_capi.py), where no kernel can run.


def _case(lib, B, H, T, d, seed):
    scale = default_scale(d)
    q, k, v, do = (to_dev(x) for x in ref.seeded_inputs(B, H, T, d, seed=seed))
    r = B * H * T
    o, m, l = torch.empty_like(q), q.new_empty(r), q.new_empty(r)
    lib.tiled_causal_attention_forward(q, k, v, o, B, H, T, d, scale, m, l)
    want = [torch.empty_like(q) for _ in range(3)]
    ws = q.new_empty(r)
    lib.tiled_causal_attention_backward(q, k, v, o, do, m, l, *want, ws, B, H, T, d, scale)
    got = [torch.full_like(q, float("nan")) for _ in range(3)]
    lib.tiled_causal_attention_backward_noalloc(q, k, v, o, do, m, l, *got, B, H, T, d, scale)
    torch.cuda.synchronize()
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        assert torch.equal(g, w), f"{name}: no-alloc differs from the workspace entry point"
    # the scratch held D of this call: the workspace entry point's D, bitwise
    return ws


@pytest.mark.gpu
def test_noalloc_backward_two_calls_second_smaller(lib):
    _case(lib, 4, 12, 1024, 64, seed=5)   # 49,152 rows of D
    _case(lib, 2, 3, 333, 128, seed=6)    # 1,998 rows: a stale D from above would show
    _case(lib, 1, 2, 77, 32, seed=7)


@pytest.mark.gpu
def test_noalloc_backward_at_scratch_limit(lib):
    # B*H*T = 2^22 rows exactly: the largest problem the scratch holds
    _case(lib, 32, 1024, 128, 32, seed=8)
