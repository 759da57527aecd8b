"""bf16 fast path on the GPU.  Tolerance: rel-L2 <= 2e-2
(scripts/compare_parity.py:17 definition) on O, dQ, dK, dV against the fp32 restated
reference evaluated on the same bf16-rounded inputs.

At full config sizes the CPU oracle runs on a subset of heads (seconds), and every head
is compared with the fp32 GPU path on the same inputs, which the fp32 tests pin to the
oracle at max-abs <= 1e-5."""
import math

import numpy as np
import pytest
import torch

from gpu_util import default_scale, gpu_fwd_bwd, max_abs, rel_l2
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _rounded(B, H, T, d, seed, qk_scale=1.0):
    q, k, v, do = ref.seeded_inputs(B, H, T, d, seed=seed, qk_scale=qk_scale)
    return tuple(ref.bf16_round(x) for x in (q, k, v, do))


ZERO_ATOL = 1e-4  # where the exact answer is 0 (T = 1: dQ = dK = 0), rel-L2 is undefined


def _check(got, want, names=("o", "dq", "dk", "dv"), tol=TOL, tag=""):
    """rel-L2 <= tol per tensor; a reference that is zero to fp32 precision (its L2 norm
    below 1e-6 per element) is checked in max-abs against ZERO_ATOL instead."""
    errs = {}
    for n in names:
        w = want[n] if isinstance(want, dict) else getattr(want, n).numpy()
        if np.linalg.norm(np.asarray(w, np.float64)) <= 1e-6 * np.sqrt(w.size):
            e = max_abs(got[n], w)
            print(tag, n, f"reference ~0: max-abs {e:.2e}")
            assert e <= ZERO_ATOL, f"{tag} {n}: max-abs {e:.3e} > {ZERO_ATOL} (reference ~0)"
            continue
        errs[n] = rel_l2(got[n], w)
    print(tag, {k: f"{e:.2e}" for k, e in errs.items()})
    for n, e in errs.items():
        assert e <= tol, f"{tag} {n}: rel-L2 {e:.3e} > {tol}"
    return errs


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("T", [1, 17, 33, 64, 100, 160, 257])
def test_shapes_vs_oracle(lib, T, d):
    B, H = 2, 2
    q, k, v, do = _rounded(B, H, T, d, seed=T + d)
    scale = default_scale(d)
    want = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float32)
    got = gpu_fwd_bwd(lib, q, k, v, do, scale, dtype=torch.bfloat16)
    _check(got, want, tag=f"T={T} d={d}")
    # The forward holds Q times c = scale*log2 e rounded to bf16 (2^-9 relative per element),
    # so a score scale*q.k moves by at most 2^-9 scale sum_e |q_e k_e|, and the log-sum-exp
    # m + ln l by at most the largest such bound over the row's keys.  m is the forward's
    # reference value: the maximum over the row's first 32 keys (its scores moved the same
    # way, and carried to 16 bits), at most the row maximum.
    aq, ak = np.abs(q.astype(np.float64)), np.abs(k.astype(np.float64))
    bound = 2.0 ** -9 * scale * aq @ np.swapaxes(ak, -1, -2)
    causal = np.tril(np.ones((T, T), bool))
    bound = np.where(causal, bound, 0.0).max(-1) + 1e-6
    s = scale * q.astype(np.float64) @ np.swapaxes(k.astype(np.float64), -1, -2)
    first32 = np.where(causal & (np.arange(T) < 32)[None, :], s, -np.inf).max(-1)
    mag = np.abs(want.m.numpy()) * 2.0 ** -15
    assert np.all(got["m"] >= first32 - bound - mag), "m: at least the maximum over keys 0..31"
    assert np.all(got["m"] <= want.m.numpy() + bound + mag), "m: at most the row maximum"
    lse = got["m"] + np.log(got["l"])
    assert np.all(np.abs(lse - want.lse.numpy()) <= bound), "m + ln l"


@pytest.mark.parametrize("B,H,T,d", [(2, 4, 300, 64), (1, 8, 160, 128), (2, 8, 383, 32),
                                     (1, 16, 640, 64), (4, 64, 200, 64)])
def test_xcd_block_order_ragged_vs_oracle(lib, B, H, T, d):
    """B*H a multiple of 8: every kernel maps workgroups to heads XCD by XCD (serpentine
    rounds where the grid fits on the device at once, rank order where it does not; the
    head groups start at config 3's size, test_config3_full), at lengths that leave the last
    block of each head partly past T."""
    q, k, v, do = _rounded(B, H, T, d, seed=B * H + T + d)
    scale = default_scale(d)
    want = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float32)
    got = gpu_fwd_bwd(lib, q, k, v, do, scale, dtype=torch.bfloat16)
    _check(got, want, tag=f"B={B} H={H} T={T} d={d}")


def test_reference_kat(lib):
    T, d = 8, 32
    q = np.full((1, 1, T, d), 0.1, np.float32)
    v = np.ones_like(q)
    do = np.full_like(q, 0.5)
    got = gpu_fwd_bwd(lib, q, q, v, do, 1 / math.sqrt(d), dtype=torch.bfloat16)
    np.testing.assert_allclose(got["o"], 1.0, atol=0)
    np.testing.assert_allclose(got["dq"], 0.0, atol=1e-6)
    np.testing.assert_allclose(got["dk"], 0.0, atol=1e-6)
    want = np.array([sum(0.5 / (i + 1) for i in range(j, T)) for j in range(T)])
    np.testing.assert_allclose(got["dv"][0, 0], np.repeat(want[:, None], d, 1), rtol=8e-3)


def _full_config(lib, B, H, T, d, seed, qk_scale, oracle_heads):
    q, k, v, do = _rounded(B, H, T, d, seed, qk_scale)
    scale = default_scale(d)
    got = gpu_fwd_bwd(lib, q, k, v, do, scale, dtype=torch.bfloat16)
    for n in ("o", "dq", "dk", "dv"):
        assert np.isfinite(got[n]).all(), n
    # every head: against the fp32 GPU path on the same (bf16-valued) inputs
    f32 = gpu_fwd_bwd(lib, q, k, v, do, scale, dtype=torch.float32)
    _check(got, f32, tag="all heads vs fp32 path")
    # a subset of heads: against the CPU oracle
    for b, h in oracle_heads:
        sl = lambda x: x[b:b + 1, h:h + 1]
        want = ref.attention_fwd_bwd(sl(q), sl(k), sl(v), sl(do), scale, dtype=torch.float32)
        sub = {n: sl(got[n]) for n in ("o", "dq", "dk", "dv")}
        _check(sub, want, tag=f"head ({b},{h}) vs oracle")
        # The fp32 GPU path on this head, judged against fp64: at long T the fp32
        # summation noise of any fp32 implementation grows with T, so the bar is the
        # restated reference's own fp32 error (torch fp32 vs fp64), within 2x, floored at
        # the 1e-5 gate.
        want64 = ref.attention_fwd_bwd(sl(q), sl(k), sl(v), sl(do), scale, dtype=torch.float64)
        for n in ("o", "dq", "dk", "dv"):
            w64 = getattr(want64, n).numpy()
            ours = max_abs(sl(f32[n]), w64)
            theirs = max_abs(getattr(want, n).numpy(), w64)
            print(f"head ({b},{h}) fp32 {n}: |gpu-fp64| {ours:.2e}  |torch32-fp64| {theirs:.2e}")
            assert ours <= max(1e-5, 2.0 * theirs), n


def test_config3_full(lib):
    """B16 H16 T2048 d64, bf16 inputs from N(0,1), seed 42."""
    _full_config(lib, 16, 16, 2048, 64, 42, 1.0, oracle_heads=[(0, 0), (7, 9), (15, 15)])


def test_config4_full(lib):
    """B2 H16 T8192 d128, Q and K scaled by 0.5 (peaky softmax)."""
    _full_config(lib, 2, 16, 8192, 128, 42, 0.5, oracle_heads=[(0, 0), (1, 15)])


def _bf16(x):
    return ref.bf16_round(np.asarray(x, np.float32))


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("jump", [2.5, 9.0])
def test_reference_raise(lib, d, jump):
    """Scores that rise far above the first 32 keys' maximum later in the row: the first 32
    keys point away from q, every later key along it (scale*q.k = -jump^2, then +jump^2, in
    natural units, plus noise).  jump 2.5: rows from 32 on see their second block of keys
    ~18 (log2 units) above the first block's maximum, so the forward raises its reference
    value from the LDS tile; jump 9: ~234 above it, where 2^(s - m) overflows to inf before
    the raise.  O and the log-sum-exp are checked against a float64 restatement that rounds
    c*q to bf16 as the kernel holds it (the difference left is the bf16 P of the PV
    products); the backward's dK and dV against the fp32 oracle at the bf16 gate."""
    B, H, T = 1, 2, 256
    rng = np.random.default_rng(7 + d)
    u = rng.standard_normal((B, H, 1, d)).astype(np.float32)
    u /= np.linalg.norm(u, axis=-1, keepdims=True)
    a = jump * np.sqrt(np.sqrt(d))  # scale*q.k = a^2 / sqrt(d) = jump^2 along u
    noise = lambda n: 0.1 * rng.standard_normal((B, H, n, d)).astype(np.float32)
    q = _bf16(a * u + noise(T))
    k = np.concatenate([-a * u + noise(32), a * u + noise(T - 32)], axis=2)
    k = _bf16(k)
    v = _bf16(rng.standard_normal((B, H, T, d)))
    do = _bf16(rng.standard_normal((B, H, T, d)))
    scale = default_scale(d)
    got = gpu_fwd_bwd(lib, q, k, v, do, scale, dtype=torch.bfloat16)
    for n in ("o", "m", "l", "dq", "dk", "dv"):
        assert np.isfinite(got[n]).all(), n
    # forward against float64 with the kernel's bf16(c*q)
    c = np.float32(scale * math.log2(math.e))
    qc = _bf16(q * c).astype(np.float64) / np.float64(c)
    s = scale * qc @ np.swapaxes(k.astype(np.float64), -1, -2)
    s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
    lse = np.log(np.exp(s - s.max(-1, keepdims=True)).sum(-1)) + s.max(-1)
    o = np.exp(s - lse[..., None]) @ v.astype(np.float64)
    e = rel_l2(got["o"], o)
    rise = (s[..., 32:, :].max(-1) - s[..., 32:, :32].max(-1)).min() * math.log2(math.e)
    print(f"d={d} jump={jump}: O rel-L2 {e:.2e}, rows 32+: row max - first-32 max >= "
          f"{float(rise):.1f} (log2)")
    assert e <= 1e-2
    glse = got["m"] + np.log(got["l"])
    assert np.abs(glse - lse).max() <= 1e-3 * np.abs(lse).max() + 1e-3
    # The backward from these statistics: dK and dV (which take P from them directly)
    # within the bf16 gate of the fp32 oracle.  dQ is printed only: with scores of +-jump^2
    # its error is the backward's own bf16 rounding of c*K, 2^-9 of each score, multiplied by
    # the large keys it sums (2.8e-2 at d = 32, jump 2.5), whatever statistics it is given.
    want = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float32)
    print(f"raise d={d} jump={jump}: dQ rel-L2 {rel_l2(got['dq'], want.dq.numpy()):.2e}")
    if jump <= 2.5:
        _check(got, want, names=("dk", "dv"), tag=f"raise d={d}")
