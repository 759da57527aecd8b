"""Pins the CPU oracle (oracle/attention_ref.py) against facts that do not come from its
own formulas: the reference's known-answer tests, closed forms, fp64 central finite
differences, invariants, and an element-by-element loop restatement.  A planted mistake
in a copy of the oracle must fail at least one of these checks."""
import math

import numpy as np
import pytest
import torch

from oracle import attention_ref as ref


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


# ---------------------------------------------------------------------------- reference KATs
def test_reference_kat_causal_softmax():
    """tests/test_kernels.cu:91-120: B=H=1, T=4, all scores 1, scale 1."""
    T = 4
    att = torch.ones(1, 1, T, T).masked_fill(ref.causal_mask(T) == 0, float("-inf"))
    p = torch.softmax(att, dim=-1)[0, 0]
    assert abs(p[0, 0] - 1.0) < 1e-5 and abs(p[0, 1]) < 1e-5
    assert abs(p[1, 0] - 0.5) < 1e-4 and abs(p[1, 1] - 0.5) < 1e-4 and abs(p[1, 2]) < 1e-5


def test_reference_kat_tiled_attention_exact():
    """tests/test_kernels.cu:210-284 (T=8, d=32, q=k=0.1, v=1, dO=0.5), with its exact
    answer: O = 1, dQ = dK = 0, dV_j = 0.5 * sum_{i=j}^{7} 1/(i+1)."""
    T, d = 8, 32
    q = np.full((1, 1, T, d), 0.1)
    v = np.ones((1, 1, T, d))
    do = np.full((1, 1, T, d), 0.5)
    r = ref.attention_fwd_bwd(q, q, v, do, 1 / math.sqrt(d), dtype=torch.float64)
    np.testing.assert_allclose(r.o.numpy(), 1.0, atol=1e-12)
    np.testing.assert_allclose(r.dq.numpy(), 0.0, atol=1e-12)
    np.testing.assert_allclose(r.dk.numpy(), 0.0, atol=1e-12)
    want = np.array([sum(0.5 / (i + 1) for i in range(j, T)) for j in range(T)])
    np.testing.assert_allclose(r.dv.numpy()[0, 0], np.repeat(want[:, None], d, 1), rtol=1e-12)


# ----------------------------------------------------------------------------- closed forms
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_zero_query_prefix_means(dtype):
    """Q = 0 => P_ij = 1/(i+1): O_i = mean(v_0..v_i), m_i = 0, l_i = i+1, LSE_i = ln(i+1)."""
    B, H, T, d = 2, 3, 37, 16
    k, v = _rand((B, H, T, d), 1), _rand((B, H, T, d), 2)
    q = np.zeros_like(k)
    r = ref.attention_fwd_bwd(q, k, v, v, 0.25, dtype=dtype)
    tol = 1e-6 if dtype == torch.float32 else 1e-13
    prefix = np.cumsum(v, axis=2) / np.arange(1, T + 1)[:, None]
    np.testing.assert_allclose(r.o.numpy(), prefix, atol=tol)
    np.testing.assert_allclose(r.m.numpy(), 0.0, atol=0)
    np.testing.assert_allclose(r.l.numpy(), np.broadcast_to(np.arange(1, T + 1), (B, H, T)),
                               rtol=tol)
    np.testing.assert_allclose(r.lse.numpy(), np.log(np.arange(1, T + 1)) + 0 * r.lse.numpy(),
                               atol=tol)


def test_single_position_returns_v():
    q, k, v, do = (_rand((2, 2, 1, 8), s) for s in range(4))
    r = ref.attention_fwd_bwd(q, k, v, do, 0.3, dtype=torch.float64)
    np.testing.assert_allclose(r.o.numpy(), v, atol=0)
    np.testing.assert_allclose(r.dq.numpy(), 0.0, atol=1e-15)  # softmax of one entry
    np.testing.assert_allclose(r.dv.numpy(), do, atol=1e-15)


def test_constant_v_gives_zero_dq_dk():
    q, k, do = (_rand((1, 2, 19, 8), s) for s in range(3))
    v = np.full_like(q, 1.75)
    r = ref.attention_fwd_bwd(q, k, v, do, 0.5, dtype=torch.float64)
    np.testing.assert_allclose(r.o.numpy(), 1.75, atol=1e-14)
    np.testing.assert_allclose(r.dq.numpy(), 0.0, atol=1e-13)
    np.testing.assert_allclose(r.dk.numpy(), 0.0, atol=1e-13)


def test_zero_upstream_gives_zero_grads():
    q, k, v = (_rand((1, 1, 9, 4), s) for s in range(3))
    r = ref.attention_fwd_bwd(q, k, v, np.zeros_like(q), 0.5, dtype=torch.float64)
    for g in (r.dq, r.dk, r.dv):
        assert float(g.abs().max()) == 0.0


def test_dominant_diagonal_selects_own_value():
    """Large scale and q_i = k_i with orthogonal keys: each query attends to itself."""
    T = 6
    e = np.eye(T)[None, None]  # orthonormal keys, d = T
    v = _rand((1, 1, T, T), 7)
    r = ref.attention_fwd_bwd(e, e, v, v, 60.0, dtype=torch.float64)
    np.testing.assert_allclose(r.o.numpy(), v, atol=1e-20 + 1e-12)


# ------------------------------------------------------------------ finite differences (fp64)
def test_gradients_match_finite_differences():
    B, H, T, d = 1, 2, 5, 3
    q, k, v, do = (_rand((B, H, T, d), s) for s in range(10, 14))
    scale = 0.7
    fd = ref.finite_difference_grads(q, k, v, do, scale)
    r = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float64)
    an = ref.attention_numpy64(q, k, v, do, scale)
    for got_t, got_n, want in zip((r.dq, r.dk, r.dv), (an["dq"], an["dk"], an["dv"]), fd):
        np.testing.assert_allclose(got_t.numpy(), want, atol=1e-8)
        np.testing.assert_allclose(got_n, want, atol=1e-8)


# --------------------------------------------------------------------------------- invariants
def test_softmax_rows_sum_to_one_and_ds_rows_sum_to_zero():
    q, k, v, do = (_rand((2, 2, 23, 8), s) for s in range(20, 24))
    an = ref.attention_numpy64(q, k, v, do, 0.35)
    np.testing.assert_allclose(an["p"].sum(-1), 1.0, atol=1e-13)
    np.testing.assert_allclose(an["ds"].sum(-1), 0.0, atol=1e-12)
    assert np.all(np.triu(an["p"][0, 0], 1) == 0)  # causal
    np.testing.assert_allclose(an["D"], (an["o"] * do).sum(-1), atol=1e-13)


# ---------------------------------------------------------------- independent restatements
def test_loops_match_torch_fp64():
    q, k, v = (_rand((4, 3), s) for s in range(30, 33))
    o, ms, ls = ref.attention_loops(q.tolist(), k.tolist(), v.tolist(), 0.8)
    r = ref.attention_fwd_bwd(q[None, None], k[None, None], v[None, None], v[None, None], 0.8,
                              dtype=torch.float64, with_grad=False)
    np.testing.assert_allclose(r.o.numpy()[0, 0], np.array(o), atol=1e-14)
    np.testing.assert_allclose(r.m.numpy()[0, 0], ms, atol=1e-14)
    np.testing.assert_allclose(r.l.numpy()[0, 0], ls, atol=1e-14)


def test_torch_fp32_close_to_fp64_at_config2_slice():
    """Distance of the fp32 oracle from fp64 on one config-2 head: the floor any fp32
    implementation is judged against (the gate is 1e-5)."""
    q, k, v, do = ref.seeded_inputs(1, 1, 1024, 64, seed=42)
    r32 = ref.attention_fwd_bwd(q, k, v, do, 0.125, dtype=torch.float32)
    r64 = ref.attention_fwd_bwd(q, k, v, do, 0.125, dtype=torch.float64)
    for a, b in ((r32.o, r64.o), (r32.dq, r64.dq), (r32.dk, r64.dk), (r32.dv, r64.dv)):
        assert float((a.double() - b).abs().max()) < 5e-6


# -------------------------------------------------------------------------- planted mistakes
def _mutant_forward(kind):
    def fwd(q, k, v, scale):
        T = q.shape[-2]
        att = (q @ k.transpose(-2, -1)) * (scale if kind != "no_scale" else 1.0)
        keep = ref.causal_mask(T)
        if kind == "strict_mask":
            keep = torch.tril(torch.ones(T, T), -1)  # j < i: diagonal dropped
            keep[0, 0] = 1
        if kind == "transposed_mask":
            keep = keep.T
        att = att.masked_fill(keep.to(att.dtype) == 0, float("-inf"))
        p = torch.softmax(att, dim=-1)
        if kind == "swapped_qk_in_pv":
            return p @ k
        return p @ v
    return fwd


@pytest.mark.parametrize("kind", ["no_scale", "strict_mask", "transposed_mask", "swapped_qk_in_pv"])
def test_planted_mistake_is_caught(kind):
    """Each plausible mistake, planted in a copy of the oracle's forward, fails one of the
    pins used above (KAT, Q=0 closed form, dominant diagonal, fp64 cross-check)."""
    fwd = _mutant_forward(kind)
    caught = []
    T, d = 8, 32
    q = torch.full((1, 1, T, d), 0.1, dtype=torch.float64)
    v = torch.ones_like(q)
    caught.append(not torch.allclose(fwd(q, q, v, 1 / math.sqrt(d)), v))
    k, vv = (torch.from_numpy(_rand((1, 1, 11, 4), s)) for s in (40, 41))
    prefix = torch.cumsum(vv, 2) / torch.arange(1, 12, dtype=torch.float64)[:, None]
    caught.append(not torch.allclose(fwd(torch.zeros_like(k), k, vv, 0.5), prefix))
    e = torch.eye(6, dtype=torch.float64)[None, None]
    v6 = torch.from_numpy(_rand((1, 1, 6, 6), 42))
    caught.append(not torch.allclose(fwd(e, e, v6, 60.0), v6, atol=1e-9))
    qq, kk, v5 = (torch.from_numpy(_rand((1, 1, 9, 5), s)) for s in (43, 44, 45))
    an = ref.attention_numpy64(qq, kk, v5, v5, 0.9)["o"]
    caught.append(not np.allclose(fwd(qq, kk, v5, 0.9).numpy(), an, atol=1e-12))
    assert any(caught), f"planted mistake {kind!r} passed every pin"


# ---------------------------------------------------------------------- config-1 fixture
def test_c1_fixture_is_consistent_with_oracle():
    """The committed layer-0 tensors satisfy the oracle: O and dQ/dK/dV recomputed from
    (q, k, v, dO) in fp64 match the fp32 fixture."""
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "c1_layer0_attention.npz")
    f = np.load(path)
    assert f["q"].shape == (4, 4, 64, 32)
    an = ref.attention_numpy64(f["q"], f["k"], f["v"], f["do"], 1 / math.sqrt(32))
    np.testing.assert_allclose(f["o"], an["o"], atol=2e-6)
    for n in ("dq", "dk", "dv"):
        scale = np.abs(an[n]).max()
        np.testing.assert_allclose(f[n], an[n], atol=1e-6 * scale + 1e-12)
    assert abs(float(f["loss"]) - math.log(256)) < 0.1  # untrained model: loss ~ ln V


# --------------------------------------------------------------- parity metrics (the gate)
def _metric_pin_failures(metrics):
    """Closed-form checks of the parity metrics of scripts/compare_parity.py:11-26
    (max, mean and RMS of |a - b|, rel = ||a - b||_2 / (||b||_2 + 1e-12)); returns the
    names of the checks that `metrics` fails."""
    failed = []

    def close(x, y, rtol=1e-12):
        return math.isclose(x, y, rel_tol=rtol, abs_tol=0.0)

    b = _rand((3, 5, 7), 50)
    m = metrics(b.copy(), b)
    if any(m[n] != 0.0 for n in ("max_err", "mean_err", "rms_err", "rel_err")):
        failed.append("a == b gives zeros")
    if m["elements"] != b.size:
        failed.append("element count")
    # a = b (1 + e): |a - b| = e |b| elementwise, so rel = e and max/mean/RMS scale |b|'s
    e = 0.03125
    m = metrics(b * (1 + e), b)
    nb = float(np.linalg.norm(b.ravel()))
    if not close(m["rel_err"], e * nb / (nb + 1e-12), 1e-12):
        failed.append("relative perturbation gives rel = e")
    if not close(m["max_err"], e * float(np.abs(b).max())):
        failed.append("relative perturbation max")
    if not close(m["mean_err"], e * float(np.abs(b).mean())):
        failed.append("relative perturbation mean")
    if not close(m["rms_err"], e * float(np.sqrt((b ** 2).mean()))):
        failed.append("relative perturbation rms")
    # one element off by delta among n
    n = b.size
    a = b.copy()
    a[1, 2, 3] += 0.5
    m = metrics(a, b)
    if not (close(m["max_err"], 0.5, 1e-12) and close(m["mean_err"], 0.5 / n, 1e-9) and
            close(m["rms_err"], 0.5 / math.sqrt(n), 1e-9) and
            close(m["rel_err"], 0.5 / (nb + 1e-12), 1e-9)):
        failed.append("single perturbed element")
    # hand vector: |a - b| = (0, 2, 0, 4)
    m = metrics(np.array([1.0, 2.0, 3.0, 4.0]), np.array([1.0, 0.0, 3.0, 8.0]))
    if not (m["max_err"] == 4.0 and m["mean_err"] == 1.5 and close(m["rms_err"], math.sqrt(5.0))
            and close(m["rel_err"], math.sqrt(20.0) / (math.sqrt(74.0) + 1e-12))):
        failed.append("hand vector")
    # b = 0: rel = ||a|| / 1e-12 (the guard term), finite
    a = np.array([3.0, 4.0])
    m = metrics(a, np.zeros(2))
    if not (np.isfinite(m["rel_err"]) and close(m["rel_err"], 5.0 / 1e-12, 1e-9)):
        failed.append("zero reference")
    # normalised by the second argument (the reference tensor), not the first
    x, y = np.array([1.0, 1.0]), np.array([2.0, 2.0])
    if not (close(metrics(x, y)["rel_err"], math.sqrt(2.0) / (math.sqrt(8.0) + 1e-12)) and
            close(metrics(y, x)["rel_err"], math.sqrt(2.0) / (math.sqrt(2.0) + 1e-12))):
        failed.append("normalised by b")
    # signs cancel in nothing: |a - b| of mixed signs
    m = metrics(np.array([1.0, -1.0]), np.array([0.0, 0.0]) + np.array([2.0, -2.0]))
    if not close(m["mean_err"], 1.0):
        failed.append("absolute differences")
    return failed


def test_parity_metrics_closed_forms():
    assert _metric_pin_failures(ref.compute_metrics) == []


def _mutant_metrics(kind):
    def metrics(a, b):
        a = np.asarray(a, dtype=np.float64)
        b = np.asarray(b, dtype=np.float64)
        diff = a - b if kind == "signed_diff" else np.abs(a - b)
        denom = np.linalg.norm((a if kind == "norm_of_a" else b).ravel())
        num = np.linalg.norm(diff.ravel())
        if kind == "max_for_norm":
            num = np.abs(diff).max()
        if kind == "squared_norm":
            num, denom = num ** 2, denom ** 2
        rms = np.sqrt((diff ** 2).mean())
        if kind == "rms_without_sqrt":
            rms = (diff ** 2).mean()
        return {
            "max_err": float(np.abs(diff).max()),
            "mean_err": float(diff.mean()),
            "rms_err": float(rms),
            "rel_err": float(num / (denom + (0.0 if kind == "no_guard" else 1e-12))),
            "elements": int(a.size),
        }
    return metrics


@pytest.mark.parametrize("kind", ["norm_of_a", "max_for_norm", "squared_norm", "rms_without_sqrt",
                                  "signed_diff", "no_guard"])
def test_parity_metrics_planted_mistake_is_caught(kind):
    """Each plausible slip in a copy of the metric function fails a closed-form pin."""
    with np.errstate(divide="ignore", invalid="ignore"):
        failed = _metric_pin_failures(_mutant_metrics(kind))
    assert failed, f"planted metric mistake {kind!r} passed every pin"
