"""Materialised attention mode on the GPU: the strided-batched fp32 GEMM against fp64
products, and the reference's materialised forward/backward sequences (src/model.cu:313-332,
617-650) against the CPU oracle and the tiled fp32 path."""
import math

import numpy as np
import pytest
import torch

from gpu_util import default_scale, max_abs, to_dev
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu


def gemm_ref(a, b, M, N, K, sA, sB, sC, batch, ta, tb, alpha, beta, c0):
    """fp64 restatement of the row-major strided-batched GEMM (matmul.cu:167-207)."""
    c = c0.astype(np.float64).copy()
    for i in range(batch):
        A = a[i * sA:i * sA + M * K].astype(np.float64)
        B = b[i * sB:i * sB + K * N].astype(np.float64)
        A = A.reshape(K, M).T if ta else A.reshape(M, K)
        B = B.reshape(N, K).T if tb else B.reshape(K, N)
        prev = c[i * sC:i * sC + M * N].reshape(M, N)
        out = alpha * (A @ B) + (beta * prev if beta != 0 else 0.0)
        c[i * sC:i * sC + M * N] = out.reshape(-1)
    return c


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (17, 33, 5), (64, 64, 16), (100, 70, 130),
                                   (65, 129, 64), (256, 256, 1024)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_vs_fp64(lib, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 1000 + N * 10 + K + 2 * ta + tb)
    batch = 3
    pad = 7  # strides larger than one matrix: batches are not packed
    sA, sB, sC = M * K + pad, K * N + pad, M * N + pad
    a = rng.standard_normal(batch * sA).astype(np.float32)
    b = rng.standard_normal(batch * sB).astype(np.float32)
    c0 = rng.standard_normal(batch * sC).astype(np.float32)
    for alpha, beta in ((1.0, 0.0), (0.5, -1.25)):
        cg = to_dev(c0)
        if beta == 0.0:
            cg.fill_(float("nan"))  # beta = 0 must not read C
        lib.matmul_batched_strided(to_dev(a), to_dev(b), cg, M, N, K, sA, sB, sC, batch, ta, tb,
                                   alpha, beta)
        torch.cuda.synchronize()
        got = cg.cpu().numpy()
        want = gemm_ref(a, b, M, N, K, sA, sB, sC, batch, ta, tb, alpha, beta, c0)
        for i in range(batch):
            g = got[i * sC:i * sC + M * N]
            w = want[i * sC:i * sC + M * N]
            assert np.isfinite(g).all()
            np.testing.assert_allclose(g, w, rtol=0, atol=2e-6 * K + 1e-6,
                                       err_msg=f"batch {i} alpha {alpha} beta {beta}")
        # the padding between batch matrices is never written
        for i in range(batch - 1):
            gap = got[i * sC + M * N:(i + 1) * sC]
            ref_gap = c0[i * sC + M * N:(i + 1) * sC]
            if beta == 0.0:
                assert np.isnan(gap).all()
            else:
                np.testing.assert_array_equal(gap, ref_gap)


@pytest.mark.parametrize("M,N,K", [(4, 4, 4), (100, 68, 132), (260, 64, 1024), (132, 200, 36),
                                   (512, 516, 64), (36, 8, 20), (100, 200, 48), (36, 8, 16),
                                   (300, 60, 160)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("pad", [0, 4])
def test_gemm_vectorized_vs_fp64(lib, M, N, K, ta, tb, pad):
    """Operands whose contiguous dimension is a multiple of 4 elements, with 16-byte aligned
    batch strides, take the 16-byte-load kernels (128 x 128 tiles, or 128 x 64 for N <= 64),
    the copy-pipelined one where K is a multiple of 16: ragged against both tile shapes, every
    transpose combination, packed and padded batches."""
    rng = np.random.default_rng(M * 7919 + N * 31 + K + 2 * ta + tb + pad)
    batch = 3
    sA, sB, sC = M * K + pad, K * N + pad, M * N + pad
    a = rng.standard_normal(batch * sA).astype(np.float32)
    b = rng.standard_normal(batch * sB).astype(np.float32)
    c0 = rng.standard_normal(batch * sC).astype(np.float32)
    for alpha, beta in ((1.0, 0.0), (0.75, 0.5)):
        cg = to_dev(c0)
        if beta == 0.0:
            cg.fill_(float("nan"))
        lib.matmul_batched_strided(to_dev(a), to_dev(b), cg, M, N, K, sA, sB, sC, batch, ta, tb,
                                   alpha, beta)
        torch.cuda.synchronize()
        got = cg.cpu().numpy()
        want = gemm_ref(a, b, M, N, K, sA, sB, sC, batch, ta, tb, alpha, beta, c0)
        for i in range(batch):
            g = got[i * sC:i * sC + M * N]
            assert np.isfinite(g).all()
            np.testing.assert_allclose(g, want[i * sC:i * sC + M * N], rtol=0,
                                       atol=2e-6 * K + 1e-6, err_msg=f"batch {i} beta {beta}")
        for i in range(batch - 1):  # the padding between batch matrices is never written
            gap = got[i * sC + M * N:(i + 1) * sC]
            if beta == 0.0:
                assert np.isnan(gap).all()
            else:
                np.testing.assert_array_equal(gap, c0[i * sC + M * N:(i + 1) * sC])


def materialized(lib, q, k, v, do, B, H, T, d, scale):
    qg, kg, vg, dog = (to_dev(x) for x in (q, k, v, do))
    nan = lambda shape: torch.full(shape, float("nan"), device="cuda:0")
    scores, probs = nan((B * H * T, T)), nan((B * H * T, T))
    out = nan((B, H, T, d))
    lib.materialized_causal_attention_forward(qg, kg, vg, scores, probs, out, B, H, T, d, scale)
    dprobs, dscores = nan((B * H * T, T)), nan((B * H * T, T))
    dq, dk, dv = nan((B, H, T, d)), nan((B, H, T, d)), nan((B, H, T, d))
    lib.materialized_causal_attention_backward(qg, kg, vg, probs, dog, dprobs, dscores, dq, dk,
                                               dv, B, H, T, d, scale)
    torch.cuda.synchronize()
    f = lambda t: t.cpu().numpy()
    return dict(o=f(out), dq=f(dq), dk=f(dk), dv=f(dv), probs=f(probs).reshape(B, H, T, T))


@pytest.mark.parametrize("B,H,T,d", [(1, 1, 1, 32), (2, 3, 17, 64), (1, 2, 100, 128),
                                     (2, 2, 257, 64), (1, 1, 64, 48)])
def test_materialized_vs_oracle(lib, B, H, T, d):
    q, k, v, do = ref.seeded_inputs(B, H, T, d, seed=T + d)
    scale = default_scale(d)
    got = materialized(lib, q, k, v, do, B, H, T, d, scale)
    want = ref.attention_fwd_bwd(q, k, v, do, scale)
    for name in ("o", "dq", "dk", "dv"):
        err = max_abs(got[name], getattr(want, name).numpy())
        assert err <= 1e-5, f"{name}: max-abs {err:.3e}"
    # probs: zeros above the diagonal up to the end of its 128-column block, untouched after
    i = np.arange(T)
    inside = i[None, :] < np.minimum((i[:, None] // 128 + 1) * 128, T)
    upper = np.triu(np.ones((T, T), bool), 1)
    assert np.all(got["probs"][..., upper & inside] == 0)
    assert np.isnan(got["probs"][..., ~inside]).all()


def test_materialized_config2_vs_oracle_and_tiled(lib):
    """Config 2 (B8 H12 T1024 d64, fp32): the materialised mode against the oracle on three
    heads and against the tiled fp32 path on every head."""
    B, H, T, d = 8, 12, 1024, 64
    q, k, v, do = ref.seeded_inputs(B, H, T, d, seed=42)
    scale = default_scale(d)
    got = materialized(lib, q, k, v, do, B, H, T, d, scale)
    from gpu_util import gpu_fwd_bwd
    tiled = gpu_fwd_bwd(lib, q, k, v, do, scale)
    for name in ("o", "dq", "dk", "dv"):
        err = max_abs(got[name], tiled[name])
        assert err <= 2e-5, f"{name} vs tiled: max-abs {err:.3e}"
    for b, h in ((0, 0), (3, 7), (B - 1, H - 1)):
        sl = lambda x: x[b:b + 1, h:h + 1]
        want = ref.attention_fwd_bwd(sl(q), sl(k), sl(v), sl(do), scale)
        for name in ("o", "dq", "dk", "dv"):
            err = max_abs(sl(got[name]), getattr(want, name).numpy())
            assert err <= 1e-5, f"{name} head ({b},{h}): max-abs {err:.3e}"


@pytest.mark.parametrize("T,d", [(1024, 64), (300, 32), (129, 128)])
def test_causal_gemm_equals_full_product(lib, T, d):
    """attn_matmul_batched_strided_causal_f32 on causally structured operands: the outputs it
    writes equal the full product's bitwise (the terms it skips are exact zeros, the outputs
    it skips lie in 128 x 128 blocks above the diagonal, which stay as they were)."""
    BH = 3
    g = torch.Generator(device="cpu").manual_seed(T + d)
    x = torch.randn((BH, T, d), generator=g).to("cuda:0")
    y = torch.randn((BH, T, d), generator=g).to("cuda:0")
    lower = torch.tril(torch.randn((BH, T, T), generator=g)).to("cuda:0").contiguous()
    sh, ss = T * d, T * T
    cases = [  # (A, B, M, N, K, sA, sB, transA, transB, causal)
        (x, y, T, T, d, sh, sh, False, True, lib.GEMM_LOWER_OUT),   # Q K^T
        (lower, y, T, d, T, ss, sh, False, False, lib.GEMM_LOWER_A),  # P V, dS K
        (lower, y, T, d, T, ss, sh, True, False, lib.GEMM_UPPER_A),   # P^T dO, dS^T Q
    ]
    for A, Bm, M, N, K, sA, sB, ta, tb, causal in cases:
        full = torch.full((BH, M, N), float("nan"), device="cuda:0")
        part = torch.full((BH, M, N), float("nan"), device="cuda:0")
        lib.matmul_batched_strided(A, Bm, full, M, N, K, sA, sB, M * N, BH, ta, tb)
        lib.matmul_batched_strided_causal(A, Bm, part, M, N, K, sA, sB, M * N, BH, ta, tb,
                                          causal)
        torch.cuda.synchronize()
        if causal == lib.GEMM_LOWER_OUT:
            i = torch.arange(M, device="cuda:0")
            blk = (i[None, :] // 128) > (i[:, None] // 128)  # blocks wholly above the diagonal
            assert torch.isnan(part[:, blk]).all(), "skipped blocks must stay unwritten"
            assert torch.equal(part[:, ~blk], full[:, ~blk]), f"causal {causal}"
        else:
            assert torch.equal(part, full), f"causal {causal}"


def test_materialized_equals_its_launch_sequence(lib):
    """The materialised entry points equal, bitwise, their launch sequence run through the
    public pieces (the causal GEMM and the softmax kernels with zero_block 128), which is what
    bench.py times launch by launch."""
    B, H, T, d = 2, 3, 256, 64
    q, k, v, do = (to_dev(x) for x in ref.seeded_inputs(B, H, T, d, seed=3))
    scale = default_scale(d)
    got = materialized(lib, *(x.cpu().numpy() for x in (q, k, v, do)), B, H, T, d, scale)
    BH, sh, ss = B * H, T * d, T * T
    sq = lambda: torch.full((BH * T, T), float("nan"), device="cuda:0")
    scores, probs, dprobs, dscores = sq(), sq(), sq(), sq()
    out, dq, dk, dv = (torch.empty_like(q) for _ in range(4))
    gm = lib.matmul_batched_strided_causal
    gm(q, k, scores, T, T, d, sh, sh, ss, BH, False, True, lib.GEMM_LOWER_OUT)
    lib.causal_softmax_forward(scores, probs, B, H, T, scale, zero_block=128)
    gm(probs, v, out, T, d, T, ss, sh, sh, BH, False, False, lib.GEMM_LOWER_A)
    gm(do, v, dprobs, T, T, d, sh, sh, ss, BH, False, True, lib.GEMM_LOWER_OUT)
    gm(probs, do, dv, T, d, T, ss, sh, sh, BH, True, False, lib.GEMM_UPPER_A)
    lib.causal_softmax_backward(dprobs, probs, dscores, B, H, T, scale, zero_block=128)
    gm(dscores, k, dq, T, d, T, ss, sh, sh, BH, False, False, lib.GEMM_LOWER_A)
    gm(dscores, q, dk, T, d, T, ss, sh, sh, BH, True, False, lib.GEMM_UPPER_A)
    torch.cuda.synchronize()
    for name, t in (("o", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert np.array_equal(got[name], t.cpu().numpy()), name
