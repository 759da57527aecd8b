"""fp32 parity path on the GPU: the tiled MFMA kernels against the restated reference
(torch fp32 on the CPU, pytorch_src/model.py:43-52) at the reference gate, max-abs <= 1e-5
on O, LSE, dQ, dK, dV (scripts/compare_parity.py:108-116), plus exact
closed forms and the reference's known-answer test."""
import math
import os

import numpy as np
import pytest
import torch

from gpu_util import default_scale, gpu_fwd_bwd, max_abs, to_dev
from oracle import attention_ref as ref
from oracle import c_oracle as co

pytestmark = pytest.mark.gpu

TOL = 1e-5  # the reference's forward gate, applied to every tensor here


@pytest.fixture(scope="module")
def config2():
    """B8 H12 T1024 d64, N(0,1) from seed 42, scale 1/8."""
    q, k, v, do = ref.seeded_inputs(8, 12, 1024, 64, seed=42)
    want = ref.attention_fwd_bwd(q, k, v, do, 0.125, dtype=torch.float32)
    return (q, k, v, do), want


def test_config2_parity(lib, config2):
    (q, k, v, do), want = config2
    got = gpu_fwd_bwd(lib, q, k, v, do, 0.125)
    lse = got["m"] + np.log(got["l"])
    errs = {n: max_abs(got[n], getattr(want, n).numpy()) for n in ("o", "dq", "dk", "dv")}
    errs["lse"] = max_abs(lse, want.lse.numpy())
    print("config2 max-abs vs torch fp32:", {k: f"{e:.2e}" for k, e in errs.items()})
    # distance of both fp32 results to fp64 (reported; the gate is the one above)
    w64 = ref.attention_fwd_bwd(q, k, v, do, 0.125, dtype=torch.float64)
    d64 = {n: (max_abs(got[n], getattr(w64, n).numpy()),
               max_abs(getattr(want, n).numpy(), getattr(w64, n).numpy()))
           for n in ("o", "dq", "dk", "dv")}
    print("config2 max-abs to fp64 (gpu, torch fp32):",
          {k: f"{a:.2e}, {b:.2e}" for k, (a, b) in d64.items()})
    for n, e in errs.items():
        assert e <= TOL, f"{n}: max-abs {e:.3e} > {TOL}"


def test_config2_deterministic(lib, config2):
    (q, k, v, do), _ = config2
    a = gpu_fwd_bwd(lib, q, k, v, do, 0.125)
    b = gpu_fwd_bwd(lib, q, k, v, do, 0.125)
    for n in ("o", "m", "l", "dq", "dk", "dv"):
        np.testing.assert_array_equal(a[n], b[n])


def test_config1_fixture(lib):
    """layer-0 attention of the tiny GPT (tests/golden)."""
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "c1_layer0_attention.npz"))
    got = gpu_fwd_bwd(lib, f["q"], f["k"], f["v"], f["do"], 1 / math.sqrt(32))
    for n in ("o", "dq", "dk", "dv"):
        e = max_abs(got[n], f[n])
        rel = ref.compute_metrics(got[n], f[n])["rel_err"]
        print(f"config1 {n}: max-abs {e:.2e} rel-L2 {rel:.2e}")
        assert e <= TOL
        assert rel <= 1e-5


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("T", [1, 5, 31, 32, 33, 100, 129, 257, 300])
def test_shapes_vs_oracle(lib, T, d):
    B, H = 2, 3
    q, k, v, do = ref.seeded_inputs(B, H, T, d, seed=T * 131 + d)
    scale = default_scale(d)
    want = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float32)
    got = gpu_fwd_bwd(lib, q, k, v, do, scale)
    for n in ("o", "dq", "dk", "dv"):
        assert max_abs(got[n], getattr(want, n).numpy()) <= TOL, n
    assert max_abs(got["m"], want.m.numpy()) <= TOL
    np.testing.assert_allclose(got["l"], want.l.numpy(), rtol=1e-5)


@pytest.mark.parametrize("B,H,T,d", [(2, 4, 300, 64), (1, 8, 160, 128), (2, 8, 383, 32),
                                     (4, 64, 200, 64)])
def test_xcd_block_order_ragged_vs_oracle(lib, B, H, T, d):
    """B*H a multiple of 8, where the shared-tile kernels map workgroups to heads XCD by XCD
    and the persistent ones fill per-XCD task queues, at lengths that leave the last block
    of each head partly past T."""
    q, k, v, do = ref.seeded_inputs(B, H, T, d, seed=B * H + T + d)
    scale = default_scale(d)
    want = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float32)
    got = gpu_fwd_bwd(lib, q, k, v, do, scale)
    for n in ("o", "dq", "dk", "dv"):
        assert max_abs(got[n], getattr(want, n).numpy()) <= TOL, n
    assert max_abs(got["m"], want.m.numpy()) <= TOL
    np.testing.assert_allclose(got["l"], want.l.numpy(), rtol=1e-5)


@pytest.mark.parametrize("d,T", [(64, 2048), (64, 2080), (128, 2080)])
def test_shared_tile_boundary_vs_oracle(lib, d, T):
    """Either side of the sequence length where the fp32 kernels change form (d = 64: the
    forward, dQ and dK/dV on tiles shared by a 128-row workgroup up to T = 2048, the
    persistent per-wave kernels beyond; d = 128: shared at every T)."""
    B, H = 1, 2
    q, k, v, do = ref.seeded_inputs(B, H, T, d, seed=T + d)
    scale = default_scale(d)
    want = ref.attention_fwd_bwd(q, k, v, do, scale, dtype=torch.float32)
    got = gpu_fwd_bwd(lib, q, k, v, do, scale)
    for n in ("o", "dq", "dk", "dv"):
        e = max_abs(got[n], getattr(want, n).numpy())
        print(f"T={T} d={d} {n}: max-abs {e:.2e}")
        assert e <= TOL, n
    assert max_abs(got["m"], want.m.numpy()) <= TOL
    np.testing.assert_allclose(got["l"], want.l.numpy(), rtol=1e-5)


def test_reference_kat_exact(lib):
    """tests/test_kernels.cu:210-284 with the exact answer (O=1, dQ=dK=0, dV closed form)."""
    T, d = 8, 32
    q = np.full((1, 1, T, d), 0.1, np.float32)
    v = np.ones_like(q)
    do = np.full_like(q, 0.5)
    got = gpu_fwd_bwd(lib, q, q, v, do, 1 / math.sqrt(d))
    np.testing.assert_allclose(got["o"], 1.0, atol=1e-6)
    np.testing.assert_allclose(got["dq"], 0.0, atol=1e-6)
    np.testing.assert_allclose(got["dk"], 0.0, atol=1e-6)
    want = np.array([sum(0.5 / (i + 1) for i in range(j, T)) for j in range(T)])
    np.testing.assert_allclose(got["dv"][0, 0], np.repeat(want[:, None], d, 1), rtol=1e-6)
    np.testing.assert_allclose(got["l"][0, 0], np.arange(1, T + 1), rtol=1e-6)


@pytest.mark.parametrize("d,T", [(64, 1000), (128, 77), (32, 515)])
def test_closed_forms(lib, d, T):
    B, H = 1, 2
    rng = np.random.default_rng(d + T)
    k, v, do = (rng.standard_normal((B, H, T, d)).astype(np.float32) for _ in range(3))
    got = gpu_fwd_bwd(lib, np.zeros_like(k), k, v, do, default_scale(d))
    prefix = np.cumsum(v.astype(np.float64), 2) / np.arange(1, T + 1)[:, None]
    np.testing.assert_allclose(got["o"], prefix, atol=2e-6)
    assert np.all(got["m"] == 0)
    np.testing.assert_allclose(got["l"], np.broadcast_to(np.arange(1, T + 1), (B, H, T)), rtol=1e-6)
    q = rng.standard_normal((B, H, T, d)).astype(np.float32)
    got = gpu_fwd_bwd(lib, q, k, np.full_like(q, 0.75), do, default_scale(d))
    # O = sum_j p_j * 0.75 / sum_j p_j: the two sums run over up to T terms in different
    # orders (MFMA vs VALU), so fp32 leaves ~sqrt(T)*eps relative: 4e-6 bounds T = 1000.
    np.testing.assert_allclose(got["o"], 0.75, atol=4e-6)
    np.testing.assert_allclose(got["dq"], 0.0, atol=1e-5)
    np.testing.assert_allclose(got["dk"], 0.0, atol=1e-5)
    got = gpu_fwd_bwd(lib, q, k, v, np.zeros_like(q), default_scale(d))
    for n in ("dq", "dk", "dv"):
        assert np.all(got[n] == 0)


def test_stats_and_stages_match_reference_kernels(lib):
    """m/l follow the reference tiled kernel's contract (C restatement of attention.cu:
    518-624); the standalone D launcher and the two backward stages equal the composite."""
    B, H, T, d = 2, 2, 70, 64
    q, k, v, do = ref.seeded_inputs(B, H, T, d, seed=5)
    scale = default_scale(d)
    c_o, c_m, c_l = co.tiled_fwd(q, k, v, scale)
    got = gpu_fwd_bwd(lib, q, k, v, do, scale)
    # m is a max of fp32 dot products whose summation order differs (MFMA vs a C loop)
    np.testing.assert_allclose(got["m"], c_m, rtol=2e-6, atol=1e-6)
    np.testing.assert_allclose(got["l"], c_l, rtol=2e-6)
    np.testing.assert_allclose(got["o"], c_o, atol=1e-5)
    c_dq, c_dk, c_dv, c_D = co.tiled_bwd(q, k, v, got["o"], do, got["m"], got["l"], scale)
    np.testing.assert_allclose(got["D"], c_D, atol=1e-5)
    for n, c in (("dq", c_dq), ("dk", c_dk), ("dv", c_dv)):
        assert max_abs(got[n], c) <= TOL, n

    qg, kg, vg, dog = (to_dev(x) for x in (q, k, v, do))
    og, mg, lg = to_dev(got["o"]), to_dev(got["m"]), to_dev(got["l"])
    D = torch.empty((B, H, T), device="cuda:0")
    lib.attention_precompute_dot_do_o(dog, og, D, B, H, T, d)
    ws = torch.empty_like(D)
    dq = torch.empty_like(qg)
    dk = torch.empty_like(qg)
    dv = torch.empty_like(qg)
    lib.tiled_causal_attention_backward_dq(qg, kg, vg, og, dog, mg, lg, dq, ws, B, H, T, d, scale)
    lib.tiled_causal_attention_backward_dkdv(qg, kg, vg, dog, mg, lg, ws, dk, dv, B, H, T, d, scale)
    torch.cuda.synchronize()
    np.testing.assert_allclose(D.cpu().numpy(), ws.cpu().numpy(), atol=2e-6)
    full = gpu_fwd_bwd(lib, q, k, v, do, scale)
    np.testing.assert_array_equal(dq.cpu().numpy(), full["dq"])
    np.testing.assert_array_equal(dk.cpu().numpy(), full["dk"])
    np.testing.assert_array_equal(dv.cpu().numpy(), full["dv"])


def test_optional_stats_pointers(lib):
    B, H, T, d = 1, 2, 40, 32
    q, k, v, _ = ref.seeded_inputs(B, H, T, d, seed=9)
    qg, kg, vg = (to_dev(x) for x in (q, k, v))
    out = torch.empty_like(qg)
    lib.tiled_causal_attention_forward(qg, kg, vg, out, B, H, T, d, default_scale(d))
    torch.cuda.synchronize()
    want = ref.attention_fwd_bwd(q, k, v, q, default_scale(d), with_grad=False)
    assert max_abs(out.cpu().numpy(), want.o.numpy()) <= TOL


def test_concurrent_streams_match_serial(lib):
    """The persistent kernels take their tasks from a per-launch queue slot: launches that run
    at the same time on different streams must not take each other's tasks."""
    B, H, T, d = 2, 8, 512, 64  # B*H = 16: per-XCD queues
    ins = [ref.seeded_inputs(B, H, T, d, seed=100 + i) for i in range(4)]
    serial = [gpu_fwd_bwd(lib, *x, 0.125) for x in ins]
    streams = [torch.cuda.Stream() for _ in ins]
    outs = []
    for x, st in zip(ins, streams):
        with torch.cuda.stream(st):
            qg, kg, vg, dog = (to_dev(a) for a in x)
            o, m, l = lib.attention_forward(qg, kg, vg, 0.125)
            dq, dk, dv, _ = lib.attention_backward(qg, kg, vg, o, dog, m, l, 0.125)
            outs.append((o, dq, dk, dv))
    torch.cuda.synchronize()
    for got, want in zip(outs, serial):
        for t, n in zip(got, ("o", "dq", "dk", "dv")):
            np.testing.assert_array_equal(t.cpu().numpy(), want[n])
