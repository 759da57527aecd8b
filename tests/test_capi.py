"""The C-ABI library without a GPU: it loads, exports every symbol the headers declare,
and validates arguments on the host (status codes, no launch)."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CAPI = os.path.join(REPO, "include", "attn_capi.h")

FAKE = 0x10000  # never dereferenced: every call below fails validation before launching
MISALIGNED = 0x10004

OK, INVALID_DIM, BAD_HEAD_DIM, NULLPTR, MISALIGN, LAUNCH, BAD_VALUE, SCRATCH_LIMIT = range(8)


def declared_symbols():
    text = open(CAPI).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(attn_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib):
    syms = declared_symbols()
    assert len(syms) >= 20
    handle = lib.raw()
    for s in syms:
        assert hasattr(handle, s), f"{s} declared in attn_capi.h but not exported"
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", lib.LIB_PATH], capture_output=True,
                             text=True, check=True).stdout
        exported = set(re.findall(r"\bT (attn_\w+)", out))
        assert set(syms) <= exported


def test_binding_covers_header(lib):
    declared = set(declared_symbols()) - {"attn_status_string", "attn_version",
                                          "attn_f32x3_workspace_bytes",
                                          "attn_f32x3_planes_bytes",
                                          "attn_f32x3_ds_workspace_bytes",
                                          "attn_f32x3_backward_uses_ds",
                                          "attn_f32_ds_workspace_bytes",
                                          "attn_f32_backward_uses_ds"}
    assert declared == set(lib.SIGNATURES)


def test_status_strings(lib):
    assert lib.status_string(0) == "success"
    for s in range(1, 8):
        assert lib.status_string(s) not in ("success", "unknown status")
    assert lib.status_string(99) == "unknown status"
    assert lib.raw().attn_version() >= 100


def fwd(lib, q=FAKE, out=FAKE, B=1, H=1, T=8, d=64, scale=0.125):
    return lib.call("attn_tiled_causal_forward_f32", q, FAKE, FAKE, out, B, H, T, d,
                    ctypes.c_float(scale), None, None, None)


def test_forward_validation(lib):
    assert fwd(lib, d=48) == BAD_HEAD_DIM          # reference silently mis-runs d=48
    assert fwd(lib, d=256) == BAD_HEAD_DIM
    assert fwd(lib, B=0) == INVALID_DIM
    assert fwd(lib, T=-1) == INVALID_DIM
    assert fwd(lib, q=None) == NULLPTR
    assert fwd(lib, out=None) == NULLPTR
    assert fwd(lib, q=MISALIGNED) == MISALIGN
    assert fwd(lib, scale=0.0) == BAD_VALUE
    assert fwd(lib, scale=float("nan")) == BAD_VALUE
    assert fwd(lib, scale=float("inf")) == BAD_VALUE
    assert fwd(lib, B=1 << 16, H=1 << 16) == INVALID_DIM


def test_backward_validation(lib):
    def bwd(name, d=64, ws=FAKE, dk=FAKE):
        args = [FAKE] * 7 + [FAKE, dk, FAKE, ws, 1, 1, 8, d, ctypes.c_float(0.125), None]
        return lib.call(name, *args)
    for name in ("attn_tiled_causal_backward_f32", "attn_tiled_causal_backward_bf16"):
        assert bwd(name, d=128 + 32) == BAD_HEAD_DIM   # reference: silent no-op for d=128
        assert bwd(name, ws=None) == NULLPTR
        assert bwd(name, dk=None) == NULLPTR
        assert bwd(name, dk=MISALIGNED) == MISALIGN


def test_split_and_softmax_validation(lib):
    f = ctypes.c_float
    assert lib.call("attn_qkv_split_transpose_forward_f32", FAKE, FAKE, None, FAKE, 1, 4, 2, 8,
                    None) == NULLPTR
    assert lib.call("attn_qkv_split_transpose_forward_f32", FAKE, FAKE, FAKE, FAKE, 1, 0, 2, 8,
                    None) == INVALID_DIM
    assert lib.call("attn_qkv_split_transpose_backward_bf16", FAKE, FAKE, FAKE, FAKE, 1, 4, 2,
                    0, None) == INVALID_DIM
    assert lib.call("attn_causal_softmax_forward_f32", FAKE, None, 1, 1, 4, f(1.0),
                    None) == NULLPTR
    assert lib.call("attn_causal_softmax_backward_f32", FAKE, FAKE, FAKE, 1, 1, 4,
                    f(float("nan")), None) == BAD_VALUE
    for zb in (-1, 6):
        assert lib.call("attn_causal_softmax_forward_blocked_f32", FAKE, FAKE, 1, 1, 4, f(1.0),
                        zb, None) == BAD_VALUE
    assert lib.call("attn_causal_softmax_backward_blocked_f32", FAKE, None, FAKE, 1, 1, 4,
                    f(1.0), 128, None) == NULLPTR
    assert lib.call("attn_causal_softmax_backward_blocked_f32", FAKE, FAKE, FAKE, 1, 0, 4,
                    f(1.0), 128, None) == INVALID_DIM
    assert lib.call("attn_head_merge_transpose_forward_f32", FAKE, FAKE, 0, 1, 4, 8,
                    None) == INVALID_DIM


def test_gemm_handle_without_gpu(lib):
    """The handle argument of matmul_batched_strided (include/kernels/matmul.cuh:44-58):
    a NULL handle is rejected before anything else; creating one needs a current device."""
    f = ctypes.c_float
    assert lib.call("attn_matmul_batched_strided_f32_h", None, FAKE, FAKE, FAKE, 4, 4, 4, 16,
                    16, 16, 2, 0, 1, f(1.0), f(0.0), None) == NULLPTR
    assert lib.call("attn_gemm_create", None) == NULLPTR
    assert lib.call("attn_gemm_destroy", None) == OK
    assert lib.raw().attn_gemm_device(None) == -1


def test_noalloc_backward_validation(lib):
    """attn_tiled_causal_backward_f32_noalloc checks its arguments, and the size against its
    fixed scratch, before it looks anything up on a device."""
    f = ctypes.c_float
    call = lambda *p, B=1, H=1, T=8, d=64, scale=0.125: lib.call(
        "attn_tiled_causal_backward_f32_noalloc", *p, B, H, T, d, f(scale), None)
    ten = [FAKE] * 10
    for i in range(10):
        args = list(ten)
        args[i] = None
        assert call(*args) == NULLPTR
    assert call(*ten, d=48) == BAD_HEAD_DIM
    assert call(*ten, T=0) == INVALID_DIM
    assert call(*ten, scale=0.0) == BAD_VALUE
    limit = 1 << 22
    assert call(*ten, B=1, H=1, T=limit + 1) == SCRATCH_LIMIT
    assert call(*ten, B=64, H=16, T=4097) == SCRATCH_LIMIT
    args = list(ten)
    args[7] = MISALIGNED
    assert call(*args) == MISALIGN


def test_materialized_validation(lib):
    f = ctypes.c_float
    gemm = lambda A=FAKE, M=4, N=4, K=4, sA=16, batch=2, alpha=1.0, beta=0.0: lib.call(
        "attn_matmul_batched_strided_f32", A, FAKE, FAKE, M, N, K, sA, 16, 16, batch, 0, 1,
        f(alpha), f(beta), None)
    assert gemm(A=None) == NULLPTR
    assert gemm(M=0) == INVALID_DIM
    assert gemm(K=-3) == INVALID_DIM
    assert gemm(batch=0) == BAD_VALUE
    assert gemm(sA=-1) == BAD_VALUE
    assert gemm(alpha=float("inf")) == BAD_VALUE
    assert gemm(beta=float("nan")) == BAD_VALUE
    assert gemm(M=1 << 20, N=1 << 20, batch=16) == INVALID_DIM  # grid beyond 2^31 tiles
    assert lib.call("attn_materialized_causal_forward_f32", FAKE, FAKE, FAKE, FAKE, None, FAKE,
                    1, 1, 8, 32, f(0.1), None) == NULLPTR
    assert lib.call("attn_materialized_causal_forward_f32", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                    1, 1, 8, 32, f(0.0), None) == BAD_VALUE
    assert lib.call("attn_materialized_causal_backward_f32", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                    FAKE, FAKE, FAKE, FAKE, 1, 0, 8, 32, f(0.1), None) == INVALID_DIM
    assert lib.call("attn_materialized_causal_backward_f32", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                    FAKE, FAKE, None, FAKE, 1, 1, 8, 32, f(0.1), None) == NULLPTR


def test_f32x3_validation(lib):
    """The three-plane fp32 entry points validate before any HIP call."""
    f = ctypes.c_float
    raw = lib.raw()
    # planes of q, k, v, dO (3 x bf16 each) and, at d = 64, the one-call backward's dS (64 x 64
    # fp32 per head: T rounded up to 32)
    assert raw.attn_f32x3_workspace_bytes(2, 3, 40, 64) == 4 * 3 * 2 * 3 * 40 * 64 * 2 + 6 * 64 * 64 * 4
    assert raw.attn_f32x3_workspace_bytes(2, 3, 40, 32) == 4 * 3 * 2 * 3 * 40 * 32 * 2
    assert raw.attn_f32x3_workspace_bytes(0, 3, 40, 64) == 0
    assert lib.f32x3_backward_uses_ds(2, 3, 40, 64) and not lib.f32x3_backward_uses_ds(2, 3, 40, 32)
    # dS above 16 GiB: the two-stage order, no dS in the workspace
    assert lib.f32x3_backward_uses_ds(1, 16, 16384, 64)          # 16 GiB exactly
    assert not lib.f32x3_backward_uses_ds(1, 16, 16416, 64)
    assert raw.attn_f32x3_workspace_bytes(1, 16, 16416, 64) == 4 * 3 * 16 * 16416 * 64 * 2
    assert not lib.f32x3_backward_uses_ds(0, 16, 1024, 64)
    fwd = lambda d=64, planes=FAKE, qkv=FAKE, scale=0.125: lib.call(
        "attn_packed_causal_forward_f32x3", qkv, FAKE, 1, 2, 8, d, f(scale), None, None,
        planes, None)
    assert fwd(d=128) == BAD_HEAD_DIM   # plane tiles of d = 128 do not fit the LDS
    assert fwd(d=48) == BAD_HEAD_DIM
    assert fwd(planes=None) == NULLPTR
    assert fwd(planes=MISALIGNED) == MISALIGN
    assert fwd(qkv=None) == NULLPTR
    assert fwd(scale=0.0) == BAD_VALUE
    assert lib.call("attn_fused_causal_forward_f32x3", FAKE, FAKE, 1, 2, 8, 32, f(0.1), None,
                    None, None, None) == NULLPTR
    bwd = lambda name, planes=FAKE, ws=FAKE, d=64: lib.call(
        name, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, ws, 1, 2, 8, d, f(0.125), planes, 1, None)
    for name in ("attn_packed_causal_backward_f32x3", "attn_fused_causal_backward_dq_f32x3"):
        assert bwd(name, planes=None) == NULLPTR
        assert bwd(name, ws=None) == NULLPTR
        assert bwd(name, d=128) == BAD_HEAD_DIM
    assert lib.call("attn_causal_backward_dkdv_f32x3", FAKE, FAKE, FAKE, FAKE, FAKE, 1, 2, 8,
                    64, f(0.125), None, None) == NULLPTR
    # the three stages of the one-call backward
    for name in ("attn_packed_causal_backward_prep_f32x3", "attn_fused_causal_backward_prep_f32x3"):
        prep = lambda planes=FAKE, ws=FAKE, d=64: lib.call(name, FAKE, FAKE, FAKE, ws, 1, 2, 8, d,
                                                           planes, 1, None)
        assert prep(planes=None) == NULLPTR
        assert prep(ws=None) == NULLPTR
        assert prep(d=128) == BAD_HEAD_DIM
        assert prep(planes=MISALIGNED) == MISALIGN
    dkdv = lambda planes=FAKE, d=64, scale=0.125: lib.call(
        "attn_causal_backward_dkdv_ds_f32x3", FAKE, FAKE, FAKE, FAKE, FAKE, 1, 2, 8, d, f(scale),
        planes, None)
    assert dkdv(planes=None) == NULLPTR
    assert dkdv(d=48) == BAD_HEAD_DIM
    assert dkdv(scale=0.0) == BAD_VALUE
    assert dkdv(d=32) == BAD_HEAD_DIM  # d = 32 takes the two-stage order: no dS
    dq = lambda dqkv=FAKE, planes=FAKE, d=64, T=8: lib.call(
        "attn_causal_backward_dq_ds_f32x3", dqkv, 1, 2, T, d, f(0.125), planes, None)
    assert dq(dqkv=None) == NULLPTR
    assert dq(planes=None) == NULLPTR
    assert dq(d=128) == BAD_HEAD_DIM
    assert dq(d=32) == BAD_HEAD_DIM
    assert dq(T=100000) == INVALID_DIM  # dS above 16 GiB
    assert dq(dqkv=MISALIGNED) == MISALIGN
    # the fp32 MFMA backward in the dS-first order
    assert raw.attn_f32_ds_workspace_bytes(2, 3, 40, 64) == 6 * 64 * 64 * 4
    assert raw.attn_f32_ds_workspace_bytes(2, 3, 0, 64) == 0
    # shapes the dimension checks accept but whose dS bytes pass SIZE_MAX: reported as 0
    # and rejected before any launch (T = 2^26 - 1 at d = 32; 4 * 4095 * 2^52 > 2^64)
    big_T = (1 << 26) - 1
    assert raw.attn_f32_ds_workspace_bytes(1, 4095, big_T, 32) == 0
    assert raw.attn_f32_ds_workspace_bytes(1, 1023, big_T, 32) == 1023 * 4 << 52
    assert lib.call("attn_packed_causal_backward_ds_f32", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                    FAKE, FAKE, 1, 4095, big_T, 32, f(0.125), None) == INVALID_DIM
    assert lib.call("attn_fused_causal_backward_dkdv_ds_f32", FAKE, FAKE, FAKE, FAKE, FAKE,
                    FAKE, FAKE, 1, 4095, big_T, 32, f(0.125), None) == INVALID_DIM
    assert lib.call("attn_causal_backward_dq_ds_f32", FAKE, FAKE, FAKE, 1, 4095, big_T, 32,
                    f(0.125), None) == INVALID_DIM
    for fam in ("packed", "fused"):
        one = lambda ds=FAKE, ws=FAKE, d=64: lib.call(
            f"attn_{fam}_causal_backward_ds_f32", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, ws, ds, 1,
            2, 8, d, f(0.125), None)
        assert one(ds=None) == NULLPTR
        assert one(ws=None) == NULLPTR
        assert one(d=48) == BAD_HEAD_DIM
        assert one(ds=MISALIGNED) == MISALIGN
        assert lib.call(f"attn_{fam}_causal_backward_prep_f32", FAKE, FAKE, None, 1, 2, 8, 64,
                        None) == NULLPTR
        assert lib.call(f"attn_{fam}_causal_backward_dkdv_ds_f32", FAKE, FAKE, FAKE, FAKE, FAKE,
                        FAKE, None, 1, 2, 8, 64, f(0.125), None) == NULLPTR
    dqf = lambda ds=FAKE, scale=0.125: lib.call("attn_causal_backward_dq_ds_f32", FAKE, FAKE, ds,
                                                1, 2, 8, 64, f(scale), None)
    assert dqf(ds=None) == NULLPTR
    assert dqf(scale=0.0) == BAD_VALUE
    assert dqf(ds=MISALIGNED) == MISALIGN
    assert lib.call("attn_tiled_causal_forward_f32x3", FAKE, FAKE, FAKE, FAKE, 1, 2, 8, 64,
                    f(0.125), None, None, MISALIGNED, None) == MISALIGN
    assert lib.call("attn_tiled_causal_backward_f32x3", *([FAKE] * 11), 1, 2, 8, 128,
                    f(0.125), FAKE, 1, None) == BAD_HEAD_DIM


def test_causal_gemm_validation(lib):
    """attn_matmul_batched_strided_causal_f32 rejects, before any launch, an unknown causal
    structure and shapes that do not fit the one given."""
    g = lambda causal=1, M=64, N=64, K=64, A=FAKE: lib.call(
        "attn_matmul_batched_strided_causal_f32", A, FAKE, FAKE, M, N, K, M * K, K * N, M * N,
        2, 0, 0, causal, None)
    assert g(causal=4) == BAD_VALUE and g(causal=-1) == BAD_VALUE
    assert g(causal=lib.GEMM_LOWER_OUT, N=32) == INVALID_DIM      # needs M == N
    assert g(causal=lib.GEMM_LOWER_A, K=32) == INVALID_DIM        # needs M == K
    assert g(causal=lib.GEMM_UPPER_A, K=32) == INVALID_DIM
    assert g(A=None) == NULLPTR
    assert g(M=0, N=0) == INVALID_DIM


def test_f32x3_separate_ds_validation(lib):
    """The workspace split into planes and dS, and the one-call backwards that take them
    apart: sizes add up, dS is required exactly where the dS-first order runs."""
    f = ctypes.c_float
    raw = lib.raw()
    for shape in ((2, 3, 40, 64), (2, 3, 40, 32), (1, 16, 16416, 64), (8, 12, 1024, 64)):
        planes, ds = raw.attn_f32x3_planes_bytes(*shape), raw.attn_f32x3_ds_workspace_bytes(*shape)
        assert planes == 4 * 3 * shape[0] * shape[1] * shape[2] * shape[3] * 2
        assert planes + ds == raw.attn_f32x3_workspace_bytes(*shape)
        assert (ds > 0) == lib.f32x3_backward_uses_ds(*shape)
    assert raw.attn_f32x3_ds_workspace_bytes(2, 3, 40, 64) == 6 * 64 * 64 * 4
    assert raw.attn_f32x3_planes_bytes(0, 3, 40, 64) == 0
    for fam in ("packed", "fused"):
        one = lambda ds=FAKE, planes=FAKE, d=64, T=8: lib.call(
            f"attn_{fam}_causal_backward_ds_f32x3", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, ds,
            1, 2, T, d, f(0.125), planes, 1, None)
        assert one(ds=None) == NULLPTR           # d = 64: the dS-first order needs dS
        assert one(ds=MISALIGNED) == MISALIGN
        assert one(planes=None) == NULLPTR
        assert one(d=128) == BAD_HEAD_DIM
        assert one(planes=MISALIGNED, ds=None, d=32) == MISALIGN  # two-stage: dS not needed


def test_f32_backward_order_gate(lib):
    """attn_f32_backward_uses_ds: the dS-first order of the fp32 MFMA backward where its dS
    fits 16 GiB, at every supported head size; the two-stage order beyond."""
    assert lib.f32_backward_uses_ds(8, 12, 1024, 64)
    assert lib.f32_backward_uses_ds(8, 12, 1024, 32) and lib.f32_backward_uses_ds(2, 16, 2048, 128)
    assert lib.f32_backward_uses_ds(1, 16, 16384, 64)        # 16 GiB exactly
    assert not lib.f32_backward_uses_ds(1, 16, 16416, 64)
    assert not lib.f32_backward_uses_ds(1, 4095, (1 << 26) - 1, 32)  # bytes past SIZE_MAX
    assert not lib.f32_backward_uses_ds(8, 12, 1024, 48)
    assert not lib.f32_backward_uses_ds(0, 12, 1024, 64)


def test_python_launchers_reject_host_tensors(lib):
    import torch
    x = torch.zeros(2, 2, 8, 32)
    with pytest.raises(ValueError):
        lib.tiled_causal_attention_forward(x, x, x, x, 2, 2, 8, 32, 0.1)


@pytest.mark.parametrize("lang", ["c", "c++"])
def test_headers_compile_standalone(tmp_path, lang):
    """attn_capi.h is a C header; kernels/attention.h and kernels/matmul.h compile as C++17
    (syntax only)."""
    if lang == "c":
        src = tmp_path / "t.c"
        src.write_text('#include "attn_capi.h"\nint main(void){return attn_version() > 0 ? 0 : 1;}\n')
        cmd = ["gcc", "-std=c11", "-fsyntax-only"]
    else:
        src = tmp_path / "t.cpp"
        src.write_text('#include "kernels/attention.h"\n#include "kernels/matmul.h"\n#include "common.h"\nint main(){return 0;}\n')
        cmd = ["g++", "-std=c++17", "-fsyntax-only"]
    cmd += ["-D__HIP_PLATFORM_AMD__", f"-I{REPO}/include", "-I/opt/rocm/include", str(src)]
    subprocess.run(cmd, check=True)
