"""Python binding of the MI355X causal attention library (libtcamd_attn.so).

The product is the HIP library and its C ABI (include/attn_capi.h); this module binds
that ABI with ctypes so Python callers (tests, bench) drive exactly the entry points a
C/C++ caller would.  torch is used only for device memory and the current stream.

Launcher functions keep the reference's names and argument order
(include/kernels/attention.cuh:5-105) and take torch tensors for the pointer arguments;
they raise RuntimeError on a non-zero status, like the reference's callers do via
CUDA_CHECK.  There is no CPU fallback: if the library is missing, importing this module
fails.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtcamd_attn.so")
REPO_ROOT = os.path.dirname(_HERE)
CAPI_HEADER = os.path.join(REPO_ROOT, "include", "attn_capi.h")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C transformer-cuda_amd)")

# One HIP runtime per process.  torch bundles its own libamdhip64 (the same soname as the
# system one this library links against): loaded after this library, it would come in as a
# second runtime, whose device memory and streams this library's runtime does not see (its
# launches then fail with hipErrorNoDevice).  torch first makes this library bind to torch's.
try:
    import torch  # noqa: F401
except ImportError:  # no torch: the system runtime (C callers, the host-only tests)
    pass

_lib = ctypes.CDLL(LIB_PATH)

STATUS = {
    0: "ATTN_SUCCESS",
    1: "ATTN_ERROR_INVALID_DIM",
    2: "ATTN_ERROR_UNSUPPORTED_HEAD_DIM",
    3: "ATTN_ERROR_NULL_POINTER",
    4: "ATTN_ERROR_MISALIGNED",
    5: "ATTN_ERROR_LAUNCH",
    6: "ATTN_ERROR_INVALID_VALUE",
    7: "ATTN_ERROR_SCRATCH_LIMIT",
}

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_L = ctypes.c_longlong

# name -> argument types (the trailing _P is the hipStream_t)
SIGNATURES = {
    "attn_qkv_split_transpose_forward_f32": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "attn_qkv_split_transpose_backward_f32": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "attn_qkv_split_transpose_forward_bf16": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "attn_qkv_split_transpose_forward_f32_bf16": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "attn_qkv_split_transpose_backward_bf16": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "attn_qkv_split_transpose_backward_bf16_f32": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "attn_head_merge_transpose_forward_f32": [_P, _P, _I, _I, _I, _I, _P],
    "attn_head_merge_transpose_backward_f32": [_P, _P, _I, _I, _I, _I, _P],
    "attn_causal_softmax_forward_f32": [_P, _P, _I, _I, _I, _F, _P],
    "attn_causal_softmax_backward_f32": [_P, _P, _P, _I, _I, _I, _F, _P],
    "attn_causal_softmax_forward_blocked_f32": [_P, _P, _I, _I, _I, _F, _I, _P],
    "attn_causal_softmax_backward_blocked_f32": [_P, _P, _P, _I, _I, _I, _F, _I, _P],
    "attn_matmul_batched_strided_f32":
        [_P, _P, _P, _I, _I, _I, _L, _L, _L, _I, _I, _I, _F, _F, _P],
    "attn_gemm_create": [_P],
    "attn_gemm_destroy": [_P],
    "attn_gemm_device": [_P],
    "attn_matmul_batched_strided_f32_h":
        [_P, _P, _P, _P, _I, _I, _I, _L, _L, _L, _I, _I, _I, _F, _F, _P],
    "attn_matmul_batched_strided_causal_f32":
        [_P, _P, _P, _I, _I, _I, _L, _L, _L, _I, _I, _I, _I, _P],
    "attn_materialized_causal_forward_f32": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_packed_causal_forward_f32": [_P, _P, _I, _I, _I, _I, _F, _P, _P, _P],
    "attn_packed_causal_backward_f32": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_packed_causal_backward_dq_f32":
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_packed_causal_backward_dkdv_f32": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_packed_causal_backward_dq_bf16":
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_packed_causal_backward_dkdv_bf16": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_packed_causal_forward_bf16": [_P, _P, _I, _I, _I, _I, _F, _P, _P, _P],
    "attn_packed_causal_backward_bf16": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_fused_causal_forward_f32": [_P, _P, _I, _I, _I, _I, _F, _P, _P, _P],
    "attn_fused_causal_backward_f32": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_fused_causal_backward_dq_f32": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_fused_causal_backward_dkdv_f32": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_fused_causal_forward_bf16": [_P, _P, _I, _I, _I, _I, _F, _P, _P, _P],
    "attn_fused_causal_backward_bf16": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_fused_causal_backward_dq_bf16": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_fused_causal_backward_dkdv_bf16": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_materialized_causal_backward_f32":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_tiled_causal_forward_f32": [_P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P, _P],
    "attn_precompute_dot_do_o_f32": [_P, _P, _P, _I, _I, _I, _I, _P],
    "attn_tiled_causal_backward_f32":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_tiled_causal_backward_f32_noalloc":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_tiled_causal_backward_dq_f32":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_tiled_causal_backward_dkdv_f32":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_tiled_causal_forward_bf16": [_P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P, _P],
    "attn_tiled_causal_backward_bf16":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_tiled_causal_backward_dq_bf16":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_tiled_causal_backward_dkdv_bf16":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_packed_causal_forward_f32x3": [_P, _P, _I, _I, _I, _I, _F, _P, _P, _P, _P],
    "attn_fused_causal_forward_f32x3": [_P, _P, _I, _I, _I, _I, _F, _P, _P, _P, _P],
    "attn_packed_causal_backward_f32x3":
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P],
    "attn_fused_causal_backward_f32x3":
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P],
    "attn_packed_causal_backward_ds_f32x3":
        [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P],
    "attn_fused_causal_backward_ds_f32x3":
        [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P],
    "attn_packed_causal_backward_ds_f32":
        [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_fused_causal_backward_ds_f32":
        [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_packed_causal_backward_prep_f32": [_P, _P, _P, _I, _I, _I, _I, _P],
    "attn_fused_causal_backward_prep_f32": [_P, _P, _P, _I, _I, _I, _I, _P],
    "attn_packed_causal_backward_dkdv_ds_f32": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_fused_causal_backward_dkdv_ds_f32": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_causal_backward_dq_ds_f32": [_P, _P, _P, _I, _I, _I, _I, _F, _P],
    "attn_packed_causal_backward_prep_f32x3": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P],
    "attn_fused_causal_backward_prep_f32x3": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P],
    "attn_causal_backward_dkdv_ds_f32x3": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P],
    "attn_causal_backward_dq_ds_f32x3": [_P, _I, _I, _I, _I, _F, _P, _P],
    "attn_packed_causal_backward_dq_f32x3":
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P],
    "attn_fused_causal_backward_dq_f32x3":
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P],
    "attn_causal_backward_dkdv_f32x3": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P],
    "attn_tiled_causal_forward_f32x3": [_P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P, _P, _P],
    "attn_tiled_causal_backward_f32x3":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P],
    "attn_tiled_causal_backward_dq_f32x3":
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P],
    "attn_tiled_causal_backward_dkdv_f32x3":
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P],
}

for _name, _args in SIGNATURES.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = ctypes.c_int
_lib.attn_status_string.argtypes = [_I]
_lib.attn_status_string.restype = ctypes.c_char_p
_lib.attn_version.argtypes = []
_lib.attn_version.restype = ctypes.c_int
_lib.attn_f32x3_workspace_bytes.argtypes = [_I, _I, _I, _I]
_lib.attn_f32x3_workspace_bytes.restype = ctypes.c_size_t
_lib.attn_f32_ds_workspace_bytes.argtypes = [_I, _I, _I, _I]
_lib.attn_f32_ds_workspace_bytes.restype = ctypes.c_size_t
_lib.attn_f32x3_backward_uses_ds.argtypes = [_I, _I, _I, _I]
_lib.attn_f32x3_backward_uses_ds.restype = ctypes.c_int
_lib.attn_f32x3_planes_bytes.argtypes = [_I, _I, _I, _I]
_lib.attn_f32x3_planes_bytes.restype = ctypes.c_size_t
_lib.attn_f32x3_ds_workspace_bytes.argtypes = [_I, _I, _I, _I]
_lib.attn_f32x3_ds_workspace_bytes.restype = ctypes.c_size_t
_lib.attn_f32_backward_uses_ds.argtypes = [_I, _I, _I, _I]
_lib.attn_f32_backward_uses_ds.restype = ctypes.c_int


def raw():
    """The ctypes handle of libtcamd_attn.so (every symbol of include/attn_capi.h)."""
    return _lib


def status_string(status: int) -> str:
    return _lib.attn_status_string(int(status)).decode()


class AttnError(RuntimeError):
    def __init__(self, what: str, status: int):
        super().__init__(f"{what}: {status_string(status)} ({STATUS.get(status, status)})")
        self.status = status


def check(status: int, what: str) -> None:
    if status != 0:
        raise AttnError(what, status)


def call(name: str, *args) -> int:
    """Call a C-ABI entry point with raw arguments; returns its status."""
    return getattr(_lib, name)(*args)


# ---------------------------------------------------------------------------------------
# torch-tensor launchers (reference names and argument order)
# ---------------------------------------------------------------------------------------
def _torch():
    import torch
    return torch


def _ptr(t, dtype=None, numel=None, what=""):
    if t is None:
        return None
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{what}: expected a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{what}: tensor must be on a GPU device, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{what}: expected {dtype}, got {t.dtype}")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{what}: needs {numel} elements, has {t.numel()}")
    return t.data_ptr()


def _stream(stream):
    if stream is None:
        return _torch().cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _dt(bf16: bool):
    torch = _torch()
    return torch.bfloat16 if bf16 else torch.float32


def qkv_split_transpose_forward(qkv, q, k, v, B, T, H, d_head, stream=None):
    """Reference: include/kernels/attention.cuh:5-11.  dtype pair chosen from the tensors:
    f32->f32, bf16->bf16 or f32->bf16 (cast fused)."""
    torch = _torch()
    n = B * T * H * d_head
    src_bf = qkv.dtype == torch.bfloat16
    dst_bf = q.dtype == torch.bfloat16
    if src_bf and not dst_bf:
        raise ValueError("bf16 -> f32 split is not provided")
    name = ("attn_qkv_split_transpose_forward_bf16" if src_bf else
            "attn_qkv_split_transpose_forward_f32_bf16" if dst_bf else
            "attn_qkv_split_transpose_forward_f32")
    check(call(name, _ptr(qkv, _dt(src_bf), 3 * n, "qkv"), _ptr(q, _dt(dst_bf), n, "q"),
               _ptr(k, _dt(dst_bf), n, "k"), _ptr(v, _dt(dst_bf), n, "v"),
               B, T, H, d_head, _stream(stream)), "qkv_split_transpose_forward")


def qkv_split_transpose_backward(dq, dk, dv, dqkv, B, T, H, d_head, stream=None):
    """Reference: include/kernels/attention.cuh:13-19.  f32->f32, bf16->bf16 or bf16->f32."""
    torch = _torch()
    n = B * T * H * d_head
    src_bf = dq.dtype == torch.bfloat16
    dst_bf = dqkv.dtype == torch.bfloat16
    if dst_bf and not src_bf:
        raise ValueError("f32 -> bf16 backward split is not provided")
    name = ("attn_qkv_split_transpose_backward_bf16" if dst_bf else
            "attn_qkv_split_transpose_backward_bf16_f32" if src_bf else
            "attn_qkv_split_transpose_backward_f32")
    check(call(name, _ptr(dq, _dt(src_bf), n, "dq"), _ptr(dk, _dt(src_bf), n, "dk"),
               _ptr(dv, _dt(src_bf), n, "dv"), _ptr(dqkv, _dt(dst_bf), 3 * n, "dqkv"),
               B, T, H, d_head, _stream(stream)), "qkv_split_transpose_backward")


def head_merge_transpose_forward(inp, out, B, H, T, d_head, stream=None):
    """Reference: include/kernels/attention.cuh:91-97."""
    n = B * H * T * d_head
    f32 = _dt(False)
    check(call("attn_head_merge_transpose_forward_f32", _ptr(inp, f32, n, "in"),
               _ptr(out, f32, n, "out"), B, H, T, d_head, _stream(stream)),
          "head_merge_transpose_forward")


def head_merge_transpose_backward(dout, din, B, H, T, d_head, stream=None):
    """Reference: include/kernels/attention.cuh:99-105."""
    n = B * H * T * d_head
    f32 = _dt(False)
    check(call("attn_head_merge_transpose_backward_f32", _ptr(dout, f32, n, "dout"),
               _ptr(din, f32, n, "din"), B, H, T, d_head, _stream(stream)),
          "head_merge_transpose_backward")


def causal_softmax_forward(scores, probs, B, H, T, scale, stream=None, zero_block=None):
    """Reference: include/kernels/attention.cuh:21-31.  zero_block (no counterpart in the
    reference): write the zeros above the diagonal only up to the end of the zero_block-column
    block that holds it (attn_causal_softmax_forward_blocked_f32)."""
    n = B * H * T * T
    f32 = _dt(False)
    args = (_ptr(scores, f32, n, "scores"), _ptr(probs, f32, n, "probs"), B, H, T, float(scale))
    if zero_block is None:
        check(call("attn_causal_softmax_forward_f32", *args, _stream(stream)),
              "causal_softmax_forward")
    else:
        check(call("attn_causal_softmax_forward_blocked_f32", *args, int(zero_block),
                   _stream(stream)), "causal_softmax_forward_blocked")


def causal_softmax_backward(dprobs, probs, dscores, B, H, T, scale, stream=None,
                            zero_block=None):
    """Reference: include/kernels/attention.cuh:80-89.  zero_block as in
    causal_softmax_forward (attn_causal_softmax_backward_blocked_f32)."""
    n = B * H * T * T
    f32 = _dt(False)
    args = (_ptr(dprobs, f32, n, "dprobs"), _ptr(probs, f32, n, "probs"),
            _ptr(dscores, f32, n, "dscores"), B, H, T, float(scale))
    if zero_block is None:
        check(call("attn_causal_softmax_backward_f32", *args, _stream(stream)),
              "causal_softmax_backward")
    else:
        check(call("attn_causal_softmax_backward_blocked_f32", *args, int(zero_block),
                   _stream(stream)), "causal_softmax_backward_blocked")


def matmul_batched_strided(A, B, C, M, N, K, strideA, strideB, strideC, batch_count, transA,
                           transB, alpha=1.0, beta=0.0, stream=None):
    """Reference: include/kernels/matmul.cuh:44 (src/kernels/matmul.cu:167-207) without the
    cuBLAS handle.  Row-major C_b (M x N) = alpha*op(A_b)*op(B_b) + beta*C_b; A, B, C are
    fp32 tensors holding `batch_count` matrices at the given element strides."""
    f32 = _dt(False)
    last = batch_count - 1
    check(call("attn_matmul_batched_strided_f32",
               _ptr(A, f32, last * strideA + M * K, "A"), _ptr(B, f32, last * strideB + K * N, "B"),
               _ptr(C, f32, last * strideC + M * N, "C"), M, N, K, strideA, strideB, strideC,
               batch_count, int(bool(transA)), int(bool(transB)), float(alpha), float(beta),
               _stream(stream)), "matmul_batched_strided")


GEMM_FULL, GEMM_LOWER_OUT, GEMM_LOWER_A, GEMM_UPPER_A = range(4)  # attn_gemm_causal


def matmul_batched_strided_causal(A, B, C, M, N, K, strideA, strideB, strideC, batch_count,
                                  transA, transB, causal, stream=None):
    """matmul_batched_strided (alpha 1, beta 0) skipping what a causal structure makes unused
    (attn_matmul_batched_strided_causal_f32: GEMM_LOWER_OUT, GEMM_LOWER_A, GEMM_UPPER_A)."""
    f32 = _dt(False)
    last = batch_count - 1
    check(call("attn_matmul_batched_strided_causal_f32",
               _ptr(A, f32, last * strideA + M * K, "A"), _ptr(B, f32, last * strideB + K * N, "B"),
               _ptr(C, f32, last * strideC + M * N, "C"), M, N, K, strideA, strideB, strideC,
               batch_count, int(bool(transA)), int(bool(transB)), int(causal), _stream(stream)),
          "matmul_batched_strided_causal")


def materialized_causal_attention_forward(q, k, v, scores, probs, out, B, H, T, d_head, scale,
                                          stream=None):
    """The reference's materialised forward, src/model.cu:313-332 (fp32)."""
    f32 = _dt(False)
    n, nn = B * H * T * d_head, B * H * T * T
    check(call("attn_materialized_causal_forward_f32", _ptr(q, f32, n, "q"), _ptr(k, f32, n, "k"),
               _ptr(v, f32, n, "v"), _ptr(scores, f32, nn, "scores"), _ptr(probs, f32, nn, "probs"),
               _ptr(out, f32, n, "out"), B, H, T, d_head, float(scale), _stream(stream)),
          "materialized_causal_attention_forward")


def materialized_causal_attention_backward(q, k, v, probs, dout, dprobs, dscores, dq, dk, dv,
                                           B, H, T, d_head, scale, stream=None):
    """The reference's materialised backward, src/model.cu:617-650 (fp32)."""
    f32 = _dt(False)
    n, nn = B * H * T * d_head, B * H * T * T
    check(call("attn_materialized_causal_backward_f32", _ptr(q, f32, n, "q"),
               _ptr(k, f32, n, "k"), _ptr(v, f32, n, "v"), _ptr(probs, f32, nn, "probs"),
               _ptr(dout, f32, n, "dout"), _ptr(dprobs, f32, nn, "dprobs"),
               _ptr(dscores, f32, nn, "dscores"), _ptr(dq, f32, n, "dq"), _ptr(dk, f32, n, "dk"),
               _ptr(dv, f32, n, "dv"), B, H, T, d_head, float(scale), _stream(stream)),
          "materialized_causal_attention_backward")


def tiled_causal_attention_forward(q, k, v, out, B, H, T, d_head, scale, m_out=None,
                                   l_out=None, stream=None):
    """Reference: include/kernels/attention.cuh:33-49.  fp32 or bf16 by the tensors' dtype."""
    torch = _torch()
    bf = q.dtype == torch.bfloat16
    n = B * H * T * d_head
    r = B * H * T
    dt = _dt(bf)
    f32 = _dt(False)
    name = "attn_tiled_causal_forward_bf16" if bf else "attn_tiled_causal_forward_f32"
    check(call(name, _ptr(q, dt, n, "q"), _ptr(k, dt, n, "k"), _ptr(v, dt, n, "v"),
               _ptr(out, dt, n, "out"), B, H, T, d_head, float(scale),
               _ptr(m_out, f32, r, "m_out"), _ptr(l_out, f32, r, "l_out"), _stream(stream)),
          "tiled_causal_attention_forward")


def _qkv_forward(family, qkv, out, B, H, T, d_head, scale, m_out, l_out, stream):
    torch = _torch()
    bf = qkv.dtype == torch.bfloat16
    n, r = B * H * T * d_head, B * H * T
    dt, f32 = _dt(bf), _dt(False)
    check(call(f"attn_{family}_causal_forward_" + ("bf16" if bf else "f32"),
               _ptr(qkv, dt, 3 * n, "qkv"), _ptr(out, dt, n, "out"), B, H, T, d_head,
               float(scale), _ptr(m_out, f32, r, "m_out"), _ptr(l_out, f32, r, "l_out"),
               _stream(stream)), f"{family}_causal_attention_forward")


def _qkv_backward(family, stage, qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                  stream):
    torch = _torch()
    bf = qkv.dtype == torch.bfloat16
    n, r = B * H * T * d_head, B * H * T
    dt, f32 = _dt(bf), _dt(False)
    name = f"attn_{family}_causal_backward{stage}_" + ("bf16" if bf else "f32")
    if stage == "_dkdv":
        args = (_ptr(qkv, dt, 3 * n, "qkv"), _ptr(dO, dt, n, "dO"), _ptr(m, f32, r, "m"),
                _ptr(l, f32, r, "l"), _ptr(workspace, f32, r, "workspace"),
                _ptr(dqkv, dt, 3 * n, "dqkv"))
    else:
        args = (_ptr(qkv, dt, 3 * n, "qkv"), _ptr(o, dt, n, "o"), _ptr(dO, dt, n, "dO"),
                _ptr(m, f32, r, "m"), _ptr(l, f32, r, "l"), _ptr(dqkv, dt, 3 * n, "dqkv"),
                _ptr(workspace, f32, r, "workspace"))
    check(call(name, *args, B, H, T, d_head, float(scale), _stream(stream)),
          f"{family}_causal_attention_backward{stage}")


def packed_causal_attention_forward(qkv, out, B, H, T, d_head, scale, m_out=None,
                                    l_out=None, stream=None):
    """Attention straight from the QKV projection's packed output qkv (B, T, 3*H*d): the
    split-transpose (include/kernels/attention.cuh:5-11) happens in the kernels' tile
    copies.  out (B, H, T, d); fp32 or bf16 by the tensors' dtype."""
    _qkv_forward("packed", qkv, out, B, H, T, d_head, scale, m_out, l_out, stream)


def packed_causal_attention_backward(qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                                     stream=None):
    """Backward from the packed qkv, writing dq, dk, dv straight into dqkv (B, T, 3*H*d), the
    layout qkv_split_transpose_backward (include/kernels/attention.cuh:13-19) produces."""
    _qkv_backward("packed", "", qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                  stream)


def packed_causal_attention_backward_dq(qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head,
                                        scale, stream=None):
    """Stage 1 of the packed backward: D into workspace, dq into the q block of dqkv."""
    _qkv_backward("packed", "_dq", qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                  stream)


def packed_causal_attention_backward_dkdv(qkv, dO, m, l, workspace, dqkv, B, H, T, d_head,
                                          scale, stream=None):
    """Stage 2 of the packed backward: dk, dv into the k and v blocks of dqkv."""
    _qkv_backward("packed", "_dkdv", qkv, None, dO, m, l, dqkv, workspace, B, H, T, d_head,
                  scale, stream)


def f32_ds_workspace_bytes(B, H, T, d_head):
    """Bytes of the dS workspace of the fp32 dS-first backward (include/attn_capi.h)."""
    return int(_lib.attn_f32_ds_workspace_bytes(B, H, T, d_head))


def _ds_ptr(ds, B, H, T, d_head):
    need = f32_ds_workspace_bytes(B, H, T, d_head)
    if ds is not None and ds.numel() * ds.element_size() < need:
        raise ValueError(f"ds_workspace: needs {need} bytes")
    return _ptr(ds, None, None, "ds_workspace")


def _backward_ds_f32(family, qkv, o, dO, m, l, dqkv, workspace, ds, B, H, T, d_head, scale,
                     stream):
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call(f"attn_{family}_causal_backward_ds_f32", _ptr(qkv, f32, 3 * n, "qkv"),
               _ptr(o, f32, n, "o"), _ptr(dO, f32, n, "dO"), _ptr(m, f32, r, "m"),
               _ptr(l, f32, r, "l"), _ptr(dqkv, f32, 3 * n, "dqkv"),
               _ptr(workspace, f32, r, "workspace"), _ds_ptr(ds, B, H, T, d_head), B, H, T,
               d_head, float(scale), _stream(stream)), f"{family}_causal_attention_backward_ds")


def packed_causal_attention_backward_ds(qkv, o, dO, m, l, dqkv, workspace, ds_workspace, B, H,
                                        T, d_head, scale, stream=None):
    """packed_causal_attention_backward (fp32) in the dS-first order: dK/dV write dS into
    ds_workspace (f32_ds_workspace_bytes bytes) and dQ is computed from it."""
    _backward_ds_f32("packed", qkv, o, dO, m, l, dqkv, workspace, ds_workspace, B, H, T, d_head,
                     scale, stream)


def fused_causal_attention_backward_ds(qkv, o, dO, m, l, dqkv, workspace, ds_workspace, B, H,
                                       T, d_head, scale, stream=None):
    """fused_causal_attention_backward (fp32) in the dS-first order."""
    _backward_ds_f32("fused", qkv, o, dO, m, l, dqkv, workspace, ds_workspace, B, H, T, d_head,
                     scale, stream)


def _backward_prep_f32(family, o, dO, workspace, B, H, T, d_head, stream):
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call(f"attn_{family}_causal_backward_prep_f32", _ptr(o, f32, n, "o"),
               _ptr(dO, f32, n, "dO"), _ptr(workspace, f32, r, "workspace"), B, H, T, d_head,
               _stream(stream)), f"{family}_causal_attention_backward_prep")


def packed_causal_attention_backward_prep(o, dO, workspace, B, H, T, d_head, stream=None):
    """Stage 1 of packed_causal_attention_backward_ds: D = rowsum(dO o O) into workspace."""
    _backward_prep_f32("packed", o, dO, workspace, B, H, T, d_head, stream)


def fused_causal_attention_backward_prep(o, dO, workspace, B, H, T, d_head, stream=None):
    """Stage 1 of fused_causal_attention_backward_ds."""
    _backward_prep_f32("fused", o, dO, workspace, B, H, T, d_head, stream)


def _backward_dkdv_ds_f32(family, qkv, dO, m, l, workspace, dqkv, ds, B, H, T, d_head, scale,
                          stream):
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call(f"attn_{family}_causal_backward_dkdv_ds_f32", _ptr(qkv, f32, 3 * n, "qkv"),
               _ptr(dO, f32, n, "dO"), _ptr(m, f32, r, "m"), _ptr(l, f32, r, "l"),
               _ptr(workspace, f32, r, "workspace"), _ptr(dqkv, f32, 3 * n, "dqkv"),
               _ds_ptr(ds, B, H, T, d_head), B, H, T, d_head, float(scale), _stream(stream)),
          f"{family}_causal_attention_backward_dkdv_ds")


def packed_causal_attention_backward_dkdv_ds(qkv, dO, m, l, workspace, dqkv, ds_workspace, B, H,
                                             T, d_head, scale, stream=None):
    """Stage 2 of packed_causal_attention_backward_ds: dk, dv into dqkv, dS into ds_workspace."""
    _backward_dkdv_ds_f32("packed", qkv, dO, m, l, workspace, dqkv, ds_workspace, B, H, T,
                          d_head, scale, stream)


def fused_causal_attention_backward_dkdv_ds(qkv, dO, m, l, workspace, dqkv, ds_workspace, B, H,
                                            T, d_head, scale, stream=None):
    """Stage 2 of fused_causal_attention_backward_ds."""
    _backward_dkdv_ds_f32("fused", qkv, dO, m, l, workspace, dqkv, ds_workspace, B, H, T,
                          d_head, scale, stream)


def causal_attention_backward_dq_ds(qkv, dqkv, ds_workspace, B, H, T, d_head, scale,
                                    stream=None):
    """Stage 3 of the fp32 dS-first backwards: dq = scale * dS k into the q block of dqkv."""
    n = B * H * T * d_head
    f32 = _dt(False)
    check(call("attn_causal_backward_dq_ds_f32", _ptr(qkv, f32, 3 * n, "qkv"),
               _ptr(dqkv, f32, 3 * n, "dqkv"), _ds_ptr(ds_workspace, B, H, T, d_head), B, H, T,
               d_head, float(scale), _stream(stream)), "causal_attention_backward_dq_ds")


def fused_causal_attention_forward(qkv, out, B, H, T, d_head, scale, m_out=None, l_out=None,
                                   stream=None):
    """As packed_causal_attention_forward, with out in the merged-heads layout (B, T, H*d)
    that head_merge_transpose_forward (include/kernels/attention.cuh:91-97) produces."""
    _qkv_forward("fused", qkv, out, B, H, T, d_head, scale, m_out, l_out, stream)


def fused_causal_attention_backward(qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                                    stream=None):
    """As packed_causal_attention_backward, with o and dO in the merged-heads layout
    (B, T, H*d) (dO as head_merge_transpose_backward's input, attention.cuh:99-105)."""
    _qkv_backward("fused", "", qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                  stream)


def fused_causal_attention_backward_dq(qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head,
                                       scale, stream=None):
    """Stage 1 of the fused backward."""
    _qkv_backward("fused", "_dq", qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                  stream)


def fused_causal_attention_backward_dkdv(qkv, dO, m, l, workspace, dqkv, B, H, T, d_head,
                                         scale, stream=None):
    """Stage 2 of the fused backward."""
    _qkv_backward("fused", "_dkdv", qkv, None, dO, m, l, dqkv, workspace, B, H, T, d_head,
                  scale, stream)


def f32x3_workspace_bytes(B, H, T, d_head):
    """Bytes of the plane workspace of the *_f32x3 entry points (include/attn_capi.h)."""
    return int(_lib.attn_f32x3_workspace_bytes(B, H, T, d_head))


def f32x3_backward_uses_ds(B, H, T, d_head):
    """Whether the one-call *_f32x3 backwards take the dS-first order (include/attn_capi.h)."""
    return bool(_lib.attn_f32x3_backward_uses_ds(B, H, T, d_head))


def f32x3_planes_bytes(B, H, T, d_head):
    """Bytes of the planes alone (without the dS area) of the *_f32x3 workspace."""
    return int(_lib.attn_f32x3_planes_bytes(B, H, T, d_head))


def f32x3_ds_workspace_bytes(B, H, T, d_head):
    """Bytes of the dS area of the *_f32x3 backward (0 where it takes the two-stage order)."""
    return int(_lib.attn_f32x3_ds_workspace_bytes(B, H, T, d_head))


def f32_backward_uses_ds(B, H, T, d_head):
    """Whether a per-shape caller should take the fp32 dS-first order (include/attn_capi.h)."""
    return bool(_lib.attn_f32_backward_uses_ds(B, H, T, d_head))


def _planes_ptr(planes, B, H, T, d_head, need=None):
    need = f32x3_workspace_bytes(B, H, T, d_head) if need is None else need
    if planes is not None and planes.numel() * planes.element_size() < need:
        raise ValueError(f"planes: needs {need} bytes")
    return _ptr(planes, None, None, "planes")


def _planes_only_ptr(planes, B, H, T, d_head):
    """A workspace that entry points reading no dS take: the planes alone suffice."""
    return _planes_ptr(planes, B, H, T, d_head, f32x3_planes_bytes(B, H, T, d_head))


def _qkv_forward_f32x3(family, qkv, out, B, H, T, d_head, scale, planes, m_out, l_out,
                       stream):
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call(f"attn_{family}_causal_forward_f32x3", _ptr(qkv, f32, 3 * n, "qkv"),
               _ptr(out, f32, n, "out"), B, H, T, d_head, float(scale),
               _ptr(m_out, f32, r, "m_out"), _ptr(l_out, f32, r, "l_out"),
               _planes_only_ptr(planes, B, H, T, d_head), _stream(stream)),
          f"{family}_causal_attention_forward_f32x3")


def packed_causal_attention_forward_f32x3(qkv, out, B, H, T, d_head, scale, planes, m_out=None,
                                          l_out=None, stream=None):
    """packed_causal_attention_forward for fp32 on the bf16 matrix cores (operands as three
    bf16 planes in `planes`, f32x3_workspace_bytes bytes)."""
    _qkv_forward_f32x3("packed", qkv, out, B, H, T, d_head, scale, planes, m_out, l_out, stream)


def fused_causal_attention_forward_f32x3(qkv, out, B, H, T, d_head, scale, planes, m_out=None,
                                         l_out=None, stream=None):
    """fused_causal_attention_forward for fp32 on the bf16 matrix cores."""
    _qkv_forward_f32x3("fused", qkv, out, B, H, T, d_head, scale, planes, m_out, l_out, stream)


def _qkv_backward_f32x3(family, qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                        planes, kv_planes_ready, stream, stage=""):
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call(f"attn_{family}_causal_backward{stage}_f32x3", _ptr(qkv, f32, 3 * n, "qkv"),
               _ptr(o, f32, n, "o"), _ptr(dO, f32, n, "dO"), _ptr(m, f32, r, "m"),
               _ptr(l, f32, r, "l"), _ptr(dqkv, f32, 3 * n, "dqkv"),
               _ptr(workspace, f32, r, "workspace"), B, H, T, d_head, float(scale),
               _planes_ptr(planes, B, H, T, d_head), 1 if kv_planes_ready else 0,
               _stream(stream)), f"{family}_causal_attention_backward_f32x3")


def packed_causal_attention_backward_f32x3(qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head,
                                           scale, planes, kv_planes_ready=False, stream=None):
    """packed_causal_attention_backward for fp32 on the bf16 matrix cores; kv_planes_ready
    reuses the q/k/v planes the forward left in `planes` (qkv unchanged since)."""
    _qkv_backward_f32x3("packed", qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                        planes, kv_planes_ready, stream)


def fused_causal_attention_backward_f32x3(qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head,
                                          scale, planes, kv_planes_ready=False, stream=None):
    """fused_causal_attention_backward for fp32 on the bf16 matrix cores."""
    _qkv_backward_f32x3("fused", qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                        planes, kv_planes_ready, stream)


def _backward_ds_f32x3(family, qkv, o, dO, m, l, dqkv, workspace, ds_workspace, B, H, T,
                       d_head, scale, planes, kv_planes_ready, stream):
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    need = f32x3_ds_workspace_bytes(B, H, T, d_head)
    if need and (ds_workspace is None or ds_workspace.numel() * ds_workspace.element_size() < need):
        raise ValueError(f"ds_workspace: needs {need} bytes")
    check(call(f"attn_{family}_causal_backward_ds_f32x3", _ptr(qkv, f32, 3 * n, "qkv"),
               _ptr(o, f32, n, "o"), _ptr(dO, f32, n, "dO"), _ptr(m, f32, r, "m"),
               _ptr(l, f32, r, "l"), _ptr(dqkv, f32, 3 * n, "dqkv"),
               _ptr(workspace, f32, r, "workspace"),
               _ptr(ds_workspace, None, None, "ds_workspace"), B, H, T, d_head, float(scale),
               _planes_only_ptr(planes, B, H, T, d_head),
               1 if kv_planes_ready else 0, _stream(stream)),
          f"{family}_causal_attention_backward_ds_f32x3")


def packed_causal_attention_backward_ds_f32x3(qkv, o, dO, m, l, dqkv, workspace, ds_workspace,
                                              B, H, T, d_head, scale, planes,
                                              kv_planes_ready=False, stream=None):
    """packed_causal_attention_backward_f32x3 with the planes (f32x3_planes_bytes) and dS
    (f32x3_ds_workspace_bytes; None where that is 0) in separate buffers."""
    _backward_ds_f32x3("packed", qkv, o, dO, m, l, dqkv, workspace, ds_workspace, B, H, T,
                       d_head, scale, planes, kv_planes_ready, stream)


def fused_causal_attention_backward_ds_f32x3(qkv, o, dO, m, l, dqkv, workspace, ds_workspace,
                                             B, H, T, d_head, scale, planes,
                                             kv_planes_ready=False, stream=None):
    """fused_causal_attention_backward_f32x3 with the planes and dS in separate buffers."""
    _backward_ds_f32x3("fused", qkv, o, dO, m, l, dqkv, workspace, ds_workspace, B, H, T,
                       d_head, scale, planes, kv_planes_ready, stream)


def _backward_prep_f32x3(family, qkv, o, dO, workspace, B, H, T, d_head, planes,
                         kv_planes_ready, stream):
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call(f"attn_{family}_causal_backward_prep_f32x3", _ptr(qkv, f32, 3 * n, "qkv"),
               _ptr(o, f32, n, "o"), _ptr(dO, f32, n, "dO"),
               _ptr(workspace, f32, r, "workspace"), B, H, T, d_head,
               _planes_only_ptr(planes, B, H, T, d_head), 1 if kv_planes_ready else 0,
               _stream(stream)), f"{family}_causal_attention_backward_prep_f32x3")


def packed_causal_attention_backward_prep_f32x3(qkv, o, dO, workspace, B, H, T, d_head, planes,
                                                kv_planes_ready=False, stream=None):
    """Stage 1 of packed_causal_attention_backward_f32x3: D and the planes of dO (and of q, k,
    v unless kv_planes_ready)."""
    _backward_prep_f32x3("packed", qkv, o, dO, workspace, B, H, T, d_head, planes,
                         kv_planes_ready, stream)


def fused_causal_attention_backward_prep_f32x3(qkv, o, dO, workspace, B, H, T, d_head, planes,
                                               kv_planes_ready=False, stream=None):
    """Stage 1 of fused_causal_attention_backward_f32x3."""
    _backward_prep_f32x3("fused", qkv, o, dO, workspace, B, H, T, d_head, planes,
                         kv_planes_ready, stream)


def causal_attention_backward_dkdv_ds_f32x3(qkv, m, l, workspace, dqkv, B, H, T, d_head, scale,
                                            planes, stream=None):
    """Stage 2 of the one-call *_f32x3 backwards: dK, dV into dqkv, dS into `planes`."""
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call("attn_causal_backward_dkdv_ds_f32x3", _ptr(qkv, f32, 3 * n, "qkv"),
               _ptr(m, f32, r, "m"), _ptr(l, f32, r, "l"), _ptr(workspace, f32, r, "workspace"),
               _ptr(dqkv, f32, 3 * n, "dqkv"), B, H, T, d_head, float(scale),
               _planes_ptr(planes, B, H, T, d_head), _stream(stream)),
          "causal_attention_backward_dkdv_ds_f32x3")


def causal_attention_backward_dq_ds_f32x3(dqkv, B, H, T, d_head, scale, planes, stream=None):
    """Stage 3 of the one-call *_f32x3 backwards: dQ into dqkv from dS and k's planes."""
    n = B * H * T * d_head
    check(call("attn_causal_backward_dq_ds_f32x3", _ptr(dqkv, _dt(False), 3 * n, "dqkv"), B, H,
               T, d_head, float(scale), _planes_ptr(planes, B, H, T, d_head), _stream(stream)),
          "causal_attention_backward_dq_ds_f32x3")


def packed_causal_attention_backward_dq_f32x3(qkv, o, dO, m, l, dqkv, workspace, B, H, T,
                                              d_head, scale, planes, kv_planes_ready=False,
                                              stream=None):
    """Stage 1 of the two-stage order of packed_causal_attention_backward_f32x3 (D, dQ, planes
    of dO; computes S and dP itself)."""
    _qkv_backward_f32x3("packed", qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                        planes, kv_planes_ready, stream, "_dq")


def fused_causal_attention_backward_dq_f32x3(qkv, o, dO, m, l, dqkv, workspace, B, H, T,
                                             d_head, scale, planes, kv_planes_ready=False,
                                             stream=None):
    """Stage 1 of fused_causal_attention_backward_f32x3."""
    _qkv_backward_f32x3("fused", qkv, o, dO, m, l, dqkv, workspace, B, H, T, d_head, scale,
                        planes, kv_planes_ready, stream, "_dq")


def causal_attention_backward_dkdv_f32x3(qkv, m, l, workspace, dqkv, B, H, T, d_head, scale,
                                         planes, stream=None):
    """Stage 2 of the two-stage order (dK, dV from the planes stage 1 wrote)."""
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call("attn_causal_backward_dkdv_f32x3", _ptr(qkv, f32, 3 * n, "qkv"),
               _ptr(m, f32, r, "m"), _ptr(l, f32, r, "l"), _ptr(workspace, f32, r, "workspace"),
               _ptr(dqkv, f32, 3 * n, "dqkv"), B, H, T, d_head, float(scale),
               _planes_only_ptr(planes, B, H, T, d_head), _stream(stream)),
          "causal_attention_backward_dkdv_f32x3")


def tiled_causal_attention_forward_f32x3(q, k, v, out, B, H, T, d_head, scale, planes,
                                         m_out=None, l_out=None, stream=None):
    """tiled_causal_attention_forward (include/kernels/attention.cuh:39-49) for fp32 on the
    bf16 matrix cores (operands as three bf16 planes in `planes`)."""
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call("attn_tiled_causal_forward_f32x3", _ptr(q, f32, n, "q"), _ptr(k, f32, n, "k"),
               _ptr(v, f32, n, "v"), _ptr(out, f32, n, "out"), B, H, T, d_head, float(scale),
               _ptr(m_out, f32, r, "m_out"), _ptr(l_out, f32, r, "l_out"),
               _planes_only_ptr(planes, B, H, T, d_head), _stream(stream)),
          "tiled_causal_attention_forward_f32x3")


def tiled_causal_attention_backward_f32x3(q, k, v, o, dO, m, l, dq, dk, dv, workspace, B, H, T,
                                          d_head, scale, planes, kv_planes_ready=False,
                                          stream=None):
    """tiled_causal_attention_backward (attention.cuh:63-78) for fp32 on the bf16 matrix
    cores; kv_planes_ready reuses the q/k/v planes the forward left in `planes`."""
    n, r = B * H * T * d_head, B * H * T
    f32 = _dt(False)
    check(call("attn_tiled_causal_backward_f32x3", _ptr(q, f32, n, "q"), _ptr(k, f32, n, "k"),
               _ptr(v, f32, n, "v"), _ptr(o, f32, n, "o"), _ptr(dO, f32, n, "dO"),
               _ptr(m, f32, r, "m"), _ptr(l, f32, r, "l"), _ptr(dq, f32, n, "dq"),
               _ptr(dk, f32, n, "dk"), _ptr(dv, f32, n, "dv"),
               _ptr(workspace, f32, r, "workspace"), B, H, T, d_head, float(scale),
               _planes_ptr(planes, B, H, T, d_head), 1 if kv_planes_ready else 0,
               _stream(stream)), "tiled_causal_attention_backward_f32x3")


def attention_precompute_dot_do_o(dO, O, D, B, H, T, d_head, stream=None):
    """Reference: include/kernels/attention.cuh:51-58."""
    n = B * H * T * d_head
    f32 = _dt(False)
    check(call("attn_precompute_dot_do_o_f32", _ptr(dO, f32, n, "dO"), _ptr(O, f32, n, "O"),
               _ptr(D, f32, B * H * T, "D"), B, H, T, d_head, _stream(stream)),
          "attention_precompute_dot_do_o")


def tiled_causal_attention_backward(q, k, v, o, do, m, l, dq, dk, dv, d_workspace, B, H, T,
                                    d_head, scale, stream=None):
    """Reference: include/kernels/attention.cuh:60-78.  fp32 or bf16 by q's dtype."""
    torch = _torch()
    bf = q.dtype == torch.bfloat16
    n = B * H * T * d_head
    r = B * H * T
    dt = _dt(bf)
    f32 = _dt(False)
    name = "attn_tiled_causal_backward_bf16" if bf else "attn_tiled_causal_backward_f32"
    check(call(name, _ptr(q, dt, n, "q"), _ptr(k, dt, n, "k"), _ptr(v, dt, n, "v"),
               _ptr(o, dt, n, "o"), _ptr(do, dt, n, "do"), _ptr(m, f32, r, "m"),
               _ptr(l, f32, r, "l"), _ptr(dq, dt, n, "dq"), _ptr(dk, dt, n, "dk"),
               _ptr(dv, dt, n, "dv"), _ptr(d_workspace, f32, r, "d_workspace"),
               B, H, T, d_head, float(scale), _stream(stream)),
          "tiled_causal_attention_backward")


def tiled_causal_attention_backward_noalloc(q, k, v, o, do, m, l, dq, dk, dv, B, H, T, d_head,
                                            scale, stream=None):
    """tiled_causal_attention_backward (fp32) without a caller workspace: D lives in the
    library's fixed device scratch (attn_tiled_causal_backward_f32_noalloc)."""
    n = B * H * T * d_head
    r = B * H * T
    f32 = _dt(False)
    check(call("attn_tiled_causal_backward_f32_noalloc", _ptr(q, f32, n, "q"),
               _ptr(k, f32, n, "k"), _ptr(v, f32, n, "v"), _ptr(o, f32, n, "o"),
               _ptr(do, f32, n, "do"), _ptr(m, f32, r, "m"), _ptr(l, f32, r, "l"),
               _ptr(dq, f32, n, "dq"), _ptr(dk, f32, n, "dk"), _ptr(dv, f32, n, "dv"),
               B, H, T, d_head, float(scale), _stream(stream)),
          "tiled_causal_attention_backward_noalloc")


def tiled_causal_attention_backward_dq(q, k, v, o, do, m, l, dq, d_workspace, B, H, T, d_head,
                                       scale, stream=None):
    """Stage 1 of the backward (D and dQ)."""
    torch = _torch()
    bf = q.dtype == torch.bfloat16
    n = B * H * T * d_head
    r = B * H * T
    dt = _dt(bf)
    f32 = _dt(False)
    name = "attn_tiled_causal_backward_dq_bf16" if bf else "attn_tiled_causal_backward_dq_f32"
    check(call(name, _ptr(q, dt, n, "q"), _ptr(k, dt, n, "k"), _ptr(v, dt, n, "v"),
               _ptr(o, dt, n, "o"), _ptr(do, dt, n, "do"), _ptr(m, f32, r, "m"),
               _ptr(l, f32, r, "l"), _ptr(dq, dt, n, "dq"),
               _ptr(d_workspace, f32, r, "d_workspace"), B, H, T, d_head, float(scale),
               _stream(stream)), "tiled_causal_attention_backward_dq")


def tiled_causal_attention_backward_dkdv(q, k, v, do, m, l, d_workspace, dk, dv, B, H, T,
                                         d_head, scale, stream=None):
    """Stage 2 of the backward (dK, dV from D in d_workspace)."""
    torch = _torch()
    bf = q.dtype == torch.bfloat16
    n = B * H * T * d_head
    r = B * H * T
    dt = _dt(bf)
    f32 = _dt(False)
    name = ("attn_tiled_causal_backward_dkdv_bf16" if bf else
            "attn_tiled_causal_backward_dkdv_f32")
    check(call(name, _ptr(q, dt, n, "q"), _ptr(k, dt, n, "k"), _ptr(v, dt, n, "v"),
               _ptr(do, dt, n, "do"), _ptr(m, f32, r, "m"), _ptr(l, f32, r, "l"),
               _ptr(d_workspace, f32, r, "d_workspace"), _ptr(dk, dt, n, "dk"),
               _ptr(dv, dt, n, "dv"), B, H, T, d_head, float(scale), _stream(stream)),
          "tiled_causal_attention_backward_dkdv")


# ---------------------------------------------------------------------------------------
# Allocating conveniences for tests and the bench (not part of the reference API).
# ---------------------------------------------------------------------------------------
def attention_forward(q, k, v, scale):
    """(out, m, l) for (B, H, T, d) GPU tensors."""
    torch = _torch()
    B, H, T, d = q.shape
    out = torch.empty_like(q)
    m = torch.empty((B, H, T), device=q.device, dtype=torch.float32)
    l = torch.empty_like(m)
    tiled_causal_attention_forward(q, k, v, out, B, H, T, d, scale, m, l)
    return out, m, l


def attention_backward(q, k, v, o, do, m, l, scale):
    """(dq, dk, dv, D) for (B, H, T, d) GPU tensors."""
    torch = _torch()
    B, H, T, d = q.shape
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    ws = torch.empty((B, H, T), device=q.device, dtype=torch.float32)
    tiled_causal_attention_backward(q, k, v, o, do, m, l, dq, dk, dv, ws, B, H, T, d, scale)
    return dq, dk, dv, ws
