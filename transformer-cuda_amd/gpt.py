"""Python binding of the GPT training-step harness (libtcamd_gpt.so, include/gpt_capi.h).

The harness is the caller of the attention path in the reference: TransformerModel's
forward/backward (src/model.cu:248-704) and the fused clip + AdamW step
(src/optimizer.cu:117-154), fp32, with rocBLAS GEMMs and the attention of every block on
libtcamd_attn.  This module binds the C ABI with ctypes; torch supplies device memory for
tokens, targets and the loss.  There is no CPU fallback: importing it fails if the library
is not built.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import LIB_PATH as _ATTN_LIB, check  # noqa: F401  (loads libtcamd_attn first)

_HERE = os.path.dirname(os.path.abspath(__file__))
GPT_LIB_PATH = os.path.join(_HERE, "libtcamd_gpt.so")
GPT_HEADER = os.path.join(os.path.dirname(_HERE), "include", "gpt_capi.h")

if not os.path.exists(GPT_LIB_PATH):
    raise ImportError(
        f"{GPT_LIB_PATH} is not built; run __graft_entry__.build() (make -C transformer-cuda_amd)")

_lib = ctypes.CDLL(GPT_LIB_PATH)

ATTN_FUSED, ATTN_TILED_SPLIT, ATTN_MATERIALIZED, ATTN_FUSED_X3 = 0, 1, 2, 3
MODES = {"fused": ATTN_FUSED, "tiled_split": ATTN_TILED_SPLIT,
         "materialized": ATTN_MATERIALIZED, "fused_x3": ATTN_FUSED_X3}


class GptConfig(ctypes.Structure):
    """Mirrors gpt_config (include/config.h's TransformerConfig fields on the path)."""
    _fields_ = [(n, ctypes.c_int) for n in ("vocab_size", "max_seq_len", "d_model",
                                            "num_layers", "num_heads", "d_ff", "batch_size")] + \
               [(n, ctypes.c_float) for n in ("layernorm_eps", "learning_rate", "weight_decay",
                                              "beta1", "beta2", "adam_eps", "grad_clip")] + \
               [("attention_mode", ctypes.c_int)]


_P, _I, _L = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
SIGNATURES = {
    "gpt_default_config": ([ctypes.POINTER(GptConfig), _I, _I, _I, _I, _I, _I, _I], None),
    "gpt_create": ([ctypes.POINTER(GptConfig), ctypes.POINTER(_P)], _I),
    "gpt_destroy": ([_P], None),
    "gpt_num_parameters": ([_P], _L),
    "gpt_set_parameters": ([_P, _P, _L], _I),
    "gpt_get_parameters": ([_P, _P, _L], _I),
    "gpt_get_gradients": ([_P, _P, _L], _I),
    "gpt_get_logits": ([_P, _P, _L], _I),
    "gpt_forward_backward": ([_P, _P, _P, _P, _P], _I),
    "gpt_optimizer_step": ([_P, _P], _I),
    "gpt_set_attention_timing": ([_P, _I], _I),
    "gpt_last_attention_ms": ([_P, ctypes.POINTER(ctypes.c_float)], _I),
}
for _name, (_args, _ret) in SIGNATURES.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = _ret


def raw():
    return _lib


def default_config(V, T, C, L, H, d_ff, B, attention="fused") -> GptConfig:
    cfg = GptConfig()
    _lib.gpt_default_config(ctypes.byref(cfg), V, T, C, L, H, d_ff, B)
    cfg.attention_mode = MODES[attention]
    return cfg


def param_layout(V, T, C, L, d_ff):
    """(name, shape) of every tensor of the flat parameter buffer, in order
    (src/model.cu:185-217); weights are stored (in, out)."""
    out = [("tok_emb", (V, C)), ("pos_emb", (T, C))]
    for i in range(L):
        out += [(f"l{i}.ln1_g", (C,)), (f"l{i}.ln1_b", (C,)), (f"l{i}.qkv_w", (C, 3 * C)),
                (f"l{i}.qkv_b", (3 * C,)), (f"l{i}.proj_w", (C, C)), (f"l{i}.proj_b", (C,)),
                (f"l{i}.ln2_g", (C,)), (f"l{i}.ln2_b", (C,)), (f"l{i}.ffn1_w", (C, d_ff)),
                (f"l{i}.ffn1_b", (d_ff,)), (f"l{i}.ffn2_w", (d_ff, C)),
                (f"l{i}.ffn2_b", (C,))]
    out += [("lnf_g", (C,)), ("lnf_b", (C,)), ("head_w", (C, V))]
    return out


class GPT:
    """One model instance on the current device."""

    def __init__(self, cfg: GptConfig):
        self.cfg = cfg
        h = _P()
        check(_lib.gpt_create(ctypes.byref(cfg), ctypes.byref(h)), "gpt_create")
        self._h = h
        self.n_params = int(_lib.gpt_num_parameters(h))

    def close(self):
        if self._h:
            _lib.gpt_destroy(self._h)
            self._h = _P()

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass

    def set_parameters(self, flat: np.ndarray):
        flat = np.ascontiguousarray(flat, dtype=np.float32)
        check(_lib.gpt_set_parameters(self._h, flat.ctypes.data, flat.size), "gpt_set_parameters")

    def parameters(self) -> np.ndarray:
        out = np.empty(self.n_params, np.float32)
        check(_lib.gpt_get_parameters(self._h, out.ctypes.data, out.size), "gpt_get_parameters")
        return out

    def gradients(self) -> np.ndarray:
        out = np.empty(self.n_params, np.float32)
        check(_lib.gpt_get_gradients(self._h, out.ctypes.data, out.size), "gpt_get_gradients")
        return out

    def logits(self) -> np.ndarray:
        c = self.cfg
        out = np.empty(c.batch_size * c.max_seq_len * c.vocab_size, np.float32)
        check(_lib.gpt_get_logits(self._h, out.ctypes.data, out.size), "gpt_get_logits")
        return out

    def forward_backward(self, tokens, targets, loss, stream=None):
        """tokens, targets: int32 device tensors (B, T); loss: float32 device tensor (1,)."""
        import torch
        for t, dt in ((tokens, torch.int32), (targets, torch.int32), (loss, torch.float32)):
            if not t.is_cuda or t.dtype != dt or not t.is_contiguous():
                raise ValueError("tokens/targets must be contiguous int32 and loss float32 on the GPU")
        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        check(_lib.gpt_forward_backward(self._h, tokens.data_ptr(), targets.data_ptr(),
                                        loss.data_ptr(), s), "gpt_forward_backward")

    def optimizer_step(self, stream=None):
        import torch
        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        check(_lib.gpt_optimizer_step(self._h, s), "gpt_optimizer_step")

    def set_attention_timing(self, on: bool):
        check(_lib.gpt_set_attention_timing(self._h, 1 if on else 0), "gpt_set_attention_timing")

    def last_attention_ms(self) -> float:
        v = ctypes.c_float()
        check(_lib.gpt_last_attention_ms(self._h, ctypes.byref(v)), "gpt_last_attention_ms")
        return float(v.value)
