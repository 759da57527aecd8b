"""Restatement of the reference attention, for checking the HIP path (test use only).

Forward, op for op as pytorch_src/model.py:43-52:
    att   = (q @ k^T) * scale                                   (model.py:44-45)
    att   = att.masked_fill(tril == 0, -inf)                    (model.py:47-48)
    probs = softmax(att, dim=-1)                                (model.py:50-51)
    y     = probs @ v                                           (model.py:52)
Backward = torch autograd of that forward w.r.t. q, k, v given dO (what the reference's
PyTorch training step computes, pytorch_src/utils.py:226-227).

The statistics follow the reference's tiled kernel contract (src/kernels/attention.cu:
615-622): m_i = max_{j<=i} scale*q_i.k_j, l_i = sum_{j<=i} exp(scale*q_i.k_j - m_i),
so that P_ij = exp(scale*q_i.k_j - m_i)/l_i and LSE_i = m_i + ln(l_i).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch


def causal_mask(T: int) -> torch.Tensor:
    """tril(ones(T, T)) as registered in model.py:26-29 (1 = keep, 0 = masked)."""
    return torch.tril(torch.ones(T, T))


def forward_torch(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """y = softmax(mask((q @ k^T) * scale)) @ v on (B, H, T, d) tensors (model.py:44-52)."""
    T = q.shape[-2]
    att = (q @ k.transpose(-2, -1)) * scale
    att = att.masked_fill(causal_mask(T).to(att.dtype) == 0, float("-inf"))
    probs = torch.softmax(att, dim=-1)
    return probs @ v


@dataclass
class AttnResult:
    o: torch.Tensor
    m: torch.Tensor
    l: torch.Tensor
    lse: torch.Tensor
    dq: torch.Tensor | None = None
    dk: torch.Tensor | None = None
    dv: torch.Tensor | None = None


def stats_torch(q: torch.Tensor, k: torch.Tensor, scale: float):
    """m, l, lse of the reference stats contract (attention.cu:599-622), same dtype as q."""
    T = q.shape[-2]
    att = (q @ k.transpose(-2, -1)) * scale
    att = att.masked_fill(causal_mask(T).to(att.dtype) == 0, float("-inf"))
    m = att.amax(dim=-1)
    l = torch.exp(att - m.unsqueeze(-1)).sum(dim=-1)
    return m, l, m + torch.log(l)


def attention_fwd_bwd(q, k, v, do, scale: float, dtype=torch.float32, with_grad=True) -> AttnResult:
    """Forward + autograd backward of the restated reference on the CPU in `dtype`.

    Inputs may be numpy arrays or tensors of shape (B, H, T, d); they are converted to
    `dtype` on the CPU first.
    """
    def t(x):
        x = torch.as_tensor(x)
        return x.detach().to(device="cpu", dtype=dtype).clone()

    qt, kt, vt = t(q), t(k), t(v)
    if with_grad:
        qt.requires_grad_(True)
        kt.requires_grad_(True)
        vt.requires_grad_(True)
    o = forward_torch(qt, kt, vt, scale)
    dq = dk = dv = None
    if with_grad:
        o.backward(t(do))
        dq, dk, dv = qt.grad.detach(), kt.grad.detach(), vt.grad.detach()
    with torch.no_grad():
        m, l, lse = stats_torch(qt.detach(), kt.detach(), scale)
    return AttnResult(o=o.detach(), m=m, l=l, lse=lse, dq=dq, dk=dk, dv=dv)


# ----------------------------------------------------------------------------------------
# Independent fp64 restatement with the analytic backward (numpy, no autograd).
#   S = scale * Q K^T, P = softmax over j <= i, O = P V
#   dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dP * P)), dQ = scale dS K, dK = scale dS^T Q
# (the closed-form backward the reference's materialised path evaluates,
#  src/model.cu:617-650 with causal_softmax_backward, attention.cu:242-305)
# ----------------------------------------------------------------------------------------
def attention_numpy64(q, k, v, do, scale: float):
    q, k, v, do = (np.asarray(x, dtype=np.float64) for x in (q, k, v, do))
    T = q.shape[-2]
    s = np.einsum("...id,...jd->...ij", q, k) * scale
    mask = np.tril(np.ones((T, T), dtype=bool))
    s = np.where(mask, s, -np.inf)
    m = s.max(axis=-1)
    e = np.exp(s - m[..., None])
    l = e.sum(axis=-1)
    p = e / l[..., None]
    o = p @ v
    dv = np.swapaxes(p, -1, -2) @ do
    dp = do @ np.swapaxes(v, -1, -2)
    dsum = (dp * p).sum(axis=-1, keepdims=True)
    ds = p * (dp - dsum)
    dq = scale * (ds @ k)
    dk = scale * (np.swapaxes(ds, -1, -2) @ q)
    D = (do * o).sum(axis=-1)
    return dict(o=o, m=m, l=l, lse=m + np.log(l), p=p, ds=ds, dq=dq, dk=dk, dv=dv, D=D)


# ----------------------------------------------------------------------------------------
# Pure-Python loops for tiny shapes: the definitions written element by element.
# ----------------------------------------------------------------------------------------
def attention_loops(q, k, v, scale: float):
    """O and (m, l) by explicit loops over one (T, d) head (fp64 Python floats)."""
    T, d = len(q), len(q[0])
    o = [[0.0] * d for _ in range(T)]
    ms, ls = [], []
    for i in range(T):
        scores = [scale * sum(q[i][e] * k[j][e] for e in range(d)) for j in range(i + 1)]
        mx = max(scores)
        ex = [math.exp(s - mx) for s in scores]
        tot = sum(ex)
        for e in range(d):
            o[i][e] = sum(ex[j] * v[j][e] for j in range(i + 1)) / tot
        ms.append(mx)
        ls.append(tot)
    return o, ms, ls


def finite_difference_grads(q, k, v, do, scale: float, eps: float = 1e-6):
    """Central differences of L = sum(O * dO) w.r.t. every element of q, k, v (fp64).
    O(#elements) forward evaluations: tiny shapes only."""
    q, k, v, do = (np.array(x, dtype=np.float64) for x in (q, k, v, do))

    def loss(qq, kk, vv):
        return float((attention_numpy64(qq, kk, vv, do, scale)["o"] * do).sum())

    grads = []
    for which in range(3):
        base = [q, k, v]
        g = np.zeros_like(base[which])
        it = np.nditer(base[which], flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            plus = [x.copy() for x in base]
            minus = [x.copy() for x in base]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            g[idx] = (loss(*plus) - loss(*minus)) / (2 * eps)
        grads.append(g)
    return grads


# ----------------------------------------------------------------------------------------
# Parity metrics of the reference gate (scripts/compare_parity.py:11-26).
# ----------------------------------------------------------------------------------------
def compute_metrics(a, b) -> dict:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    diff = np.abs(a - b)
    return {
        "max_err": float(diff.max()) if diff.size else 0.0,
        "mean_err": float(diff.mean()) if diff.size else 0.0,
        "rms_err": float(np.sqrt((diff ** 2).mean())) if diff.size else 0.0,
        "rel_err": float(np.linalg.norm(diff.ravel()) / (np.linalg.norm(b.ravel()) + 1e-12)),
        "elements": int(a.size),
    }


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 (nearest even) and return them as fp32 (torch's cast)."""
    return torch.as_tensor(np.asarray(x, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def seeded_inputs(B: int, H: int, T: int, d: int, seed: int = 42, qk_scale: float = 1.0):
    """Q, K, V, dO ~ N(0, 1) fp32 drawn in that order from torch.Generator(cpu).manual_seed
    (seed 42 = the reference default, pytorch_src/utils.py:183); Q and K multiplied by
    qk_scale (0.5 for config 4)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    shape = (B, H, T, d)
    q = torch.randn(shape, generator=g, dtype=torch.float32)
    k = torch.randn(shape, generator=g, dtype=torch.float32)
    v = torch.randn(shape, generator=g, dtype=torch.float32)
    do = torch.randn(shape, generator=g, dtype=torch.float32)
    if qk_scale != 1.0:
        q = q * qk_scale
        k = k * qk_scale
    return q.numpy(), k.numpy(), v.numpy(), do.numpy()
