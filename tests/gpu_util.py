"""Shared helpers of the GPU parity tests (not collected as tests)."""
import math

import numpy as np
import torch

from oracle import attention_ref as ref


def to_dev(x, dtype=torch.float32):
    return torch.as_tensor(np.ascontiguousarray(x)).to(device="cuda:0", dtype=dtype).contiguous()


def gpu_fwd_bwd(lib, q, k, v, do, scale, dtype=torch.float32):
    """Run the product's forward + backward on (B,H,T,d) numpy inputs; returns numpy fp32
    (o, m, l, dq, dk, dv, D)."""
    qg, kg, vg, dog = (to_dev(x, dtype) for x in (q, k, v, do))
    o, m, l = lib.attention_forward(qg, kg, vg, scale)
    dq, dk, dv, D = lib.attention_backward(qg, kg, vg, o, dog, m, l, scale)
    torch.cuda.synchronize()
    f = lambda t: t.float().cpu().numpy()
    return dict(o=f(o), m=f(m), l=f(l), dq=f(dq), dk=f(dk), dv=f(dv), D=f(D))


def max_abs(a, b):
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max())


def rel_l2(a, b):
    return ref.compute_metrics(a, b)["rel_err"]


def default_scale(d):
    return 1.0 / math.sqrt(d)
