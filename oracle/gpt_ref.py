"""Restatement of the reference's tiny GPT (pytorch_src/model.py:61-136) with its golden
init recipe (pytorch_src/utils.py:183-213), used to capture the layer-0 attention tensors
of config 1 (B4 T64 C128 H4 L2 d_ff512 V256).  Test use only.

Module construction order and types follow model.py (nn.Embedding x2, then per block
LayerNorm, Linear qkv, Linear out, LayerNorm, Linear ffn_1, Linear ffn_2, then LayerNorm,
Linear head) so that, after torch.manual_seed(seed), construction and the
`p.normal_(0, 0.02)` pass over model.parameters() consume the generator in the same order
as the reference's generate_golden_reference.  Bit-identity with the reference's own
fixture stream is not verified (the reference is not imported): the fixture's inputs are
what this restatement draws, and the parity target is the attention output/gradients for
those inputs.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F


class _Attn(nn.Module):
    def __init__(self, C: int, H: int, max_T: int):
        super().__init__()
        self.C, self.H, self.d = C, H, C // H
        self.qkv_proj = nn.Linear(C, 3 * C, bias=True)
        self.out_proj = nn.Linear(C, C, bias=True)
        self.register_buffer("mask", torch.tril(torch.ones(max_T, max_T)).view(1, 1, max_T, max_T))
        self.capture = None  # dict filled for the captured layer

    def forward(self, x):
        B, T, C = x.shape
        q, k, v = self.qkv_proj(x).chunk(3, dim=-1)
        q = q.view(B, T, self.H, self.d).transpose(1, 2)
        k = k.view(B, T, self.H, self.d).transpose(1, 2)
        v = v.view(B, T, self.H, self.d).transpose(1, 2)
        if self.capture is not None:
            for t in (q, k, v):
                t.retain_grad()
        att = (q @ k.transpose(-2, -1)) * (1.0 / math.sqrt(self.d))
        att = att.masked_fill(self.mask[:, :, :T, :T] == 0, float("-inf"))
        y = F.softmax(att, dim=-1) @ v
        if self.capture is not None:
            y.retain_grad()
            self.capture.update(q=q, k=k, v=v, o=y)
        y = y.transpose(1, 2).contiguous().view(B, T, C)
        return self.out_proj(y)


class _Block(nn.Module):
    def __init__(self, C, H, d_ff, max_T, eps):
        super().__init__()
        self.ln_1 = nn.LayerNorm(C, eps=eps)
        self.attn = _Attn(C, H, max_T)
        self.ln_2 = nn.LayerNorm(C, eps=eps)
        self.ffn_1 = nn.Linear(C, d_ff, bias=True)
        self.ffn_2 = nn.Linear(d_ff, C, bias=True)

    def forward(self, x):
        x = x + self.attn(self.ln_1(x))
        return x + self.ffn_2(F.gelu(self.ffn_1(self.ln_2(x)), approximate="tanh"))


class TinyGPT(nn.Module):
    def __init__(self, V, max_T, C, L, H, d_ff, eps=1e-5):
        super().__init__()
        self.V = V
        self.tok_emb = nn.Embedding(V, C)
        self.pos_emb = nn.Embedding(max_T, C)
        self.blocks = nn.ModuleList([_Block(C, H, d_ff, max_T, eps) for _ in range(L)])
        self.ln_f = nn.LayerNorm(C, eps=eps)
        self.head = nn.Linear(C, V, bias=False)

    def forward(self, idx, targets):
        B, T = idx.shape
        x = self.tok_emb(idx) + self.pos_emb(torch.arange(T))
        for blk in self.blocks:
            x = blk(x)
        logits = self.head(self.ln_f(x))
        return logits, F.cross_entropy(logits.view(-1, self.V), targets.view(-1))


def layer0_attention_tensors(B=4, T=64, C=128, L=2, H=4, d_ff=512, V=256, seed=42):
    """One fwd+bwd step of the tiny GPT in fp32 on the CPU; returns layer 0's attention
    q, k, v, O (B,H,T,d), the upstream gradient dO of O, and dQ, dK, dV, as numpy."""
    torch.manual_seed(seed)
    model = TinyGPT(V, T, C, L, H, d_ff)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(mean=0.0, std=0.02)
        for blk in model.blocks:
            blk.ln_1.weight.fill_(1.0)
            blk.ln_1.bias.zero_()
            blk.attn.qkv_proj.bias.zero_()
            blk.attn.out_proj.bias.zero_()
            blk.ln_2.weight.fill_(1.0)
            blk.ln_2.bias.zero_()
            blk.ffn_1.bias.zero_()
            blk.ffn_2.bias.zero_()
        model.ln_f.weight.fill_(1.0)
        model.ln_f.bias.zero_()
    x = torch.randint(0, V, (B, T), dtype=torch.long)
    y = torch.randint(0, V, (B, T), dtype=torch.long)
    cap = {}
    model.blocks[0].attn.capture = cap
    _, loss = model(x, y)
    loss.backward()
    out = {n: cap[n].detach().contiguous().numpy() for n in ("q", "k", "v", "o")}
    out["do"] = cap["o"].grad.detach().contiguous().numpy()
    out["dq"] = cap["q"].grad.detach().contiguous().numpy()
    out["dk"] = cap["k"].grad.detach().contiguous().numpy()
    out["dv"] = cap["v"].grad.detach().contiguous().numpy()
    out["loss"] = float(loss.item())
    return out


# ---- the flat-buffer training step (checker of the GPT harness, libtcamd_gpt) -------------

def flat_layout(V, T, C, L, d_ff):
    """(name, shape) of the reference's flat parameter buffer in order (src/model.cu:185-217):
    weights stored (in, out), row-major."""
    out = [("tok_emb", (V, C)), ("pos_emb", (T, C))]
    for i in range(L):
        out += [(f"l{i}.ln1_g", (C,)), (f"l{i}.ln1_b", (C,)), (f"l{i}.qkv_w", (C, 3 * C)),
                (f"l{i}.qkv_b", (3 * C,)), (f"l{i}.proj_w", (C, C)), (f"l{i}.proj_b", (C,)),
                (f"l{i}.ln2_g", (C,)), (f"l{i}.ln2_b", (C,)), (f"l{i}.ffn1_w", (C, d_ff)),
                (f"l{i}.ffn1_b", (d_ff,)), (f"l{i}.ffn2_w", (d_ff, C)),
                (f"l{i}.ffn2_b", (C,))]
    out += [("lnf_g", (C,)), ("lnf_b", (C,)), ("head_w", (C, V))]
    return out


def _tensor_map(model: TinyGPT):
    """name -> (module parameter, stored transposed?) for flat_layout's names."""
    m = {"tok_emb": (model.tok_emb.weight, False), "pos_emb": (model.pos_emb.weight, False),
         "lnf_g": (model.ln_f.weight, False), "lnf_b": (model.ln_f.bias, False),
         "head_w": (model.head.weight, True)}
    for i, blk in enumerate(model.blocks):
        m.update({f"l{i}.ln1_g": (blk.ln_1.weight, False), f"l{i}.ln1_b": (blk.ln_1.bias, False),
                  f"l{i}.qkv_w": (blk.attn.qkv_proj.weight, True),
                  f"l{i}.qkv_b": (blk.attn.qkv_proj.bias, False),
                  f"l{i}.proj_w": (blk.attn.out_proj.weight, True),
                  f"l{i}.proj_b": (blk.attn.out_proj.bias, False),
                  f"l{i}.ln2_g": (blk.ln_2.weight, False), f"l{i}.ln2_b": (blk.ln_2.bias, False),
                  f"l{i}.ffn1_w": (blk.ffn_1.weight, True), f"l{i}.ffn1_b": (blk.ffn_1.bias, False),
                  f"l{i}.ffn2_w": (blk.ffn_2.weight, True),
                  f"l{i}.ffn2_b": (blk.ffn_2.bias, False)})
    return m


def model_from_flat(flat, V, T, C, L, H, d_ff, eps=1e-5, dtype=torch.float64) -> TinyGPT:
    """A TinyGPT whose parameters are the flat buffer's (nn.Linear holds (out, in))."""
    model = TinyGPT(V, T, C, L, H, d_ff, eps).to(dtype)
    tm = _tensor_map(model)
    off = 0
    with torch.no_grad():
        for name, shape in flat_layout(V, T, C, L, d_ff):
            n = int(torch.tensor(shape).prod())
            x = torch.as_tensor(flat[off:off + n], dtype=dtype).view(shape)
            p, tr = tm[name]
            p.copy_(x.t() if tr else x)
            off += n
    assert off == len(flat)
    return model


def flat_from_model(model: TinyGPT, V, T, C, L, d_ff, grads=False):
    """The model's parameters (or their .grad) in the flat layout, as a float64 numpy array."""
    tm = _tensor_map(model)
    parts = []
    for name, _ in flat_layout(V, T, C, L, d_ff):
        p, tr = tm[name]
        x = (p.grad if grads else p).detach()
        parts.append((x.t() if tr else x).contiguous().reshape(-1).double().numpy())
    import numpy as np
    return np.concatenate(parts)


def training_step_outputs(flat, tokens, targets, V, T, C, L, H, d_ff, eps=1e-5):
    """Logits (B*T, V), mean cross-entropy and its gradient for every parameter, in fp64 on
    the CPU: the tensors the reference's parity audit dumps (src/parity_audit.cu:64-89)."""
    model = model_from_flat(flat, V, T, C, L, H, d_ff, eps)
    logits, loss = model(torch.as_tensor(tokens, dtype=torch.long),
                         torch.as_tensor(targets, dtype=torch.long))
    loss.backward()
    return (logits.detach().reshape(-1, V).numpy(), float(loss.item()),
            flat_from_model(model, V, T, C, L, d_ff, grads=True))


def training_step_grads(flat, tokens, targets, V, T, C, L, H, d_ff, eps=1e-5):
    """Mean cross-entropy and its gradient for every parameter, in fp64 on the CPU:
    (loss, flat gradient)."""
    _, loss, grads = training_step_outputs(flat, tokens, targets, V, T, C, L, H, d_ff, eps)
    return loss, grads


def clip_adamw(params, grads, m, v, step, lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8,
               weight_decay=0.01, max_norm=1.0):
    """The reference's fused optimizer step (src/optimizer.cu:117-154) in fp64 numpy: scale
    the gradient by max_norm/||g|| when ||g|| > max_norm, Adam moments with bias correction,
    decoupled weight decay on the old parameter.  Returns (params, m, v)."""
    import numpy as np
    g = np.asarray(grads, np.float64)
    norm = float(np.sqrt((g * g).sum()))
    if norm > max_norm and norm > 1e-6:
        g = g * (max_norm / norm)
    m = beta1 * np.asarray(m, np.float64) + (1 - beta1) * g
    v = beta2 * np.asarray(v, np.float64) + (1 - beta2) * g * g
    mh = m / (1 - beta1 ** step)
    vh = v / (1 - beta2 ** step)
    p = np.asarray(params, np.float64)
    p = p - lr * (mh / (np.sqrt(vh) + eps) + weight_decay * p)
    return p, m, v
