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
