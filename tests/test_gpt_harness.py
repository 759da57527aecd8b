"""The GPT training-step harness without a GPU: library exports, configuration validation,
and the pins of its oracle (oracle/gpt_ref.py's flat-buffer step and clip + AdamW)."""
import ctypes
import re

import numpy as np
import pytest
import torch

from oracle import gpt_ref


@pytest.fixture(scope="module")
def gpt():
    import __graft_entry__
    return __graft_entry__.load_gpt()


def declared(gpt):
    text = re.sub(r"/\*.*?\*/", "", open(gpt.GPT_HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"\b(gpt_[a-z_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound(gpt):
    names = declared(gpt)
    assert len(names) >= 10
    for n in names:
        assert hasattr(gpt.raw(), n), n
    assert set(names) == set(gpt.SIGNATURES)


def test_config_validation_without_gpu(gpt):
    def create(**kw):
        cfg = gpt.default_config(256, 64, 128, 2, 4, 512, 4)
        for k, v in kw.items():
            setattr(cfg, k, v)
        h = ctypes.c_void_p()
        return gpt.raw().gpt_create(ctypes.byref(cfg), ctypes.byref(h))
    assert create(d_model=100) == 2            # d = 25: unsupported head dimension
    assert create(num_heads=3) == 1            # C % H != 0
    assert create(batch_size=0) == 1
    assert create(attention_mode=7) == 6
    assert create(attention_mode=3, d_model=512) == 2  # fused_x3 at d = 128: unsupported
    assert create(layernorm_eps=0.0) == 6
    assert gpt.raw().gpt_create(None, None) == 3


def test_defaults_are_the_reference_config(gpt):
    c = gpt.default_config(50257, 1024, 768, 12, 12, 3072, 8)
    assert (c.learning_rate, c.weight_decay, c.beta1, c.beta2, c.adam_eps, c.grad_clip) == \
        pytest.approx((3e-4, 0.01, 0.9, 0.999, 1e-8, 1.0))       # include/config.h:16-22
    assert c.layernorm_eps == pytest.approx(1e-5)
    layout = gpt.param_layout(50257, 1024, 768, 12, 3072)
    assert sum(int(np.prod(s)) for _, s in layout) == 163_037_184  # GPT-2-small, untied head
    assert layout == gpt_ref.flat_layout(50257, 1024, 768, 12, 3072)


SMALL = dict(V=16, T=8, C=32, L=1, H=1, d_ff=64)


def random_flat(V, T, C, L, H, d_ff, seed=0):
    rng = np.random.default_rng(seed)
    return rng.normal(0, 0.3, sum(int(np.prod(s)) for _, s in
                                  gpt_ref.flat_layout(V, T, C, L, d_ff)))


def test_flat_layout_round_trip():
    s = SMALL
    flat = random_flat(**s)
    model = gpt_ref.model_from_flat(flat, s["V"], s["T"], s["C"], s["L"], s["H"], s["d_ff"])
    back = gpt_ref.flat_from_model(model, s["V"], s["T"], s["C"], s["L"], s["d_ff"])
    np.testing.assert_array_equal(back, flat)
    # the (in, out) storage: the head maps ln_f output (C) to V logits
    assert model.head.weight.shape == (s["V"], s["C"])


def test_training_step_gradient_matches_finite_differences():
    """The flat gradient is d(loss)/d(flat): central differences on a few coordinates of
    every tensor class (embedding, LN, QKV, FFN, head) in fp64."""
    s = SMALL
    flat = random_flat(**s, seed=1)
    rng = np.random.default_rng(2)
    tokens = rng.integers(0, s["V"], (2, s["T"]))
    targets = rng.integers(0, s["V"], (2, s["T"]))
    loss, grad = gpt_ref.training_step_grads(flat, tokens, targets, **s)
    layout = gpt_ref.flat_layout(s["V"], s["T"], s["C"], s["L"], s["d_ff"])
    offs, o = {}, 0
    for name, shape in layout:
        offs[name] = o
        o += int(np.prod(shape))
    picks = [offs["tok_emb"] + tokens[0, 3] * s["C"] + 5, offs["pos_emb"] + 2 * s["C"] + 7,
             offs["l0.ln1_g"] + 3, offs["l0.qkv_w"] + 40, offs["l0.qkv_b"] + 70,
             offs["l0.proj_w"] + 11, offs["l0.ffn1_w"] + 100, offs["l0.ffn2_b"] + 4,
             offs["lnf_b"] + 9, offs["head_w"] + 33]
    h = 1e-6
    for i in picks:
        fp, fm = flat.copy(), flat.copy()
        fp[i] += h
        fm[i] -= h
        lp, _ = gpt_ref.training_step_grads(fp, tokens, targets, **s)
        lm, _ = gpt_ref.training_step_grads(fm, tokens, targets, **s)
        fd = (lp - lm) / (2 * h)
        assert abs(fd - grad[i]) <= 1e-6 + 1e-5 * abs(fd), (i, fd, grad[i])


def test_clip_adamw_equals_torch_adamw_without_clipping():
    rng = np.random.default_rng(3)
    p0 = rng.normal(0, 1, 50)
    g1, g2 = rng.normal(0, 0.01, 50), rng.normal(0, 0.01, 50)   # norm < 1: no clipping
    p = torch.tensor(p0, requires_grad=True)
    opt = torch.optim.AdamW([p], lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    mine, m, v = p0, np.zeros(50), np.zeros(50)
    for step, g in enumerate((g1, g2), 1):
        p.grad = torch.tensor(g)
        opt.step()
        mine, m, v = gpt_ref.clip_adamw(mine, g, m, v, step)
    np.testing.assert_allclose(mine, p.detach().numpy(), rtol=0, atol=1e-15)


def test_clip_scales_to_max_norm():
    g = np.array([3.0, 4.0])  # norm 5
    _, m, v = gpt_ref.clip_adamw(np.zeros(2), g, np.zeros(2), np.zeros(2), 1, max_norm=1.0)
    np.testing.assert_allclose(m / 0.1, [0.6, 0.8])           # (1 - beta1) * g / 5
    _, m, _ = gpt_ref.clip_adamw(np.zeros(2), g, np.zeros(2), np.zeros(2), 1, max_norm=10.0)
    np.testing.assert_allclose(m / 0.1, g)                     # below the threshold
