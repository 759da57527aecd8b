"""The GPT training-step harness on the GPU against its fp64 CPU oracle (oracle/gpt_ref.py):
loss and every parameter gradient of one forward + backward, and the clip + AdamW update,
for each attention mode (this build's fused path on the fp32 MFMA and on the bf16 MFMA with
three-plane fp32 operands, the reference's tiled sequence, the reference's materialised
default).  Shapes of config 1 (the tiny GPT), a d = 64 variant, a vocabulary of more than
16 d_model (the split-K product of the output head's input gradient) and 4096 tokens (the
split-K weight gradients).
Tolerances are the reference's own parity gates (scripts/compare_parity.py:108-117): loss
within 1e-5, gradients within 5e-5."""
import numpy as np
import pytest
import torch

from oracle import gpt_ref

pytestmark = pytest.mark.gpu

C1 = dict(V=256, T=64, C=128, L=2, H=4, d_ff=512, B=4)
D64 = dict(V=97, T=130, C=128, L=2, H=2, d_ff=256, B=3)
# V >= 16 C: the output head's input gradient takes the split-K product (V = 8 * 256 + 5,
# so the remainder product runs too)
VOC = dict(V=2053, T=32, C=64, L=1, H=2, d_ff=128, B=2)
# B*T >= 4096: the weight gradients take the split-K product (four slices over the tokens)
TOK = dict(V=97, T=512, C=64, L=1, H=2, d_ff=128, B=8)
SHAPES = {"c1": C1, "d64": D64, "vocab": VOC, "tokens": TOK}


@pytest.fixture(scope="module")
def gpt():
    import __graft_entry__
    return __graft_entry__.load_gpt()


def init_flat(V, T, C, L, d_ff, seed):
    """N(0, 0.02) weights, LayerNorm gamma 1, beta and biases 0 (src/model.cu:219-241)."""
    rng = np.random.default_rng(seed)
    parts = []
    for name, shape in gpt_ref.flat_layout(V, T, C, L, d_ff):
        leaf = name.split(".")[-1]
        if leaf.endswith("_g"):
            parts.append(np.ones(shape))
        elif leaf.endswith("_b"):
            parts.append(np.zeros(shape))
        else:
            parts.append(rng.normal(0, 0.02, shape))
    return np.concatenate([p.reshape(-1) for p in parts]).astype(np.float32)


def make(gpt, s, mode, seed=0):
    cfg = gpt.default_config(s["V"], s["T"], s["C"], s["L"], s["H"], s["d_ff"], s["B"], mode)
    model = gpt.GPT(cfg)
    flat = init_flat(s["V"], s["T"], s["C"], s["L"], s["d_ff"], seed)
    model.set_parameters(flat)
    rng = np.random.default_rng(seed + 100)
    tokens = rng.integers(0, s["V"], (s["B"], s["T"]))
    targets = rng.integers(0, s["V"], (s["B"], s["T"]))
    return model, flat, tokens, targets


def run_fb(model, tokens, targets):
    tk = torch.as_tensor(tokens, dtype=torch.int32).cuda()
    tg = torch.as_tensor(targets, dtype=torch.int32).cuda()
    loss = torch.full((1,), float("nan"), device="cuda:0")
    model.forward_backward(tk, tg, loss)
    torch.cuda.synchronize()
    return float(loss.item()), model.gradients()


@pytest.mark.parametrize("shape", ["c1", "d64", "vocab", "tokens"])
@pytest.mark.parametrize("mode", ["fused", "fused_x3", "tiled_split", "materialized"])
def test_loss_and_gradients_vs_oracle(gpt, mode, shape):
    s = SHAPES[shape]
    model, flat, tokens, targets = make(gpt, s, mode, seed=7)
    loss, grads = run_fb(model, tokens, targets)
    want_loss, want = gpt_ref.training_step_grads(flat.astype(np.float64), tokens, targets,
                                                  s["V"], s["T"], s["C"], s["L"], s["H"],
                                                  s["d_ff"])
    assert abs(loss - want_loss) <= 1e-5, (loss, want_loss)
    err = np.abs(grads.astype(np.float64) - want)
    worst = int(err.argmax())
    assert err.max() <= 5e-5, f"grad max-abs {err.max():.3e} at flat index {worst}"
    model.close()


def test_optimizer_step_vs_oracle_two_steps(gpt):
    """Two steps: the update from the GPU's own gradients equals the fp64 clip + AdamW of
    those gradients (moments carried over), and the gradients are zeroed after each step."""
    s = C1
    model, flat, tokens, targets = make(gpt, s, "fused", seed=3)
    p, m, v = flat.astype(np.float64), np.zeros(flat.size), np.zeros(flat.size)
    for step in (1, 2):
        _, grads = run_fb(model, tokens, targets)
        model.optimizer_step()
        torch.cuda.synchronize()
        p, m, v = gpt_ref.clip_adamw(p, grads.astype(np.float64), m, v, step)
        got = model.parameters()
        err = np.abs(got.astype(np.float64) - p).max()
        assert err <= 2e-7, f"step {step}: params max-abs {err:.3e}"
        assert not model.gradients().any(), "gradients not zeroed by the optimizer step"
        p = got.astype(np.float64)  # continue from the device's fp32 parameters
    model.close()


def test_modes_agree_and_attention_timing(gpt):
    """The four attention modes give the same loss and gradients to fp32 rounding, and the
    attention timing reports a positive time below the step's."""
    s = D64
    out = {}
    for mode in ("fused", "fused_x3", "tiled_split", "materialized"):
        model, flat, tokens, targets = make(gpt, s, mode, seed=11)
        model.set_attention_timing(True)
        out[mode] = run_fb(model, tokens, targets)
        assert model.last_attention_ms() > 0.0
        model.close()
    for mode in ("fused_x3", "tiled_split", "materialized"):
        assert abs(out[mode][0] - out["fused"][0]) <= 1e-5
        assert np.abs(out[mode][1] - out["fused"][1]).max() <= 2e-5, mode
    # The fused mode's backward takes the dS-first order (dQ from the dK/dV kernel's dS) and
    # the reference's tiled sequence the two-stage one: the same forward kernels, so the same
    # loss bitwise, and gradients within fp32 rounding (above).
    assert out["tiled_split"][0] == out["fused"][0]


C5 = dict(V=50257, T=1024, C=768, L=12, H=12, d_ff=3072, B=8)


def _host_cross_entropy(logits, targets):
    """fp64 mean cross entropy of (B*T, V) fp32 logits (rows in chunks)."""
    total = 0.0
    tg = targets.reshape(-1)
    for r0 in range(0, logits.shape[0], 512):
        z = logits[r0:r0 + 512].astype(np.float64)
        mx = z.max(axis=1, keepdims=True)
        lse = mx[:, 0] + np.log(np.exp(z - mx).sum(axis=1))
        total += float((lse - z[np.arange(z.shape[0]), tg[r0:r0 + 512]]).sum())
    return total / logits.shape[0]


def test_config5_full_shape_fused_and_x3(gpt):
    """BASELINE config 5 at its own shape (GPT-2 small: L12 C768 H12 d_ff 3072, T 1024, B 8,
    V 50257; N(0, 0.02) weights, uniform tokens and targets), the fp32 MFMA attention and the
    three-plane attention: the loss equals the fp64 cross entropy of the GPU's own logits
    (1e-5) and sits just above ln V (random logits of spread s give ln V + s^2/2, s ~ 0.5 here);
    the two modes agree on the loss (1e-5) and on every gradient (5e-5); one clip + AdamW
    step zeroes the gradients and moves the parameters."""
    out = {}
    for mode in ("fused_x3", "fused"):
        model, flat, tokens, targets = make(gpt, C5, mode, seed=21)
        assert model.n_params == flat.size == 163_037_184
        loss, grads = run_fb(model, tokens, targets)
        assert np.isfinite(loss) and np.isfinite(grads).all(), mode
        logits = model.logits().reshape(C5["B"] * C5["T"], C5["V"])
        want = _host_cross_entropy(logits, targets)
        assert abs(loss - want) <= 1e-5, (mode, loss, want)
        del logits
        assert np.log(C5["V"]) - 0.01 <= loss <= np.log(C5["V"]) + 0.3, (mode, loss)
        out[mode] = (loss, grads)
        if mode == "fused":
            model.optimizer_step()
            torch.cuda.synchronize()
            assert not model.gradients().any(), "gradients not zeroed by the optimizer step"
            moved = np.abs(model.parameters() - flat)
            assert moved.max() > 0 and np.isfinite(moved).all()
        model.close()
    assert abs(out["fused_x3"][0] - out["fused"][0]) <= 1e-5
    err = np.abs(out["fused_x3"][1] - out["fused"][1])
    assert err.max() <= 5e-5, f"grad max-abs {err.max():.3e} at flat index {int(err.argmax())}"
