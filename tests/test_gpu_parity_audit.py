"""The reference's end-to-end parity gate (scripts/compare_parity.py) on this build: a data
directory in the parity-audit file protocol (src/parity_audit.cu, pytorch_src/utils.py:7-42)
drives bin/parity_audit; its logits, loss and gradients are compared with the fp64 oracle
at the gate's tolerances (logits and loss 1e-5, gradients 5e-5, compare_parity.py:108-117).
Shapes: the gate's own configuration (B4 T16 C64 L2 H4 V65, d_head 16: the materialised
mode, which the reference's audit runs by default) and a d_head 32 one for all modes."""
import os
import subprocess

import numpy as np
import pytest

from oracle import gpt_ref

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
AUDIT = os.path.join(REPO, "transformer-cuda_amd", "bin", "parity_audit")


def write_case(d, B, T, C, L, H, V, seed):
    rng = np.random.default_rng(seed)
    parts = []
    for name, shape in gpt_ref.flat_layout(V, T, C, L, 4 * C):
        leaf = name.split(".")[-1]
        parts.append(np.ones(shape) if leaf.endswith("_g") else
                     np.zeros(shape) if leaf.endswith("_b") else rng.normal(0, 0.02, shape))
    flat = np.concatenate([p.reshape(-1) for p in parts]).astype(np.float32)
    tokens = rng.integers(0, V, B * T).astype(np.int32)
    targets = rng.integers(0, V, B * T).astype(np.int32)
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "config.txt"), "w") as f:
        f.write(f"{B} {T} {C} {L} {H} {V}\n")
    flat.tofile(os.path.join(d, "pytorch_params.bin"))
    tokens.tofile(os.path.join(d, "inputs.bin"))
    targets.tofile(os.path.join(d, "targets.bin"))
    return flat, tokens.reshape(B, T), targets.reshape(B, T)


@pytest.mark.parametrize("shape,flag", [((4, 16, 64, 2, 4, 65), None),
                                        ((2, 48, 128, 2, 4, 101), None),
                                        ((2, 48, 128, 2, 4, 101), "--tiled_attn"),
                                        ((2, 48, 128, 2, 4, 101), "--fused_attn"),
                                        ((2, 48, 128, 2, 4, 101), "--fused_x3_attn")])
def test_parity_audit_protocol(tmp_path, shape, flag):
    B, T, C, L, H, V = shape
    d = str(tmp_path / "parity_data")
    flat, tokens, targets = write_case(d, B, T, C, L, H, V, seed=42)
    cmd = [AUDIT, d] + ([flag] if flag else [])
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    logits = np.fromfile(os.path.join(d, "cuda_logits.bin"), np.float32).reshape(B * T, V)
    loss = float(np.fromfile(os.path.join(d, "cuda_loss.bin"), np.float32)[0])
    grads = np.fromfile(os.path.join(d, "cuda_grads.bin"), np.float32)
    w_logits, w_loss, w_grads = gpt_ref.training_step_outputs(
        flat.astype(np.float64), tokens, targets, V, T, C, L, H, 4 * C)
    assert np.abs(logits - w_logits).max() <= 1e-5
    assert abs(loss - w_loss) <= 1e-5
    assert grads.shape == w_grads.shape
    assert np.abs(grads - w_grads).max() <= 5e-5
