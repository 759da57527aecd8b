"""Writes tests/golden/c1_layer0_attention.npz: the layer-0 causal attention tensors of
BASELINE config 1 (tiny GPT, B4 T64 C128 H4 (d=32) L2 d_ff512 V256, fp32, seed 42, N(0,0.02)
weights, LayerNorm gamma=1 beta=0, zero biases, uniform tokens/targets in [0,256)).

Produced by oracle/gpt_ref.py (a restatement of pytorch_src/model.py:61-136 and the init
recipe of pytorch_src/utils.py:183-213); the reference itself is not imported.

Arrays (float32, (B, H, T, d) = (4, 4, 64, 32)): q, k, v, o, do, dq, dk, dv.

    python tests/golden/make_c1_fixture.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.gpt_ref import layer0_attention_tensors  # noqa: E402

PATH = os.path.join(HERE, "c1_layer0_attention.npz")


def main():
    t = layer0_attention_tensors()
    arrays = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in t.items() if k != "loss"}
    np.savez_compressed(PATH, **arrays, loss=np.float32(t["loss"]))
    print(f"wrote {PATH}: loss {t['loss']:.6f}, q {arrays['q'].shape}")


if __name__ == "__main__":
    main()
