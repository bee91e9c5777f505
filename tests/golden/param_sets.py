"""Small parameter sets and per-step gradients shared by the golden-fixture
generator and the tests that replay the fixtures.

All values come from ``gefen_amd.synthetic`` (integer-exact generator), so the
fixture only needs to store seeds; checksums of the generated arrays are kept in
the fixtures to catch any drift of the generator.
"""

from __future__ import annotations

import numpy as np

from gefen_amd import synthetic as syn

# name, shape, grad scale mode ("row": one factor per row, "tensor": one per tensor)
GPT2_MINI = [
    ("wte", (256, 48), "row"),
    ("wpe", (64, 48), "row"),
    ("h0.ln_1.weight", (48,), "row"),
    ("h0.ln_1.bias", (48,), "row"),
    ("h0.attn.c_attn.weight", (48, 144), "row"),
    ("h0.attn.c_attn.bias", (144,), "row"),
    ("h0.attn.c_proj.weight", (48, 48), "row"),
    ("h0.mlp.c_fc.weight", (48, 192), "row"),
    ("h0.mlp.c_proj.weight", (192, 48), "row"),
    ("ln_f.weight", (48,), "row"),
]

LLAMA_MINI = [
    ("embed_tokens", (512, 32), "tensor"),
    ("q_proj", (32, 32), "tensor"),
    ("k_proj", (8, 32), "row"),
    ("v_proj", (8, 32), "tensor"),
    ("o_proj", (32, 32), "row"),
    ("gate_proj", (96, 32), "row"),
    ("up_proj", (96, 32), "tensor"),
    ("down_proj", (32, 96), "row"),
    ("input_layernorm", (32,), "tensor"),
    ("lm_head", (512, 32), "row"),
]

FP16_MINI = [
    ("w1", (64, 96), "row"),
    ("w2", (96, 40), "row"),
    ("b1", (96,), "tensor"),
]

MUON_MINI = [
    ("q_proj", (64, 64), "tensor"),
    ("k_proj", (32, 64), "row"),
    ("v_proj", (32, 64), "tensor"),
    ("gate_proj", (96, 64), "row"),
    ("down_proj", (64, 96), "row"),
]

TINY_E2E = [
    ("a", (16, 24), "row"),
    ("b", (40,), "tensor"),
    ("c", (6, 10), "row"),
]


def init_param(seed: int, index: int, shape, dtype: str) -> np.ndarray:
    """N(0, 0.02) initial values, rounded to the storage dtype."""
    n = int(np.prod(shape))
    z = syn.normal(syn.make_key(seed, 1_000_000 + index), n) * 0.02
    return syn.round_to(z, dtype).reshape(shape)


def grad_for_step(seed: int, index: int, step: int, shape, dtype: str, mode: str,
                  e_lo: int = -14, e_hi: int = -4) -> np.ndarray:
    n = int(np.prod(shape))
    rows = shape[0] if (mode == "row" and len(shape) > 1) else 1
    cols = n // rows
    stream = step * 4096 + index
    g = syn.row_scaled_normal(seed, stream, rows, cols, e_lo, e_hi)
    return syn.round_to(g, dtype).reshape(shape)
