"""Write tests/golden/variants_S96.npz: seeded bf16 inputs and the fp32 oracle's
outputs for the ten variants at parameters scaled to S = 96 (window 24, local
window 16, dilation 3, block 32, prefix 20, softcap 5, per-head temperature
and ALiBi slopes).  The reference holds no tensor-valued vectors, so these are
our own oracle's outputs: they freeze it (tests/test_golden.py) and give the
GPU tests a reference that needs no oracle run on the box.

Run from the repository root: python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402

B, H, S, D = 1, 2, 96, 64
SEED = 20269696
PARAMS = {
    "sigmoid_attn": dict(causal=True, bias=-1.0),
    "relu_attn": dict(causal=False, post_scale=1.0 / 96),
    "temp_perhead": dict(temperature=[0.6, 1.7], mode="div"),
    "bias_alibi": dict(slopes=[0.25, 0.0625]),
    "bias_dilated": dict(dilation=3),
    "bias_local": dict(window=16),
    "bias_block_diagonal": dict(block=32),
    "bias_prefix_lm": dict(prefix=20),
    "softcap_gemma2": dict(softcap=5.0),
    "bias_sliding_window": dict(window=24),
}


def make():
    g = torch.Generator("cpu").manual_seed(SEED)
    q, k, v = (torch.randn(B, H, S, D, generator=g).to(torch.bfloat16) for _ in range(3))
    out = {f"in_{n}": t.view(torch.int16).numpy() for n, t in (("q", q), ("k", k), ("v", v))}
    for op, p in PARAMS.items():
        out[f"out_{op}"] = oracle.variant_ref(op, q, k, v, **p).numpy().astype(np.float16)
    return out


if __name__ == "__main__":
    path = Path(__file__).resolve().parent / "variants_S96.npz"
    np.savez_compressed(path, **make())
    print(path, path.stat().st_size, "bytes")
