"""Seeded workloads: the BASELINE configurations and the benchmark suites.

Inputs are drawn on the CPU with a seeded generator (the reference uses
unseeded device randn, extra_bench.py:79-81): q, k, v in that order as fp32
N(0, 1) [B, H, S, D], cast to bf16; per-head temperatures, when a case needs
them, are drawn after v as 0.5 + 1.5 * U[0, 1).  Configuration k of
BASELINE.json uses seed 20260000 + k; the headline / north-star / S-sweep
suites use seed 20261000 + S; the reference-shape suites seed 20260000 + S.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

from .variants._spec import OP_NAMES, standard_alibi_slopes


@dataclass(frozen=True)
class Case:
    name: str
    op: str
    B: int
    H: int
    S: int
    D: int
    seed: int
    params: Dict = field(default_factory=dict)
    temperature: bool = False  # draw t_h ~ U[0.5, 2] after v and pass it as `temperature`

    @property
    def shape(self) -> Tuple[int, int, int, int]:
        return (self.B, self.H, self.S, self.D)


def draw_inputs(case: Case, device: Optional[str] = None, dtype: torch.dtype = torch.bfloat16):
    """(q, k, v, params) for `case`; params includes the drawn temperatures."""
    g = torch.Generator("cpu").manual_seed(case.seed)
    shp = case.shape
    q = torch.randn(shp, generator=g, dtype=torch.float32)
    k = torch.randn(shp, generator=g, dtype=torch.float32)
    v = torch.randn(shp, generator=g, dtype=torch.float32)
    params = dict(case.params)
    if case.temperature:
        params["temperature"] = 0.5 + 1.5 * torch.rand(case.H, generator=g, dtype=torch.float32)
    q, k, v = (t.to(dtype) for t in (q, k, v))
    if device is not None:
        q, k, v = (t.to(device) for t in (q, k, v))
    return q, k, v, params


def baseline_params(op: str, S: int, H: int) -> Dict:
    """BASELINE.json's parameters for variant `op` at sequence length S."""
    return {
        "bias_sliding_window": dict(window=256),
        "bias_local": dict(window=129),  # +-128: |i-j| <= 128  <=>  |i-j| < 129
        "bias_dilated": dict(dilation=2, window=1024),
        "bias_block_diagonal": dict(block=256, causal=True),
        "bias_prefix_lm": dict(prefix=1024),
        "bias_alibi": dict(slopes=standard_alibi_slopes(H)),
        "softcap_gemma2": dict(softcap=50.0),
        "temp_perhead": dict(mode="div"),
        "relu_attn": dict(causal=False, post_scale=1.0 / S),
        "sigmoid_attn": dict(causal=False, bias=-math.log(S)),
    }[op]


def suite(B: int, H: int, S: int, D: int, seed: Optional[int] = None, tag: str = "") -> List[Case]:
    """All ten variants at one shape with BASELINE parameters."""
    seed = 20261000 + S if seed is None else seed
    return [
        Case(name=f"{tag}{op}", op=op, B=B, H=H, S=S, D=D, seed=seed, params=baseline_params(op, S, H),
             temperature=(op == "temp_perhead"))
        for op in OP_NAMES
    ]


def headline_suite() -> List[Case]:
    """The metric's workload: all ten variants at B4 H16 S2048 D64 bf16."""
    return suite(4, 16, 2048, 64, tag="headline:")


def north_star_suite() -> List[Case]:
    """The north-star target: all ten variants at B4 H16 S4096 D64 bf16."""
    return suite(4, 16, 4096, 64, tag="northstar:")


def reference_suite(S: int = 2048) -> List[Case]:
    """The reference's own benchmark shape and constants: all ten variants at
    B2 H32 S D128 bf16 with the constants baked into its eager closures
    (extra_bench.py:5,32-62; sigmoid_fix.py:34-40) -- window 256, dilation 4,
    block 512, prefix 256, ALiBi slope h+1, temperature 0.5+h/H, softcap 30,
    causal sigmoid and ReLU.  S = 2048 is its benchmark; its sequence sweep
    (extra_bench.py:166) adds S = 1024 and 4096 with the same constants.
    Seed 20260000 + S (20262048 at the benchmark; the reference draws unseeded)."""
    return [Case(name=f"reference:{op}:S{S}", op=op, B=2, H=32, S=S, D=128, seed=20260000 + S) for op in OP_NAMES]


REFERENCE_SWEEP_S = (1024, 2048, 4096)  # extra_bench.py:166


def baseline_configs() -> List[Case]:
    """The five configurations of BASELINE.json, expanded into cases."""
    cases = [
        Case("c1_softcap50_B1H8S512D64", "softcap_gemma2", 1, 8, 512, 64, 20260001, dict(softcap=50.0)),
        Case("c2_window256_B4H16S2048D64", "bias_sliding_window", 4, 16, 2048, 64, 20260002, dict(window=256)),
        Case("c3_alibi_B4H16S2048D64", "bias_alibi", 4, 16, 2048, 64, 20260003,
             dict(slopes=standard_alibi_slopes(16))),
        Case("c3_temp_B4H16S2048D64", "temp_perhead", 4, 16, 2048, 64, 20260003, dict(mode="div"),
             temperature=True),
        Case("c4a_prefix1024_B2H16S4096D64", "bias_prefix_lm", 2, 16, 4096, 64, 20260004, dict(prefix=1024)),
        Case("c4b_block256_causal_B2H16S4096D64", "bias_block_diagonal", 2, 16, 4096, 64, 20260004,
             dict(block=256, causal=True)),
        Case("c4b_block256_full_B2H16S4096D64", "bias_block_diagonal", 2, 16, 4096, 64, 20260004,
             dict(block=256, causal=False)),
        Case("c4c_dilated2_w1024_B2H16S4096D64", "bias_dilated", 2, 16, 4096, 64, 20260004,
             dict(dilation=2, window=1024)),
        Case("c4d_local128_B2H16S4096D64", "bias_local", 2, 16, 4096, 64, 20260004, dict(window=129)),
    ]
    for S in (1024, 2048, 4096):
        cases.append(Case(f"c5_sigmoid_B4H16S{S}D128", "sigmoid_attn", 4, 16, S, 128, 20260005,
                          dict(causal=False, bias=-math.log(S))))
        cases.append(Case(f"c5_relu_B4H16S{S}D128", "relu_attn", 4, 16, S, 128, 20260005,
                          dict(causal=False, post_scale=1.0 / S)))
    return cases
