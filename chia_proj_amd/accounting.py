"""FLOP and byte accounting against MI355X's published peaks.

Algorithmic work (what the roofline fraction uses):
  FLOPs = 4 * D * (exact number of visible (i, j) pairs) * B * H   (2*D for q.k, 2*D for p.v)
  bytes = 4 * B * H * S * D * 2                                    (q, k, v read once, o written once, bf16)
Also reported: visited-tile FLOPs (tiles the kernel actually computes, at its
wavefront tile of wave_m x block_n and at its workgroup tile of
block_m x block_n) and dense-equivalent FLOPs 4 * D * S^2 * B * H.
The visible-pair and tile counts come from chia_attn_plan, i.e. from the
same mask functions the kernel runs.
"""
from __future__ import annotations

from typing import Dict

from .attention import plan
from .variants._spec import core_kwargs

PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 bf16 FLOP/clk/CU (dense)
PEAK_HBM_GBPS = 8000.0     # HBM3E


def core_plan_kwargs(op: str, H: int, params: Dict) -> Dict:
    kw = core_kwargs(op, H, **params)
    out = {k: kw[k] for k in ("norm", "causal", "window", "dilation", "block", "prefix", "softcap", "bias",
                              "post_scale") if k in kw}
    out["alibi"] = kw.get("alibi_slopes") is not None
    out["head_scale"] = kw.get("head_scale") is not None
    return out


def work(op: str, B: int, H: int, S: int, D: int, params: Dict) -> Dict:
    p = plan(batch=B, heads=H, seqlen=S, head_dim=D, **core_plan_kwargs(op, H, params))
    alg = 4.0 * D * p["pairs_visible"]
    dense = 4.0 * D * S * S * B * H
    wave_tile = 4.0 * D * p["wave_m"] * p["block_n"]
    wg_tile = 4.0 * D * p["block_m"] * p["block_n"]
    nbytes = 4.0 * B * H * S * D * 2
    t_mfma = alg / (PEAK_BF16_TFLOPS * 1e12)
    t_hbm = nbytes / (PEAK_HBM_GBPS * 1e9)
    return {
        "pairs_visible": p["pairs_visible"],
        "visible_frac": p["pairs_visible"] / float(S * S * B * H),
        "flops_alg": alg,
        "flops_dense": dense,
        "flops_visited_wave": wave_tile * p["wave_tiles_visited"],
        "flops_visited_wg": wg_tile * p["tiles_visited"],
        "tile_wave": f"{p['wave_m']}x{p['block_n']}",
        "tile_wg": f"{p['block_m']}x{p['block_n']}",
        "bytes": nbytes,
        "t_mfma_us": t_mfma * 1e6,
        "t_hbm_us": t_hbm * 1e6,
        "bound": "mfma" if t_mfma >= t_hbm else "hbm",
        "plan": p,
    }


def rates(w: Dict, us: float) -> Dict:
    """Throughput figures for one measured call of `us` microseconds."""
    s = us * 1e-6
    t_roof = max(w["t_mfma_us"], w["t_hbm_us"]) * 1e-6
    return {
        "us": us,
        "tflops_alg": w["flops_alg"] / s / 1e12,
        "tflops_visited": w["flops_visited_wave"] / s / 1e12,
        "tflops_dense": w["flops_dense"] / s / 1e12,
        "frac_mfma_alg": w["flops_alg"] / s / 1e12 / PEAK_BF16_TFLOPS,
        "frac_mfma_visited": w["flops_visited_wave"] / s / 1e12 / PEAK_BF16_TFLOPS,
        "gbps": w["bytes"] / s / 1e9,
        "frac_hbm": w["bytes"] / s / 1e9 / PEAK_HBM_GBPS,
        "frac_roofline": t_roof / s,
    }
