"""Numerical gate and status taxonomy for variant kernels.

Two criteria:
  * the north-star gate: bf16 output against an fp32 reference within
    max-abs 2e-2 and mean-abs 2e-3;
  * the reference's own gate (synth10.py:173-184): at input scales 1.0 and
    0.01, rel = max|r - o| / (max|r| + 1e-6) must stay below 3e-2
    (REL_TOL, synth10.py:11), after checking for exceptions, shape mismatch,
    NaN and Inf in that order.
``classify`` reproduces the per-shape status classes of shape_gen.py:97-110
(OK / wrong shape / NaN / Inf / incorrect / AssertionError / <exception name>).

The gate takes the reference as a callable or tensor; it never computes one.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Dict, Tuple

import torch

GATE_MAX_ABS = 2e-2
GATE_MEAN_ABS = 2e-3
REL_TOL = 3e-2
# Scale-aware tolerances (unnormalised sigmoid / ReLU outputs), relative to
# M = max|ref|: about twice the largest ratio the GPU suite's 563 scale-aware
# checks measure (max-abs 5.3e-3 M, mean-abs 5.3e-4 M), never below the
# absolute gate.  Rounding an output to bf16 alone moves it by up to 2^-8 M.
SCALED_MAX_ABS = 1e-2
SCALED_MEAN_ABS = 1e-3
SCALES = (("standard", 1.0), ("small", 0.01))


def relerr(ref: torch.Tensor, out: torch.Tensor) -> float:
    """max|r - o| / (max|r| + 1e-6) (extra_bench.py:29)."""
    r = ref.detach().float().cpu()
    o = out.detach().float().cpu()
    return ((r - o).abs().max() / (r.abs().max() + 1e-6)).item()


def error_stats(ref: torch.Tensor, out: torch.Tensor) -> Dict[str, float]:
    r = ref.detach().float().cpu()
    o = out.detach().float().cpu()
    d = (r - o).abs()
    return {
        "max_abs": d.max().item(),
        "mean_abs": d.mean().item(),
        "rel": (d.max() / (r.abs().max() + 1e-6)).item(),
    }


@dataclass
class GateResult:
    ok: bool
    status: str
    stats: Dict[str, float] = field(default_factory=dict)

    def __bool__(self) -> bool:
        return self.ok


def _finite_status(ref: torch.Tensor, out) -> str:
    if not isinstance(out, torch.Tensor) or tuple(out.shape) != tuple(ref.shape):
        return "wrong shape"
    if torch.isnan(out).any():
        return "NaN"
    if torch.isinf(out).any():
        return "Inf"
    return ""


def north_star_gate(ref: torch.Tensor, out: torch.Tensor, max_abs: float = GATE_MAX_ABS,
                    mean_abs: float = GATE_MEAN_ABS, scale_aware: bool = False,
                    scaled_max_abs: float = SCALED_MAX_ABS, scaled_mean_abs: float = SCALED_MEAN_ABS) -> GateResult:
    """bf16 `out` against fp32 `ref`: max-abs <= 2e-2 and mean-abs <= 2e-3.

    scale_aware=True allows max(max_abs, scaled_max_abs M) and
    max(mean_abs, scaled_mean_abs M), M = max|ref|.  It is for the unnormalised
    sigmoid / ReLU outputs at the reference's default parameters (no 1/S or
    -log S), whose magnitude grows like sqrt(S): rounding an output of
    magnitude 32 to bf16 alone moves it by up to 0.0625.
    """
    st = _finite_status(ref, out)
    if st:
        return GateResult(False, st)
    stats = error_stats(ref, out)
    mag = max(1.0, ref.detach().float().abs().max().item()) if scale_aware else 1.0
    stats["tol_scale"] = mag
    tol_max = max(max_abs, scaled_max_abs * mag) if scale_aware else max_abs
    tol_mean = max(mean_abs, scaled_mean_abs * mag) if scale_aware else mean_abs
    stats["tol_max_abs"], stats["tol_mean_abs"] = tol_max, tol_mean
    ok = stats["max_abs"] <= tol_max and stats["mean_abs"] <= tol_mean
    return GateResult(ok, "OK" if ok else "incorrect", stats)


def verify(fn: Callable, ref_fn: Callable, q, k, v) -> Tuple[bool, float, str]:
    """The reference's gate (synth10.py:173-184): scales 1.0 and 0.01, worst rel < 3e-2."""
    worst, msgs = 0.0, []
    for name, sc in SCALES:
        qq, kk, vv = q * sc, k * sc, v * sc
        try:
            out, r = fn(qq, kk, vv), ref_fn(qq, kk, vv)
        except Exception as e:  # noqa: BLE001 -- every failure is a gate outcome
            return False, 9e9, f"{name}: {type(e).__name__}: {e}"
        st = _finite_status(r, out)
        if st:
            return False, 9e9, f"{name}: {st}"
        rel = relerr(r, out)
        worst = max(worst, rel)
        msgs.append(f"{name} rel={rel:.2e}")
    return worst < REL_TOL, worst, "; ".join(msgs)


def classify(fn: Callable, ref_fn: Callable, q, k, v) -> Tuple[str, float]:
    """Per-shape status of shape_gen.py:97-110: (status, relerr or nan)."""
    try:
        out = fn(q, k, v)
        if not isinstance(out, torch.Tensor) or tuple(out.shape) != tuple(q.shape):
            return "wrong shape", float("nan")
        if torch.isnan(out).any():
            return "NaN", float("nan")
        if torch.isinf(out).any():
            return "Inf", float("nan")
        rel = relerr(ref_fn(q, k, v), out)
        return ("incorrect" if rel >= REL_TOL else "OK"), rel
    except AssertionError:
        return "AssertionError", float("nan")
    except Exception as e:  # noqa: BLE001
        return type(e).__name__[:13], float("nan")
