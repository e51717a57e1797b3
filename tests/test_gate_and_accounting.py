"""CPU tests of the gate (status taxonomy of shape_gen.py:97-110 and the gate of
synth10.py:173-184, forced with fake kernels) and of the FLOP/byte accounting."""
import math

import pytest
import torch

from chia_proj_amd import gate
from chia_proj_amd.accounting import PEAK_BF16_TFLOPS, PEAK_HBM_GBPS, rates, work
from chia_proj_amd.workloads import baseline_configs, draw_inputs, headline_suite, north_star_suite

REF = lambda q, k, v: q + k + v  # noqa: E731 -- any deterministic "reference"


def _qkv():
    g = torch.Generator().manual_seed(0)
    return tuple(torch.randn(1, 2, 16, 8, generator=g) for _ in range(3))


def test_classify_every_outcome():
    q, k, v = _qkv()

    def raises(exc):
        def f(*a):
            raise exc
        return f

    assert gate.classify(REF, REF, q, k, v)[0] == "OK"
    assert gate.classify(lambda q, k, v: q[:, :1], REF, q, k, v)[0] == "wrong shape"
    assert gate.classify(lambda q, k, v: REF(q, k, v) * float("nan"), REF, q, k, v)[0] == "NaN"
    assert gate.classify(lambda q, k, v: REF(q, k, v) + float("inf"), REF, q, k, v)[0] == "Inf"
    assert gate.classify(lambda q, k, v: REF(q, k, v) * 1.5, REF, q, k, v)[0] == "incorrect"
    assert gate.classify(raises(AssertionError("shape")), REF, q, k, v)[0] == "AssertionError"
    assert gate.classify(raises(RuntimeError("hip")), REF, q, k, v)[0] == "RuntimeError"


def test_reference_verify_uses_both_scales():
    q, k, v = _qkv()
    ok, worst, msg = gate.verify(REF, REF, q, k, v)
    assert ok and worst == 0.0 and "standard" in msg and "small" in msg
    # an error that only shows at scale 0.01 (an absolute offset) fails the relative gate there
    ok, worst, msg = gate.verify(lambda q, k, v: REF(q, k, v) + 0.01, REF, q, k, v)
    assert not ok and worst > 3e-2
    ok, _, msg = gate.verify(lambda q, k, v: q[:, :1], REF, q, k, v)
    assert not ok and "shape" in msg


def test_north_star_gate_thresholds():
    r = torch.zeros(4, 64)
    assert gate.north_star_gate(r, r + 0.019).ok is False  # mean-abs 1.9e-2 > 2e-3
    o = r.clone()
    o[0, 0] = 0.019
    assert gate.north_star_gate(r, o).ok
    o[0, 0] = 0.021
    assert not gate.north_star_gate(r, o).ok
    big = torch.full((4, 64), 30.0)
    o = big + 0.05
    assert not gate.north_star_gate(big, o).ok
    assert not gate.north_star_gate(big, o).ok
    o2 = big.clone()
    o2[0, 0] += 0.1
    assert gate.north_star_gate(big, o2, scale_aware=True).ok  # 0.1 <= 1e-2 * 30
    o2[0, 0] = 30.0 + 0.31
    assert not gate.north_star_gate(big, o2, scale_aware=True).ok  # 0.31 > 1e-2 * 30
    # never tighter than the absolute gate: M = 1.5 keeps max-abs 2e-2
    small = torch.full((4, 64), 1.5)
    o3 = small.clone()
    o3[0, 0] += 0.019
    assert gate.north_star_gate(small, o3, scale_aware=True).ok
    assert gate.north_star_gate(r, r[:, :3]).status == "wrong shape"
    assert gate.north_star_gate(r, r * float("nan")).status == "NaN"


def test_relerr_matches_reference_formula():
    r = torch.tensor([1.0, -2.0, 3.0])
    o = torch.tensor([1.0, -2.5, 3.0])
    assert gate.relerr(r, o) == pytest.approx(0.5 / (3.0 + 1e-6))


@pytest.mark.parametrize("case", baseline_configs()[1:10], ids=lambda c: c.name)
def test_work_accounting_closed_forms(case):
    w = work(case.op, case.B, case.H, case.S, case.D, case.params)
    assert w["bytes"] == 4 * case.B * case.H * case.S * case.D * 2
    assert w["flops_dense"] == 4 * case.D * case.S ** 2 * case.B * case.H
    assert w["flops_alg"] == 4 * case.D * w["pairs_visible"]
    assert w["flops_alg"] <= w["flops_visited_wave"] <= w["flops_dense"] * 1.0001 + 4 * case.D * 32 * 64 * 64
    assert w["bound"] == ("mfma" if w["t_mfma_us"] >= w["t_hbm_us"] else "hbm")


def test_configuration_figures():
    # visible fractions and bounds of the BASELINE configurations (closed forms in
    # tests/test_oracle_pins.py); window-256 at S=2048 is 11.72 % and HBM-bound,
    # ALiBi causal at S=2048 is MFMA-bound.
    c = {x.name: x for x in baseline_configs()}
    w = work("bias_sliding_window", 4, 16, 2048, 64, c["c2_window256_B4H16S2048D64"].params)
    assert abs(w["visible_frac"] - 0.1172) < 1e-4 and w["bound"] == "hbm"
    w = work("bias_alibi", 4, 16, 2048, 64, c["c3_alibi_B4H16S2048D64"].params)
    assert abs(w["visible_frac"] - 0.5002) < 1e-4 and w["bound"] == "mfma"
    assert abs(w["flops_alg"] / 1e9 - 34.38) < 0.01


def test_rates():
    w = {"flops_alg": 1e12, "flops_visited_wave": 2e12, "flops_dense": 4e12, "bytes": 8e9,
         "t_mfma_us": 1e12 / (PEAK_BF16_TFLOPS * 1e12) * 1e6, "t_hbm_us": 8e9 / (PEAK_HBM_GBPS * 1e9) * 1e6}
    r = rates(w, 1000.0)
    assert r["tflops_alg"] == pytest.approx(1000.0)
    assert r["gbps"] == pytest.approx(8000.0)
    assert r["frac_hbm"] == pytest.approx(1.0)


def test_suites_and_seeds():
    hs, ns = headline_suite(), north_star_suite()
    assert [c.op for c in hs] == [c.op for c in ns] and len(hs) == 10
    assert all(c.shape == (4, 16, 2048, 64) for c in hs)
    assert all(c.shape == (4, 16, 4096, 64) for c in ns)
    small = [c for c in baseline_configs() if c.name.startswith("c1")][0]
    q, k, v, p = draw_inputs(small)
    g = torch.Generator("cpu").manual_seed(20260001)
    assert torch.equal(q, torch.randn(1, 8, 512, 64, generator=g).to(torch.bfloat16))
    temp_case = [c for c in headline_suite() if c.op == "temp_perhead"][0]
    _, _, _, p = draw_inputs(temp_case)
    t = p["temperature"]
    assert t.shape == (16,) and (t >= 0.5).all() and (t < 2.0).all()
    sig = [c for c in headline_suite() if c.op == "sigmoid_attn"][0]
    assert sig.params["bias"] == pytest.approx(-math.log(2048)) and sig.params["causal"] is False
