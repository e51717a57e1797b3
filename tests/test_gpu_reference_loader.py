"""The reference's own harness protocol on the GPU: `<op>_BEST.py` modules found
by glob and loaded with importlib exactly as extra_bench.py:24-27,65-70 does,
then called as launch_kernel(q, k, v) at the reference's benchmark shape and
constants (B2 H32 S2048 D128 bf16, extra_bench.py:5,32-62; sigmoid_fix.py:34-40).
Every (batch, head) slice is gated against the CPU oracle, and the whole output
against the reference's own statistic (relerr < 3e-2, extra_bench.py:29,121).
The same modules are then called at the other lengths of the reference's
sequence sweep, S = 1024 and 4096 (extra_bench.py:166-201)."""
import glob
import importlib.util
import os
from pathlib import Path

import pytest
import torch

import oracle
from chia_proj_amd import gate
from chia_proj_amd.workloads import REFERENCE_SWEEP_S, draw_inputs, reference_suite

pytestmark = pytest.mark.gpu
DEV = "cuda"
KERNEL_DIR = Path(__file__).resolve().parent.parent / "chia_proj_amd" / "kernels_mi355x"


def _say(msg):
    print(msg, flush=True)


def _discover():
    """op -> path, by the reference's rule (extra_bench.py:65-70)."""
    found = {}
    for p in glob.glob(os.path.join(KERNEL_DIR, "*_BEST.py")):
        bn = os.path.basename(p).replace("_BEST.py", "")
        op = "sigmoid_attn" if bn.startswith("sigmoid_") else bn.split("_gemini")[0]
        found.setdefault(op, []).append(p)
    return found


def _load(p):
    """extra_bench.py:24-27."""
    sp = importlib.util.spec_from_file_location("k" + str(abs(hash(p))), p)
    m = importlib.util.module_from_spec(sp)
    sp.loader.exec_module(m)
    return m.launch_kernel


_INPUTS = {}


def _shared_inputs(case):
    # one q, k, v draw serves every variant, as in extra_bench.py:79-81
    if "qkv" not in _INPUTS:
        q, k, v, _ = draw_inputs(case, DEV)
        _INPUTS["qkv"] = (q, k, v)
    return _INPUTS["qkv"]


def test_every_variant_is_discovered():
    found = _discover()
    assert sorted(found) == sorted(c.op for c in reference_suite())
    assert all(len(v) == 1 for v in found.values())


@pytest.mark.parametrize("case", reference_suite(), ids=lambda c: c.op)
def test_reference_loader_at_reference_shape(case):
    _say(f"[loader] {case.op} B{case.B} H{case.H} S{case.S} D{case.D}")
    (path,) = _discover()[case.op]
    launch_kernel = _load(path)
    q, k, v = _shared_inputs(case)
    o = launch_kernel(q, k, v)
    torch.cuda.synchronize()
    assert o.shape == q.shape and o.dtype == torch.bfloat16
    assert bool(torch.isfinite(o).all())
    qc, kc, vc, oc = q.cpu(), k.cpu(), v.cpu(), o.float().cpu()
    # sigmoid / ReLU at the reference constants are unnormalised (no -log S, no 1/S):
    # their outputs grow like sqrt(S), so both tolerances scale with max |ref|
    unnorm = case.op in ("sigmoid_attn", "relu_attn")
    worst_rel = 0.0
    for b in range(case.B):
        ref = oracle.variant_ref(case.op, qc[b:b + 1], kc[b:b + 1], vc[b:b + 1])
        worst_rel = max(worst_rel, gate.relerr(ref[0], oc[b]))
        for h in range(case.H):
            res = gate.north_star_gate(ref[0, h], oc[b, h], scale_aware=unnorm)
            assert res.ok, f"{case.op} b={b} h={h}: {res.status} {res.stats}"
    assert worst_rel < gate.REL_TOL, (case.op, worst_rel)
    _say(f"  {case.op}: {case.B * case.H} slices within the gate, reference relerr {worst_rel:.2e}")


_SWEEP_INPUTS = {}


@pytest.mark.parametrize("S", [s for s in REFERENCE_SWEEP_S if s != 2048])
@pytest.mark.parametrize("op", [c.op for c in reference_suite()])
def test_reference_loader_at_swept_lengths(op, S):
    """The reference's sequence sweep (extra_bench.py:166-201) calls the same modules
    at S = 1024 and 4096 with the constants unchanged and keeps a kernel whose output
    passes relerr < 3e-2 ("generalises").  Every slice is gated at S = 1024; at
    S = 4096 sixteen (batch, head) slices spread over both batch entries and all heads."""
    case = next(c for c in reference_suite(S) if c.op == op)
    _say(f"[loader-sweep] {op} B{case.B} H{case.H} S{S} D{case.D}")
    (path,) = _discover()[op]
    launch_kernel = _load(path)
    if _SWEEP_INPUTS.get("S") != S:
        _SWEEP_INPUTS.clear()
        q, k, v, _ = draw_inputs(case, DEV)
        _SWEEP_INPUTS.update(S=S, qkv=(q, k, v), cpu=(q.cpu(), k.cpu(), v.cpu()))
    q, k, v = _SWEEP_INPUTS["qkv"]
    qc, kc, vc = _SWEEP_INPUTS["cpu"]
    o = launch_kernel(q, k, v)
    torch.cuda.synchronize()
    assert o.shape == q.shape and o.dtype == torch.bfloat16
    assert bool(torch.isfinite(o).all())
    if S <= 1024:
        heads = [(b, h) for b in range(case.B) for h in range(case.H)]
    else:
        heads = [(b, h) for b in range(case.B) for h in range(b, case.H, 4)]
    refs = oracle.variant_ref_heads(op, qc, kc, vc, heads)
    unnorm = op in ("sigmoid_attn", "relu_attn")
    worst_rel = 0.0
    for (b, h), ref in zip(heads, refs):
        out = o[b, h].float().cpu()
        worst_rel = max(worst_rel, gate.relerr(ref, out))
        res = gate.north_star_gate(ref, out, scale_aware=unnorm)
        assert res.ok, f"{op} S={S} b={b} h={h}: {res.status} {res.stats}"
    assert worst_rel < gate.REL_TOL, (op, S, worst_rel)
    _say(f"  {op} S{S}: {len(heads)} slices within the gate, reference relerr {worst_rel:.2e}")
