"""Golden fixtures (tests/golden/variants_S96.npz, written by make_golden.py).

CPU: the oracle still reproduces the committed vectors (it has not drifted).
GPU: the HIP core, called through the C ABI, meets the north-star gate
against the committed vectors without running the oracle on the box.
"""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden  # noqa: E402

DATA = np.load(GOLDEN / "variants_S96.npz")


def _inputs():
    return tuple(torch.from_numpy(DATA[f"in_{n}"]).view(torch.bfloat16) for n in ("q", "k", "v"))


@pytest.mark.parametrize("op", list(make_golden.PARAMS))
def test_oracle_reproduces_golden(op):
    import oracle

    q, k, v = _inputs()
    got = oracle.variant_ref(op, q, k, v, **make_golden.PARAMS[op]).numpy()
    want = DATA[f"out_{op}"].astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-4)


def test_golden_inputs_are_the_seeded_draw():
    g = torch.Generator("cpu").manual_seed(make_golden.SEED)
    q = torch.randn(1, 2, 96, 64, generator=g).to(torch.bfloat16)
    assert torch.equal(q, _inputs()[0])


@pytest.mark.gpu
@pytest.mark.parametrize("op", list(make_golden.PARAMS))
def test_kernel_matches_golden(op):
    from chia_proj_amd import OPS, gate

    print(f"[golden] {op}", flush=True)
    q, k, v = (t.to("cuda") for t in _inputs())
    o = OPS[op](q, k, v, **make_golden.PARAMS[op])
    torch.cuda.synchronize()
    want = torch.from_numpy(DATA[f"out_{op}"].astype(np.float32))
    res = gate.north_star_gate(want, o.float().cpu(), scale_aware=op == "sigmoid_attn")
    assert res.ok, (op, res.stats)
