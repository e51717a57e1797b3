"""The reference's published A100 latencies that bench.py prints beside its own
reference-shape figures must equal the reference's result files:
results/FINAL_flexattention.csv (the S = 2048 benchmark, extra_bench.py:83-157)
and results/FINAL_seqsweep.csv (the sequence sweep, extra_bench.py:166-201),
where a sweep row counts only if its status is "generalises".  Skipped where the
reference tree is absent (it never travels to the GPU box)."""
import csv
import importlib.util
from pathlib import Path

import pytest

from chia_proj_amd.workloads import REFERENCE_SWEEP_S, reference_suite

REPO = Path(__file__).resolve().parent.parent
RESULTS = Path("/root/reference/results")


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", REPO / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _rows(name):
    path = RESULTS / name
    if not path.is_file():
        pytest.skip(f"{path} not present")
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


def _num(x):
    return float(x) if x not in ("", None) else None


def test_flexattention_table_matches_reference_file():
    bench = _bench()
    rows = {r["op"]: r for r in _rows("FINAL_flexattention.csv")}
    assert set(bench.A100_PUBLISHED_US) == set(rows) == {c.op for c in reference_suite()}
    for op, (gs, flex) in bench.A100_PUBLISHED_US.items():
        assert gs == _num(rows[op]["graphsynth_us"]), op
        assert flex == _num(rows[op]["flex_us"]), op


def test_seqsweep_table_matches_reference_file():
    bench = _bench()
    rows = _rows("FINAL_seqsweep.csv")
    assert {int(r["S"]) for r in rows} == set(REFERENCE_SWEEP_S)
    assert set(bench.A100_SEQSWEEP_US) == {c.op for c in reference_suite()}
    for r in rows:
        want = _num(r["graphsynth_us"]) if r["status"] == "generalises" else None
        assert bench.A100_SEQSWEEP_US[r["op"]][int(r["S"])] == want, (r["op"], r["S"], r["status"])


def test_reference_suites_keep_the_reference_shape():
    for S in REFERENCE_SWEEP_S:
        cases = reference_suite(S)
        assert [c.op for c in cases] == [c.op for c in reference_suite()]
        assert all((c.B, c.H, c.S, c.D) == (2, 32, S, 128) and c.params == {} for c in cases)
    assert reference_suite()[0].seed == 20262048  # the benchmark's draw is unchanged
