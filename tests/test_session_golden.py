"""recap_amd's step loop against the reference's own decisions: the 40 scenarios of
tests/golden/session_cases.py (budgets, prefix floor and cap, exact tails, passing, failing
and non-finite refinement errors, one and two streams, two samples with a reset between,
three output wrappings and two dtypes) replayed through recap_amd.RecapSession must give
the records the reference's RecapSession wrote (tests/golden/session_golden.json, made by
tests/golden/make_session_golden.py): the same action at every step, the same h and
validation ages and verdicts, m, g and errors within 1e-6, and the same outputs returned
to the pipeline (REUSE extrapolations included)."""

from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

from session_cases import run_case  # noqa: E402

import recap_amd.config as config_module  # noqa: E402
from recap_amd import RecapSession  # noqa: E402

DATA = json.loads((GOLDEN / "session_golden.json").read_text())


def _close(a, b, tol=1e-6) -> bool:
    if isinstance(a, float) or isinstance(b, float):
        a, b = float(a), float(b)
        if math.isnan(a) or math.isnan(b):
            return math.isnan(a) and math.isnan(b)
        if math.isinf(a) or math.isinf(b):
            return a == b
        return abs(a - b) <= tol * max(1.0, abs(a), abs(b))
    return a == b


def _same_record(got: dict, want: dict) -> bool:
    if set(got) != set(want):
        return False
    for key, value in want.items():
        if isinstance(value, dict):
            if not _same_record(got[key], value):
                return False
        elif not _close(got[key], value):
            return False
    return True


def test_golden_covers_every_action():
    actions = {row["a"] for r in DATA["results"] for s in r["samples"] for row in s["actions"]}
    verdicts = {row["validation"]["passed"] for r in DATA["results"] for s in r["samples"]
                for row in s["actions"] if "validation" in row}
    assert actions == {"exact", "refresh", "sparse", "reuse"} and verdicts == {True, False}


@pytest.mark.parametrize("index", range(len(DATA["cases"])))
def test_session_matches_reference_records(index):
    case, want = DATA["cases"][index], DATA["results"][index]
    got = run_case(case, RecapSession, config_module)
    assert len(got["samples"]) == len(want["samples"])
    for n, (g, w) in enumerate(zip(got["samples"], want["samples"])):
        where = f"{case['name']} sample {n}"
        assert [r["a"] for r in g["actions"]] == [r["a"] for r in w["actions"]], where
        for gr, wr in zip(g["actions"], w["actions"]):
            assert _same_record(gr, wr), (where, gr, wr)
        assert g["kinds"] == w["kinds"], where
        assert g["counts"] == w["counts"], where
        assert _close(g["gain"], w["gain"]), where
        assert len(g["validation_history"]) == len(w["validation_history"]), where
        for gv, wv in zip(g["validation_history"], w["validation_history"]):
            assert _same_record(gv, wv), (where, gv, wv)
        for i, (gs, ws) in enumerate(zip(g["output_sums"], w["output_sums"])):
            assert gs[2] == ws[2] and _close(gs[0], ws[0], 1e-5) and _close(gs[1], ws[1], 1e-5), \
                (where, i, gs, ws)
