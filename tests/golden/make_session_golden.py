"""Writes tests/golden/session_golden.json: the reference's step loop (RecapSession and
Controller, recap/session.py:46-359, recap/controller.py:20-131) driven through the
scenarios of session_cases.py, imported from the reference tree in the development
container only.  The decisions are a function of the measured mismatches and refinement
errors that nothing but the reference's own code fixes, so its records are the fixture.

    python tests/golden/make_session_golden.py [/root/reference]
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

from session_cases import make_cases, run_case  # noqa: E402


def main(reference: str = "/root/reference") -> None:
    sys.path.insert(0, reference)
    import recap.config as config_module
    from recap.session import RecapSession

    cases = make_cases()
    out = {"generator": "tests/golden/session_cases.py make_cases()",
           "cases": cases,
           "results": [run_case(case, RecapSession, config_module) for case in cases]}
    path = HERE / "session_golden.json"
    path.write_text(json.dumps(out, indent=None, separators=(",", ":")))
    total = sum(len(s["actions"]) for r in out["results"] for s in r["samples"])
    print(f"wrote {path} ({len(cases)} cases, {total} step records)")


if __name__ == "__main__":
    main(*sys.argv[1:])
