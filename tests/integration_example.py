"""The kernel-level ctypes example of INTEGRATION.md, read out of that file so that the
tests run the text a maintainer copies."""

from __future__ import annotations

import os
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def example_source() -> str:
    """The first python code block after the "## 2. Kernel level" heading."""
    text = (ROOT / "INTEGRATION.md").read_text()
    section = text[text.index("## 2. Kernel level"):]
    start = section.index("```python\n") + len("```python\n")
    return section[start:section.index("```", start)]


def load_example() -> dict:
    """Executes the block (from the repository root, as its relative library path
    assumes) and returns its namespace."""
    namespace: dict = {}
    cwd = os.getcwd()
    os.chdir(ROOT)
    try:
        exec(compile(example_source(), "INTEGRATION.md:kernel-level", "exec"), namespace)
    finally:
        os.chdir(cwd)
    return namespace
