"""Build librecap_hip.so in-tree for gfx950 with hipcc.

    python -m recap_amd.build_lib          # or __graft_entry__.build()

Every kernel source compiles to its own object in parallel, then the objects link into
``recap_amd/librecap_hip.so``.  Packed-fp32 instructions are disabled for all device code.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "librecap_hip.so"
ARCH = os.environ.get("RECAP_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; a ROCm toolchain is required to build librecap_hip.so")


def _compile(src: Path, obj: Path) -> tuple[Path, int, str]:
    cmd = [hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    log = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line)
    return src, proc.returncode, log


def build(verbose: bool = True) -> Path:
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with tempfile.TemporaryDirectory(prefix="recap_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in sources]
        with ThreadPoolExecutor(max_workers=min(len(sources), os.cpu_count() or 4)) as pool:
            results = list(pool.map(_compile, sources, objs))
        failed = [(s, log) for s, rc, log in results if rc != 0]
        for s, rc, log in results:
            if log.strip() and (verbose or rc):
                print(f"[{s.name}]\n{log}", file=sys.stderr)
        if failed:
            raise RuntimeError("hipcc failed: " + ", ".join(s.name for s, _ in failed))
        tmp_lib = LIB.with_suffix(".so.tmp")
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp_lib),
               *map(str, objs)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode:
            raise RuntimeError("link failed:\n" + proc.stdout + proc.stderr)
        missing = undefined_own_symbols(tmp_lib)
        if missing:
            raise RuntimeError("librecap_hip.so would leave symbols of its own undefined (a "
                               "kernel's host launch stub was not emitted): " + ", ".join(missing))
        os.replace(tmp_lib, LIB)
    return LIB


def undefined_own_symbols(lib: Path) -> list[str]:
    """Symbols of the `recap` namespace that ``lib`` references but does not define.  The host
    pass of a HIP source can drop a kernel's launch stub without an error; the library then
    links and fails only when it is loaded."""
    nm = shutil.which("nm") or "/opt/rocm/llvm/bin/llvm-nm"
    proc = subprocess.run([nm, "-D", "--undefined-only", str(lib)], capture_output=True,
                          text=True)
    if proc.returncode:
        raise RuntimeError(f"{nm} failed on {lib}: {proc.stderr}")
    names = [line.split()[-1] for line in proc.stdout.splitlines() if line.strip()]
    return [n for n in names if n.startswith("_ZN5recap")]


if __name__ == "__main__":
    print(build())
