"""Build libfracture_hip.so for gfx950 in-tree with hipcc.

Every HIP source under ``csrc/`` compiles to an object under ``_build/`` and links into
``fracture_amd/libfracture_hip.so``. HIP code is built with packed fp32 ops disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``); the host-only TurboQuant table code
is built with ``-ffp-contract=off`` so its double arithmetic is not fused.

Usage: ``python -m fracture_amd.build`` (or ``build()`` from Python).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libfracture_hip.so"
ARCH = os.environ.get("FHIP_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
]
PER_FILE = {
    "tq_host.cpp": ["-ffp-contract=off"],
}
SOURCES = ["elementwise.hip", "reduce.hip", "turboquant.hip", "attention_tq.hip",
           "attention_paged.hip", "matmul.cpp",
           "tq_host.cpp", "runtime.cpp"]

_NOISE = "'-packed-fp32-ops' is not a recognized feature for this target"


def _clean(text: str) -> str:
    return "\n".join(l for l in text.splitlines() if _NOISE not in l).strip()


def _compile(src: str) -> Path:
    obj = BUILD / (src.replace(".", "_") + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *COMMON, *PER_FILE.get(src, []), *lang, "-c", str(CSRC / src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    msg = _clean(p.stdout + p.stderr)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    if msg:
        print(f"[build] {src}:\n{msg}", file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    """Compile every HIP source for gfx950 and link libfracture_hip.so (always rebuilds)."""
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    # -z defs: a symbol that no object or linked library defines fails the link here rather
    # than the library's load on the device host
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", str(tmp),
           *map(str, objs), "-lrocblas", "-ldl"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + _clean(p.stdout + p.stderr))
    os.replace(tmp, LIB)
    if verbose:
        print(f"[build] {LIB.relative_to(ROOT)} ({LIB.stat().st_size // 1024} KiB)")
    return LIB


if __name__ == "__main__":
    build()
