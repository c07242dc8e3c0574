"""Build libfracture_hip.so for gfx950 in-tree with hipcc.

Every HIP source under ``csrc/`` compiles to an object under ``_build/`` and links into
``fracture_amd/libfracture_hip.so``. HIP code is built with packed fp32 ops disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``); the host-only TurboQuant table code
is built with ``-ffp-contract=off`` so its double arithmetic is not fused.

Usage: ``python -m fracture_amd.build`` (or ``build()`` from Python).

``python -m fracture_amd.build --host-sanitize`` builds a second copy,
``fracture_amd/_san/libfracture_hip.so``, whose host code carries AddressSanitizer and
UndefinedBehaviorSanitizer (the device code is unchanged): a CPU-only check of the host-side
argument handling and table code, loaded with ``FHIP_LIBRARY`` and clang's ASan runtime
preloaded (``oracle/Makefile``'s ``sanitize`` target builds the oracle to match).
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
           "attention_paged.hip", "probes.hip", "matmul.cpp",
           "tq_host.cpp", "runtime.cpp"]

_NOISE = "'-packed-fp32-ops' is not a recognized feature for this target"


def _clean(text: str) -> str:
    return "\n".join(l for l in text.splitlines() if _NOISE not in l).strip()


# host code only: each option behind -Xarch_host, so no GPU code is built with a sanitizer
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=all"]
SAN_BUILD = PKG / "_build_san"
SAN_LIB = PKG / "_san" / "libfracture_hip.so"
# The host build of the decode-attention kernel's index helpers (tq_attn_index.h), which the
# CPU bounds check of that kernel's accesses calls. Plain C++: no GPU code, no HIP runtime.
INDEX_LIB = PKG / "libfracture_hip_index.so"
CXX = os.environ.get("CXX", "g++")


def _compile(src: str, san: bool = False) -> Path:
    obj = (SAN_BUILD if san else BUILD) / (src.replace(".", "_") + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    extra = HOST_SAN if san else []
    cmd = [HIPCC, *COMMON, *extra, *PER_FILE.get(src, []), *lang, "-c", str(CSRC / src), "-o",
           str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    msg = _clean(p.stdout + p.stderr)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    if msg:
        print(f"[build] {src}:\n{msg}", file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = True, host_sanitize: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link libfracture_hip.so (always rebuilds);
    host_sanitize builds the host-sanitized copy instead (see the module docstring)."""
    out = SAN_LIB if host_sanitize else LIB
    (SAN_BUILD if host_sanitize else BUILD).mkdir(exist_ok=True)
    out.parent.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, host_sanitize), SOURCES))
    tmp = out.with_suffix(".so.tmp")
    # -z defs: a symbol that no object or linked library defines fails the link here rather
    # than the library's load on the device host (the sanitized copy takes its runtime's
    # symbols from the shared ASan runtime, preloaded when it is used)
    link = (["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-shared-libasan"] if host_sanitize else ["-Wl,-z,defs"])
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *link, "-o", str(tmp),
           *map(str, objs), "-lrocblas", "-ldl"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + _clean(p.stdout + p.stderr))
    os.replace(tmp, out)
    if verbose:
        print(f"[build] {out.relative_to(ROOT)} ({out.stat().st_size // 1024} KiB)")
    if not host_sanitize:
        build_index(verbose)
    return out


def build_index(verbose: bool = True) -> Path:
    """libfracture_hip_index.so from tq_attn_index_host.cpp (host C++ only)."""
    tmp = INDEX_LIB.with_suffix(".so.tmp")
    cmd = [CXX, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", f"-I{CSRC}", "-o", str(tmp),
           str(CSRC / "tq_attn_index_host.cpp")]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("index helper build failed:\n" + p.stdout + p.stderr)
    os.replace(tmp, INDEX_LIB)
    if verbose:
        print(f"[build] {INDEX_LIB.relative_to(ROOT)}")
    return INDEX_LIB


if __name__ == "__main__":
    build(host_sanitize="--host-sanitize" in sys.argv[1:])
