"""Builds libjanus_moe_hip.so in-tree from the HIP sources under janus_amd/csrc for gfx950.

    python -m janus_amd.build          # compile every source, link the library

hipcc compiles each source to an object (in parallel), then links the shared library next to this file, where
janus_amd._lib loads it. The library exports only the extern "C" entry points of include/janus_moe.h.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libjanus_moe_hip.so"
SOURCES = ("align.hip", "router.hip", "gemm.hip", "norm.hip", "api.hip")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # packed fp32 VALU ops stay off: plain fp32 code only
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # atomics stay one instruction per wave: the optimizer's broadcast of a returned value waits for the atomic where
    # it is issued, and the persistent GEMM launch takes its next ticket early so that the wait falls a unit later
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if candidate and (Path(candidate).exists() or candidate == "hipcc"):
            return candidate
    raise RuntimeError("hipcc not found")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(jobs: int | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    objects = [BUILD / (src.replace(".hip", ".o")) for src in SOURCES]
    cmds = [[cc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)] for src, obj in zip(SOURCES, objects)]
    with ThreadPoolExecutor(max_workers=jobs or min(len(cmds), os.cpu_count() or 1)) as pool:
        list(pool.map(_run, cmds))
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)])
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
