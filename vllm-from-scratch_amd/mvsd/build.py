"""Build recipe for libmvsd.so (the HIP kernels + C ABI declared in include/mvsd.h).

Compiles every ``csrc/*.hip`` for gfx950 with hipcc (one object per source, in parallel) and
links them into one shared library next to this file.  Flags:
  * ``-fhip-fp32-correctly-rounded-divide-sqrt``: IEEE fp32 division, so the temperature
    divide and ``p / q`` round like the reference's fp32 arithmetic;
  * ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed-FP32 VALU instructions;
  * ``-mllvm -amdgpu-atomic-optimizer-strategy=None``: single-lane counter atomics stay plain
    atomics whose results are waited for where they are used, instead of being rewritten
    into a wave reduction that waits for the result (and every older load) at once;
  * no fast-math.

Run ``python -m mvsd.build`` (from ``vllm-from-scratch_amd/``) or call :func:`build`.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR.parent / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parent.parent / "include"
LIB_NAME = "libmvsd.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME

OFFLOAD_ARCH = os.environ.get("MVSD_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm under /opt/rocm")


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; that is expected.
    noise = "packed-fp32-ops"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd)}\n{stderr}")
    return stderr


def build(verbose: bool = False) -> Path:
    """Compile libmvsd.so in place (always rebuilds) and return its path.  Each source is
    compiled to an object of its own, in parallel, and the objects are linked into the
    library (every translation unit carries its own device code; none calls device code of
    another)."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1)), 16))
    with tempfile.TemporaryDirectory(prefix="mvsd_build_") as tmpdir:
        objs = [Path(tmpdir) / (src.stem + ".o") for src in srcs]
        cmds = [[hipcc(), *compile_flags, f"-I{INCLUDE_DIR}", "-c", "-o", str(obj), str(src)]
                for src, obj in zip(srcs, objs)]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            logs = list(pool.map(_run, cmds))
        tmp = LIB_PATH.with_suffix(".so.tmp")
        link = [hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp),
                *map(str, objs)]
        logs.append(_run(link))
    if verbose:
        for cmd in cmds + [link]:
            print(" ".join(cmd), flush=True)
        for log in logs:
            if log.strip():
                print(log, file=sys.stderr)
    tmp.replace(LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
