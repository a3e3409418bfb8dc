"""Build recipe for `hexlib_amd/libhexlib_gpu.so` (gfx950 only).

Regenerates the entry adapters from the RunnerSpec table, compiles every
`csrc/*.hip` and `csrc/*.cpp` with hipcc in parallel, and links one shared
library in-tree. Every HIP translation unit is built with packed-FP32
instruction selection switched off (`-target-feature -packed-fp32-ops`).

    python -m hexlib_amd.build
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD_DIR = os.path.join(ROOT, "_build")
LIB_PATH = os.path.join(PKG, "libhexlib_gpu.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


# Per-source flags. attention.hip: MFMA accumulators in VGPRs -- its kernels
# rescale and read the accumulators with VALU code every key tile, and the
# AGPR form spent ~250 accvgpr moves per loop and an occupancy step on it.
EXTRA_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


class BuildError(RuntimeError):
    pass


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".cpp")))


def _headers_mtime() -> float:
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    hs += [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]
    return max(os.path.getmtime(h) for h in hs)


def _compile(src: str, changed_only: bool = False) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    if changed_only and os.path.exists(obj) and \
            os.path.getmtime(obj) > max(os.path.getmtime(src), _headers_mtime()):
        return obj
    # .cpp files hold host code only (runtime, generated entries): no device pass.
    host_only = ["--offload-host-only"] if src.endswith(".cpp") else []
    extra = EXTRA_FLAGS.get(os.path.basename(src), [])
    cmd = [HIPCC, *CFLAGS, *extra, *host_only, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise BuildError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False, changed_only: bool = False) -> str:
    """Compile every source (or, with `changed_only`, those newer than their
    object or any header) and link the library."""
    from hexlib_amd.exec import genentry

    genentry.write()
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = max(1, min(len(sources()), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(lambda src: _compile(src, changed_only), sources()))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise BuildError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    build_replay()
    if verbose:
        print(f"built {LIB_PATH} from {len(objs)} sources, and {REPLAY_PATH}")
    return LIB_PATH


REPLAY_SRC = os.path.join(PKG, "replay", "hxplan_replay.c")
REPLAY_PATH = os.path.join(PKG, "hxplan_replay")


def build_replay() -> str:
    """The plan-file replay program: plain C against the library (host code
    only, gcc), found beside it at run time through its rpath."""
    tmp = REPLAY_PATH + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-Wall", f"-I{INCLUDE}", REPLAY_SRC, "-o", tmp,
           f"-L{PKG}", "-lhexlib_gpu", "-Wl,-rpath,$ORIGIN"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise BuildError(f"replay build failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, REPLAY_PATH)
    return REPLAY_PATH


if __name__ == "__main__":
    build(verbose=True, changed_only="--changed" in sys.argv[1:])
    sys.exit(0)
