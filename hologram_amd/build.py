"""Build the HIP backend in place: hologram_amd/libholo_hip.so.

Device sources (*.hip) are compiled by hipcc for gfx950 only; host sources
(*.cpp) by g++ for x86-64 (SSE2, no FMA contraction: the activation tables are
defined by x86-64 IEEE semantics). Everything links into one shared library
whose exported surface is include/holo_hip.h.

    python -m hologram_amd.build
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
OBJ = PKG / "_build"
LIB = PKG / "libholo_hip.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # No contraction anywhere: the quantizer's t = x*inv, t +- 0.5 must round
    # as two separate IEEE operations. Kernels that want FMA call fmaf().
    "-ffp-contract=off",
    # Packed FP32 instructions stay disabled: some of their forms have given
    # wrong results on these boxes without any error.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
CXX_FLAGS = [
    "-O2", "-fPIC", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-fsignaling-nans", "-msse2",
    "-mfpmath=sse", "-D__HIP_PLATFORM_AMD__", "-Wall",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n"
                           f"{proc.stdout}\n{proc.stderr}")


def _compile(src: Path, obj_dir: Path = OBJ) -> Path:
    out = obj_dir / (src.name + ".o")
    inc = [f"-I{ROOT / 'include'}", f"-I{CSRC}", f"-I{ROCM / 'include'}"]
    if src.suffix == ".hip":
        _run([str(HIPCC), *HIP_FLAGS, *inc, "-c", str(src), "-o", str(out)])
    else:
        _run(["g++", *CXX_FLAGS, *inc, "-c", str(src), "-o", str(out)])
    return out


def build(verbose: bool = True) -> Path:
    """Compile every source under csrc/ and link libholo_hip.so (always rebuilds)."""
    if not HIPCC.exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    out, obj_dir = LIB, OBJ
    obj_dir.mkdir(parents=True, exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda p: _compile(p, obj_dir), srcs))
    tmp = out.with_suffix(".so.tmp")
    _run([str(HIPCC), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
          "-o", str(tmp), f"-L{ROCM / 'lib'}", "-lamdhip64",
          f"-Wl,-rpath,{ROCM / 'lib'}"])
    tmp.replace(out)
    if verbose:
        print(f"built {out} from {len(srcs)} sources", file=sys.stderr)
    return out


if __name__ == "__main__":
    build()
