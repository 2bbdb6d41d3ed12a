"""Build libkvq.so (the gfx950 kernels and their C ABI) in-tree.

The HIP sources under ``csrc/`` are compiled for gfx950 with hipcc and linked against the HIP
runtime that PyTorch ships (``torch/lib/libamdhip64.so``), so the library, torch's allocator and
torch's streams all live in one HIP runtime instance. The library is written next to this file
(``libkvq.so``) so it travels with the source tree.

Usage: ``python -m myinfer_amd._build`` or ``myinfer_amd._build.build()``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libkvq.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unknown-pragmas",
    # packed fp32 VALU forms are kept out of the generated code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


# Per-source additions. wide.hip keeps its MFMA accumulators in VGPRs: one wave per SIMD has 512
# registers, and with AGPR accumulators the compiler copied all 128 of them between the two files on
# every tile step.
SOURCE_FLAGS = {"wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall"]


def _torch_lib_dir() -> Path:
    import importlib.util

    spec = importlib.util.find_spec("torch")
    if spec is None or spec.origin is None:
        raise RuntimeError("PyTorch is required: libkvq.so links against torch's HIP runtime")
    return Path(spec.origin).resolve().parent / "lib"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in (res.stderr or "").splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every ``csrc/*.hip`` for gfx950 (and the host-only ``csrc/*.cpp`` with g++) and link
    ``libkvq.so``. Always recompiles."""
    hipcc = _hipcc()
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    host_sources = sorted(CSRC.glob("*.cpp"))  # host-only code (no device code): g++
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    objs = [OBJ / (s.stem + ".o") for s in sources]
    host_objs = [OBJ / (s.stem + ".host.o") for s in host_sources]
    jobs = jobs or min(len(sources) + len(host_sources), max(1, os.cpu_count() or 1), 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [hipcc, *HIPCC_FLAGS, *SOURCE_FLAGS.get(s.name, []), "-c", str(s), "-o", str(o)], verbose)
                for s, o in zip(sources, objs)]
        futs += [ex.submit(_run, ["g++", *HOST_FLAGS, "-c", str(s), "-o", str(o)], verbose)
                 for s, o in zip(host_sources, host_objs)]
        for f in futs:
            f.result()
    objs += host_objs
    tlib = _torch_lib_dir()
    tmp = LIB.with_suffix(".so.tmp")
    link = [
        "g++",
        "-shared",
        "-o",
        str(tmp),
        *map(str, objs),
        f"-L{tlib}",
        "-l:libamdhip64.so",
        f"-Wl,-rpath,{tlib}",
        "-Wl,--disable-new-dtags",
        "-Wl,--no-undefined",
    ]
    _run(link, verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
