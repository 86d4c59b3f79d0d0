"""Build libsmx.so, the gfx950 C-ABI library of the decode path, in place.

Every HIP source is compiled for gfx950 only, with packed-FP32 code
generation disabled, and linked into ``native/libsmx.so`` next to this file.
Each HIP source's device code is also written as a code object
(``native/libsmx.<source>.co``), which the step runner loads into its own
HSA executables.  The benchmark's streaming-read probe (csrc/probe/) is a
measurement instrument, not part of the decode path: it is built into a
library of its own, ``native/libsmx_probe.so``.  Run as ``python build.py``
or call :func:`build`.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libsmx.so"
PROBE_LIB = HERE / "libsmx_probe.so"
PROBE_SOURCE = CSRC / "probe" / "read_probe.hip"
OBJ_DIR = HERE / "_build"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ROCM_LIB = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib"
COMMON = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # leading scalar/pointer kernel arguments arrive in SGPRs (gfx950 kernarg
    # preloading): no scalar-load round trip before a kernel's first loads
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]
SOURCES = ["q4_0_gemv.hip", "q4_0_gemm.hip", "splitkv_attention.hip", "small_ops.hip",
           "abi.cpp", "step_runner.cpp"]
DEVICE_SOURCES = [s for s in SOURCES if s.endswith(".hip")]


def code_object_paths() -> list[Path]:
    """The device code objects the step runner loads, one per HIP source."""
    return [HERE / f"libsmx.{Path(s).stem}.co" for s in DEVICE_SOURCES]


def _compile(src: str) -> Path:
    out = OBJ_DIR / (Path(src).stem + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *COMMON, *lang, "-c", str(CSRC / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return out


def _code_object(src: str) -> Path:
    out = HERE / f"libsmx.{Path(src).stem}.co"
    tmp = out.with_suffix(".co.tmp")
    cmd = [HIPCC, *COMMON, "-x", "hip", "--cuda-device-only", "--no-gpu-bundle-output",
           str(CSRC / src), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc (device code object) failed for {src}:\n{res.stderr}")
    os.replace(tmp, out)
    return out


def _probe_library() -> Path:
    """libsmx_probe.so: the streaming-read probe alone (bench only)."""
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *COMMON, "-x", "hip", "-shared", str(PROBE_SOURCE), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SOURCE.name}:\n{res.stderr}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build(verbose: bool = False) -> Path:
    """Compile all sources, link libsmx.so, write the device code objects and
    build the benchmark's probe library; returns libsmx.so's path."""
    OBJ_DIR.mkdir(exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as pool:
        objs_f = [pool.submit(_compile, s) for s in SOURCES]
        cos_f = [pool.submit(_code_object, s) for s in DEVICE_SOURCES]
        probe_f = pool.submit(_probe_library)
        objs = [f.result() for f in objs_f]
        for f in cos_f:
            f.result()
        probe_f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp),
           f"-L{ROCM_LIB}", f"-Wl,-rpath,{ROCM_LIB}", "-lhsa-runtime64"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} and {PROBE_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
