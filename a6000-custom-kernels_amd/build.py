"""Build the gfx950 C-ABI library in-tree with hipcc.

    python a6000-custom-kernels_amd/build.py        # -> a6000-custom-kernels_amd/lib/libggml_hip_moe_cache.so

The library is plain hipcc output (no torch extension): kernels, the HIP
device layer and the C++ host registry linked into one shared object whose
exported symbols are exactly the functions of include/ggml_hip_moe_cache.h.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libggml_hip_moe_cache.so"

ARCH = os.environ.get("MC_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# Device-code flags: gfx950 only, -O3, no packed-FP32 instructions (their
# results have been unreliable on these boards), IEEE division/rounding.
DEVICE_FLAGS = ["--offload-arch=" + ARCH, "-mcode-object-version=5", "-O3", "-std=c++17", "-fPIC",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-fno-fast-math", "-ffp-contract=fast-honor-pragmas",
                "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function"]

SOURCES = [
    ("mc_kernels.hip", "hip"),
    ("mc_mmq.hip", "hip"),
    ("mc_ffn.hip", "hip"),
    ("mc_ssm_conv.hip", "hip"),
    ("mc_noalloc.hip", "hip"),
    ("mc_device_hip.cpp", "hiphost"),
    ("mc_host.cpp", "cxx"),
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    out = (r.stdout or "") + (r.stderr or "")
    # hipcc's host pass does not know the packed-fp32 feature: harmless, drop the noise
    out = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(str(c) for c in cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build(verbose: bool = False) -> Path:
    """Compile every source (always: this is the build check) and link the library."""
    BUILD.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    inc = ["-I", str(INCLUDE), "-I", str(CSRC)]
    jobs = []
    for src, kind in SOURCES:
        obj = BUILD / (src + ".o")
        if kind == "hip":
            cmd = [HIPCC, *DEVICE_FLAGS, *inc, "-c", CSRC / src, "-o", obj]
        elif kind == "hiphost":
            cmd = [HIPCC, *HOST_FLAGS, *inc, "-c", CSRC / src, "-o", obj]
        else:
            cmd = ["g++", *HOST_FLAGS, *inc, "-c", CSRC / src, "-o", obj]
        jobs.append((cmd, obj))
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        list(ex.map(lambda j: _run(j[0], verbose), jobs))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp, *[o for _, o in jobs],
          "-Wl,--version-script=" + str(CSRC / "exports.map")], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_single(src: Path, lib: Path, verbose: bool = False) -> Path:
    """One self-contained HIP source (the bench's read-floor probe) as its own shared library,
    with the library's device flags."""
    tmp = lib.with_suffix(".so.tmp")
    _run([HIPCC, *DEVICE_FLAGS, "-shared", "-o", tmp, src], verbose)
    os.replace(tmp, lib)
    return lib


def build_hostsim(verbose: bool = False) -> Path:
    """Test-only: the same registry/step code linked against a host-memory
    simulated device (tests/native/sim_device.cpp); no kernels, no GPU."""
    out_dir = ROOT / "tests" / "native" / "_build"
    out_dir.mkdir(parents=True, exist_ok=True)
    lib = out_dir / "libmc_hostsim.so"
    tmp = lib.with_suffix(".so.tmp")
    _run(["g++", *HOST_FLAGS, "-I", str(INCLUDE), "-I", str(CSRC), "-shared", "-o", tmp,
          CSRC / "mc_host.cpp", ROOT / "tests" / "native" / "sim_device.cpp"], verbose)
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    v = "-v" in sys.argv
    print(build(verbose=v))
    if "--hostsim" in sys.argv:
        print(build_hostsim(verbose=v))
