"""Build libpsquant.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python comfyui-powershard_amd/powershard_amd/build_lib.py [-j N]

Each ``csrc/*.hip`` compiles to an object under ``_build/``; the objects link into
``lib/libpsquant.so``.  Flags:

* ``--offload-arch=gfx950`` only: no other target, no CUDA path.
* ``-ffp-contract=off``: no silent FMA fusion (the kernels call fmaf where the convention
  fuses), so the quantization and epilogue arithmetic matches the CPU oracle bit for bit.
* ``-fhip-fp32-correctly-rounded-divide-sqrt``: IEEE division for the per-row 127/absmax.
* ``-fno-gpu-flush-denormals-to-zero``: fp32 denormals are kept, as on the CPU.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32 VALU instructions.
"""
import argparse
import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "lib" / "libpsquant.so"
INCLUDE = PKG.parent.parent / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++20",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function", f"-I{INCLUDE}",
]


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src):
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    # surface warnings other than the known host-pass note about the packed-fp32 feature
    for line in r.stderr.splitlines():
        if "warning" in line and "packed-fp32-ops" not in line:
            print(line, file=sys.stderr)
    return obj


def _check_stubs(lib):
    """Fail on an undefined symbol of the library's own namespace.  When the host pass of a .hip
    file rejects a kernel body (a target builtin it cannot check there), clang drops the kernel's
    launch stub without an error, and the library then fails to load on the GPU host."""
    r = subprocess.run(["nm", "-D", "--undefined-only", str(lib)], capture_output=True, text=True)
    if r.returncode != 0:
        return   # no binutils: the ABI test's load of the library still catches it
    missing = [line.split()[-1] for line in r.stdout.splitlines() if "_ZN3psq" in line]
    if missing:
        raise RuntimeError("kernel launch stubs missing (host pass dropped them): " + ", ".join(missing[:4]))


def build(jobs=None, verbose=False):
    """Compile every csrc/*.hip for gfx950 and link lib/libpsquant.so. Returns the library path."""
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 1, 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    _check_stubs(tmp)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    build(ap.parse_args().j, verbose=True)
