"""Build libds4hip.so (the gfx950 HIP kernels + C-ABI) and the CPU oracle.

`python -m ds4cuda_amd.build` compiles every ds4cuda_amd/csrc/*.hip with
hipcc for gfx950 into ds4cuda_amd/libds4hip.so, in-tree, so the library
travels with the source tree to the GPU box. The oracle under oracle/ is test
infrastructure and is built by its own Makefile (build_oracle).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libds4hip.so"
OBJ = ROOT / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("DS4HIP_ARCH", "gfx950")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-munsafe-fp-atomics",
    # packed fp32 VALU ops are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-I", str(ROOT / "include"), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


# Kernels whose copy ring counts outstanding vector-memory operations: a
# register spill store inside the ring could complete ahead of older copies
# and break that count, so the build refuses any spill store that a path can
# reach while a copy is outstanding (ds4cuda_amd/spill_check.py). Spills
# outside the ring (before the first copy, after a vmcnt(0)) and reloads
# (in order with the copies) are allowed.
NO_SPILL_KERNELS = ("decode_fp8_kernelILb0E", "decode_flat_kernel")


def check_spills(src: Path) -> None:
    import re
    import tempfile
    from .spill_check import ring_violations
    with tempfile.TemporaryDirectory() as td:
        out = Path(td) / "k.s"
        cmd = [HIPCC, *FLAGS, "-I", str(ROOT / "include"), "--cuda-device-only", "-S", str(src),
               "-o", str(out)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc -S failed for {src.name}:\n{r.stderr}")
        asm = out.read_text()
    syms = sorted(set(re.findall(r"^(_Z\w+):", asm, re.M)))
    for sym in syms:
        if any(k in sym for k in NO_SPILL_KERNELS):
            bad = ring_violations(asm, sym)
            if bad:
                raise RuntimeError(f"{sym}: {len(bad)} spill stores while ring copies may be "
                                   f"outstanding (first: {bad[0]}); its copy-ring waits require none")


def build_lib(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    check_spills(CSRC / "flash_attn.hip")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_native_checks(verbose: bool = False) -> Path:
    """The C++ caller of the launcher shims used by the GPU tests
    (tests/native/forward_layer_check.cpp), linked against libds4hip.so."""
    out_dir = ROOT / "tests" / "native" / "_bin"
    out_dir.mkdir(parents=True, exist_ok=True)
    exe = out_dir / "forward_layer_check"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-I", str(ROOT / "include"),
           str(ROOT / "tests" / "native" / "forward_layer_check.cpp"), "-o", str(exe),
           f"-L{PKG}", "-lds4hip", f"-Wl,-rpath,{PKG}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"forward_layer_check build failed:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {exe}")
    return exe


def build_oracle(verbose: bool = False) -> Path:
    r = subprocess.run(["make", "-C", str(ROOT / "oracle"), "-B", "-j8"], capture_output=True,
                       text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print("built oracle/libds4oracle.so")
    return ROOT / "oracle" / "libds4oracle.so"


if __name__ == "__main__":
    build_lib(verbose=True)
    if "--lib-only" not in sys.argv:
        build_native_checks(verbose=True)
        if shutil.which("make"):
            build_oracle(verbose=True)
