"""Build ``libcacheir_hip.so`` (the C-ABI kernel library) in-tree with hipcc for gfx950.

Usage: ``python -m cacheir_amd.build`` (also called by ``__graft_entry__.build()``).
Objects go to ``cacheir_amd/_build/``; the library to ``cacheir_amd/_lib/``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB_DIR = PKG / "_lib"
LIB = LIB_DIR / "libcacheir_hip.so"
SOURCES = ["attention.hip", "qgemm.hip", "rowops.hip", "probe.hip"]
ARCH = os.environ.get("CACHEIR_HIP_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-mcode-object-version=5",
        f"-I{ROOT / 'include'}", f"-I{SRC}",
        # Packed-FP32 VALU forms stay off in generated code (hardware notes).
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA results in VGPRs (no accumulator-register copies before the scale FMAs).
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-Wno-unused-result",
    ]


def _compile(src: Path, obj: Path, verbose: bool, defines: tuple[str, ...] = ()) -> None:
    cmd = [hipcc(), *common_flags(), *(f"-D{d}" for d in defines), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = False, defines: tuple[str, ...] = (), lib: Path = LIB, obj_dir: Path = OBJ) -> Path:
    """Compile every source and link ``lib``.  ``defines`` (``NAME=VALUE``) and another
    ``lib``/``obj_dir`` build a variant of the library beside the default one."""
    obj_dir.mkdir(parents=True, exist_ok=True)
    lib.parent.mkdir(parents=True, exist_ok=True)
    objs = [obj_dir / (s.replace(".hip", ".o")) for s in SOURCES]
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        futs = [ex.submit(_compile, SRC / s, o, verbose, tuple(defines)) for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
