"""Build libgoda_attn.so in-tree with hipcc for gfx950.

`python -m goda_amd.build` compiles every `goda_amd/csrc/*.hip` file to an
object (in parallel) and links them into `goda_amd/lib/libgoda_attn.so`.
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
INCLUDE = ROOT / "include"
LIBDIR = PKG / "lib"
LIBNAME = "libgoda_attn.so"
OFFLOAD_ARCH = "gfx950"

# Packed fp32 VALU forms are turned off for all device code; hipcc's host pass
# warns that it does not know the feature, which is harmless.
HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # The kernels type-pun through vector pointers (element arrays read as
    # 16-byte vectors and back); keep type-based alias analysis out of it.
    "-fno-strict-aliasing",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def lib_path() -> Path:
    return LIBDIR / LIBNAME


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [hipcc(), *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    noise = "is not a recognized feature for this target"
    errs = [ln for ln in res.stderr.splitlines() if ln.strip() and noise not in ln]
    if verbose and errs:
        print("\n".join(errs), flush=True)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all HIP sources and link the shared library; returns its path."""
    LIBDIR.mkdir(parents=True, exist_ok=True)
    objdir = LIBDIR / "obj"
    objdir.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [objdir / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, verbose) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    out = lib_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
