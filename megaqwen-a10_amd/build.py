"""Build the gfx950 HIP library ``lib/libmegaqwen_a10.so`` in-tree with hipcc.

Usage: ``python megaqwen-a10_amd/build.py [--asm DIR]``. Each ``csrc/*.hip``
compiles to an object in parallel, then one shared library is linked.
``--asm DIR`` also writes the device assembly of every source to DIR (for
inspecting the generated gfx950 code).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIBNAME = "libmegaqwen_a10.so"
OBJDIR = PKG / "_build"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Keep the compiler from forming packed fp32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def build(verbose: bool = False, asm_dir: Path | None = None) -> Path:
    cc = hipcc()
    OBJDIR.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sources()
    objs = [OBJDIR / (s.stem + ".o") for s in srcs]
    jobs = []
    for s, o in zip(srcs, objs):
        jobs.append([cc, *HIPCC_FLAGS, "-c", str(s), "-o", str(o)])
        if asm_dir is not None:
            asm_dir.mkdir(parents=True, exist_ok=True)
            jobs.append([cc, *HIPCC_FLAGS, "--cuda-device-only", "-S", str(s), "-o", str(asm_dir / (s.stem + ".s"))])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for cmd, fut in zip(jobs, [ex.submit(_run, j) for j in jobs]):
            if verbose:
                print(" ".join(cmd))
            fut.result()
    out = LIBDIR / LIBNAME
    tmp = LIBDIR / (LIBNAME + ".tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--asm", type=Path, default=None, help="also write device assembly here")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args(argv)
    build(verbose=args.verbose, asm_dir=args.asm)
    return 0


if __name__ == "__main__":
    sys.exit(main())
