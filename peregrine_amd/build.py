"""Build libperegrine_hip.so (gfx950) in-tree, plus the CPU oracle library.

    python -m peregrine_amd.build            # everything
    python -m peregrine_amd.build --lib      # HIP library only

Every HIP translation unit under peregrine_amd/csrc is compiled with hipcc for
gfx950 only, in parallel, then linked into peregrine_amd/libperegrine_hip.so.
The oracle (test infrastructure) is compiled with gcc into oracle/liboracle.so.
Both .so files are git-ignored build products.
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
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB = PKG / "libperegrine_hip.so"
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "liboracle.so"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-FP32 VALU ops are disabled for all device code on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libperegrine_hip.so)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")


def build_lib(jobs: int | None = None, incremental: bool = False) -> Path:
    """Compile every translation unit and link. incremental: recompile only
    sources newer than their object (any header change recompiles all)."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    objs = [BUILD / (s.stem + ".o") for s in sources]
    headers = max(p.stat().st_mtime for p in [*CSRC.glob("*.hpp"), *INCLUDE.glob("*.h")])

    def stale(s: Path, o: Path) -> bool:
        return not incremental or not o.exists() or o.stat().st_mtime < max(s.stat().st_mtime, headers)

    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [hipcc, *HIPCC_FLAGS, "-c", str(s), "-o", str(o)])
                for s, o in zip(sources, objs) if stale(s, o)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    cc = os.environ.get("CC", "gcc")
    src = ORACLE_DIR / "peregrine_oracle.c"
    tmp = ORACLE_LIB.with_suffix(".so.tmp")
    _run([cc, "-O2", "-std=c11", "-fPIC", "-shared", "-pthread", "-ffp-contract=off",
          "-fno-fast-math", str(src), "-o", str(tmp), "-lm"])
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib", action="store_true", help="HIP library only")
    ap.add_argument("--oracle", action="store_true", help="oracle only")
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--incremental", action="store_true", help="recompile only out-of-date objects")
    a = ap.parse_args(argv)
    if not a.oracle:
        print("built", build_lib(a.j, a.incremental))
    if not a.lib:
        print("built", build_oracle())
    return 0


if __name__ == "__main__":
    sys.exit(main())
