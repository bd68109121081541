"""Builds libtnpa.so (HIP kernels + C ABI) for gfx950 in-tree with hipcc.

    python -m tensor_train_ing_amd.build [--jobs N] [--incremental]

Kernel instantiations are split into one translation unit per (element type, key head dim) so they compile in
parallel; objects go to tensor_train_ing_amd/_build/, the library to tensor_train_ing_amd/libtnpa.so.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtnpa.so"
ARCH = "gfx950"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# Packed FP32 VALU ops are disabled for all device code (known-bad on this machine pool).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-variable",
          "-Wno-unused-but-set-variable", "-Wno-unknown-pragmas", *DEVICE_FLAGS]

ELEMENT_TYPES = {"bf16": "__bf16", "f16": "_Float16", "f32": "float"}
HEAD_DIMS = (16, 32, 64, 128, 256)
HEADERS = ("tnpa_device.hpp", "tnpa_kernels.hpp", "tnpa_params.hpp", "tnpa_internal.h", "tnpa_error.hpp")


def _units():
    """Translation units, longest compiles first (larger head dims, fp32 first; 40-140 s each) so the parallel
    build's last unit to start is a short one."""
    units = []
    for dk in sorted(HEAD_DIMS, reverse=True):
        for tag in ("f32", "bf16", "f16"):
            units.append((f"tnpa_inst_{tag}_dk{dk}", CSRC / "tnpa_inst.hip",
                          [f"-DTNPA_INST_T={ELEMENT_TYPES[tag]}", f"-DTNPA_INST_DK={dk}"]))
    return units + [("tnpa_api", CSRC / "tnpa_api.hip", []), ("tnce", CSRC / "tnce.hip", [])]


def _stale(obj: Path, src: Path) -> bool:
    if not obj.exists():
        return True
    deps = [src, *(CSRC / h for h in HEADERS), *(PKG.parent / "include").glob("*.h"), Path(__file__)]
    return any(d.stat().st_mtime > obj.stat().st_mtime for d in deps)


def _compile(name: str, src: Path, defs: list[str]) -> tuple[str, int, str]:
    obj = BUILD / f"{name}.o"
    cmd = [HIPCC, *COMMON, *defs, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    return name, r.returncode, msg


def build(jobs: int | None = None, incremental: bool = False, verbose: bool = False) -> Path:
    """Compiles every translation unit (all of them unless `incremental`) and links libtnpa.so."""
    BUILD.mkdir(exist_ok=True)
    units = _units()
    todo = [u for u in units if not incremental or _stale(BUILD / f"{u[0]}.o", u[1])]
    jobs = jobs or min(16, os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(lambda u: _compile(*u), todo))
    failed = [(n, m) for n, rc, m in results if rc != 0]
    for n, rc, m in results:
        if verbose and m.strip():
            print(f"[{n}]\n{m}", file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(f"[{n}]\n{m}" for n, m in failed))
    objs = [str(BUILD / f"{u[0]}.o") for u in units]
    tmp = LIB.with_suffix(".so.tmp")
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--incremental", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args(argv)
    print(build(a.jobs, a.incremental, a.verbose))


if __name__ == "__main__":
    main()
