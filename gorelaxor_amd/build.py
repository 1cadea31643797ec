"""Build libgrx.so (gfx950) in-tree with hipcc.

    python -m gorelaxor_amd.build

The library lands next to this file (gorelaxor_amd/libgrx.so) so that it
travels with the source tree; nothing is installed.
"""
from __future__ import annotations

import glob
import os
import re
import shutil
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libgrx.so")
BUILD_DIR = os.path.join(PKG, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=off: a product followed by a sum is never fused unless the
# source asks for it (__fmaf_rn), which parity with the reference needs.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 are generated.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    "-I" + os.path.join(ROOT, "include"),
]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _compile_one(src: str, build_dir: str, extra: list[str]) -> tuple[str, subprocess.Popen]:
    obj = os.path.join(build_dir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *extra, "-c", src, "-o", obj]
    p = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    return obj, p


def _local_includes(path: str, seen: set[str] | None = None) -> set[str]:
    """The in-tree headers `path` includes with #include "...", transitively."""
    seen = set() if seen is None else seen
    try:
        text = open(path).read()
    except OSError:
        return seen
    for name in re.findall(r'^\s*#\s*include\s+"([^"]+)"', text, re.M):
        for d in (os.path.dirname(path), CSRC, os.path.join(ROOT, "include")):
            h = os.path.join(d, name)
            if os.path.exists(h) and h not in seen:
                seen.add(h)
                _local_includes(h, seen)
                break
    return seen


def _stale(src: str, build_dir: str) -> bool:
    obj = os.path.join(build_dir, os.path.basename(src) + ".o")
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(f) > t for f in [src, *_local_includes(src)])


def build(verbose: bool = True, out: str = LIB, defines: list[str] | None = None, incremental: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link gorelaxor_amd/libgrx.so
    (or `out`, with extra -D `defines`, for a variant build).  incremental:
    recompile only sources newer than their objects (or with a newer
    header), for development; the default rebuilds everything."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_dir = BUILD_DIR if out == LIB else os.path.join(os.path.dirname(os.path.abspath(out)), "_build")
    os.makedirs(build_dir, exist_ok=True)
    extra = [f"-D{d}" for d in (defines or [])]
    t0 = time.time()
    todo = [s for s in sources() if not incremental or _stale(s, build_dir)]
    jobs = [_compile_one(s, build_dir, extra) for s in todo]
    objs = [os.path.join(build_dir, os.path.basename(s) + ".o") for s in sources()]
    failed = []
    for obj, p in jobs:
        text, _ = p.communicate()
        lines = [l for l in text.splitlines() if "packed-fp32-ops" not in l]
        if p.returncode != 0:
            failed.append((obj, "\n".join(lines)))
        elif verbose and lines:
            print("\n".join(lines), file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n\n".join(f"{o}:\n{t}" for o, t in failed))
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    shutil.move(tmp, out)
    if verbose:
        print(f"built {out} in {time.time() - t0:.1f}s", file=sys.stderr)
    return out


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv[1:])
