"""Build liblik_hip.so (the gfx950 MaxSim engine) from csrc/ with hipcc.

Usage: python build_lib.py [--jobs N]

Each csrc/*.hip file is compiled to an object in parallel, then linked into
late_interaction_kernels/_lib/liblik_hip.so, in-tree so that it ships with the
package. Always rebuilds (a build is a few tens of seconds).
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
OUT_DIR = HERE / "late_interaction_kernels" / "_lib"
LIB_NAME = "liblik_hip.so"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


# Packed-FP32 VALU ops are disabled for all device code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _compile(src: Path, obj: Path, extra: list[str]) -> tuple[Path, str]:
    cmd = [hipcc(), *DEVICE_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(
        line
        for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line  # host pass does not know the feature; harmless
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msg}")
    return obj, msg


def build(jobs: int | None = None, verbose: bool = False, out_dir: Path | None = None,
          extra_flags: list[str] | None = None, incremental: bool = False) -> Path:
    """Compile and link; ``extra_flags`` (e.g. -DLIK_PROF) and ``out_dir`` are for
    instrumented side builds that must not replace the product library.
    ``incremental`` recompiles only sources newer than their object (or
    older than the newest header); the default rebuilds everything."""
    out_dir = Path(out_dir) if out_dir else OUT_DIR
    out_dir.mkdir(parents=True, exist_ok=True)
    obj_dir = HERE / ("_build" if not extra_flags else "_build_extra")
    obj_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources in {CSRC}")
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    newest_hdr = max([h.stat().st_mtime for h in CSRC.glob("*.h")] + [h.stat().st_mtime for h in INCLUDE.glob("*.h")])
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = []
        for s in sources:
            o = obj_dir / (s.stem + ".o")
            if incremental and o.exists() and o.stat().st_mtime > max(s.stat().st_mtime, newest_hdr):
                objs.append(o)
                continue
            futs.append(ex.submit(_compile, s, o, extra_flags or []))
        for f in futs:
            obj, msg = f.result()
            objs.append(obj)
            if verbose and msg.strip():
                print(msg, file=sys.stderr)
    out = out_dir / LIB_NAME
    tmp = out_dir / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, out)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--out-dir", default=None, help="side build directory (instrumented builds)")
    ap.add_argument("--define", action="append", default=[], help="extra -D macro, e.g. LIK_PROF")
    ap.add_argument("--incremental", action="store_true", help="recompile only out-of-date objects")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose, args.out_dir, [f"-D{d}" for d in args.define], args.incremental))


if __name__ == "__main__":
    main()
