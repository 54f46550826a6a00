"""Builds libllamazero_hip.so for gfx950 from the .hip sources in this folder.

Each source is compiled to an object under csrc/_build/ (in parallel), then
linked into ../lzhip/libllamazero_hip.so.  Usage:

    python csrc/build.py [--jobs N] [--arch gfx950]
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
PKG = HERE.parent
OUT_LIB = PKG / "lzhip" / "libllamazero_hip.so"

SOURCES = [
    "runtime.hip",
    "dropout.hip",
    "optim.hip",
    "norm.hip",
    "rope.hip",
    "swiglu.hip",
    "embed.hip",
    "ce.hip",
    "transpose.hip",
    "gemm.hip",
    "gemm_f32.hip",
    "attn.hip",
]

COMMON_FLAGS = [
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-fvisibility=hidden",
    # packed fp32 arithmetic is kept out of the generated code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


# Per-source extra flags.  RoPE reproduces the reference's separately rounded
# products and sum, so multiply-add contraction is off for that file.
EXTRA_FLAGS = {
    "rope.hip": ["-ffp-contract=off"],
}


def find_hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(hipcc: str, arch: str, src: Path, obj: Path) -> tuple[Path, int, str]:
    cmd = [hipcc, f"--offload-arch={arch}", *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o",
           str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 feature name; drop that notice
    msgs = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if "packed-fp32-ops" not in line
    )
    return obj, proc.returncode, msgs


def build(arch: str = "gfx950", jobs: int | None = None, verbose: bool = False) -> Path:
    hipcc = find_hipcc()
    build_dir = HERE / "_build"
    build_dir.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 4)))
    objs = []
    failures = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = [pool.submit(_compile, hipcc, arch, HERE / s, build_dir / (Path(s).stem + ".o")) for s in SOURCES]
        for fut in futs:
            obj, rc, msgs = fut.result()
            if rc != 0:
                failures.append(f"{obj.name}:\n{msgs}")
            else:
                if msgs.strip() and verbose:
                    print(msgs)
                objs.append(obj)
    if failures:
        raise RuntimeError("HIP compilation failed:\n" + "\n".join(failures))
    tmp = OUT_LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={arch}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OUT_LIB)
    return OUT_LIB


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--arch", default="gfx950")
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    out = build(arch=args.arch, jobs=args.jobs, verbose=args.verbose)
    print(f"built {out}")


if __name__ == "__main__":
    sys.exit(main())
