"""Build liblcuda_hip.so: every csrc/*.hip compiled for gfx950 and linked into
one shared library under llm_cuda/_native/.

Usage:  python llm-cuda_amd/build.py [--jobs N] [--verbose]

The library exports only the C ABI declared in include/lcuda.h. It links
against the system HIP runtime (libamdhip64.so.7); when torch has already
loaded its own copy of that soname, the dynamic loader reuses it, so kernels
launch on the runtime that owns torch's streams.
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
BUILD_DIR = PKG_ROOT / "_build"
LIB_PATH = PKG_ROOT / "llm_cuda" / "_native" / "liblcuda_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    # Packed FP32 VALU forms are kept out of every kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{REPO_ROOT / 'include'}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # The host pass warns that it does not know the packed-fp32 feature; drop that noise.
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    ).strip()
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out and verbose:
        print(out, flush=True)


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile all kernels and link the shared library; returns its path."""
    hipcc = _hipcc()
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_PATH.parent.mkdir(parents=True, exist_ok=True)
    objects = [BUILD_DIR / (src.stem + ".o") for src in sources]
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)

    def compile_one(pair):
        src, obj = pair
        _run([hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)], verbose)
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(compile_one, zip(sources, objects)))

    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run(
        [
            hipcc,
            f"--offload-arch={ARCH}",
            "-shared",
            "-fPIC",
            "-o",
            str(tmp),
            *map(str, objects),
            "-Wl,-rpath,/opt/rocm/lib",
        ],
        verbose,
    )
    # A kernel whose host-side launch stub was not emitted links fine but fails
    # at load time; catch it here.
    nm = shutil.which("nm")
    if nm:
        undef = subprocess.run([nm, "-D", "--undefined-only", str(tmp)], capture_output=True,
                               text=True).stdout
        stubs = [ln.split()[-1] for ln in undef.splitlines() if "__device_stub__" in ln]
        if stubs:
            raise RuntimeError(f"undefined kernel launch stubs in {tmp.name}: {stubs}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--jobs", type=int, default=None)
    parser.add_argument("--verbose", action="store_true")
    args = parser.parse_args()
    path = build(jobs=args.jobs, verbose=args.verbose)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
