"""Build libdexter_gfx950.so from the HIP sources in this directory.

Each ``*.hip`` file is compiled for gfx950 in parallel, then linked into one
shared library next to the Python package (``dexter_amd/libdexter_gfx950.so``),
where ``dexter_amd.ops.gfx950._lib`` loads it. Usage::

    python dexter-labs_amd/csrc/build.py [--jobs N] [--verbose] [--timeline]

``--timeline`` builds the measurement variant instead: the same sources with
``-DDX_TIMELINE`` (per-workgroup phase stamps in the decode and merge kernels,
read back through ``dx_timeline_read``) into ``libdexter_gfx950_timeline.so``
beside the product library, which it leaves alone (``bench.py --timeline``).

Flags: ``-O3``; ``-Xclang -target-feature -Xclang -packed-fp32-ops`` keeps the
compiler from emitting packed fp32 VALU instructions (the host pass warns that
it does not know the feature; that is harmless); ``-mllvm
-amdgpu-mfma-vgpr-form=1`` keeps MFMA accumulators in ordinary VGPRs.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent / "dexter_amd"
LIB_NAME = "libdexter_gfx950.so"
TIMELINE_LIB_NAME = "libdexter_gfx950_timeline.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: kernels with inline assembly
    # otherwise get them in AGPRs, and every vector op on an accumulator
    # (the softmax rescale) then costs a copy out and back.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build")
    return path


def _compile(src: Path, obj: Path, verbose: bool, defines: tuple[str, ...] = ()) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, *(f"-D{d}" for d in defines), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False, timeline: bool = False) -> Path:
    sources = sorted(HERE.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {HERE}")
    out = PKG / (TIMELINE_LIB_NAME if timeline else LIB_NAME)
    defines = ("DX_TIMELINE",) if timeline else ()
    with tempfile.TemporaryDirectory(prefix="dx_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in sources]
        workers = jobs or min(len(sources), os.cpu_count() or 4, 8)
        with cf.ThreadPoolExecutor(max_workers=workers) as ex:
            futs = [ex.submit(_compile, s, o, verbose, defines) for s, o in zip(sources, objs)]
            for f in futs:
                f.result()
        tmp_out = Path(tmp) / out.name
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp_out),
               *map(str, objs)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stderr}")
        # Replace atomically so a running process never maps a half-written file.
        staged = out.with_suffix(".so.tmp")
        shutil.copyfile(tmp_out, staged)
        os.replace(staged, out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--timeline", action="store_true",
                    help="build the phase-stamp variant (libdexter_gfx950_timeline.so)")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose, args.timeline))
