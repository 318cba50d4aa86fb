"""Build libgstar_evict.so (gfx950) from csrc/*.hip with hipcc.

Every HIP source is compiled for gfx950 only, with packed-FP32 instructions
disabled, then linked into one shared library next to the Python package, so
it ships with the source tree. Run: python cache-eviction_amd/build.py
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "gstar_evict" / "libgstar_evict.so"
BUILD = HERE.parent / "_build"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{HERE.parent / 'include'}",
]


# Per-source additions. prefill.hip: keep MFMA results in ordinary VGPRs. With the compiler's
# own choice the pass-2 tile kept them in accumulation registers and paid one v_accvgpr_read per
# logit (a fifth vector issue slot beside the FMA, the exp2 and the add); forcing the VGPR form
# removed them without spills (measured: 290 -> 302 TFLOP/s at the 79,720-token prompt).
SOURCE_FLAGS = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build gstar_evict")
    return path


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (proc.stderr or "").splitlines() if noise not in l)
    if proc.returncode:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile every csrc/*.hip and link libgstar_evict.so; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [BUILD / (s.stem + ".o") for s in sources]
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(sources)))) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], verbose), zip(sources, objs)))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
