"""Build libqmoe.so (the gfx950 kernels behind include/qmoe.h) with hipcc.

Each ``csrc/*.hip`` file is compiled to an object in parallel, then linked into
``titan_amd/lib/libqmoe.so``; ``csrc/peaks/peaks.hip`` (the bench's
measured-ceiling probes, include/qmoe_peaks.h) becomes
``titan_amd/lib/libqmoe_peaks.so``; and ``titan_amd/lib/libqmoe_stamps.so`` is
libqmoe.so with the decode GEMV's per-phase timestamps and the bf16 grouped
GEMM's per-unit timestamps compiled in (QMOE_QMV_STAMPS, QMOE_GEMM_STAMPS,
read by ``bench.py --decode-phases`` and ``--gemm-units``), a measurement
build that nothing else loads.  The libraries land in-tree so that they travel with
the source tree; nothing is installed anywhere else.

    python -m titan_amd.build            # build (always recompiles)
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
BUILD = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libqmoe.so"
PEAKS_SRC = CSRC / "peaks" / "peaks.hip"
PEAKS_LIB = LIB_DIR / "libqmoe_peaks.so"
STAMPS_LIB = LIB_DIR / "libqmoe_stamps.so"
ARCH = os.environ.get("QMOE_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: hipcc must not form v_pk_{add,mul,fma}_f32 on its own.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


# Per-source extra flags.  int8.hip: MFMA results in VGPRs, so the per-group
# rescale reads them without a v_accvgpr_read per element.
FILE_FLAGS = {"int8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libqmoe.so)")


def _compile(src: Path, variant: str = "", defines=()) -> Path:
    obj = BUILD / (src.stem + variant + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), *(f"-D{d}" for d in defines), f"-I{INCLUDE}",
           f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


def _link(objs, lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources) + 1, max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        fut_peaks = ex.submit(_compile, PEAKS_SRC)
        stamped = {"qmv": ex.submit(_compile, CSRC / "qmv.hip", "_stamps", ("QMOE_QMV_STAMPS",)),
                   "gemm_bf16": ex.submit(_compile, CSRC / "gemm_bf16.hip", "_stamps", ("QMOE_GEMM_STAMPS",))}
        objs = list(ex.map(_compile, sources))
        peaks_obj = fut_peaks.result()
        stamped = {k: f.result() for k, f in stamped.items()}
    _link(objs, LIB)
    _link([peaks_obj], PEAKS_LIB)
    _link([stamped.get(o.stem, o) for o in objs], STAMPS_LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources, {PEAKS_LIB} and {STAMPS_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
