"""Builds libturbopolar_hip.so (the C-ABI HIP library) in-tree for gfx950.

Run as ``python -m turbopolar_amd.build`` or through ``__graft_entry__.build()``.
Every call recompiles.  Objects go to ``turbopolar_amd/_build/`` and the shared
library to ``turbopolar_amd/libturbopolar_hip.so``.  A second library,
``libturbopolar_hip_timeline.so`` (the measurement library), is the same code
with the decode kernel's phase stamps compiled in (``-DTP_TIMELINE``) plus the
streaming-read probe of ``tp_measure.hip``; only ``bench.py --workload
timeline`` and ``--workload stream`` load it.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libturbopolar_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
TIMELINE_LIB_PATH = PKG_DIR / "libturbopolar_hip_timeline.so"
ARCH = os.environ.get("TP_OFFLOAD_ARCH", "gfx950")

SOURCES = ["tp_api.hip", "tp_encode.hip", "tp_attention.hip", "tp_decode.hip", "tp_append.hip", "tp_qjl.hip"]
MEASURE_SOURCES = ["tp_measure.hip"]  # measurement library only

# -ffp-contract=off and correctly rounded fp32 divide/sqrt are required for the
# encoder's bit-exact fp16 rules (SOURCE_FLAGS below relaxes contraction for
# the attention kernels only); packed fp32 VALU ops are disabled.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{REPO_DIR / 'include'}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the TurboPolar HIP library cannot be built")


# Per-source flags after the common ones.  The attention kernels compare with
# the reference within a tolerance, so their fp32 multiply-adds may contract
# into FMAs (fewer instructions and shorter dependency chains in the softmax,
# the wave fold and the split-K combine: 32k 18.29 -> 18.03 us, 131k 51.42 ->
# 51.10 us, paired); the decoded code angle keeps the reference's separate
# roundings by its own pragma (code_angle, tp_common.h).  Every other source
# stays uncontracted for the encoder's and the page decoder's bit-exact rules.
SOURCE_FLAGS = {"tp_attention.hip": ["-ffp-contract=fast-honor-pragmas"]}


def _compile(src: Path, obj: Path, defines=()) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), *[f"-D{d}" for d in defines], "-c", str(src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = True) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    objs = []
    timeline_obj = BUILD_DIR / "tp_attention_timeline.o"
    measure_objs = [BUILD_DIR / (Path(n).stem + ".o") for n in MEASURE_SOURCES]
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        futs = []
        for name in SOURCES:
            obj = BUILD_DIR / (Path(name).stem + ".o")
            objs.append(obj)
            futs.append(ex.submit(_compile, CSRC / name, obj))
        futs.append(ex.submit(_compile, CSRC / "tp_attention.hip", timeline_obj, ("TP_TIMELINE",)))
        for name, obj in zip(MEASURE_SOURCES, measure_objs):
            futs.append(ex.submit(_compile, CSRC / name, obj))
        for f in futs:
            f.result()
    _link(objs, LIB_PATH)
    _link([timeline_obj if o.stem == "tp_attention" else o for o in objs] + measure_objs, TIMELINE_LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


def _link(objs, out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)


if __name__ == "__main__":
    build()
    sys.exit(0)
