"""Builds libmoe_dispatch.so (gfx950) from the HIP sources in this directory.

    python csrc/build.py            # from the package directory, or
    python -c "import __graft_entry__ as g; g.build()"   # from the repo root

Each .hip file compiles to an object under csrc/_build/ (in parallel), then the
objects link into <package>/libmoe_dispatch.so next to the Python loader. The
measurement probes (probes.hip: bench.py --ceilings) link into a library of
their own, <package>/libmoe_probes.so, which takes the status functions from
libmoe_dispatch.so.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
REPO = PKG.parent
LIB = PKG / "libmoe_dispatch.so"
PROBE_LIB = PKG / "libmoe_probes.so"
BUILD = CSRC / "_build"

SOURCES = [
    "status.hip",
    "topk.hip",
    "row_id_map.hip",
    "permute.hip",
    "unpermute.hip",
    "index_select.hip",
    "grouped_gemm.hip",
    "grouped_gemm_bwd.hip",
    "router.hip",
    "cast.hip",
]
PROBE_SOURCES = ["probes.hip"]

ARCH = os.environ.get("MOE_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # Packed fp32 ops are kept out of the generated code (v_pk_* fp32 forms).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{REPO / 'include'}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (looked at $HIPCC, /opt/rocm/bin/hipcc, PATH)")


def _compile(src: str, hipcc: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [hipcc, *COMMON_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # The host pass warns that it does not know the packed-fp32 feature; drop that noise.
    noise = "is not a recognized feature for this target"
    for line in (r.stdout + r.stderr).splitlines():
        if line.strip() and noise not in line:
            print(f"[{src}] {line}", file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> Path:
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    every = SOURCES + PROBE_SOURCES
    jobs = jobs or min(len(every), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = dict(zip(every, ex.map(lambda s: _compile(s, hipcc), every)))
    # --no-undefined: a kernel whose host launch stub was not emitted fails here, not at load time.
    _link(hipcc, LIB, [objs[s] for s in SOURCES], [])
    _link(hipcc, PROBE_LIB, [objs[s] for s in PROBE_SOURCES],
          [f"-L{PKG}", f"-l:{LIB.name}", "-Wl,-rpath,$ORIGIN"])
    return LIB


def _link(hipcc: str, out: Path, objs: list, extra: list) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", str(tmp),
           *map(str, objs), *extra]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)


if __name__ == "__main__":
    print(build())
