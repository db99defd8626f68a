"""CPU: the grouped GEMM kernels keep every value in registers (no scratch spills).

The one-wavefront-per-SIMD GEMM kernels hold 128 or 256 fp32 accumulators in AGPRs and a K
step of operand fragments in VGPRs; the ping-pong kernels (forward and backward, two
wavefronts per SIMD) hold their 128 accumulators and fragments in the 256 registers a
wavefront gets at that occupancy, and so do the short-group kernels (wgrad sweep, 128-row
forward tiles) and the tf32 router dgrad's 128 x 128 tiles with their smaller tiles. A spill puts scratch loads (which wait on the vector-memory counter, and so on
the LDS DMA in flight) inside the MFMA stream. The compiler's kernel-resource-usage remarks
for the device code must report 0 scratch bytes per lane for every instantiation.
"""
from __future__ import annotations

import shutil
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "1188b-reference-kernels_amd" / "csrc"
sys.path.insert(0, str(CSRC))

pytestmark = pytest.mark.skipif(not (Path("/opt/rocm/bin/hipcc").exists() or shutil.which("hipcc")),
                                reason="needs hipcc (device compile only, no GPU)")


def test_gemm_kernels_do_not_spill():
    import resource_usage as ru
    hipcc = ru._hipcc()
    srcs = ["grouped_gemm.hip", "grouped_gemm_bwd.hip"]
    with ThreadPoolExecutor(max_workers=2) as ex:
        results = list(ex.map(lambda s: ru.usage(s, hipcc), srcs))
    rows = [r for res in results for r in res]
    assert len(rows) >= 15, rows
    spilled = [(name, v) for name, v in rows if v.get("scratch", 0) != 0]
    assert not spilled, spilled
    pingpong = [(name, v) for name, v in rows if "_pp_kernel" in name]
    # forward: 4 epilogue/gather forms, each with and without the 128-row tail tiles; backward: dgrad
    # with and without them, wgrad, ordered wgrad
    assert len(pingpong) == 12, pingpong
    assert all(v.get("occ") == 2 and v.get("vgpr", 0) + v.get("agpr", 0) <= 256 for _, v in pingpong), pingpong
    # the short-group wgrad sweep: two wavefronts per SIMD as well (both orientations)
    sweep = [(name, v) for name, v in rows if "_sweep_kernel" in name]
    assert len(sweep) == 2 and all(v.get("occ") == 2 and v.get("vgpr", 0) + v.get("agpr", 0) <= 256 for _, v in sweep), sweep
    # the short-group forward kernel (128-row tiles of 128, 160 and 192 columns, loading wavefronts): the same
    fwd128 = [(name, v) for name, v in rows if "_fwd128_kernel" in name]
    assert len(fwd128) == 3 and all(v.get("occ") == 2 and v.get("vgpr", 0) + v.get("agpr", 0) <= 256 for _, v in fwd128), fwd128
    # the tf32 router dgrad's 128 x 128 tiles: two workgroups per CU, its 64 accumulators in VGPRs
    dg128 = [(name, v) for name, v in rows if "dgrad128_kernel" in name and "ELi128ELi2E" in name]
    assert len(dg128) == 1 and all(v.get("occ") == 2 and v.get("vgpr", 0) + v.get("agpr", 0) <= 256 for _, v in dg128), dg128
    assert all(v.get("agpr") in (128, 256) for name, v in rows if "gemm" in name and "kernel" in name and "sum_planes" not in name
               and "split" not in name and "tails_init" not in name and "_pp_kernel" not in name
               and "_sweep_kernel" not in name and "_fwd128_kernel" not in name and (name, v) not in dg128)
