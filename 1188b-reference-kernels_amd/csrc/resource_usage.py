"""Per-kernel register and scratch usage of the gfx950 device code, as a markdown table.

    python 1188b-reference-kernels_amd/csrc/resource_usage.py [source.hip ...]

Compiles each source (default: every source build.py links) for the device only, with the
compiler's kernel-resource-usage remarks, and prints one row per kernel: VGPRs, AGPRs,
scratch bytes per lane (0 = no spills) and waves per SIMD. Nothing is written to disk.
"""
from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

from build import ARCH, COMMON_FLAGS, CSRC, PROBE_SOURCES, SOURCES, _hipcc


def usage(src: str, hipcc: str) -> list[tuple[str, dict]]:
    cmd = [hipcc, *[f for f in COMMON_FLAGS if f != "-Wall"], "--cuda-device-only", "-c", str(CSRC / src),
           "-o", "/dev/null", "-Rpass-analysis=kernel-resource-usage"]
    err = subprocess.run(cmd, capture_output=True, text=True).stderr
    rows, cur, vals = [], None, {}
    for line in err.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur, vals = m.group(1), {}
            continue
        for key, pat in (("vgpr", r"VGPRs: (\d+)"), ("agpr", r"AGPRs: (\d+)"), ("scratch", r"ScratchSize \[bytes/lane\]: (\d+)"),
                         ("occ", r"Occupancy \[waves/SIMD\]: (\d+)")):
            m = re.search(pat, line)
            if m and cur:
                vals[key] = int(m.group(1))
        if "Occupancy" in line and cur:
            rows.append((cur, dict(vals)))
    return rows


def demangle(names: list[str]) -> list[str]:
    out = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True).stdout.splitlines()
    return [n.replace("moe::(anonymous namespace)::", "").split("(moe::")[0] for n in out]


def main(argv: list[str]) -> int:
    hipcc = _hipcc()
    srcs = argv or SOURCES + PROBE_SOURCES
    print(f"| source | kernel ({ARCH}) | VGPR | AGPR | scratch B/lane | waves/SIMD |")
    print("|---|---|---|---|---|---|")
    bad = 0
    for src in srcs:
        rows = usage(src, hipcc)
        for (mangled, v), name in zip(rows, demangle([r[0] for r in rows])):
            bad += v.get("scratch", 0) > 0
            print(f"| {src} | `{name}` | {v.get('vgpr')} | {v.get('agpr')} | {v.get('scratch')} | {v.get('occ')} |")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
