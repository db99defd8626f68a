"""CPU: the public headers are valid C99 and the library links and answers from a plain C program.

tests/c_consumer.c includes include/moe_dispatch.h and include/moe_probes.h, is compiled by gcc with
-std=c99 -Wall -Wextra -Werror -pedantic, links libmoe_dispatch.so and libmoe_probes.so, and calls entry points whose argument
checks fail before any HIP call (the status codes the headers document), so no GPU is needed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

from conftest import load_pkg

REPO = Path(__file__).resolve().parents[1]

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")


def test_c99_consumer_compiles_links_and_runs(tmp_path):
    pkg = load_pkg()
    lib = Path(pkg._lib.LIB_PATH)
    exe = tmp_path / "c_consumer"
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{REPO / 'include'}",
           str(REPO / "tests" / "c_consumer.c"), "-o", str(exe), str(lib), str(pkg._lib.PROBES_PATH),
           f"-Wl,-rpath,{lib.parent}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, env={**os.environ, "HIP_VISIBLE_DEVICES": ""},
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "unexpected" not in r.stdout
