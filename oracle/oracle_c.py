"""numpy wrappers over liboracle.so (oracle/moe_oracle.c).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  build() compiles the C
restatement with gcc; load() builds it on first use if it is missing.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "moe_oracle.c"
LIB = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-Wall", "-o", str(LIB), str(SRC), "-lm"]
    subprocess.run(cmd, check=True)
    return LIB


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists() or LIB.stat().st_mtime < SRC.stat().st_mtime:
            build()
        _lib = ctypes.CDLL(str(LIB))
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        _lib.oracle_bf16_rne.restype = ctypes.c_uint16
        _lib.oracle_bf16_rne.argtypes = [ctypes.c_float]
        _lib.oracle_row_id_map.argtypes = [P, I64, I64, P, P]
        _lib.oracle_permute.argtypes = [P, I64, I64, P, I, I64, P, P, P, I64]
        _lib.oracle_unpermute.argtypes = [P, I64, I64, P, I, I64, I64, P, P, P]
        _lib.oracle_prob_gather.argtypes = [P, I64, P, I, I64, I64, P]
        _lib.oracle_topk.argtypes = [P, I64, I64, I64, P, P]
        _lib.oracle_index_select.argtypes = [P, I64, I64, P, I64, P]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """uint16 bf16 bits of fp32 values (element by element through the C routine)."""
    f = load().oracle_bf16_rne
    flat = _c(x, np.float32).ravel()
    return np.array([f(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(x))


def row_id_map(mask: np.ndarray):
    """(row_tm int64 [T,E], offsets int64 [E+1]) of a [T,E] 0/1 mask."""
    m = _c(mask, np.uint8)
    T, E = m.shape
    row = np.empty((T, E), np.int64)
    offs = np.empty(E + 1, np.int64)
    load().oracle_row_id_map(_p(m), T, E, _p(row), _p(offs))
    return row, offs


def permute(x: np.ndarray, row_map: np.ndarray, num_out: int, probs: np.ndarray | None = None,
            expert_major: bool = False):
    """(out, pp) for x [T, ...] (any dtype, copied as bytes) and an int64 map."""
    xc = np.ascontiguousarray(x)
    T = xc.shape[0]
    row_bytes = xc.nbytes // T if T else 0
    m = _c(row_map, np.int64)
    E = m.shape[0] if expert_major else m.shape[1]
    out = np.empty((num_out,) + xc.shape[1:], xc.dtype)
    pp = np.empty(num_out, np.float32) if probs is not None else None
    pr = _c(probs, np.float32) if probs is not None else None
    load().oracle_permute(_p(xc.view(np.uint8)), T, row_bytes, _p(m), int(expert_major), E, _p(pr),
                          _p(out.view(np.uint8)), _p(pp), num_out)
    return out, pp


def unpermute(pin_bits: np.ndarray, row_map: np.ndarray, probs: np.ndarray | None = None,
              expert_major: bool = True):
    """(out bf16 bits uint16 [T,H], acc fp32 [T,H]) for pin given as uint16 bf16 bits."""
    pin = _c(pin_bits, np.uint16)
    R, H = pin.shape
    m = _c(row_map, np.int64)
    E, T = (m.shape if expert_major else m.shape[::-1])
    out = np.empty((T, H), np.uint16)
    acc = np.empty((T, H), np.float32)
    pr = _c(probs, np.float32) if probs is not None else None
    load().oracle_unpermute(_p(pin), R, H, _p(m), int(expert_major), E, T, _p(pr), _p(out), _p(acc))
    return out, acc


def prob_gather(dpp: np.ndarray, row_map: np.ndarray, expert_major: bool = True) -> np.ndarray:
    d = _c(dpp, np.float32)
    m = _c(row_map, np.int64)
    E, T = (m.shape if expert_major else m.shape[::-1])
    out = np.empty((T, E), np.float32)
    load().oracle_prob_gather(_p(d), d.shape[0], _p(m), int(expert_major), E, T, _p(out))
    return out


def topk(x: np.ndarray, k: int):
    xc = _c(x, np.float32)
    T, E = xc.shape
    values = np.empty((T, k), np.float32)
    indices = np.empty((T, k), np.int64)
    load().oracle_topk(_p(xc), T, E, k, _p(values), _p(indices))
    return values, indices


def index_select(src: np.ndarray, index: np.ndarray) -> np.ndarray:
    s = np.ascontiguousarray(src)
    rows = s.shape[0]
    row_bytes = s.nbytes // rows if rows else 0
    idx = _c(index, np.int64)
    out = np.empty((idx.shape[0],) + s.shape[1:], s.dtype)
    load().oracle_index_select(_p(s.view(np.uint8)), rows, row_bytes, _p(idx), idx.shape[0], _p(out.view(np.uint8)))
    return out
