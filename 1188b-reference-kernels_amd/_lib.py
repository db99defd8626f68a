"""ctypes binding of libmoe_dispatch.so (the C ABI in include/moe_dispatch.h).

The library is loaded after `import torch`, so its NEEDED libamdhip64.so.7
resolves to the HIP runtime torch already holds (one runtime, one context,
torch streams usable as hipStream_t).  There is no fallback: if the library
is missing every op raises.
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

PKG_DIR = Path(__file__).resolve().parent
# MOE_DISPATCH_LIB may name another build of the same library (e.g. a tuning variant).
LIB_PATH = Path(os.environ.get("MOE_DISPATCH_LIB", PKG_DIR / "libmoe_dispatch.so"))
HEADER_PATH = PKG_DIR.parent / "include" / "moe_dispatch.h"

# Mirrors of the header's enums.
MOE_OK = 0
MOE_ERR_INVALID_ARG = 1
MOE_ERR_SHAPE = 2
MOE_ERR_ALIGN = 3
MOE_ERR_CAPACITY = 4
MOE_ERR_WORKSPACE = 5
MOE_ERR_LAUNCH = 6

MOE_IDX_I32 = 0
MOE_IDX_I64 = 1
MOE_MAP_TOKEN_MAJOR = 0
MOE_MAP_EXPERT_MAJOR = 1
MOE_EPILOGUE_NONE = 0
MOE_EPILOGUE_SWIGLU = 1

ABI_VERSION = 13

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every function declared in the header.
SIGNATURES = {
    "moe_abi_version": (_int, []),
    "moe_status_string": (ctypes.c_char_p, [_int]),
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_topk": (_int, [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p]),
    "moe_row_id_map_workspace_size": (_sz, [_i64, _i64]),
    "moe_row_id_map": (_int, [_p, _i64, _i64, _p, _p, _p, _p, _p, _i64, _p, _sz, _p]),
    "moe_row_id_map_noalloc": (_int, [_p, _i64, _i64, _p, _p, _p, _p, _p, _i64, _p]),
    "moe_permute_workspace_size": (_sz, [_i64]),
    "moe_map_extent_workspace_size": (_sz, [_i64]),
    "moe_map_extent": (_int, [_p, _int, _i64, _p, _p, _sz, _p]),
    "moe_permute": (_int, [_p, _i64, _i64, _p, _int, _int, _i64, _p, _p, _p, _i64, _int, _p, _sz, _p]),
    "moe_unpermute": (_int, [_p, _i64, _i64, _p, _int, _int, _i64, _i64, _p, _p, _p, _p]),
    "moe_permute_bwd": (_int, [_p, _i64, _i64, _p, _p, _int, _int, _i64, _i64, _p, _p, _p, _p]),
    "moe_index_select": (_int, [_p, _i64, _i64, _p, _int, _i64, _p, _p]),
    "moe_grouped_gemm_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "moe_grouped_gemm": (_int, [_p, _i64, _i64, _p, _i64, _i64, _p, _int, _p, _p, _sz, _p]),
    "moe_permute_index": (_int, [_p, _int, _int, _i64, _i64, _p, _i64, _int, _p]),
    "moe_grouped_gemm_gather": (_int, [_p, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _int, _p, _p, _sz, _p]),
    "moe_grouped_gemm_dgrad_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "moe_grouped_gemm_wgrad_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "moe_grouped_gemm_dgrad": (_int, [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _sz, _p]),
    "moe_grouped_gemm_wgrad": (_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _sz, _p]),
    "moe_router_workspace_size": (_sz, [_i64, _i64, _i64]),
    "moe_router_logits": (_int, [_p, _i64, _i64, _p, _i64, _p, _p, _sz, _p]),
    "moe_router_topk": (_int, [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "moe_cast_bf16_to_f32": (_int, [_p, _i64, _p, _p]),
    "moe_cast_f32_to_bf16": (_int, [_p, _i64, _p, _p]),
    "moe_router_dgrad_tf32_workspace_size": (_sz, [_i64, _i64, _i64]),
    "moe_router_dgrad_tf32": (_int, [_p, _i64, _i64, _p, _i64, _p, _p, _sz, _p]),
    "moe_router_wgrad_tf32_workspace_size": (_sz, [_i64, _i64, _i64]),
    "moe_router_wgrad_tf32": (_int, [_p, _i64, _i64, _p, _i64, _p, _p, _sz, _p]),
}

_LIB = None


class MoeError(RuntimeError):
    """A non-zero moe_status_t from the C ABI."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


def header_functions() -> list[str]:
    """Function names declared in include/moe_dispatch.h."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int|size_t|char\s*\*|const char \*)\s*\**\s*(moe_\w+)\s*\(", text, re.M)))


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                "from the repository root (hipcc --offload-arch=gfx950)")
        handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.moe_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {handle.moe_abi_version()} != {ABI_VERSION}")
        _LIB = handle
    return _LIB


PROBES_PATH = PKG_DIR / "libmoe_probes.so"
_PROBES = None


def probes() -> ctypes.CDLL:
    """The measurement probes (include/moe_probes.h: moe_probe_mfma, moe_probe_stream), a library of their own
    that takes its status functions from libmoe_dispatch.so (loaded first); used by bench.py --ceilings."""
    global _PROBES
    if _PROBES is None:
        lib()
        if not PROBES_PATH.exists():
            raise RuntimeError(f"{PROBES_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        handle = ctypes.CDLL(str(PROBES_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        P, I64 = ctypes.c_void_p, ctypes.c_int64
        handle.moe_probe_mfma.restype = ctypes.c_int
        handle.moe_probe_mfma.argtypes = [I64, I64, P, P]
        handle.moe_probe_stream.restype = ctypes.c_int
        handle.moe_probe_stream.argtypes = [ctypes.c_int, P, P, I64, I64, P]
        _PROBES = handle
    return _PROBES


def call(name: str, *args) -> None:
    """Calls C ABI function `name`; raises MoeError on a non-zero status."""
    status = getattr(lib(), name)(*args)
    if status != MOE_OK:
        msg = lib().moe_last_error().decode(errors="replace")
        raise MoeError(name, status, msg)


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None or empty tensors)."""
    if t is None:
        return None
    return t.data_ptr() if t.numel() > 0 else None


def stream_handle() -> int:
    """hipStream_t of torch's current stream on the current device."""
    return torch.cuda.current_stream().cuda_stream
