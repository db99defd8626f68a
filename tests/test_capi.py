"""CPU checks of the C ABI library: it loads, exports every declared symbol, and
rejects bad arguments before any HIP call (no GPU needed)."""
from __future__ import annotations

import ctypes
import re

import pytest
import torch

from conftest import load_pkg

pkg = load_pkg()
L = pkg._lib


def test_library_loads_and_exports_header_symbols():
    lib = L.lib()
    declared = L.header_functions()
    assert len(declared) == len(L.SIGNATURES) == 31
    assert set(declared) == set(L.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.moe_abi_version() == L.ABI_VERSION


def test_header_enums_match_python_mirror():
    text = L.HEADER_PATH.read_text()
    for name in ["MOE_OK", "MOE_ERR_INVALID_ARG", "MOE_ERR_SHAPE", "MOE_ERR_ALIGN", "MOE_ERR_CAPACITY",
                 "MOE_ERR_WORKSPACE", "MOE_ERR_LAUNCH", "MOE_IDX_I32", "MOE_IDX_I64", "MOE_MAP_TOKEN_MAJOR",
                 "MOE_MAP_EXPERT_MAJOR", "MOE_EPILOGUE_NONE", "MOE_EPILOGUE_SWIGLU"]:
        m = re.search(rf"\b{name}\s*=\s*(\d+)", text)
        assert m and int(m.group(1)) == getattr(L, name), name


def _status(name, *args):
    lib = L.lib()
    st = getattr(lib, name)(*args)
    return st, lib.moe_last_error().decode()


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


@pytest.mark.parametrize("name,args,code,needle", [
    ("moe_permute", (None, -1, 8, None, 1, 0, 4, None, None, None, 0, 0, None, 0, None), L.MOE_ERR_SHAPE, "negative"),
    ("moe_permute", (FAKE, 4, 8, FAKE, 7, 0, 4, None, FAKE, None, 16, 0, None, 0, None), L.MOE_ERR_INVALID_ARG, "idx_dtype"),
    ("moe_permute", (FAKE, 4, 8, FAKE, 1, 3, 4, None, FAKE, None, 16, 0, None, 0, None), L.MOE_ERR_INVALID_ARG, "map_layout"),
    ("moe_permute", (None, 4, 8, FAKE, 1, 0, 4, None, FAKE, None, 16, 0, None, 0, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_permute", (FAKE, 4, 8, FAKE, 1, 0, 4, None, FAKE, FAKE, 16, 0, None, 0, None), L.MOE_ERR_INVALID_ARG, "without probs"),
    ("moe_permute", (FAKE, 4, 8, FAKE, 1, 0, 4, None, FAKE, None, 16, 1, None, 0, None), L.MOE_ERR_WORKSPACE, "workspace"),
    ("moe_unpermute", (FAKE, 8, 8, FAKE, 1, 1, 5000, 4, None, FAKE, None, None), L.MOE_ERR_CAPACITY, "4096"),
    ("moe_unpermute", (FAKE, 8, -8, FAKE, 1, 1, 4, 4, None, FAKE, None, None), L.MOE_ERR_SHAPE, "negative"),
    ("moe_permute_bwd", (FAKE, 8, 8, None, FAKE, 1, 1, 4, 4, FAKE, FAKE, None, None), L.MOE_ERR_INVALID_ARG, "dpp"),
    ("moe_row_id_map", (FAKE, 16, 8000, None, None, None, None, None, 0, None, 0, None), L.MOE_ERR_CAPACITY, "4096"),
    ("moe_row_id_map", (FAKE, 16, 8, None, None, None, None, None, 0, None, 0, None), L.MOE_ERR_WORKSPACE, "workspace"),
    ("moe_row_id_map", (None, 16, 8, None, None, None, None, None, 0, FAKE, 1 << 20, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_row_id_map_noalloc", (FAKE, 1 << 20, 4096, None, None, None, None, None, 0, None), L.MOE_ERR_CAPACITY, "2^31"),
    ("moe_row_id_map_noalloc", (FAKE, 16, 8000, None, None, None, None, None, 0, None), L.MOE_ERR_CAPACITY, "4096"),
    ("moe_row_id_map_noalloc", (FAKE, -16, 8, None, None, None, None, None, 0, None), L.MOE_ERR_SHAPE, "negative"),
    ("moe_row_id_map_noalloc", (None, 16, 8, None, None, None, None, None, 0, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_row_id_map", (FAKE, 16, 8, None, None, None, None, FAKE, -1, FAKE, 1 << 20, None), L.MOE_ERR_SHAPE, "src_capacity"),
    ("moe_topk", (FAKE, 4, 16, 0, FAKE, FAKE, None, None, None), L.MOE_ERR_SHAPE, "out of range"),
    ("moe_topk", (FAKE, 4, 16, 17, FAKE, FAKE, None, None, None), L.MOE_ERR_SHAPE, "out of range"),
    ("moe_topk", (FAKE, 4, 2048, 8, FAKE, FAKE, None, None, None), L.MOE_ERR_CAPACITY, "1024"),
    ("moe_topk", (FAKE, 4, 128, 65, FAKE, FAKE, None, None, None), L.MOE_ERR_CAPACITY, "64"),
    ("moe_index_select", (FAKE, 4, 8, FAKE, 5, 2, FAKE, None), L.MOE_ERR_INVALID_ARG, "idx_dtype"),
    ("moe_index_select", (FAKE, 4, 8, None, 0, 2, FAKE, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_grouped_gemm", (FAKE, 4, 12, FAKE, 1, 8, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "multiple of 8"),
    ("moe_grouped_gemm", (FAKE, 4, 16, FAKE, 0, 8, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "G=0"),
    ("moe_grouped_gemm", (FAKE, 4, 16, FAKE, 1, 7, FAKE, 1, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "even N"),
    ("moe_grouped_gemm", (FAKE, 4, 16, FAKE, 1, 8, FAKE, 9, FAKE, None, 0, None), L.MOE_ERR_INVALID_ARG, "epilogue"),
    ("moe_grouped_gemm", (FAKE, 4, 16, FAKE, 1, 8, None, 0, FAKE, None, 0, None), L.MOE_ERR_INVALID_ARG, "group_offsets"),
    ("moe_grouped_gemm", (ctypes.c_void_p(0x1002), 4, 16, FAKE, 1, 8, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_ALIGN, "aligned"),
    ("moe_grouped_gemm", (FAKE, 4, 1 << 22, FAKE, 1, 8, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "32-bit"),
    ("moe_grouped_gemm", (FAKE, 4, 8192, FAKE, 1, 1 << 17, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "32-bit"),
    ("moe_grouped_gemm_gather", (FAKE, 8, None, 4, 16, FAKE, 1, 8, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_INVALID_ARG, "a_rows"),
    ("moe_grouped_gemm_gather", (FAKE, 1 << 27, FAKE, 4, 16, FAKE, 1, 8, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "x rows"),
    ("moe_grouped_gemm_gather", (FAKE, 0, FAKE, 4, 16, FAKE, 1, 8, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "no rows"),
    ("moe_grouped_gemm_gather", (FAKE, 8, FAKE, 4, 12, FAKE, 1, 8, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "multiple of 8"),
    ("moe_permute_index", (FAKE, 3, 0, 4, 8, FAKE, 32, 1, None), L.MOE_ERR_INVALID_ARG, "idx_dtype"),
    ("moe_permute_index", (FAKE, 1, 2, 4, 8, FAKE, 32, 1, None), L.MOE_ERR_INVALID_ARG, "map_layout"),
    ("moe_permute_index", (None, 1, 0, 4, 8, FAKE, 32, 1, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_permute_index", (FAKE, 1, 0, -4, 8, FAKE, 32, 1, None), L.MOE_ERR_SHAPE, "negative"),
    ("moe_permute_index", (FAKE, 1, 0, 1 << 31, 8, FAKE, 32, 1, None), L.MOE_ERR_CAPACITY, "int32"),
    # dgrad (dy, M, N, w, G, K, offsets, dx, ws, ws_bytes, stream)
    ("moe_map_extent", (FAKE, L.MOE_IDX_I64, -1, FAKE, FAKE, 64, None), L.MOE_ERR_SHAPE, "negative"),
    ("moe_map_extent", (FAKE, 7, 16, FAKE, FAKE, 64, None), L.MOE_ERR_INVALID_ARG, "idx_dtype"),
    ("moe_map_extent", (FAKE, L.MOE_IDX_I64, 16, None, FAKE, 64, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_map_extent", (FAKE, L.MOE_IDX_I64, 16, FAKE, FAKE, 8, None), L.MOE_ERR_WORKSPACE, "workspace"),
    ("moe_grouped_gemm_dgrad", (FAKE, -4, 16, FAKE, 1, 16, FAKE, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "negative"),
    ("moe_grouped_gemm_dgrad", (FAKE, 4, 12, FAKE, 1, 16, FAKE, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "multiples of 8"),
    ("moe_grouped_gemm_dgrad", (FAKE, 4, 16, FAKE, 1, 20, FAKE, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "multiples of 8"),
    ("moe_grouped_gemm_dgrad", (FAKE, 4, 16, FAKE, 0, 16, FAKE, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "G=0"),
    ("moe_grouped_gemm_dgrad", (FAKE, 4, 16, FAKE, 1, 16, None, FAKE, None, 0, None), L.MOE_ERR_INVALID_ARG, "group_offsets"),
    ("moe_grouped_gemm_dgrad", (FAKE, 4, 16, None, 1, 16, FAKE, FAKE, None, 0, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_grouped_gemm_dgrad", (ctypes.c_void_p(0x1008), 4, 16, FAKE, 1, 16, FAKE, FAKE, None, 0, None), L.MOE_ERR_ALIGN, "aligned"),
    ("moe_grouped_gemm_dgrad", (FAKE, 4, 1 << 22, FAKE, 1, 16, FAKE, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "32-bit"),
    ("moe_grouped_gemm_dgrad", (FAKE, 4, 1 << 16, FAKE, 1, 1 << 16, FAKE, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "32-bit"),
    # router (inp, M, K, weight, N, [k,] logits, [values, indices, map, probs,] ws, ws_bytes, stream)
    ("moe_router_logits", (FAKE, 64, 16, FAKE, 0, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "N=0"),
    ("moe_router_logits", (FAKE, 64, 16, FAKE, 513, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "512"),
    ("moe_router_logits", (FAKE, 64, 12, FAKE, 8, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "multiple of 8"),
    ("moe_router_logits", (FAKE, -1, 16, FAKE, 8, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "negative"),
    ("moe_router_logits", (FAKE, 64, 16, FAKE, 8, None, None, 0, None), L.MOE_ERR_INVALID_ARG, "null logits"),
    ("moe_router_logits", (ctypes.c_void_p(0x1002), 64, 16, FAKE, 8, FAKE, None, 0, None), L.MOE_ERR_ALIGN, "aligned"),
    ("moe_router_logits", (FAKE, 64, 1 << 22, FAKE, 8, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "32-bit"),
    ("moe_router_topk", (FAKE, 64, 16, FAKE, 8, 9, None, FAKE, FAKE, None, None, FAKE, 1 << 20, None), L.MOE_ERR_SHAPE, "out of range"),
    ("moe_router_topk", (FAKE, 64, 16, FAKE, 128, 65, None, FAKE, FAKE, None, None, FAKE, 1 << 20, None), L.MOE_ERR_CAPACITY, "64"),
    ("moe_router_topk", (FAKE, 64, 16, FAKE, 8, 2, None, None, FAKE, None, None, FAKE, 1 << 20, None), L.MOE_ERR_INVALID_ARG, "values"),
    ("moe_router_topk", (FAKE, 64, 16, FAKE, 8, 2, None, FAKE, FAKE, None, None, None, 0, None), L.MOE_ERR_WORKSPACE, "workspace"),
    ("moe_cast_f32_to_bf16", (FAKE, -1, FAKE, None), L.MOE_ERR_SHAPE, "negative"),
    ("moe_cast_f32_to_bf16", (None, 8, FAKE, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_cast_bf16_to_f32", (FAKE, 8, None, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_router_dgrad_tf32", (FAKE, 64, 12, FAKE, 64, FAKE, FAKE, 1 << 20, None), L.MOE_ERR_SHAPE, "multiples of 8"),
    ("moe_router_dgrad_tf32", (FAKE, 64, 16, FAKE, 64, FAKE, None, 0, None), L.MOE_ERR_WORKSPACE, "workspace"),
    ("moe_router_dgrad_tf32", (FAKE, 64, 16, FAKE, 64, None, FAKE, 1 << 20, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_router_dgrad_tf32", (FAKE, 64, 1 << 21, FAKE, 64, FAKE, FAKE, 1 << 20, None), L.MOE_ERR_CAPACITY, "32-bit"),
    ("moe_router_wgrad_tf32", (FAKE, 64, 16, FAKE, 20, FAKE, FAKE, 1 << 20, None), L.MOE_ERR_SHAPE, "multiples of 8"),
    ("moe_router_wgrad_tf32", (FAKE, 64, 16, FAKE, 16, FAKE, None, 0, None), L.MOE_ERR_WORKSPACE, "workspace"),
    ("moe_router_wgrad_tf32", (FAKE, 1 << 20, 1 << 10, FAKE, 16, FAKE, FAKE, 1 << 20, None), L.MOE_ERR_CAPACITY, "32-bit"),
    # wgrad (dy, x, M, N, K, G, offsets, dw, ws, ws_bytes, stream)
    ("moe_grouped_gemm_wgrad", (FAKE, FAKE, 4, 16, 16, 5000, FAKE, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "4096"),
    ("moe_grouped_gemm_wgrad", (FAKE, FAKE, 4, 16, 10, 1, FAKE, FAKE, None, 0, None), L.MOE_ERR_SHAPE, "multiples of 8"),
    ("moe_grouped_gemm_wgrad", (FAKE, None, 4, 16, 16, 1, FAKE, FAKE, None, 0, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_grouped_gemm_wgrad", (FAKE, FAKE, 4, 16, 16, 1, FAKE, None, None, 0, None), L.MOE_ERR_INVALID_ARG, "null"),
    ("moe_grouped_gemm_wgrad", (FAKE, ctypes.c_void_p(0x1004), 4, 16, 16, 1, FAKE, FAKE, None, 0, None), L.MOE_ERR_ALIGN, "aligned"),
    ("moe_grouped_gemm_wgrad", (FAKE, FAKE, 1 << 20, 1 << 12, 16, 1, FAKE, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "32-bit"),
    ("moe_grouped_gemm_wgrad", (FAKE, FAKE, 16, 1 << 16, 1 << 16, 1, FAKE, FAKE, None, 0, None), L.MOE_ERR_CAPACITY, "32-bit"),
])
def test_argument_validation(name, args, code, needle):
    st, msg = _status(name, *args)
    assert st == code, (st, msg)
    assert needle in msg, msg


def test_empty_problems_are_no_ops():
    # Nothing to do -> MOE_OK without touching the device.
    assert _status("moe_permute", None, 0, 8, None, 1, 0, 4, None, None, None, 0, 0, None, 0, None)[0] == 0
    assert _status("moe_unpermute", None, 0, 8, None, 1, 1, 4, 0, None, None, None, None)[0] == 0
    assert _status("moe_topk", None, 0, 16, 4, None, None, None, None, None)[0] == 0
    assert _status("moe_index_select", None, 0, 8, None, 1, 0, None, None)[0] == 0
    assert _status("moe_grouped_gemm", None, 0, 16, None, 1, 8, FAKE, 0, None, None, 0, None)[0] == 0
    assert _status("moe_grouped_gemm_gather", None, 4, None, 0, 16, None, 1, 8, FAKE, 0, None, None, 0, None)[0] == 0
    assert _status("moe_permute_index", None, 1, 0, 0, 8, None, 0, 1, None)[0] == 0
    assert _status("moe_grouped_gemm_dgrad", None, 0, 16, None, 1, 16, FAKE, None, None, 0, None)[0] == 0
    assert _status("moe_grouped_gemm_dgrad", None, 4, 16, None, 1, 0, FAKE, None, None, 0, None)[0] == 0
    assert _status("moe_grouped_gemm_wgrad", None, None, 4, 0, 16, 1, FAKE, None, None, 0, None)[0] == 0
    assert _status("moe_router_logits", None, 0, 16, None, 8, None, None, 0, None)[0] == 0
    assert _status("moe_cast_f32_to_bf16", None, 0, None, None)[0] == 0
    assert _status("moe_cast_bf16_to_f32", None, 0, None, None)[0] == 0
    assert _status("moe_router_topk", None, 0, 16, None, 8, 2, None, None, None, None, None, None, 0, None)[0] == 0


def test_workspace_sizes():
    lib = L.lib()
    # per super-chunk (S <= 64 of them, each a multiple of 256 tokens) the expert counts [S, E]
    # and the 32-expert group sums [S, ceil(E/32)], int32
    assert lib.moe_row_id_map_workspace_size(16384, 64) >= 64 * (64 + 2) * 4
    assert lib.moe_row_id_map_workspace_size(16385, 320) >= 65 * (320 + 10) * 4 // 2
    assert lib.moe_row_id_map_workspace_size(300001, 6) >= 62 * (6 + 1) * 4
    assert lib.moe_row_id_map_workspace_size(1 << 26, 32) <= 64 * 33 * 4 + 256
    assert lib.moe_permute_workspace_size(16384) >= 4096 * 4
    # map extent: one (max, count) int64 pair per partial block, at most 1024 blocks
    assert lib.moe_map_extent_workspace_size(0) == 256  # partials (256-byte aligned), then n bytes of row marks
    # one (max, count) pair per block, a block per 4096 entries up to 2048 blocks: 1280 at case21
    assert lib.moe_map_extent_workspace_size(320 * 16384) == 1280 * 16 + 320 * 16384
    assert lib.moe_map_extent_workspace_size(1 << 24) == 2048 * 16 + (1 << 24)
    assert lib.moe_map_extent_workspace_size(33) == 256 + 48
    assert lib.moe_map_extent_workspace_size(-1) == 0
    assert lib.moe_row_id_map_workspace_size(-1, 4) == 0
    # router: one fp32 logits plane (used when the top-k call gets no logits output)
    assert lib.moe_router_workspace_size(16384, 8192, 320) == 16384 * 320 * 4
    assert lib.moe_router_workspace_size(0, 8192, 320) == 0
    # one-group dgrad reduction split (no GPU here: the CU count reads as 256): case37
    # [288 x 5120] @ [5120 x 8192] has 2 x 32 output tiles -> 4 splits of 20 steps, fp32 planes
    assert lib.moe_grouped_gemm_dgrad_workspace_size(288, 5120, 8192, 1) == 4 * 288 * 8192 * 4
    # no split (512 tiles), a reduction of at least 4096: the tail list, 4 * (64 + G) bytes rounded to 256
    assert lib.moe_grouped_gemm_dgrad_workspace_size(4096, 5120, 8192, 1) == 512
    assert lib.moe_grouped_gemm_dgrad_workspace_size(131072, 4096, 7168, 64) == 512    # c5 fc1 dgrad
    assert lib.moe_grouped_gemm_dgrad_workspace_size(131072, 7168, 2048, 64) == 512    # c5 fc2 dgrad
    assert lib.moe_grouped_gemm_dgrad_workspace_size(131072, 4096, 7168, 4096) == 0    # 128-row tiles (32 rows a group)
    assert lib.moe_grouped_gemm_dgrad_workspace_size(131072, 2048, 7168, 64) == 0      # reduction below 4096
    assert lib.moe_grouped_gemm_dgrad_workspace_size(4096, 4160, 8192, 1) == 512       # 4160 = 65 steps
    assert lib.moe_grouped_gemm_dgrad_workspace_size(288, 5120, 8192, 2) == 0    # several groups
    assert lib.moe_grouped_gemm_dgrad_workspace_size(160, 5120, 8192, 1) == 0    # 128-row tiles
    assert lib.moe_grouped_gemm_dgrad_workspace_size(288, 320, 8192, 1) == 0     # too short a reduction
    assert lib.moe_grouped_gemm_dgrad_workspace_size(288, 5128, 8192, 1) == 0    # N % 64 != 0
    # wgrad group order: one int16 per group, for two or more groups
    # group order: int16 ids (rounded to 256 bytes), then the int32 (lo, hi) row range of each
    assert lib.moe_grouped_gemm_wgrad_workspace_size(131072, 7168, 2048, 64) == 256 + 512   # c5 fc2: 28 x 8 tiles
    assert lib.moe_grouped_gemm_wgrad_workspace_size(131072, 4096, 7168, 64) == 256 + 512   # c5 fc1: 16 x 28 tiles
    assert lib.moe_grouped_gemm_wgrad_workspace_size(4096, 64, 64, 1) == 0
    assert lib.moe_grouped_gemm_wgrad_workspace_size(4096, 64, 64, 4096) == 8192 + 32768
    # forward grouped GEMM: the tail list (counter, count, one int per group), for reductions of
    # at least 4096 in whole 64-column steps
    assert lib.moe_grouped_gemm_workspace_size(131072, 7168, 4096, 64) == 512     # c5 fc1: 4 * (64 + 64)
    assert lib.moe_grouped_gemm_workspace_size(131072, 7168, 4096, 4096) == (4 * (64 + 4096) + 255) // 256 * 256
    assert lib.moe_grouped_gemm_workspace_size(131072, 2048, 7168, 64) == 0       # c5 fc2: short reduction
    assert lib.moe_grouped_gemm_workspace_size(4096, 2560, 8192, 40) == 512        # case04: 102 rows per group
    assert lib.moe_grouped_gemm_workspace_size(4096, 4100, 256, 4) == 0           # K % 64 != 0
    assert lib.moe_grouped_gemm_workspace_size(4096, 4096, 256, 0) == 0
    # one group whose last round of 256 x 256 tiles is at most half full (256 CUs; no GPU here: the default):
    # fp32 planes of 256 x 256 for the reduction split of those tiles
    assert lib.moe_grouped_gemm_workspace_size(4096, 8192, 5120, 1) == 64 * 4 * 65536 * 4  # case10: 320 tiles
    assert lib.moe_grouped_gemm_workspace_size(1000, 1024, 1000, 1) == 16 * 5 * 65536 * 4  # 16 tiles, 5 ranges
    assert lib.moe_grouped_gemm_workspace_size(4096, 2560, 8192, 1) == 0   # case14: 512 tiles, two full rounds
    assert lib.moe_grouped_gemm_workspace_size(4096, 8192, 5120, 2) == (4 * (64 + 2) + 255) // 256 * 256
    # router tf32 wgrad: fp16 copies of both operands (M x (N + K)), the column exponents and column-max slabs
    # (64 slabs of 64 rows for each operand here), and 8 fp32 planes of N x K (8 reduction chunks of 512 rows)
    def up(b):
        return (b + 255) // 256 * 256
    want = (up(4096 * 64 * 2) + up(4096 * 1000 * 2) + up(64 * 4) + up(1000 * 4) + up(64 * 64 * 4) + up(64 * 1000 * 4)
            + up(8 * 64 * 1000 * 4))
    assert lib.moe_router_wgrad_tf32_workspace_size(4096, 64, 1000) == want
    assert lib.moe_router_wgrad_tf32_workspace_size(0, 16, 24) > 0  # one plane: the output is written through it


def test_status_strings():
    lib = L.lib()
    for code in range(7):
        assert lib.moe_status_string(code)
    assert lib.moe_status_string(99) == b"unknown status"


def test_ops_reject_cpu_tensors():
    # There is no CPU path: host tensors are refused before any launch.
    with pytest.raises(ValueError, match="GPU"):
        pkg.ops.permute(torch.zeros(2, 8, dtype=torch.bfloat16), torch.zeros(2, 2, dtype=torch.int64), num_out=4)
    with pytest.raises(ValueError, match="GPU"):
        pkg.ops.topk(torch.zeros(2, 8), 2)
    with pytest.raises(ValueError, match="GPU"):
        pkg.ops.grouped_gemm(torch.zeros(2, 8, dtype=torch.bfloat16), torch.zeros(1, 8, 8, dtype=torch.bfloat16),
                             torch.zeros(2, dtype=torch.int32))


def test_inputs_generators_cpu():
    sizes = pkg.inputs.zipf_group_sizes(32768, 16)
    assert sum(sizes) == 32768 and sizes[-1] == 0 and sizes[0] == max(sizes)
    assert pkg.inputs.uniform_group_sizes(4096, 40)[:2] == [103, 103] and sum(pkg.inputs.uniform_group_sizes(4096, 40)) == 4096
    rm, sel = pkg.inputs.reference_routing_mask(64, 16)
    assert rm.sum(1).tolist() == [6 if t % 4 == 1 else 5 for t in range(64)]


def test_probe_entry_points_validate_before_launch():
    # measurement probes (include/moe_probes.h, in libmoe_probes.so): exported, and bad arguments fail on the
    # host with the status (and the message) of libmoe_dispatch.so's status functions
    lib = L.probes()
    assert not hasattr(L.lib(), "moe_probe_mfma"), "the probes are not in the product library"
    assert lib.moe_probe_mfma(6, 10, FAKE, None) == L.MOE_ERR_SHAPE
    assert lib.moe_probe_mfma(8, 10, None, None) == L.MOE_ERR_INVALID_ARG
    assert lib.moe_probe_stream(3, FAKE, FAKE, 16, 1, None) == L.MOE_ERR_INVALID_ARG
    assert lib.moe_probe_stream(7, FAKE, FAKE, 16, 1, None) == L.MOE_ERR_INVALID_ARG
    assert lib.moe_probe_stream(0, None, FAKE, 16, 1, None) == L.MOE_ERR_INVALID_ARG
    assert lib.moe_probe_stream(2, None, ctypes.c_void_p(0x1004), 16, 1, None) == L.MOE_ERR_ALIGN
    assert b"moe_probe_stream" in L.lib().moe_last_error()
