"""moe_row_id_map_noalloc (the entry point that allocates nothing) against
moe_row_id_map (workspace from the caller), both called through the C ABI:
results bit-identical on two calls in a row, the second with a smaller input,
so stale scratch contents from the first call cannot leak into the second."""
from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import assert_bits_equal, load_pkg

pkg = load_pkg()
L = pkg._lib

pytestmark = pytest.mark.gpu


def _mask(T, E, k, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.rand(T, E, generator=g).topk(k, dim=1).indices
    return torch.zeros(T, E, dtype=torch.uint8).scatter_(1, idx, 1)


def _outputs(T, E, dev):
    return (torch.full((E, T), -7, dtype=torch.int64, device=dev),
            torch.full((T, E), -7, dtype=torch.int64, device=dev),
            torch.full((E, T), -7, dtype=torch.int32, device=dev),
            torch.full((E + 1,), -7, dtype=torch.int32, device=dev))


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("shapes", [[(4096, 320, 8), (1000, 64, 2)], [(16384, 64, 8), (257, 16, 3)]])
def test_row_id_map_noalloc_matches_workspace_entry_point(dev, shapes):
    lib = L.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, (T, E, k) in enumerate(shapes):
        print(f"call {i}: T={T} E={E} k={k}", flush=True)
        mask = _mask(T, E, k, seed=T * 7 + E).to(dev)
        ws_bytes = lib.moe_row_id_map_workspace_size(T, E)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        ref = _outputs(T, E, dev)
        got = _outputs(T, E, dev)
        st = lib.moe_row_id_map(_ptr(mask), T, E, *(_ptr(t) for t in ref), _ptr(ws), ws_bytes, stream)
        assert st == L.MOE_OK, lib.moe_last_error().decode()
        st = lib.moe_row_id_map_noalloc(_ptr(mask), T, E, *(_ptr(t) for t in got), stream)
        assert st == L.MOE_OK, lib.moe_last_error().decode()
        torch.cuda.synchronize()
        for name, g, r in zip(("expert-major", "token-major", "int32 expert-major", "offsets"), got, ref):
            assert_bits_equal(g, r, f"call {i} {name}")
        assert int(got[3][-1]) == T * k


def test_row_id_map_noalloc_rejects_oversized_input(dev):
    lib = L.lib()
    T, E = 1 << 18, 4096  # ceil(T/64) * E int32 counts = 64 MiB > the 8 MiB scratch
    st = lib.moe_row_id_map_noalloc(ctypes.c_void_p(0x1000), T, E, None, None, None, None, None)
    assert st == L.MOE_ERR_CAPACITY and "scratch" in lib.moe_last_error().decode()
