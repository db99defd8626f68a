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


def _outputs(T, E, k, dev):
    return (torch.full((E, T), -7, dtype=torch.int64, device=dev),
            torch.full((T, E), -7, dtype=torch.int64, device=dev),
            torch.full((E, T), -7, dtype=torch.int32, device=dev),
            torch.full((E + 1,), -7, dtype=torch.int32, device=dev),
            torch.full((T * k,), -7, dtype=torch.int32, device=dev))


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("shapes", [[(4096, 320, 8), (1000, 64, 2)], [(16384, 64, 8), (257, 16, 3)],
                                    [(200000, 40, 4), (70, 4096, 5)]])
def test_row_id_map_noalloc_matches_workspace_entry_point(dev, shapes):
    lib = L.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, (T, E, k) in enumerate(shapes):
        print(f"call {i}: T={T} E={E} k={k}", flush=True)
        mask = _mask(T, E, k, seed=T * 7 + E).to(dev)
        ws_bytes = lib.moe_row_id_map_workspace_size(T, E)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        ref = _outputs(T, E, k, dev)
        got = _outputs(T, E, k, dev)
        st = lib.moe_row_id_map(_ptr(mask), T, E, *(_ptr(t) for t in ref), T * k, _ptr(ws), ws_bytes, stream)
        assert st == L.MOE_OK, lib.moe_last_error().decode()
        st = lib.moe_row_id_map_noalloc(_ptr(mask), T, E, *(_ptr(t) for t in got), T * k, stream)
        assert st == L.MOE_OK, lib.moe_last_error().decode()
        torch.cuda.synchronize()
        for name, g, r in zip(("expert-major", "token-major", "int32 expert-major", "offsets", "source tokens"),
                              got, ref):
            assert_bits_equal(g, r, f"call {i} {name}")
        assert int(got[3][-1]) == T * k


def test_row_id_map_noalloc_rejects_sizes_beyond_its_limits(dev):
    # E above 4096 and T * E at 2^31 fail before any device work; everything below them fits
    # the static scratch (the largest need, E = 4096, is 64 * (4096 + 128) int32 values).
    lib = L.lib()
    for T, E, needle in ((16, 5000, "4096"), (1 << 20, 4096, "2^31")):
        st = lib.moe_row_id_map_noalloc(ctypes.c_void_p(0x1000), T, E, None, None, None, None, None, 0, None)
        assert st == L.MOE_ERR_CAPACITY and needle in lib.moe_last_error().decode(), (T, E)
    assert lib.moe_row_id_map_workspace_size((1 << 31) // 4096 - 1, 4096) <= 2 << 20


def test_row_id_map_noalloc_under_graph_capture(dev):
    # Captured once in a graph (the call allocates nothing and records only kernels), then replayed after the
    # mask changes in place; every replay, with eager work and a synchronisation between replays, is bit-equal
    # to moe_row_id_map with a workspace on the same mask.
    lib = L.lib()
    T, E, k = 4096, 64, 8
    mask = _mask(T, E, k, seed=1).to(dev)
    got = _outputs(T, E, k, dev)
    # first call outside the graph: the scratch address is looked up once per device here
    st = lib.moe_row_id_map_noalloc(_ptr(mask), T, E, *(_ptr(t) for t in got), T * k,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == L.MOE_OK, lib.moe_last_error().decode()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = lib.moe_row_id_map_noalloc(_ptr(mask), T, E, *(_ptr(t) for t in got), T * k,
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == L.MOE_OK, lib.moe_last_error().decode()
    ws_bytes = lib.moe_row_id_map_workspace_size(T, E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for rep, seed in enumerate((2, 3, 4)):
        print(f"replay {rep}: mask seed {seed}", flush=True)
        mask.copy_(_mask(T, E, k, seed=seed).to(dev))
        for t in got:
            t.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        ref = _outputs(T, E, k, dev)
        st = lib.moe_row_id_map(_ptr(mask), T, E, *(_ptr(t) for t in ref), T * k, _ptr(ws), ws_bytes, stream)
        assert st == L.MOE_OK, lib.moe_last_error().decode()
        torch.cuda.synchronize()
        for name, g, r in zip(("expert-major", "token-major", "int32 expert-major", "offsets", "source tokens"),
                              got, ref):
            assert_bits_equal(g, r, f"replay {rep} {name}")
