"""MI355X-native (gfx950) MoE expert-dispatch path.

    router top-k -> mask map -> row-id map -> permute -> grouped GEMM fc1 (+SwiGLU)
    -> grouped GEMM fc2 -> probability-weighted unpermute, plus the permute
    backward and the index_select row gather.

The compute lives in hand-written HIP kernels behind the C ABI of
include/moe_dispatch.h (libmoe_dispatch.so in this directory, built by
csrc/build.py).  `ops` is the tensor-level API, `cases` holds drop-in
counterparts of the reference's kernel cases, `moe_ffn` the composed layer and
`inputs` the seeded input generators.

The directory name is not a Python identifier; import it with
importlib.import_module("1188b-reference-kernels_amd").
"""
from . import _lib, inputs, ops  # noqa: F401
from . import moe_ffn  # noqa: F401
from . import cases  # noqa: F401

__all__ = ["ops", "inputs", "moe_ffn", "cases"]
