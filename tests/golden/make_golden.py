"""Writes tests/golden/generator_digests.json: SHA-256 digests of the reference
cases' seeded input generators, computed by importing the reference case
modules (run in the build container only, where /root/reference exists).

Only the generators are imported: they are the one part of the reference whose
exact output no golden vector, closed form or invariant pins (torch CPU RNG +
argsort streams).  Sizes are the reference's own; nothing of the reference is
copied into the repository, only the digests and shapes.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import importlib.util
import json
from pathlib import Path

import torch

REF = Path("/root/reference/kernel_cases")
OUT = Path(__file__).resolve().parent / "generator_digests.json"


def _load(name):
    spec = importlib.util.spec_from_file_location(name, REF / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def digest(t: torch.Tensor) -> dict:
    t = t.contiguous()
    raw = t.view(torch.uint8) if t.dtype != torch.bool else t.to(torch.uint8)
    return {"shape": list(t.shape), "dtype": str(t.dtype), "sha256": hashlib.sha256(raw.numpy().tobytes()).hexdigest()}


def main():
    out = {}
    c12 = _load("case12_moe_row_id_map_pass2")
    out["case12.make_routing_map"] = digest(c12.make_routing_map())
    c17 = _load("case17_moe_permute_with_mask_map")
    x, row_id_map, probs = c17.get_inputs()
    out["case17.get_inputs.x"] = digest(x)
    out["case17.get_inputs.row_id_map"] = digest(row_id_map)
    out["case17.get_inputs.probs"] = digest(probs)
    c15 = _load("case15_moe_unpermute_mask_fwd")
    pin, rmap = c15.get_inputs()
    out["case15.get_inputs.pin"] = digest(pin)
    out["case15.get_inputs.row_id_map"] = digest(rmap)
    c21 = _load("case21_ref_permute_with_mask_map_trans")
    out["case21.make_row_id_map"] = digest(c21.make_row_id_map())
    c24 = _load("case24_ref_moe_unpermute_mask_kernel_false")
    out["case24.make_row_id_map"] = digest(c24.make_row_id_map())
    c22 = _load("case22_ref_moe_permute_mask_kernel_true")
    out["case22.make_probs_seed1"] = digest(c22.make_probs(c22.make_row_id_map(), seed=1))
    c23 = _load("case23_ref_aten_topk")
    out["case23.make_inputs_seed0"] = digest(c23.make_inputs(seed=0))
    c06 = _load("case06_cp_seq_chunk_index_select")
    k_ag, v_ag, index = c06.get_inputs()
    out["case06.get_inputs.k_ag"] = digest(k_ag)
    out["case06.get_inputs.v_ag"] = digest(v_ag)
    out["case06.get_inputs.index"] = digest(index)
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {OUT} ({len(out)} digests)")


if __name__ == "__main__":
    main()
