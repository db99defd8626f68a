"""Pins the restated input generators (and the oracle's row-id map on them) to
the reference's own generator outputs, by SHA-256 digest (CPU).

tests/golden/generator_digests.json was written by tests/golden/make_golden.py,
which imports the reference case modules in the build container.  A digest
match means the tensor is bit-identical to the reference's at the reference's
full size.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import pytest
import torch

from conftest import load_pkg
from oracle import ref_torch

DIGESTS = json.loads((Path(__file__).resolve().parent / "golden" / "generator_digests.json").read_text())
inputs = load_pkg().inputs


def _digest(t: torch.Tensor) -> dict:
    t = t.contiguous()
    raw = t.view(torch.uint8) if t.dtype != torch.bool else t.to(torch.uint8)
    return {"shape": list(t.shape), "dtype": str(t.dtype), "sha256": hashlib.sha256(raw.numpy().tobytes()).hexdigest()}


def _check(name, t):
    assert _digest(t) == DIGESTS[name], name


def test_case12_routing_mask_and_row_id_map():
    rm, _ = inputs.reference_routing_mask(16384, 320)
    _check("case12.make_routing_map", rm)


def test_case17_inputs_and_oracle_row_id_map():
    rm, sel = inputs.reference_routing_mask(16384, 320)
    _, row_tm = ref_torch.row_id_map(rm)  # the oracle's map equals the reference generator's map
    _check("case17.get_inputs.row_id_map", row_tm)
    x, probs = inputs.case17_x_probs(sel, 8192, 320)
    _check("case17.get_inputs.x", x)
    _check("case17.get_inputs.probs", probs)


def test_case15_inputs_and_oracle_row_id_map():
    rm, _ = inputs.reference_routing_mask(16384, 320)
    row_em, _ = ref_torch.row_id_map(rm)
    _check("case15.get_inputs.row_id_map", row_em)
    _check("case15.get_inputs.pin", inputs.case15_pin(int(rm.sum()), 8192))


def test_modular_maps_case21_case24():
    _check("case21.make_row_id_map", ref_torch.modular_row_id_map(16384, 320, 8))
    # the same map from the oracle's cumsum construction on the modular mask
    em, _ = ref_torch.row_id_map(inputs.modular_routing_mask(16384, 320, 8).t().contiguous())
    _check("case21.make_row_id_map", em)
    _check("case24.make_row_id_map", em.to(torch.int32))


def test_case22_probs_case23_logits():
    sel = ref_torch.modular_row_id_map(16384, 320, 8) >= 0
    _check("case22.make_probs_seed1", inputs.case22_probs(sel, seed=1))
    _check("case23.make_inputs_seed0", inputs.case23_logits(16384, 320, seed=0))


@pytest.mark.parametrize("which", ["k_ag", "v_ag", "index"])
def test_case06_inputs(which):
    torch.manual_seed(20261111)
    k_ag = torch.randn(2, 65536, 16, 192).to(torch.bfloat16)
    if which == "k_ag":
        return _check("case06.get_inputs.k_ag", k_ag)
    v_ag = torch.randn(2, 65536, 16, 128).to(torch.bfloat16)
    if which == "v_ag":
        return _check("case06.get_inputs.v_ag", v_ag)
    _check("case06.get_inputs.index", torch.arange(2, dtype=torch.int32))
