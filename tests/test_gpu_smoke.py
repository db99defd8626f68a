"""GPU: the build entry's smoke() (one small MoE FFN forward, every stage against the oracle)."""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def test_graft_entry_smoke(dev):
    import __graft_entry__

    __graft_entry__.smoke()
