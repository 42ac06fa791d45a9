"""The hardware reciprocal's error bound that the selection chain's candidate margin assumes.

A chain step forms the state after a pick with v_rcp_f32 and no Newton step; the argument at
raised_key (csrc/tree_select.hip) takes |rcp(d) * d - 1| <= 2^-23.38 for every float d in
[1, 2^24].  This checks that bound exhaustively on the GPU (201,326,593 values)."""
import os
import subprocess

import pytest

from tests.golden.rcp_bound import BIN

pytestmark = pytest.mark.gpu


def test_rcp_bound_over_every_denominator():
    if not os.path.exists(BIN):
        pytest.fail("tests/golden/rcp_bound is not built (__graft_entry__.build() builds it)")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    f = r.stdout.split()
    vals = dict(zip(f[0::2], f[1::2]))
    assert int(vals["floats"]) == 0x0C000001
    assert int(vals["over_2^-23"]) == 0
    assert float(vals["max_rel_err"]) <= 2.0 ** -23.38, r.stdout
