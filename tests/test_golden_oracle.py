"""The oracle reproduces the committed golden fixture (tests/golden/ppo_update_small.npz, written by
tests/golden/make_golden.py): guards against drift between the torch build that wrote it and the one running."""

from __future__ import annotations

from pathlib import Path

import numpy as np

from tests.golden import make_golden

FIXTURE = Path(__file__).resolve().parent / "golden" / "ppo_update_small.npz"


def test_oracle_reproduces_golden_fixture():
    ref = np.load(FIXTURE)
    got = make_golden.compute()
    assert sorted(got) == sorted(ref.files)
    assert np.array_equal(got["perm"], ref["perm"]), "randperm of the seeded CPU generator"
    assert np.array_equal(got["returns"], ref["returns"]), "GAE returns are elementwise: bit-exact"
    np.testing.assert_allclose(got["advantages"], ref["advantages"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(got["losses"], ref["losses"], rtol=1e-5)
    np.testing.assert_array_equal(got["trace.lr"], ref["trace.lr"])
    for k in ref.files:
        if k.startswith("final.") or k.startswith("init."):
            np.testing.assert_allclose(got[k], ref[k], rtol=1e-4, atol=1e-6, err_msg=k)
