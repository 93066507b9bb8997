"""The oracle reproduces the committed golden fixtures (tests/golden/*.npz):
binning and forward outputs bit for bit, float64 gradient sums and losses to
rounding.  A change of the oracle that moves any result fails here."""
from __future__ import annotations

import numpy as np
import pytest

from golden import make_fixtures as G


def load(case):
    with np.load(G.fixture_path(case)) as z:
        return {k: z[k] for k in z.files}


def inputs(fx):
    return {k[3:]: v for k, v in fx.items() if k.startswith("in_")}


@pytest.mark.parametrize("case", list(G.CASES))
def test_oracle_reproduces_fixture(case):
    fx = load(case)
    exp = G.expected(inputs(fx), G.CASES[case])
    assert set(exp) == {k for k in fx if not k.startswith("in_")}
    for k, v in exp.items():
        ref = fx[k]
        if k.startswith("bin_") or k.startswith("fwd_"):
            assert v.dtype == ref.dtype and v.shape == ref.shape, k
            np.testing.assert_array_equal(v.view(np.uint8), ref.view(np.uint8), err_msg=k)
        else:
            np.testing.assert_allclose(v, ref, rtol=1e-9, atol=1e-12, err_msg=k)


def test_tied_depths_keep_primitive_order():
    """Equal depths: each tile's list is in ascending primitive id (the stable
    order the build defines for the reference's torch.sort ties)."""
    fx = load("ties_fill")
    ids = fx["bin_primitive_ids_sorted"]
    bins = fx["bin_tile_bins"]
    multi = 0
    for t0, t1 in bins:
        seg = ids[t0:t1]
        assert np.all(np.diff(seg) > 0)
        multi += len(seg) > 1
    assert multi > 0


def test_fixture_invariants():
    for case in G.CASES:
        fx = load(case)
        bins = fx["bin_tile_bins"]
        n = fx["bin_primitive_ids_sorted"].size
        assert int(fx["bin_num_tiles_hit"].sum()) == n
        nz = bins[bins[:, 1] > bins[:, 0]]
        assert nz[:, 1].max() == n and nz[:, 0].min() == 0
        T = fx["fwd_final_T"]
        assert np.all((T >= 0) & (T <= 1))
