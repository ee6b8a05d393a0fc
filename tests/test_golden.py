"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from seeded inputs) against the C oracle now:
every output must come out bit for bit, so any change to the oracle's
arithmetic (which the GPU parity tests rely on) shows here."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402


def load(name):
    with np.load(os.path.join(HERE, "golden", name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", sorted(make_golden.CASES))
def test_oracle_reproduces_golden_fixture(name):
    want = load(name)
    got = make_golden.make(name)
    assert sorted(got) == sorted(want)
    for key in want:
        g = np.asarray(got[key])
        assert g.dtype == want[key].dtype and g.shape == want[key].shape, key
        assert g.tobytes() == want[key].tobytes(), (name, key)


def test_golden_fixtures_are_small():
    total = sum(os.path.getsize(os.path.join(HERE, "golden", f))
                for f in os.listdir(os.path.join(HERE, "golden")) if f.endswith(".npz"))
    assert total < 512 * 1024
