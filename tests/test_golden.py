"""The committed fixtures under tests/golden/ (CPU): each file matches its
manifest digest, and the oracle re-derives every array bit for bit from the
same seeds, so a change to the oracle's arithmetic cannot pass unnoticed."""
import json
import os
import sys

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)

import make_golden  # noqa: E402


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", ["q8_0_codec.npz", "linear.npz", "sampler.npz"])
def test_fixture_matches_manifest(name):
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        manifest = json.load(f)
    assert make_golden.digest(load(name)) == manifest[name]


def test_oracle_rederives_every_fixture(orc):
    for name, arrays in make_golden.build_all(orc).items():
        have = load(name)
        assert sorted(have) == sorted(arrays), name
        for key, want in arrays.items():
            got = have[key]
            assert got.dtype == np.asarray(want).dtype and got.shape == np.asarray(want).shape, (name, key)
            assert got.tobytes() == np.ascontiguousarray(want).tobytes(), (name, key)  # bit for bit, NaNs included
