"""The oracle against golden vectors written by the reference implementation itself: the reference's gpuq.hip,
compiled from its own source into oracle/_ref/ and run on an MI355X by tests/golden/make_ref_golden.py over a row
subset of the reference's self-test fixture (gpuq/test_gpuq.py:57-73), with this repository's search tables.
Every type and imatrix mode must match byte for byte, and the i-quant dequantizers bit for bit (sha256)."""
import os

import numpy as np
import pytest

from conftest import TABLES

import tables

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def golden():
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from make_ref_golden import golden_inputs, sha
    g = np.load(GOLDEN, allow_pickle=False)
    xs, ims = golden_inputs()
    assert str(g["meta_inputs"]) == sha(np.stack(xs)) + sha(np.stack(ims)), "fixture inputs changed"
    assert str(g["meta_tables"]) == tables.content_sha(TABLES), "tables changed"
    return g, xs, ims, sha


def keys():
    g = np.load(GOLDEN, allow_pickle=False)
    return sorted(k for k in g.files if k.startswith("q_"))


@pytest.mark.parametrize("key", keys())
def test_quantize_matches_reference_vectors(oracle_lib, golden, key):
    g, xs, ims, _ = golden
    _, t, mode = key.split("_")
    t = int(t)
    want = g[key]
    for m, (x, im) in enumerate(zip(xs, ims)):
        got = oracle_lib.quantize(t, x, im if mode == "im" else None).reshape(-1)
        bb = oracle_lib.block_bytes(t)
        same = (got.reshape(-1, bb) == want[m].reshape(-1, bb)).all(axis=1)
        assert same.all(), "%s matrix %d: %d blocks differ, first %d" % (key, m, int((~same).sum()),
                                                                         int(np.argmin(same)))


@pytest.mark.parametrize("t", [16, 17, 22, 18, 21, 19, 29, 23])
def test_dequantize_matches_reference_vectors(oracle_lib, golden, t):
    g, xs, ims, sha = golden
    q = g["q_%d_im" % t]
    f = oracle_lib.dequantize(t, q.reshape(-1), q.size // oracle_lib.block_bytes(t) * 256)
    assert sha(f) == str(g["dq_%d" % t])
