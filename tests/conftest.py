"""Shared test setup: the `gpu` marker, repository paths and the seeded fixtures of the reference's own tests."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "trench-gguf_amd")
for p in (os.path.join(ROOT, "oracle"), os.path.join(PKG, "gpuq"), PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

TABLES = os.path.join(PKG, "gpuq", "gpuq_tables.bin")
# the repository's table file holds stand-in IQ codebooks (ggml's are not available here): the library loads them
# only when asked to, which the tests do
os.environ["GPUQ_ALLOW_SYNTHETIC_TABLES"] = "1"
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libgpuq_ref.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


def selftest_matrices(ne1=256, ne0=2304, seed=1234):
    """The reference's self-test fixture (gpuq/test_gpuq.py:57-73): Gaussian, a coarse copy with ties, heavy tails,
    and edge rows (zeros, constants, one-signed, x^2 subnormal, sparse zeros); one gamma(1,1) imatrix each."""
    rng = np.random.default_rng(seed)
    g = rng.standard_normal((ne1, ne0)).astype(np.float32) * 0.02
    coarse = (np.round(g / 0.005) * 0.005).astype(np.float32)
    heavy = (rng.standard_t(3, (ne1, ne0)) * 0.01).astype(np.float32)
    edge = g.copy()
    edge[0:8] = 0
    edge[8:16, :1024] = 0.01
    edge[16:32] = np.abs(edge[16:32])
    edge[32:48] = -np.abs(edge[32:48])
    edge[48:64] *= 1e-20
    edge[64:80, ::16] = 0
    xs = [g, coarse, heavy, edge]
    ims = [rng.gamma(1.0, 1.0, ne0).astype(np.float32) for _ in xs]
    return xs, ims


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import Oracle
    if not os.path.exists(TABLES):
        pytest.skip("tables not built: run __graft_entry__.build()")
    return Oracle(tables=TABLES)
