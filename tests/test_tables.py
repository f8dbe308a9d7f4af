"""The search-table generator: determinism, the layout rules the GPU loader enforces, and ggml's neighbour rule
checked by brute force on sampled keys."""
import hashlib
import os

import numpy as np
import pytest

from conftest import TABLES

import tables as T


@pytest.fixture(scope="module")
def recs():
    if not os.path.exists(TABLES):
        pytest.skip("tables not built")
    return T.read_tables(TABLES)


def test_file_is_the_generator_output(recs, tmp_path):
    p = T.write_tables(str(tmp_path / "t.bin"))
    assert hashlib.sha256(open(p, "rb").read()).hexdigest() == hashlib.sha256(open(TABLES, "rb").read()).hexdigest()


SHAPES = {16: (256, 8, 2, 3), 17: (512, 8, 2, 3), 19: (2048, 8, 2, 2), 22: (1024, 8, 2, 3), 18: (256, 4, 3, 7),
          21: (512, 4, 3, 7)}


@pytest.mark.parametrize("typ", sorted(SHAPES))
def test_layout_rules(recs, typ):
    """every point's key maps back to it; every key the trial rounding reaches has a point or a non-empty list"""
    grid, kmap, neigh = recs[typ]
    G, nv, bits, maxlev = SHAPES[typ]
    assert len(grid) == G and len(kmap) == (43692 if nv == 8 else 4096)
    lv = np.stack([((grid >> np.uint64(8 * i)) & np.uint64(0xff)).astype(np.int64) for i in range(nv)], axis=1)
    assert ((lv % 2 == 1) & (lv >= 1) & (lv <= 2 * maxlev + 1)).all()
    keys = (((lv - 1) // 2) << (bits * np.arange(nv))).sum(axis=1)
    assert (kmap[keys] == np.arange(G)).all()
    reach = range(3 ** 8) if nv == 8 else range(4096)
    for k in reach:
        u = k
        if nv == 8:
            u, r = 0, k
            for i in range(8):
                u |= (r % 3) << (2 * i)
                r //= 3
        m = int(kmap[u])
        if m >= 0:
            assert m < G
        else:
            off = -m - 1
            cnt = int(neigh[off])
            assert cnt >= 1 and off + cnt < len(neigh)
            assert (neigh[off + 1:off + 1 + cnt] < G).all()
    dq = recs[1000 + typ][0]
    assert len(dq) == G


@pytest.mark.parametrize("typ,nwant", [(16, 2), (19, 3), (22, 1), (18, 2)])
def test_neighbour_rule_brute_force(recs, typ, nwant):
    """a list holds every point within the nwant smallest distinct squared distances, ordered by (distance, index)"""
    grid, kmap, neigh = recs[typ]
    G, nv, bits, _ = SHAPES[typ]
    pts = [[2 * (((int(g) >> (8 * i)) & 0xff) - 1) // 2 + 1 for i in range(nv)] for g in grid]
    rng = np.random.default_rng(11)
    off_keys = np.nonzero(kmap < 0)[0]
    for u in rng.choice(off_keys, 40, replace=False):
        kp = [2 * ((int(u) >> (bits * i)) & ((1 << bits) - 1)) + 1 for i in range(nv)]
        d2 = [sum((a - b) ** 2 for a, b in zip(kp, p)) for p in pts]
        shells = sorted(set(d2))[:nwant]
        want = sorted([j for j in range(G) if d2[j] <= shells[-1]], key=lambda j: (d2[j], j))
        off = -int(kmap[u]) - 1
        cnt = int(neigh[off])
        assert list(neigh[off + 1:off + 1 + cnt]) == want, int(u)
