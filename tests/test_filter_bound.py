"""The filtered search's decision rule (trench-gguf_amd/csrc/filter.cuh: the key of a candidate, the two least keys of
a list and filt_pick's margin test), restated in float32 numpy and checked against ggml's serial scan
(iq2_find_best_neighbour, gpuq/gpuq.hip:178-197, as oracle/gq_oracle.c's nb_iq2 restates it): whenever the test
decides, its pick must be the scan's. Inputs: random groups, weights over many decades, zero weights, a sign-flipped
value; built near-ties (values halfway between two scaled grid points, nudged by 2^-26 .. 2^-14, so that two
candidates' distances straddle the margin); and values on a scaled grid point (ggml's distance 0, the filter's value
rounding to either side of 0). The IQ2_XXS stand-in grid's points are the candidates.

Planted mistakes in the restatement are caught: the cross term's sign flipped, and keys that keep the value's sign
(a value rounded below 0 then ranks last).

(numpy has no fused multiply-add: fma(a, b, c) is formed in float64, where a*b is exact, and rounded to float32; the
sum's own float64 rounding can move the result by one unit in the last place in rare cases, far inside the margin.)"""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "trench-gguf_amd"))

F = np.float32
IB = 8                                  # IQ2_XXS: 256 grid points, 8 index bits in a key
KM = np.uint32((1 << IB) - 1)
KHI = np.uint32(0x7FFFFFFF & ~((1 << IB) - 1))
NONE = np.uint32(0xFFFFFFFF)
FLT_MAX = np.finfo(np.float32).max


def fma(a, b, c):
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(F)


def grid_levels():
    from gpuq import tables
    import gpuq
    grid = tables.read_tables(gpuq.tables_path())[16][0]
    q = ((grid[:, None] >> (8 * np.arange(8, dtype=np.uint64))) & np.uint64(0xFF)).astype(F)   # q = 2l+1
    return q


def ggml_pick(q, cand, x, w, s):
    """the serial scan: d2 += w * diff * diff in index order, strict < from FLT_MAX (first wins); -1: none"""
    qc = q[cand]                                    # [G, L, 8]
    d2 = np.zeros(cand.shape, F)
    for i in range(8):
        diff = (s[:, None] * qc[:, :, i]).astype(F) - x[:, None, i]
        d2 = (d2 + (w[:, None, i] * diff).astype(F) * diff).astype(F)
    best = np.full(cand.shape[0], FLT_MAX, F)
    pick = np.full(cand.shape[0], -1)
    for j in range(cand.shape[1]):
        b = d2[:, j] < best
        best = np.where(b, d2[:, j], best)
        pick = np.where(b, cand[:, j], pick)
    return pick


def filter_keys(q, cand, x, w, s, plant=None):
    """each candidate's key: bits(|fma(s, fma(s, A, B'), C)|) with the low IB bits replaced by its grid index"""
    qc = q[cand]
    wx = (w * x).astype(F)
    nwx = (F(2 if plant == "cross_sign" else -2) * wx).astype(F)
    A = (w[:, None, 0] * (qc[:, :, 0] * qc[:, :, 0])).astype(F)
    B = (nwx[:, None, 0] * qc[:, :, 0]).astype(F)
    C = np.zeros(x.shape[0], F)
    for i in range(8):
        if i:
            A = fma(w[:, None, i], (qc[:, :, i] * qc[:, :, i]).astype(F), A)
            B = fma(nwx[:, None, i], qc[:, :, i], B)
        C = fma(wx[:, i], x[:, i], C)
    D = fma(s[:, None], fma(s[:, None], A, B), C[:, None])
    if plant == "keep_sign":
        return (D.view(np.uint32) & (KHI | np.uint32(0x80000000))) | cand.astype(np.uint32)
    return (np.abs(D).view(np.uint32) & KHI) | cand.astype(np.uint32)


def filter_pick(keys, x, w, s, margin=F(2.002)):
    ks = np.sort(keys, axis=1)
    k1 = ks[:, 0]
    k2 = ks[:, 1] if ks.shape[1] > 1 else np.full(ks.shape[0], NONE)
    sw = np.zeros(x.shape[0], F)
    swx = np.zeros(x.shape[0], F)
    swxx = np.zeros(x.shape[0], F)
    for i in range(8):
        sw = (sw + w[:, i]).astype(F)
        swx = fma(w[:, i], np.abs(x[:, i]), swx)
        swxx = fma((w[:, i] * x[:, i]).astype(F), x[:, i], swxx)
    smax = fma((s * s).astype(F), (F(49) * sw).astype(F), fma((F(14) * s).astype(F), swx, swxx))
    delta = (smax * F(2.0 ** -19)).astype(F)
    ok = (smax >= F(2.0 ** -60)) & (smax <= F(2.0 ** 100)) & (k1 != NONE)
    up1 = ((k1 & ~KM) + KM + np.uint32(1)).view(F)
    with np.errstate(over="ignore", invalid="ignore"):
        ok &= (up1 + delta).astype(F) < FLT_MAX
        lo2 = (k2 & ~KM).view(F)
        ok &= (k2 == NONE) | ((lo2 - up1).astype(F) > (margin * delta).astype(F))
    return np.where(ok, (k1 & KM).astype(np.int64), -1)


def cases(q, rng, n=6000, kind="random"):
    """n groups: values, weights (w >= 0), a trial scale s = 1/id and a list of distinct candidates"""
    G = n
    L = int(rng.integers(2, 40))
    cand = np.argsort(rng.random((G, q.shape[0])), axis=1)[:, :L]
    mag = F(10.0) ** rng.uniform(-6, 3, G).astype(F)
    idv = (F(1) / (mag * F(rng.uniform(0.2, 0.6)))).astype(F)
    s = (F(1) / idv).astype(F)
    w = (F(10.0) ** rng.uniform(-3, 3, (G, 8))).astype(F)
    w[rng.random((G, 8)) < 0.1] = 0
    if kind == "exact":                                     # on the first candidate's scaled point
        x = (s[:, None] * q[cand[:, 0]]).astype(F)
    elif kind == "near":
        a, b = cand[:, 0], cand[:, 1]                       # two candidates: x halfway between their scaled points
        x = (s[:, None] * ((q[a] + q[b]) * F(0.5))).astype(F)
        e = (rng.choice([-1.0, 1.0], (G, 8)) * 2.0 ** -rng.uniform(14, 26, (G, 8))).astype(F)  # relative nudges
        x = (x * (F(1) + e)).astype(F)
        w[:] = w[:, :1]                                     # equal weights: the two distances nearly tie
    else:
        x = (mag[:, None] * rng.uniform(0, 3, (G, 8)).astype(F)).astype(F)
    flip = rng.random(G) < 0.2                              # ggml's parity flip can make one value negative
    x[flip, 0] = -x[flip, 0]
    return cand, x, w, s


@pytest.fixture(scope="module")
def q():
    return grid_levels()


FLOOR = {"random": 0.8, "near": 0.1, "exact": 0.6}     # the share of searches the test must decide


@pytest.mark.parametrize("kind", sorted(FLOOR))
def test_decided_picks_are_the_scans(q, kind):
    rng = np.random.default_rng({"random": 10, "near": 11, "exact": 13}[kind])
    decided = total = 0
    for _ in range(12):
        cand, x, w, s = cases(q, rng, kind=kind)
        want = ggml_pick(q, cand, x, w, s)
        got = filter_pick(filter_keys(q, cand, x, w, s), x, w, s)
        d = got >= 0
        bad = np.nonzero(d & (got != want))[0]
        assert bad.size == 0, ("filter pick differs from the scan", bad[:5], got[bad[:5]], want[bad[:5]])
        decided += int(d.sum())
        total += d.size
    # most searches are decided (zero weights make exact ties); built near-ties mostly go to the exact search
    assert decided > FLOOR[kind] * total, (decided, total)


@pytest.mark.parametrize("plant,kind", [("cross_sign", "random"), ("keep_sign", "exact")])
def test_planted_mistakes_are_caught(q, plant, kind):
    rng = np.random.default_rng(12)
    wrong = 0
    for _ in range(4):
        cand, x, w, s = cases(q, rng, kind=kind)
        want = ggml_pick(q, cand, x, w, s)
        got = filter_pick(filter_keys(q, cand, x, w, s, plant=plant), x, w, s)
        wrong += int(((got >= 0) & (got != want)).sum())
    assert wrong > 0
