"""The filtered neighbour search of IQ2_XXS and IQ2_XS (csrc/filter.cuh, window_group in csrc/iq2.cuh) on inputs
built to reach the cases it hands elsewhere, against the oracle byte for byte (IQ2_S, whose searches are exact, on
the same inputs):

- exact ties between candidates (the least distance shared): the filter's margin test cannot decide them and the
  exact cooperative search repeats ggml's first-wins scan (|x| equal within a row, weights equal or zero, so
  candidates that permute one another's levels tie);
- sub-blocks whose acceptance chain ends at a negative scale (a tiny value of the opposite sign with a huge importance
  in a group of equal values: its sign flip makes the accepted sum of w*x*q negative), where the final pass does not
  run and the accepted trial's grid points are kept;
- magnitudes where the filter's bound is out of its range (tiny and huge rows) and everything in between.

The CPU test pins that each construction reaches its case, with the oracle's path counters (gq_oracle.h); the GPU
test compares the library's bytes with the oracle's on the same inputs."""
import numpy as np
import pytest

IQ2_XXS, IQ2_XS, IQ2_S, F32 = 16, 17, 22, 0
TYPES = {16: "iq2_xxs", 17: "iq2_xs", 22: "iq2_s"}
NEGCHAIN = {16: "iq2xxs_negchain", 17: "iq2x16_negchain"}  # (IQ2_S keeps each sign: no flipped value)


def negchain(nrow=16, ncol=2048, seed=0):
    rng = np.random.default_rng(seed)
    im = np.ones(ncol, np.float32)
    cols = np.arange(0, ncol, 32) + rng.integers(0, 32, ncol // 32)      # one special column a sub-block
    im[cols] = np.array([1e4, 1e5, 3e5, 1e6], np.float32)[np.arange(cols.size) % 4]
    eps = np.array([1e-3, 3e-3, 1e-2, 1e-3])[np.arange(nrow) % 4]
    mag = np.array([0.02, 1.0, 3e-4, 50.0])[(np.arange(nrow) // 4) % 4]
    x = np.ones((nrow, ncol)) * mag[:, None]
    x[:, cols] = -(eps * mag)[:, None]
    return x.astype(np.float32), im


def symmetric(nrow=16, ncol=2048, seed=1):
    rng = np.random.default_rng(seed)
    a = np.array([0.02, 1.0, 0.5, 3e-3])[np.arange(nrow) % 4]
    x = (rng.choice([-1.0, 1.0], (nrow, ncol)) * a[:, None]).astype(np.float32)
    im = np.ones(ncol, np.float32)
    im[::7] = 0.0
    return x, im


def magnitudes(nrow=16, ncol=2048, seed=2):
    rng = np.random.default_rng(seed)
    mag = np.array([1e-14, 1e-12, 1e-10, 1e6, 1e8, 1e9, 2e9, 1.0])[np.arange(nrow) % 8]
    x = (rng.standard_normal((nrow, ncol)) * mag[:, None]).astype(np.float32)
    im = rng.lognormal(0, 1.5, ncol).astype(np.float32)
    return x, im


CASES = {"negchain": negchain, "symmetric": symmetric, "magnitudes": magnitudes}


@pytest.mark.parametrize("typ", sorted(TYPES), ids=[TYPES[t] for t in sorted(TYPES)])
def test_constructions_reach_their_cases(oracle_lib, typ):
    bb = {16: 66, 17: 74, 22: 82}[typ]
    want = {"negchain": NEGCHAIN.get(typ, "nb8_ties"), "symmetric": "nb8_ties", "magnitudes": "nb8_searches"}
    for name, make in CASES.items():
        x, im = make()
        oracle_lib.stats_read_reset()
        q = oracle_lib.quantize(typ, x, im)
        st = oracle_lib.stats_read_reset()
        assert q.size == x.size // 256 * bb, name                 # (no trap: every search accepted a point)
        assert st[want[name]] > 0, (name, st)
    if typ in NEGCHAIN:
        x, im = negchain()
        oracle_lib.stats_read_reset()
        oracle_lib.quantize(typ, x, im)
        st = oracle_lib.stats_read_reset()
        per = 32 if typ == 16 else 16                           # (weights a sub-block)
        assert st[NEGCHAIN[typ]] >= x.size // per // 8 and st["nb8_ties"] > st["nb8_searches"] // 2, st


@pytest.mark.gpu
@pytest.mark.parametrize("typ", sorted(TYPES), ids=[TYPES[t] for t in sorted(TYPES)])
@pytest.mark.parametrize("name", sorted(CASES))
def test_filter_cases_match_oracle(oracle_lib, name, typ):
    import torch
    import gpuq
    gq = gpuq.load_gpuq(0)
    x, im = CASES[name]()
    want = oracle_lib.quantize(typ, x, im).reshape(-1)
    d_x = torch.from_numpy(x).cuda()
    d_im = torch.from_numpy(im).cuda()
    d_out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    print("case filter %s %s" % (TYPES[typ], name), flush=True)
    got = gq.gpuq_requantize_dev(F32, d_x.data_ptr(), typ, d_out.data_ptr(), 1, x.shape[0], x.shape[1],
                                 d_im.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert got == want.size
    out = d_out.cpu().numpy()
    assert np.array_equal(out, want), "%d bytes differ" % int((out != want).sum())
    assert gq.gpuq_take_error() == 0
