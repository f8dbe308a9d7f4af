"""The two variants of IQ1_S's partition scan (csrc/iq1.cuh): a wave whose scanning lanes all have weights 0 or in
[2^-100, 2^100] drops the scan's `sumq2 > 0` test (and starts a lane of zero weights from +inf); any other wave keeps
it. Inputs that put waves on both sides, against the oracle byte for byte (IQ1_M, whose scan keeps the test, on the
same inputs):

- blocks whose weights are all 0 (importance 0 over the whole block) beside ordinary blocks, and scattered zero
  importances: the test-free variant with +inf starts;
- rows of magnitude 1e-6 where a few columns have importance 1e-25 (weights ~1e-31, below 2^-100) beside rows of
  magnitude 0.02 (the same columns' weights ~3e-27): waves of the first kind keep the test, of the second drop it,
  and the waves that hold one row of each keep it.

The CPU test pins that the constructions produce those weights."""
import numpy as np
import pytest

IQ1_S, IQ1_M, F32 = 19, 29, 0
NAMES = {19: "iq1_s", 29: "iq1_m"}
PLAIN_LO, PLAIN_HI = 2.0 ** -100, 2.0 ** 100


def zero_weight_blocks(nrow=16, ncol=2048, seed=5):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((nrow, ncol)) * 0.02).astype(np.float32)
    im = rng.lognormal(0, 1.5, ncol).astype(np.float32)
    for b in range(0, ncol, 256):
        im[b + 96:b + 128] = 0          # a whole 32-block (two IQ1_M 16-blocks)
        im[b + 208:b + 224] = 0         # one IQ1_M 16-block, half of an IQ1_S block
    im[rng.integers(0, ncol, 40)] = 0
    return x, im


def tiny_weight_rows(nrow=16, ncol=2048, seed=6):
    rng = np.random.default_rng(seed)
    mag = np.array([0.02, 1e-6, 1e-6, 1e-6, 0.02, 0.02, 1e-6, 0.02])[np.arange(nrow) % 8]
    x = (rng.standard_normal((nrow, ncol)) * mag[:, None]).astype(np.float32)
    im = rng.lognormal(0, 1.0, ncol).astype(np.float32)
    im[rng.integers(0, ncol, 64)] = 1e-25
    return x, im


CASES = {"zero_weight_blocks": zero_weight_blocks, "tiny_weight_rows": tiny_weight_rows}


def lane_weights(x, im, n):
    """the lanes' weights as the kernels form them: importance * sqrt(2 sum(x^2)/256 + x^2), n weights a lane"""
    xs = x.reshape(-1, 256)
    sigma2 = 2 * (xs.astype(np.float64) ** 2).sum(1) / 256
    w = np.tile(im.reshape(-1, 256), (x.shape[0], 1)) * np.sqrt(sigma2[:, None] + xs.astype(np.float64) ** 2)
    return w.reshape(-1, n)


def plain(w):
    return ((w == 0) | ((w >= PLAIN_LO) & (w <= PLAIN_HI))).all(1)


def test_constructions_reach_both_variants():
    x, im = zero_weight_blocks()
    for n in (32, 16):
        w = lane_weights(x, im, n)
        assert plain(w).all() and (w == 0).all(1).any() and ((w == 0).any(1) & (w > 0).any(1)).any(), n
    x, im = tiny_weight_rows()
    for n, lanes in ((32, 64), (16, 64)):
        ok = plain(lane_weights(x, im, n)).reshape(-1, lanes).all(1)     # a wave: 64 lanes
        assert ok.any() and not ok.all(), n
    # IQ1_S waves of one row of each magnitude (rows 0-1, 6-7)
    ok = plain(lane_weights(x, im, 32)).reshape(-1, 64)
    assert (ok.any(1) & ~ok.all(1)).any()


@pytest.mark.gpu
@pytest.mark.parametrize("typ", [IQ1_S, IQ1_M], ids=[NAMES[IQ1_S], NAMES[IQ1_M]])
@pytest.mark.parametrize("name", sorted(CASES))
def test_scan_variants_match_oracle(oracle_lib, name, typ):
    import torch
    torch.cuda.init()
    import gpuq
    gq = gpuq.load_gpuq(0)
    x, im = CASES[name]()
    want = oracle_lib.quantize(typ, x, im).reshape(-1)
    d_x = torch.from_numpy(x).cuda()
    d_im = torch.from_numpy(im).cuda()
    d_out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    print("case iq1 scan %s %s" % (NAMES[typ], name), flush=True)
    got = gq.gpuq_requantize_dev(F32, d_x.data_ptr(), typ, d_out.data_ptr(), 1, x.shape[0], x.shape[1],
                                 d_im.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert got == want.size
    out = d_out.cpu().numpy()
    assert np.array_equal(out, want), "%d bytes differ" % int((out != want).sum())
    assert gq.gpuq_take_error() == 0
