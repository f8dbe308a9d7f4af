"""The two variants of IQ1_S's partition scan (csrc/iq1.cuh): a wave whose scanning lanes all have weights 0 or in
[2^-100, 2^100] drops the scan's `sumq2 > 0` test (and starts a lane of zero weights from +inf); any other wave keeps
it. Inputs that put waves on both sides, against the oracle byte for byte (IQ1_M, whose scan keeps the test, on the
same inputs):

- blocks whose weights are all 0 (importance 0 over the whole block) beside ordinary blocks, and scattered zero
  importances: the test-free variant with +inf starts;
- rows of magnitude 1e-6 where a few columns have importance 1e-25 (weights ~1e-31, below 2^-100) beside rows of
  magnitude 0.02 (the same columns' weights ~3e-27): waves of the first kind keep the test, of the second drop it,
  and the waves that hold one row of each keep it.

IQ1_M ranks its candidates first (an approximate score, no branches) and runs the acceptance chain only on the lanes
whose best candidate does not stand clear of the second, or whose weights or sums leave the safe range
(iq1_rank_ok): the zero-weight blocks give exact ties at the top (a zero weight between two boundaries changes no
sum), the tiny-weight rows weights out of range, and both put such lanes in waves beside lanes the ranking settles.

The CPU tests pin that the constructions produce those weights and those lanes (the latter from the kernel's own
float32 sums of every candidate)."""
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


def iq1m_rank_lanes(x, im):
    """IQ1_M lanes that the ranking pass settles for certain and that certainly replay the chain: every candidate's
    sumqx and sumq2 as the kernel forms them (float32, operation by operation: sequential sigma2 sum, weights, prefix
    sums in stable rank order split by half, then csrc/iq1.cuh iq1m_sums), T = sumqx^2 / sumq2 in float64, the
    relative gap between the two largest T; the kernel's scores are T within 4 units of 2^-24, so a gap above 2^-18
    (with the range conditions met) settles and one below 2^-22 (or a condition failed) replays. Lanes skipped as
    negligible (max |x| < 1e-7) count as neither."""
    f = np.float32
    xs = x.reshape(-1, 16).astype(f)
    nl = xs.shape[0]
    sq = xs * xs
    sb = sq.reshape(-1, 256)
    acc = np.zeros(sb.shape[0], f)
    for i in range(256):
        acc = (acc + sb[:, i]).astype(f)
    sigma2 = np.repeat(f(2) * acc / f(256), 16)
    qv = np.tile(im.reshape(-1, 16).astype(f), (x.shape[0], 1))
    w = (qv * np.sqrt((sigma2[:, None] + sq).astype(f))).astype(f)
    order = np.argsort(xs, axis=1, kind="stable")
    px = [np.zeros((nl, 17), f), np.zeros((nl, 17), f)]
    pw = [np.zeros((nl, 17), f), np.zeros((nl, 17), f)]
    rows = np.arange(nl)
    for j in range(16):
        e = order[:, j]
        vx, vw, h = (w[rows, e] * xs[rows, e]).astype(f), w[rows, e], e >= 8
        for hh in (0, 1):
            sel = h == bool(hh)
            px[hh][:, j + 1] = np.where(sel, px[hh][:, j] + vx, px[hh][:, j])
            pw[hh][:, j + 1] = np.where(sel, pw[hh][:, j] + vw, pw[hh][:, j])
    txs, tws = [px[0][:, 16], px[1][:, 16]], [pw[0][:, 16], pw[1][:, 16]]
    p2, m2 = f(1.125), f(0.875)
    cp1, cp2, cm1, cm2 = f(0.75), f(-1.25), f(1.25), f(-0.75)
    T = []
    for i1 in range(17):
        for i2 in range(i1, 17):
            qx, q2 = {}, {}
            for hh in (0, 1):
                sx = px[hh][:, i1] + px[hh][:, i2]
                qx[hh, 0] = txs[hh] * p2 - sx
                qx[hh, 1] = txs[hh] * m2 - sx
                q2[hh, 0] = tws[hh] * p2 * p2 + pw[hh][:, i1] * cp1 + pw[hh][:, i2] * cp2
                q2[hh, 1] = tws[hh] * m2 * m2 + pw[hh][:, i1] * cm1 + pw[hh][:, i2] * cm2
            for k in range(4):
                sqx = (qx[0, k >> 1] + qx[1, k & 1]).astype(np.float64)
                sq2 = (q2[0, k >> 1] + q2[1, k & 1]).astype(np.float64)
                T.append(np.where(sq2 > 0, sqx * sqx / np.where(sq2 > 0, sq2, 1), -1))
    T = np.sort(np.stack(T, 1), 1)
    t1, t2 = T[:, -1], T[:, -2]
    gap = (t1 - t2) / np.where(t1 > 0, t1, 1)
    totw = (tws[0] + tws[1]).astype(f)
    mx = np.abs(xs).max(1)
    inrange = plain(w) & (totw >= 2.0 ** -40) & (totw <= 2.0 ** 40) & (mx * totw <= 2.0 ** 50)
    settle = inrange & (t1 >= 2.0 ** -58) & (t1 <= 2.0 ** 98) & (gap > 2.0 ** -18)
    replay = ~inrange | (gap < 2.0 ** -22)
    scanned = ~(mx < 1e-7)
    return settle & scanned, replay & scanned


def test_iq1m_constructions_reach_both_paths():
    for name, make in sorted(CASES.items()):
        settle, replay = iq1m_rank_lanes(*make())
        assert settle.any() and replay.any(), name
        waves = settle.size // 64
        mixed = settle[:waves * 64].reshape(waves, 64).any(1) & replay[:waves * 64].reshape(waves, 64).any(1)
        assert mixed.any(), name


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
