"""Inputs ggml does not guard against: NaN and infinite weights, NaN, infinite and negative importances.

ggml aborts where a search accepts nothing (every distance of a list NaN or at least FLT_MAX) and where a final
encode meets levels off the grid (gpuq/gpuq.hip:82-86); this library flags those cases, its host entry points answer
0 and gpuq_take_error reports the flag once. Each case's outcome is the oracle's (the CPU test pins which cases
abort); every index the kernels form from such values stays within its table (levels are clamped, grid indices come
from the validated lists, keys are checked against the map), as the oracle's bounds checks confirm for the same
inputs.

Bytes: negative importances are finite and their bytes are the oracle's - they make IQ1_S / IQ1_M's distances
negative (those searches weigh by the importance itself), which the searches order with an order-preserving key
(csrc/coop.cuh). For NaN or infinite inputs that do not abort, ggml's bytes depend on where its left-to-right MAX
folds meet the NaN and on C's conversion of NaN to an integer (undefined), while this library's reductions over a
super-block are order-free: only the abort behaviour is reproduced there."""
import numpy as np
import pytest

ALL = [8, 10, 11, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29]
NAMES = {8: "q8_0", 10: "q2_k", 11: "q3_k", 12: "q4_k", 13: "q5_k", 14: "q6_k", 16: "iq2_xxs", 17: "iq2_xs",
         18: "iq3_xxs", 19: "iq1_s", 20: "iq4_nl", 21: "iq3_s", 22: "iq2_s", 23: "iq4_xs", 29: "iq1_m"}
KINDS = ["nan", "inf", "-inf", "nan_im", "inf_im", "neg_im"]


def case(typ, kind, seed=0, nrow=4, ncol=512):
    rng = np.random.default_rng(seed + typ)
    x = (rng.standard_normal((nrow, ncol)) * 0.02).astype(np.float32)
    im = rng.gamma(1.0, 1.0, ncol).astype(np.float32)
    if kind == "nan":
        x[1, 37] = np.nan
    elif kind == "inf":
        x[1, 37] = np.inf
    elif kind == "-inf":
        x[1, 37] = -np.inf
    elif kind == "nan_im":
        im[37] = np.nan
    elif kind == "inf_im":
        im[37] = np.inf
    elif kind == "neg_im":
        im[::5] *= -1
    return x, (None if typ == 8 else im)


def oracle_outcome(orc, typ, x, im):
    """the oracle's bytes, or None where ggml traps (a search that accepts nothing)"""
    try:
        return orc.quantize(typ, x, im).reshape(-1)
    except RuntimeError:
        return None


def test_which_cases_trap(oracle_lib):
    """the cases that trap are searches whose every distance is NaN or infinite: a non-finite weight in the types
    that search with the square root of the weight, an infinite importance, a negative importance under a square
    root; the types without a grid search never trap"""
    traps = {k: sorted(t for t in ALL if oracle_outcome(oracle_lib, t, *case(t, k)) is None) for k in KINDS}
    for k in ("nan", "inf", "-inf"):
        assert traps[k] == [17, 18, 21, 22], (k, traps[k])   # IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S
    assert {17, 22} <= set(traps["nan_im"]) and {16, 19, 29} <= set(traps["inf_im"]), traps
    assert {16, 17, 22} <= set(traps["neg_im"]) and not {19, 29} & set(traps["neg_im"]), traps
    for t in (8, 10, 11, 12, 13, 14, 20, 23):
        assert all(t not in v for v in traps.values()), t


@pytest.mark.gpu
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("typ", ALL, ids=[NAMES[t] for t in ALL])
def test_failure_path_matches_oracle(oracle_lib, typ, kind):
    import torch
    torch.cuda.init()
    import gpuq
    gq = gpuq.load_gpuq(0)
    x, im = case(typ, kind)
    want = oracle_outcome(oracle_lib, typ, x, im)
    nb = x.shape[0] * gpuq.row_bytes(gq, typ, x.shape[1])
    out = np.zeros(nb, dtype=np.uint8)
    print("case failure %s %s" % (NAMES[typ], kind), flush=True)
    got = gq.gpuq_quantize(typ, x.ctypes.data, out.ctypes.data, x.shape[0], x.shape[1],
                           None if im is None else im.ctypes.data)
    exact = kind == "neg_im"                                # (finite inputs: the bytes are defined)
    if want is None:
        assert got == 0
        assert gq.gpuq_take_error() == 1
        assert gq.gpuq_take_error() == 0
    else:
        assert got == nb and (not exact or np.array_equal(out, want))
        assert gq.gpuq_take_error() == 0
    # the device entry point: the flag alone reports it
    d_x = torch.from_numpy(x).cuda()
    d_im = None if im is None else torch.from_numpy(im).cuda()
    d_out = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    n = gq.gpuq_requantize_dev(0, d_x.data_ptr(), typ, d_out.data_ptr(), 1, x.shape[0], x.shape[1],
                               None if d_im is None else d_im.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert n == nb
    assert gq.gpuq_take_error() == (1 if want is None else 0)
    if want is not None and exact:
        assert np.array_equal(d_out.cpu().numpy(), want)
    assert gq.gpuq_take_error() == 0


def negative_importance_case(typ):
    rng = np.random.default_rng(typ)
    x = (rng.standard_normal((64, 2048)) * 0.02).astype(np.float32)
    im = (rng.gamma(1.0, 1.0, 2048) * rng.choice([-1.0, 1.0], 2048, p=[0.3, 0.7])).astype(np.float32)
    return x, im


@pytest.mark.parametrize("typ", [19, 29], ids=["iq1_s", "iq1_m"])
def test_negative_importance_reaches_negative_distances(oracle_lib, typ):
    x, im = negative_importance_case(typ)
    oracle_lib.stats_read_reset()
    oracle_lib.quantize(typ, x, im)
    assert oracle_lib.stats_read_reset()["nb1_negative"] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("typ", [19, 29], ids=["iq1_s", "iq1_m"])
def test_negative_importance_iq1(oracle_lib, typ):
    """IQ1 with many negative importances: negative distances chosen as ggml chooses them"""
    import torch
    torch.cuda.init()
    import gpuq
    gq = gpuq.load_gpuq(0)
    x, im = negative_importance_case(typ)
    want = oracle_lib.quantize(typ, x, im).reshape(-1)
    d_x, d_im = torch.from_numpy(x).cuda(), torch.from_numpy(im).cuda()
    d_out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    print("case negative importance %s" % NAMES[typ], flush=True)
    n = gq.gpuq_requantize_dev(0, d_x.data_ptr(), typ, d_out.data_ptr(), 1, 64, 2048, d_im.data_ptr(),
                               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert n == want.size
    out = d_out.cpu().numpy()
    assert np.array_equal(out, want), "%d bytes differ" % int((out != want).sum())
    assert gq.gpuq_take_error() == 0


KQ = [10, 11, 12, 13, 14]
KQ_LANES = {10: 16, 11: 16, 12: 8, 13: 8, 14: 16}      # lanes a super-block: a wave holds 64 / lanes super-blocks


def mixed_wave_case(typ, seed=3):
    """a NaN and an infinite value in two super-blocks of their waves; every other super-block finite"""
    rng = np.random.default_rng(seed + typ)
    x = (rng.standard_normal((8, 2048)) * 0.02).astype(np.float32)
    x[1, 37] = np.nan
    x[5, 1500] = np.inf
    im = rng.lognormal(0.0, 1.5, 2048).astype(np.float32)
    return x, im


def test_mixed_waves_hold_finite_super_blocks():
    for typ in KQ + [16]:
        x, _ = mixed_wave_case(typ)
        sb = x.reshape(-1, 256)
        bad = ~np.isfinite(sb).all(1)
        waves = bad.reshape(-1, 64 // (8 if typ == 16 else KQ_LANES[typ]))
        mixed = waves.any(1) & ~waves.all(1)
        assert mixed.sum() == 2 and not waves[~mixed].any(), typ


@pytest.mark.gpu
@pytest.mark.parametrize("with_im", [False, True], ids=["plain", "imatrix"])
@pytest.mark.parametrize("typ", KQ, ids=[NAMES[t] for t in KQ])
def test_finite_super_blocks_beside_non_finite(oracle_lib, typ, with_im):
    """A wave holding a NaN or an infinite value rounds its symmetric trials with the integer loop (the others in
    float, csrc/kquants.cuh sym_levels); the super-blocks without such values are the oracle's bytes either way."""
    import torch
    torch.cuda.init()
    import gpuq
    gq = gpuq.load_gpuq(0)
    x, im = mixed_wave_case(typ)
    im = im if with_im else None
    want = oracle_lib.quantize(typ, x, im).reshape(-1)
    bb = gq.gpuq_block_bytes(typ)
    d_x = torch.from_numpy(x).cuda()
    d_im = None if im is None else torch.from_numpy(im).cuda()
    d_out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    print("case mixed waves %s %s" % (NAMES[typ], "imatrix" if with_im else "plain"), flush=True)
    n = gq.gpuq_requantize_dev(0, d_x.data_ptr(), typ, d_out.data_ptr(), 1, x.shape[0], x.shape[1],
                               None if d_im is None else d_im.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert n == want.size
    gq.gpuq_take_error()
    fin = np.isfinite(x.reshape(-1, 256)).all(1)
    out = d_out.cpu().numpy().reshape(-1, bb)
    assert np.array_equal(out[fin], want.reshape(-1, bb)[fin])


@pytest.mark.gpu
def test_iq2_xxs_finite_super_blocks_beside_non_finite(oracle_lib):
    """IQ2_XXS super-blocks without a NaN or infinite value, in waves (8 super-blocks) that hold one, are the oracle's
    bytes, taken from the oracle on the same rows with the non-finite values set to 0 (a super-block's bytes depend
    only on its own values and importances): the wave-wide searches a non-finite group takes part in leave its
    neighbours' results alone."""
    import torch
    torch.cuda.init()
    import gpuq
    gq = gpuq.load_gpuq(0)
    typ = 16
    x, im = mixed_wave_case(typ)
    want = oracle_lib.quantize(typ, np.where(np.isfinite(x), x, 0).astype(np.float32), im).reshape(-1)
    bb = gq.gpuq_block_bytes(typ)
    d_x = torch.from_numpy(x).cuda()
    d_im = torch.from_numpy(im).cuda()
    d_out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    print("case mixed waves iq2_xxs imatrix", flush=True)
    n = gq.gpuq_requantize_dev(0, d_x.data_ptr(), typ, d_out.data_ptr(), 1, x.shape[0], x.shape[1], d_im.data_ptr(),
                               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert n == want.size
    gq.gpuq_take_error()
    fin = np.isfinite(x.reshape(-1, 256)).all(1)
    assert fin.sum() == fin.size - 2
    out = d_out.cpu().numpy().reshape(-1, bb)
    assert np.array_equal(out[fin], want.reshape(-1, bb)[fin])
