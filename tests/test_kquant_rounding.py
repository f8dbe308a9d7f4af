"""The k-quants' trial levels formed in float (csrc/kquants.cuh: affine_levels with the imatrix, sym_levels) against
ggml's integer rule, over a dense sample of float32 bit patterns.

ggml rounds with nearest_int(v) = (bits(v + 1.5*2^23) & 0x7fffff) - 0x400000 (gpuq/gpuq.hip:108-112) and clamps the
integer. The kernels form the clamped level in float: round(c) = (c + 1.5*2^23) - 1.5*2^23 of c = min(max(v, lo), hi)
with IEEE max and min (a NaN operand gives the other one; numpy's fmax / fmin), which for the imatrix affine rule
`v > 0 ? nearest_int(v < nmax ? v : nmax) : 0` (gpuq/gpuq.hip:1556-1560) holds for every input, NaN and infinities
included, and for the symmetric rule `MAX(-nmax, MIN(nmax-1, nearest_int(v)))` (gpuq/gpuq.hip:1448-1452) for finite
|v| <= 2^21 (ggml's nearest_int stops being a rounding just below 2^22: 4194303.5 gives -4194304) - the kernels take
that path only in waves whose values are all finite, where |v| <= nmax + 0.9, and the NaN case below shows why the
guard is needed. numpy's nearest_int is checked against the oracle's first.
"""
import numpy as np

F32 = np.float32
RND = F32(12582912.0)


def ggml_nint(v):
    t = (v.astype(F32) + RND).astype(F32)
    return (t.view(np.int32) & 0x7fffff) - 0x400000


def float_round(c):
    return ((c.astype(F32) + RND).astype(F32) - RND).astype(F32)


def sample():
    bits = np.arange(0, 1 << 32, 1021, dtype=np.uint64).astype(np.uint32)
    v = bits.view(F32)
    ties = np.arange(-140, 141, dtype=F32) / F32(2)               # every half-integer tie in the levels' range
    near = np.concatenate([np.nextafter(ties, F32(np.inf)), np.nextafter(ties, F32(-np.inf))]).astype(F32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 4194303.5, 4194304.0, 8388608.0,
                        -4194304.0, 3.4028235e38, -3.4028235e38], dtype=F32)
    return np.concatenate([v, ties, near, special]).astype(F32)


def test_numpy_nearest_int_is_the_oracles(oracle_lib):
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.uniform(-200, 200, 4000), rng.standard_normal(2000) * 1e6,
                        np.arange(-70, 71) / 2.0]).astype(F32)
    want = np.array([oracle_lib.nearest_int(float(x)) for x in v])
    assert np.array_equal(ggml_nint(v), want)


def test_affine_imatrix_rule_in_float():
    v = sample()
    with np.errstate(invalid="ignore", over="ignore"):
        for nmax in (3, 15, 31, 63):
            want = np.where(v > 0, ggml_nint(np.where(v < nmax, v, F32(nmax))), 0).astype(F32)
            got = float_round(np.fmin(np.fmax(v, F32(0)), F32(nmax)))
            assert np.array_equal(got, want), nmax


def test_symmetric_rule_in_float_for_finite_values():
    v = sample()
    with np.errstate(invalid="ignore", over="ignore"):
        for nmax in (4, 32):
            want = np.maximum(-nmax, np.minimum(nmax - 1, ggml_nint(v))).astype(F32)
            got = float_round(np.fmin(np.fmax(v, F32(-nmax)), F32(nmax - 1)))
            ok = np.isfinite(v) & (np.abs(v) <= 2.0 ** 21)
            assert np.array_equal(got[ok], want[ok]), nmax
            # why waves with a NaN keep the integer loop: ggml's rounding takes a NaN's level from its payload (0 for
            # the canonical quiet NaN), the float clamp gives -nmax
            qnan = np.array([np.nan], F32)
            clamped = float_round(np.fmin(np.fmax(qnan, F32(-nmax)), F32(nmax - 1)))
            assert ggml_nint(qnan)[0] == 0 and clamped[0] == -nmax
        big = F32(4194303.5)                                               # (and where nearest_int ends)
        assert ggml_nint(np.array([big]))[0] == -4194304
