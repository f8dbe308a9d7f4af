"""The oracle's scalar arithmetic and source decoders against closed forms, exhaustively where the domain allows.

- fp32 -> fp16 (ggml's bit trick, gpuq/gpuq.hip:91-106) against IEEE round-to-nearest-even (numpy) for all 2^32
  inputs; NaN -> sign | 0x7E00.
- fp16 -> fp32 for all 65536 halves; BF16 -> fp32 for all 65536; MXFP4 for all 256 exponents x 256 code bytes.
- nearest_int (gpuq/gpuq.hip:108-112) against rint (ties to even) for |x| < 2^22, including every half-integer tie.
- Q8_0 (gpuq/gpuq.hip:1831-1838) against its closed form.
"""
import concurrent.futures

import numpy as np
import pytest

import oracle as O


def test_fp32_to_fp16_exhaustive(oracle_lib):
    lib = oracle_lib.lib
    chunk = 1 << 22
    nthr = 8
    base = np.arange(chunk, dtype=np.uint32)

    def worker(t):
        bits = np.empty(chunk, dtype=np.uint32)
        got = np.empty(chunk, dtype=np.uint16)
        want = np.empty(chunk, dtype=np.float16)
        for c in range(t, 1 << 10, nthr):
            first = c * chunk
            np.add(base, np.uint32(first), out=bits)
            lib.gqo_fp32_to_fp16_range(first, chunk, got.ctypes.data)
            f = bits.view(np.float32)
            with np.errstate(over="ignore", invalid="ignore"):
                want[:] = f
            w = want.view(np.uint16)
            bad = np.nonzero(got != w)[0]
            for i in bad:                                   # NaN inputs: sign | 0x7E00
                if not (np.isnan(f[i]) and got[i] == (((int(bits[i]) >> 16) & 0x8000) | 0x7E00)):
                    return (first + int(i), int(got[i]), int(w[i]))
        return None

    with concurrent.futures.ThreadPoolExecutor(nthr) as ex:
        res = list(ex.map(worker, range(nthr)))
    fails = [r for r in res if r is not None]
    assert not fails, "fp32 0x%08x -> 0x%04x, RNE gives 0x%04x" % fails[0]


def test_fp16_to_fp32_all(oracle_lib):
    out = np.empty(65536, dtype=np.float32)
    oracle_lib.lib.gqo_fp16_to_fp32_all(out.ctypes.data)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(out[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(out[nan]).all()


def test_nearest_int_is_rint():
    o = O.Oracle()
    rng = np.random.default_rng(5)
    xs = list(rng.uniform(-4e6, 4e6, 2000)) + list(rng.uniform(-40, 40, 2000))
    xs += [k + 0.5 for k in range(-50, 50)] + [-0.5, 0.5, -0.0, 0.0, 2.5, 3.5, 4194302.5, -4194302.5]
    for x in xs:
        x32 = float(np.float32(x))
        assert o.nearest_int(x32) == int(np.rint(np.float32(x32))), x32


def test_decode_bf16_all(oracle_lib):
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle_lib.decode_src(O.BF16, raw.view(np.uint8), 65536)
    assert np.array_equal(got.view(np.uint32), raw.astype(np.uint32) << 16)


def test_decode_f16_all(oracle_lib):
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle_lib.decode_src(O.F16, raw.view(np.uint8), 65536)
    want = raw.view(np.float16).astype(np.float32)
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


def test_decode_mxfp4_all_pairs(oracle_lib):
    """every (e8m0, code byte) pair: value = e2m1(nibble) * 2^(e-127), e2m1 = {0,.5,1,1.5,2,3,4,6} with sign"""
    e2m1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float64)
    blocks = []
    for e in range(256):
        for b0 in range(0, 256, 16):
            blocks.append(np.concatenate([[e], np.arange(b0, b0 + 16)]).astype(np.uint8))
    raw = np.concatenate(blocks)
    got = oracle_lib.decode_src(O.MXFP4, raw, len(blocks) * 32).reshape(-1, 32)
    for k, blk in enumerate(blocks):
        e = int(blk[0])
        scale = np.ldexp(1.0, e - 127)
        lo = e2m1[blk[1:] & 15] * scale
        hi = e2m1[blk[1:] >> 4] * scale
        with np.errstate(over="ignore"):                   # (the largest exponents overflow fp32 to +-inf)
            want = np.concatenate([lo, hi]).astype(np.float32)
        assert np.array_equal(got[k], want), (e, blk[1])


def test_decode_q8_0(oracle_lib):
    rng = np.random.default_rng(3)
    nb = 512
    raw = rng.integers(0, 256, size=(nb, 34), dtype=np.uint8)
    d16 = rng.uniform(-2, 2, nb).astype(np.float16)
    raw[:, 0:2] = d16.view(np.uint8).reshape(nb, 2)
    got = oracle_lib.decode_src(O.Q8_0, raw.reshape(-1), nb * 32).reshape(nb, 32)
    want = raw[:, 2:].view(np.int8).astype(np.float32) * d16.astype(np.float32)[:, None]
    assert np.array_equal(got, want)


def q8_0_closed_form(x):
    """amax/127, id = 1/d (0 for d = 0), fp16 d, qs = round half away from zero of x*id"""
    x = x.reshape(-1, 32).astype(np.float32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = (x * idv[:, None]).astype(np.float32)
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)
    out = np.empty((x.shape[0], 34), dtype=np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def test_q8_0_closed_form(oracle_lib):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((64, 4096)) * 0.02).astype(np.float32)
    x[0] = 0
    x[1, ::3] = 1e-30
    x[2] = np.float32(65504 * 127)
    x[3, 5] = -7.5
    got = oracle_lib.quantize(O.Q8_0, x).reshape(-1)
    assert np.array_equal(got, q8_0_closed_form(x))
