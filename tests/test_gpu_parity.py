"""GPU parity: libgpuq.so (HIP, gfx950) against the CPU oracle, byte for byte, on the reference's self-test fixture
(gpuq/test_gpuq.py:57-73: Gaussian, ties, heavy tails, edge rows incl. subnormal x^2), every type, with and without
an imatrix where ggml takes both (gpuq/test_gpuq.py:98-99), through the single and the batch host entry points, and
through the reference library itself built from its own source (oracle/_ref) as a third party to the comparison.
"""
import ctypes
import os

import numpy as np
import pytest

from conftest import REF_LIB, TABLES, selftest_matrices

pytestmark = pytest.mark.gpu

ALL = [8, 10, 11, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29]
NAMES = {8: "q8_0", 10: "q2_k", 11: "q3_k", 12: "q4_k", 13: "q5_k", 14: "q6_k", 16: "iq2_xxs", 17: "iq2_xs",
         18: "iq3_xxs", 19: "iq1_s", 20: "iq4_nl", 21: "iq3_s", 22: "iq2_s", 23: "iq4_xs", 29: "iq1_m"}
TAKES_NO_IM = {8, 10, 11, 12, 13, 14, 20, 23}
CASES = [(t, True) for t in ALL if t != 8] + [(t, False) for t in ALL if t in TAKES_NO_IM]


@pytest.fixture(scope="module")
def gq():
    # torch bundles its own HIP runtime under the same soname as /opt/rocm's: it has to be the one loaded first
    import torch
    torch.cuda.init()
    import gpuq
    return gpuq.load_gpuq(0)


@pytest.fixture(scope="module")
def fixture():
    return selftest_matrices()


_oracle_cache = {}


def oracle_bytes(oracle_lib, typ, with_im, xs, ims):
    key = (typ, with_im)
    if key not in _oracle_cache:
        _oracle_cache[key] = [oracle_lib.quantize(typ, x, im if with_im else None) for x, im in zip(xs, ims)]
    return _oracle_cache[key]


def first_diff(a, b, bb):
    a, b = a.reshape(-1, bb), b.reshape(-1, bb)
    eq = np.all(a == b, axis=1)
    if eq.all():
        return None
    i = int(np.argmin(eq))
    return "%d of %d blocks differ; first %d:\n  oracle %s\n  gpu    %s" % (
        int((~eq).sum()), len(eq), i, a[i].tobytes().hex(), b[i].tobytes().hex())


@pytest.mark.parametrize("typ,with_im", CASES, ids=["%s-%s" % (NAMES[t], "im" if w else "noim") for t, w in CASES])
def test_quantize_matches_oracle(gq, oracle_lib, fixture, typ, with_im):
    xs, ims = fixture
    ne1, ne0 = xs[0].shape
    bb = gq.gpuq_block_bytes(typ)
    assert gq.gpuq_can_quantize(typ, 1 if with_im else 0) == 1
    want = oracle_bytes(oracle_lib, typ, with_im, xs, ims)
    print("case %s %s: single calls" % (NAMES[typ], "im" if with_im else "noim"), flush=True)
    for e, (x, im) in enumerate(zip(xs, ims)):
        out = np.zeros_like(want[e])
        got = gq.gpuq_quantize(typ, x.ctypes.data, out.ctypes.data, ne1, ne0, im.ctypes.data if with_im else None)
        assert got == out.nbytes, (NAMES[typ], e, got)
        d = first_diff(want[e], out, bb)
        assert d is None, "%s matrix %d: %s" % (NAMES[typ], e, d)
    print("case %s %s: batch" % (NAMES[typ], "im" if with_im else "noim"), flush=True)
    xb = np.ascontiguousarray(np.stack(xs))
    ib = np.ascontiguousarray(np.stack(ims))
    out = np.zeros(sum(w.nbytes for w in want), dtype=np.uint8)
    got = gq.gpuq_quantize_batch(typ, xb.ctypes.data, out.ctypes.data, len(xs), ne1, ne0,
                                 ib.ctypes.data if with_im else None)
    assert got == out.nbytes
    d = first_diff(np.concatenate([w.reshape(-1) for w in want]), out, bb)
    assert d is None, "%s batch: %s" % (NAMES[typ], d)
    assert gq.gpuq_take_error() == 0


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_LIB):
        pytest.skip("reference library not built (oracle/_ref needs the reference source at build time)")
    lib = ctypes.CDLL(REF_LIB)
    lib.gpuq_init.argtypes = [ctypes.c_char_p, ctypes.c_int]
    lib.gpuq_quantize.restype = ctypes.c_size_t
    lib.gpuq_quantize.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                  ctypes.c_void_p]
    lib.gpuq_block_bytes.restype = ctypes.c_size_t
    assert lib.gpuq_init(TABLES.encode(), 0) == 0
    return lib


@pytest.mark.parametrize("typ,with_im", CASES, ids=["%s-%s" % (NAMES[t], "im" if w else "noim") for t, w in CASES])
def test_oracle_matches_reference_library(ref, oracle_lib, fixture, typ, with_im):
    """the oracle against the reference's own implementation (its gpuq.hip, compiled from source), same tables"""
    xs, ims = fixture
    ne1, ne0 = xs[0].shape
    bb = ref.gpuq_block_bytes(typ)
    want = oracle_bytes(oracle_lib, typ, with_im, xs, ims)
    print("case ref %s %s" % (NAMES[typ], "im" if with_im else "noim"), flush=True)
    for e, (x, im) in enumerate(zip(xs, ims)):
        out = np.zeros_like(want[e])
        got = ref.gpuq_quantize(typ, x.ctypes.data, out.ctypes.data, ne1, ne0, im.ctypes.data if with_im else None)
        assert got == out.nbytes, (NAMES[typ], e, got)
        d = first_diff(want[e], out, bb)
        assert d is None, "%s matrix %d (oracle vs reference library): %s" % (NAMES[typ], e, d)


def bf16_bytes(x):
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)      # ggml's RNE fp32 -> bf16 (finite inputs)
    return r.view(np.uint8)


def mxfp4_bytes(nblk, seed):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(nblk, 17), dtype=np.uint8)
    raw[:, 0] = 127 + rng.integers(-8, -3, size=nblk)                   # e8m0 exponents -8..-4
    return raw.reshape(-1)


@pytest.mark.parametrize("src", [0, 1, 30, 8, 39], ids=["f32", "f16", "bf16", "q8_0", "mxfp4"])
@pytest.mark.parametrize("typ", [16, 12, 29], ids=["iq2_xxs", "q4_k", "iq1_m"])
def test_requantize_sources(gq, oracle_lib, fixture, src, typ):
    """source bytes decoded on the GPU then quantized == the oracle's decode then quantize (gpuq/test_gpuq.py:143-168)"""
    xs, ims = fixture
    x, im = xs[0][:64], ims[0]
    ne1, ne0 = x.shape
    if src == 0:
        raw = x.view(np.uint8).reshape(-1)
    elif src == 1:
        raw = x.astype(np.float16).view(np.uint8).reshape(-1)
    elif src == 30:
        raw = bf16_bytes(x.reshape(-1))
    elif src == 8:
        raw = oracle_lib.quantize(8, x).reshape(-1)
    else:
        raw = mxfp4_bytes(x.size // 32, 7)
    f = oracle_lib.decode_src(src, raw, x.size).reshape(ne1, ne0)
    want = oracle_lib.quantize(typ, f, im)
    out = np.zeros_like(want)
    print("case requantize src %d -> %s" % (src, NAMES[typ]), flush=True)
    got = gq.gpuq_requantize(src, np.ascontiguousarray(raw).ctypes.data, typ, out.ctypes.data, ne1, ne0, im.ctypes.data)
    assert got == out.nbytes
    d = first_diff(want, out, gq.gpuq_block_bytes(typ))
    assert d is None, d


@pytest.mark.parametrize("typ", [16, 17, 22, 18, 21, 19, 29, 23],
                         ids=["iq2_xxs", "iq2_xs", "iq2_s", "iq3_xxs", "iq3_s", "iq1_s", "iq1_m", "iq4_xs"])
def test_dequantize_dev_matches_oracle(gq, oracle_lib, fixture, typ):
    import torch
    xs, ims = fixture
    x = xs[0][:64]
    q = oracle_lib.quantize(typ, x, ims[0])
    want = oracle_lib.dequantize(typ, q, x.size)
    dq = torch.from_numpy(q.reshape(-1).copy()).cuda()
    out = torch.empty(x.size, dtype=torch.float32, device="cuda")
    nblocks = x.size // 256
    print("case dequantize %s" % NAMES[typ], flush=True)
    got = gq.gpuq_dequantize_dev(typ, dq.data_ptr(), out.data_ptr(), nblocks, None)
    torch.cuda.synchronize()
    assert got == x.size * 4
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("typ", [16, 19, 12], ids=["iq2_xxs", "iq1_s", "q4_k"])
def test_quantize_dev_qw_layout(gq, oracle_lib, fixture, typ):
    """the device API's importance addressing: block b reads qw + ((b % qw_mod) / qw_div) * 256 (ldlq.py's layout:
    B matrices of `rows` rows, one imatrix row a matrix, qw_mod = B*rows, qw_div = rows)"""
    import torch
    xs, ims = fixture
    rows = 32
    blk = np.ascontiguousarray(np.stack([xs[0][:rows, :256], xs[2][:rows, 256:512]]))    # [B=2, rows, 256]
    qw = np.ascontiguousarray(np.stack([ims[0][:256], ims[2][256:512]]))                  # [B, 256]
    want = np.concatenate([oracle_lib.quantize(typ, blk[b], qw[b]).reshape(-1) for b in range(2)])
    d_x = torch.from_numpy(blk).cuda()
    d_qw = torch.from_numpy(qw).cuda()
    d_o = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    print("case quantize_dev %s" % NAMES[typ], flush=True)
    got = gq.gpuq_quantize_dev(typ, d_x.data_ptr(), d_o.data_ptr(), 2 * rows, d_qw.data_ptr(), 2 * rows, rows,
                               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert got == want.size
    d = first_diff(want, d_o.cpu().numpy(), gq.gpuq_block_bytes(typ))
    assert d is None, d
