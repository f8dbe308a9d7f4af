"""The device-pointer entry points this library adds or keeps, against the oracle on the same bytes:
gpuq_requantize_dev (source bytes in HBM decoded inside the quantize kernel: F32, F16, BF16, Q8_0 and MXFP4, several
matrices of an odd row count, one imatrix row a matrix, every type), gpuq_dequantize_src_dev (every source encoding,
gpuq/gpuq.hip:2323-2328 of the reference), gpuq_dequantize_dev of the k-quants, the argument checks that answer 0
before any launch, and the stand-in table guard of gpuq_init."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ALL = [8, 10, 11, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29]
NAMES = {8: "q8_0", 10: "q2_k", 11: "q3_k", 12: "q4_k", 13: "q5_k", 14: "q6_k", 16: "iq2_xxs", 17: "iq2_xs",
         18: "iq3_xxs", 19: "iq1_s", 20: "iq4_nl", 21: "iq3_s", 22: "iq2_s", 23: "iq4_xs", 29: "iq1_m"}
F32, F16, Q8_0, BF16, MXFP4 = 0, 1, 8, 30, 39


@pytest.fixture(scope="module")
def env():
    import torch
    torch.cuda.init()
    import gpuq
    return torch, gpuq.load_gpuq(0)


def source(oracle_lib, src, x, seed):
    """x: f32 [nmat, nrow, ncol] -> the source bytes of encoding src (MXFP4: random codes, not x)"""
    flat = np.ascontiguousarray(x.reshape(-1))
    if src == F32:
        return flat.view(np.uint8)
    if src == F16:
        return flat.astype(np.float16).view(np.uint8)
    if src == BF16:
        u = flat.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).view(np.uint8)
    if src == Q8_0:
        return oracle_lib.quantize(8, x.reshape(-1, x.shape[-1])).reshape(-1)
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(flat.size // 32, 17), dtype=np.uint8)
    raw[:, 0] = 127 + rng.integers(-8, -3, size=raw.shape[0])
    return raw.reshape(-1)


@pytest.mark.parametrize("src", [F32, F16, BF16, Q8_0, MXFP4], ids=["f32", "f16", "bf16", "q8_0", "mxfp4"])
@pytest.mark.parametrize("typ", ALL, ids=[NAMES[t] for t in ALL])
def test_requantize_dev_matches_oracle(env, oracle_lib, typ, src):
    torch, gq = env
    nmat, nrow, ncol = 3, 5, 512
    rng = np.random.default_rng(typ * 100 + src)
    x = (rng.standard_normal((nmat, nrow, ncol)) * rng.uniform(0.01, 0.03, (nmat, 1, 1))).astype(np.float32)
    im = rng.lognormal(0.0, 1.5, (nmat, ncol)).astype(np.float32)
    raw = np.ascontiguousarray(source(oracle_lib, src, x, seed=typ))
    f = oracle_lib.decode_src(src, raw, x.size).reshape(nmat, nrow, ncol)
    use_im = typ != 8
    want = np.concatenate([oracle_lib.quantize(typ, f[m], im[m] if use_im else None).reshape(-1)
                           for m in range(nmat)])
    d_raw = torch.from_numpy(raw).cuda()
    d_im = torch.from_numpy(im).cuda()
    d_out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    print("case requantize_dev %s src %d" % (NAMES[typ], src), flush=True)
    got = gq.gpuq_requantize_dev(src, d_raw.data_ptr(), typ, d_out.data_ptr(), nmat, nrow, ncol,
                                 d_im.data_ptr() if use_im else None, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert got == want.size
    out = d_out.cpu().numpy()
    assert np.array_equal(out, want), "%d bytes differ" % int((out != want).sum())
    assert gq.gpuq_take_error() == 0


@pytest.mark.parametrize("src", [F32, F16, BF16, Q8_0, MXFP4], ids=["f32", "f16", "bf16", "q8_0", "mxfp4"])
def test_dequantize_src_dev_matches_oracle(env, oracle_lib, src):
    torch, gq = env
    rng = np.random.default_rng(src)
    x = (rng.standard_normal((1, 8, 512)) * 0.05).astype(np.float32)
    x[0, 0, :32] = 0
    x[0, 1, :32] = 1e-20                                   # (F16 / BF16 subnormals and underflow)
    raw = np.ascontiguousarray(source(oracle_lib, src, x, seed=5))
    want = oracle_lib.decode_src(src, raw, x.size)
    d_raw = torch.from_numpy(raw).cuda()
    d_out = torch.empty(x.size, dtype=torch.float32, device="cuda")
    print("case dequantize_src_dev src %d" % src, flush=True)
    got = gq.gpuq_dequantize_src_dev(src, d_raw.data_ptr(), d_out.data_ptr(), x.size,
                                     torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert got == x.size * 4
    assert np.array_equal(d_out.cpu().numpy().view(np.uint32), want.view(np.uint32))


GUARD = 4096        # floats after the output that no launch may write


@pytest.mark.parametrize("typ", [16, 12], ids=["iq2_xxs", "q4_k"])
def test_dequantize_dev_ragged_counts(env, oracle_lib, typ):
    """block counts that end inside a wave (8 blocks a wave) and inside a workgroup (32): every value bit for bit,
    and the floats after the last block untouched (a wave's stores stop at the launch's last block)"""
    torch, gq = env
    rng = np.random.default_rng(typ + 31)
    x = (rng.standard_normal((1, 41 * 256)) * 0.02).astype(np.float32)
    im = rng.lognormal(0.0, 1.5, 41 * 256).astype(np.float32)
    q = oracle_lib.quantize(typ, x, im).reshape(-1)
    bb = gq.gpuq_block_bytes(typ)
    d_q = torch.from_numpy(q).cuda()
    st = torch.cuda.current_stream().cuda_stream
    for nblk in (1, 3, 9, 33, 41):
        want = oracle_lib.dequantize(typ, np.ascontiguousarray(q[: nblk * bb]), nblk * 256)
        d_out = torch.full((nblk * 256 + GUARD,), 7.0, dtype=torch.float32, device="cuda")
        print("case dequantize_dev %s, %d blocks" % (NAMES[typ], nblk), flush=True)
        got = gq.gpuq_dequantize_dev(typ, d_q.data_ptr(), d_out.data_ptr(), nblk, st)
        torch.cuda.synchronize()
        assert got == nblk * 256 * 4
        out = d_out.cpu().numpy()
        assert np.array_equal(out[: nblk * 256].view(np.uint32), want.view(np.uint32)), nblk
        assert (out[nblk * 256:] == 7.0).all(), nblk


@pytest.mark.parametrize("src", [BF16, MXFP4], ids=["bf16", "mxfp4"])
def test_dequantize_src_dev_ragged_counts(env, oracle_lib, src):
    """value counts of 1, 65, 257 and 300 32-value blocks (a wave decodes 64): bit for bit, nothing written past n"""
    torch, gq = env
    rng = np.random.default_rng(src + 3)
    x = (rng.standard_normal((1, 1, 32 * 300)) * 0.05).astype(np.float32)
    raw = np.ascontiguousarray(source(oracle_lib, src, x, seed=4))
    d_raw = torch.from_numpy(raw).cuda()
    st = torch.cuda.current_stream().cuda_stream
    for nb in (1, 65, 257, 300):
        n = nb * 32
        nbytes = n * 2 if src == BF16 else nb * 17
        want = oracle_lib.decode_src(src, np.ascontiguousarray(raw[:nbytes]), n)
        d_out = torch.full((n + GUARD,), 7.0, dtype=torch.float32, device="cuda")
        print("case dequantize_src_dev src %d, %d values" % (src, n), flush=True)
        got = gq.gpuq_dequantize_src_dev(src, d_raw.data_ptr(), d_out.data_ptr(), n, st)
        torch.cuda.synchronize()
        assert got == n * 4
        out = d_out.cpu().numpy()
        assert np.array_equal(out[:n].view(np.uint32), want.view(np.uint32)), n
        assert (out[n:] == 7.0).all(), n


def test_device_api_argument_checks(env):
    """calls the library refuses answer 0 and launch nothing"""
    torch, gq = env
    st = torch.cuda.current_stream().cuda_stream
    raw = torch.zeros(4 * 512 * 4 + 64, dtype=torch.uint8, device="cuda")
    out = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    im = torch.ones(512, dtype=torch.float32, device="cuda")
    p = raw.data_ptr()
    assert gq.gpuq_requantize_dev(F16, p + 2, 12, out.data_ptr(), 1, 4, 512, None, st) == 0   # unaligned source
    assert gq.gpuq_requantize_dev(Q8_0, p + 1, 12, out.data_ptr(), 1, 4, 512, None, st) == 0  # odd Q8_0 blocks
    assert gq.gpuq_requantize_dev(2, p, 12, out.data_ptr(), 1, 4, 512, None, st) == 0         # unknown source
    assert gq.gpuq_requantize_dev(F32, p + 4, 12, out.data_ptr(), 1, 4, 512, None, st) == 0   # unaligned source
    assert gq.gpuq_requantize_dev(F32, p, 16, out.data_ptr(), 1, 4, 512, None, st) == 0       # IQ2_XXS: imatrix
    assert gq.gpuq_requantize_dev(F32, p, 12, out.data_ptr(), 1, 4, 500, None, st) == 0       # row not in blocks
    assert gq.gpuq_requantize_dev(F32, p, 12, out.data_ptr(), 0, 4, 512, im.data_ptr(), st) == 0
    assert gq.gpuq_dequantize_src_dev(F32, p, out.data_ptr(), 100, st) == 0                   # n % 32
    assert gq.gpuq_dequantize_src_dev(7, p, out.data_ptr(), 64, st) == 0                      # unknown source
    assert gq.gpuq_dequantize_src_dev(F32, p, out.data_ptr() + 4, 64, st) == 0               # unaligned output
    assert gq.gpuq_dequantize_src_dev(BF16, p + 2, out.data_ptr(), 64, st) == 0              # unaligned source
    assert gq.gpuq_dequantize_dev(12, p, out.data_ptr() + 4, 1, st) == 0                     # unaligned output
    assert gq.gpuq_dequantize_dev(12, p + 1, out.data_ptr(), 1, st) == 0                     # odd block address
    torch.cuda.synchronize()
    assert gq.gpuq_take_error() == 0


KQ = [10, 11, 12, 13, 14]


@pytest.mark.parametrize("typ", KQ, ids=[NAMES[t] for t in KQ])
def test_dequantize_dev_kquants_match_oracle(env, oracle_lib, typ):
    """ggml's to_float of the k-quants on the device, bit for bit against the oracle's (both imatrix modes' bytes,
    zero and subnormal blocks included)"""
    torch, gq = env
    rng = np.random.default_rng(typ + 7)
    x = (rng.standard_normal((12, 1024)) * rng.uniform(0.005, 0.05, (12, 1))).astype(np.float32)
    x[0] = 0
    x[1] *= 1e-20
    im = rng.lognormal(0.0, 1.5, 1024).astype(np.float32)
    q = np.concatenate([oracle_lib.quantize(typ, x, None).reshape(-1), oracle_lib.quantize(typ, x, im).reshape(-1)])
    nblk = q.size // gq.gpuq_block_bytes(typ)
    want = oracle_lib.dequantize(typ, q, nblk * 256)
    d_q = torch.from_numpy(q).cuda()
    d_out = torch.empty(nblk * 256, dtype=torch.float32, device="cuda")
    print("case dequantize_dev %s" % NAMES[typ], flush=True)
    assert gq.gpuq_can_dequantize_type(typ) == 1
    got = gq.gpuq_dequantize_dev(typ, d_q.data_ptr(), d_out.data_ptr(), nblk, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert got == nblk * 256 * 4
    assert np.array_equal(d_out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_synthetic_tables_need_the_opt_in(env):
    """a table file with the stand-in mark loads its IQ tables only under GPUQ_ALLOW_SYNTHETIC_TABLES=1: without it
    the IQ1/IQ2/IQ3 types report unavailable and the rest still work; the opt-in restores them"""
    import os
    import gpuq
    torch, gq = env
    path = gpuq.tables_path().encode()
    old = os.environ.pop("GPUQ_ALLOW_SYNTHETIC_TABLES", None)
    try:
        print("case tables without the opt-in", flush=True)
        assert gq.gpuq_init(path, 0) == 0
        assert [gq.gpuq_can_quantize(t, 1) for t in (16, 17, 18, 19, 21, 22, 29)] == [0] * 7
        assert [gq.gpuq_can_dequantize_type(t) for t in (16, 19, 29)] == [0] * 3
        assert [gq.gpuq_can_quantize(t, 1) for t in (8, 12, 14, 20, 23)] == [1] * 5
        assert gq.gpuq_can_dequantize_type(23) == 1
    finally:
        os.environ["GPUQ_ALLOW_SYNTHETIC_TABLES"] = old if old is not None else "1"
        assert gq.gpuq_init(path, 0) == 0
    assert [gq.gpuq_can_quantize(t, 1) for t in (16, 17, 18, 19, 21, 22, 29)] == [1] * 7
