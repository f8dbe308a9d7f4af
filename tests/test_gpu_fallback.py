"""GPU parity of llama-quantize's fallback types (csrc/legacy.cuh): Q4_0, Q5_0, Q5_1 and F16 from every stored
source, with and without an imatrix, against the oracle byte for byte, through the host batch entry point (rows of
160 and 7200 values: whole 32-weight blocks, not whole super-blocks; F16 rows of any length) and the device entry
point (the imatrix rules' row sigma2 in a stream-ordered allocation). The reference writes these types through
ggml on the CPU (tools/requant_experts.py:180-192, 732-747)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0, Q5_0, Q5_1, F16T = 2, 6, 7, 1
F32, F16, BF16, Q8_0, MXFP4 = 0, 1, 30, 8, 39
TYPES = [Q4_0, Q5_0, Q5_1, F16T]
TNAME = {Q4_0: "q4_0", Q5_0: "q5_0", Q5_1: "q5_1", F16T: "f16"}
SNAME = {F32: "f32", F16: "f16", BF16: "bf16", Q8_0: "q8_0", MXFP4: "mxfp4"}


@pytest.fixture(scope="module")
def env():
    import torch
    torch.cuda.init()
    import gpuq
    return torch, gpuq.load_gpuq(0)


def values(rng, nmat, nrow, ncol, special=False):
    x = (rng.standard_normal((nmat, nrow, ncol)) * rng.uniform(0.005, 0.05, (nmat, nrow, 1))).astype(np.float32)
    x[:, 0] = 0                                                 # all-zero rows
    x[:, 1, ::7] *= 40                                          # spikes
    x[:, 2] = np.abs(x[:, 2])                                   # one-signed
    x[:, 3] *= np.float32(1e-18)                                # x^2 subnormal
    if special:                                                 # (F32 sources) non-finite and extreme values
        x[:, 4, 5] = np.nan
        x[:, 5, 9] = np.inf
        x[:, 6, 40] = -np.inf
        x[:, 7] *= np.float32(1e36)
        x[:, 8] = np.float32(1e-40)                             # a denormal block: its inverse scale overflows
        x[:, 8, ::2] = np.float32(-3e-41)
    return x


def bf16(x):
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def source(oracle_lib, src, x, rng):
    """(source bytes, the values they decode to)"""
    flat = np.ascontiguousarray(x.reshape(-1))
    if src == F32:
        return flat.view(np.uint8), flat.reshape(x.shape)
    if src == F16:
        with np.errstate(over="ignore"):                        # (values past the half range become inf)
            h = flat.astype(np.float16)
        return h.view(np.uint8), h.astype(np.float32).reshape(x.shape)
    if src == BF16:
        b = bf16(flat)
        return b.view(np.uint8), (b.astype(np.uint32) << 16).view(np.float32).reshape(x.shape)
    if src == Q8_0:
        raw = oracle_lib.quantize(8, x.reshape(-1, x.shape[-1])).reshape(-1)
    else:
        raw = rng.integers(0, 256, size=(flat.size // 32, 17), dtype=np.uint8)
        raw[:, 0] = 127 + rng.integers(-8, -3, size=raw.shape[0])
        raw = raw.reshape(-1)
    return raw, oracle_lib.decode_src(src, raw, flat.size).reshape(x.shape)


def want_bytes(oracle_lib, typ, f, im):
    return np.concatenate([oracle_lib.quantize(typ, f[m], None if im is None else im[m]).reshape(-1)
                           for m in range(f.shape[0])])


def first_diff(want, got, bb):
    a, b = want.reshape(-1, bb), got.reshape(-1, bb)
    eq = np.all(a == b, axis=1)
    if eq.all():
        return None
    i = int(np.argmin(eq))
    return "%d of %d blocks differ; first %d:\n  oracle %s\n  gpu    %s" % (
        int((~eq).sum()), len(eq), i, a[i].tobytes().hex(), b[i].tobytes().hex())


@pytest.mark.parametrize("with_im", [True, False], ids=["im", "noim"])
@pytest.mark.parametrize("src", [F32, F16, BF16, Q8_0, MXFP4], ids=[SNAME[s] for s in (F32, F16, BF16, Q8_0, MXFP4)])
@pytest.mark.parametrize("typ", TYPES, ids=[TNAME[t] for t in TYPES])
def test_host_batch_matches_oracle(env, oracle_lib, typ, src, with_im):
    torch, gq = env
    rng = np.random.default_rng(typ * 100 + src + with_im)
    nmat, nrow, ncol = 3, 12, 160
    x = values(rng, nmat, nrow, ncol, special=src == F32)
    raw, f = source(oracle_lib, src, x, rng)
    raw = np.ascontiguousarray(raw)
    im = rng.lognormal(0.0, 1.5, (nmat, ncol)).astype(np.float32) if with_im else None
    want = want_bytes(oracle_lib, typ, f, im)
    out = np.zeros_like(want)
    assert gq.gpuq_can_quantize(typ, 1 if with_im else 0) == 1
    print("case fallback %s src %s %s" % (TNAME[typ], SNAME[src], "im" if with_im else "noim"), flush=True)
    got = gq.gpuq_requantize_batch(src, raw.ctypes.data, typ, out.ctypes.data, nmat, nrow, ncol,
                                   None if im is None else im.ctypes.data)
    assert got == want.size
    d = first_diff(want, out, 2 if typ == F16T else gq.gpuq_block_bytes(typ))
    assert d is None, d


@pytest.mark.parametrize("typ", [Q4_0, Q5_1], ids=["q4_0", "q5_1"])
def test_long_rows_match_oracle(env, oracle_lib, typ):
    """7200-value rows (225 blocks): the row sigma2 over many blocks; chunks of rows through the streamed pipeline"""
    torch, gq = env
    rng = np.random.default_rng(typ)
    x = values(rng, 2, 40, 7200)
    im = rng.lognormal(0.0, 1.5, (2, 7200)).astype(np.float32)
    b = bf16(x.reshape(-1))
    f = (b.astype(np.uint32) << 16).view(np.float32).reshape(x.shape)
    want = want_bytes(oracle_lib, typ, f, im)
    out = np.zeros_like(want)
    print("case fallback long rows %s" % TNAME[typ], flush=True)
    got = gq.gpuq_requantize_batch(BF16, b.ctypes.data, typ, out.ctypes.data, 2, 40, 7200, im.ctypes.data)
    assert got == want.size
    d = first_diff(want, out, gq.gpuq_block_bytes(typ))
    assert d is None, d


@pytest.mark.parametrize("ncol", [1, 37, 100], ids=["n1", "n37", "n100"])
@pytest.mark.parametrize("src", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
def test_f16_rows_of_any_length(env, oracle_lib, src, ncol):
    torch, gq = env
    rng = np.random.default_rng(ncol * 10 + src)
    x = (rng.standard_normal((2, 7, ncol)) * 10.0 ** rng.uniform(-6, 5, (2, 7, ncol))).astype(np.float32)
    raw, f = source(oracle_lib, src, x, rng)
    raw = np.ascontiguousarray(raw)
    with np.errstate(over="ignore"):
        want = np.concatenate([oracle_lib.quantize(F16T, f[m]).reshape(-1) for m in range(2)])
    out = np.zeros_like(want)
    print("case fallback f16 src %s ncol %d" % (SNAME[src], ncol), flush=True)
    got = gq.gpuq_requantize_batch(src, raw.ctypes.data, F16T, out.ctypes.data, 2, 7, ncol, None)
    assert got == want.size
    assert np.array_equal(out, want), "%d bytes differ" % int((out != want).sum())


@pytest.mark.parametrize("src", [F32, BF16, MXFP4], ids=["f32", "bf16", "mxfp4"])
@pytest.mark.parametrize("typ", TYPES, ids=[TNAME[t] for t in TYPES])
def test_requantize_dev_matches_oracle(env, oracle_lib, typ, src):
    torch, gq = env
    rng = np.random.default_rng(typ * 10 + src)
    nmat, nrow, ncol = 3, 9, 96
    x = values(rng, nmat, nrow, ncol)
    raw, f = source(oracle_lib, src, x, rng)
    im = rng.lognormal(0.0, 1.5, (nmat, ncol)).astype(np.float32)
    want = want_bytes(oracle_lib, typ, f, im)
    d_raw = torch.from_numpy(np.ascontiguousarray(raw)).cuda()
    d_im = torch.from_numpy(im).cuda()
    d_out = torch.zeros(want.size, dtype=torch.uint8, device="cuda")
    print("case fallback requantize_dev %s src %s" % (TNAME[typ], SNAME[src]), flush=True)
    got = gq.gpuq_requantize_dev(src, d_raw.data_ptr(), typ, d_out.data_ptr(), nmat, nrow, ncol, d_im.data_ptr(),
                                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert got == want.size
    out = d_out.cpu().numpy()
    d = first_diff(want, out, 2 if typ == F16T else gq.gpuq_block_bytes(typ))
    assert d is None, d
