"""The host entry points' streamed pipeline: an input cut into chunks of whole matrices, or of rows of one matrix,
that run through three slots (copy in / quantize / copy out overlapped; the first two chunks a quarter and a half of
the budget) gives the bytes of the oracle over the whole input, matrix by matrix with each matrix's own imatrix row
(gpuq/gpuq.hip:2219-2250 of the reference: the batch entry points take nmat matrices and nmat imatrix rows).
GPUQ_STAGE_MB sets the chunk size; it is read on each call.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

IQ2_XXS, Q4_K, Q8_0, IQ1_M = 16, 12, 8, 29
F32, F16, BF16, SQ8_0 = 0, 1, 30, 8


@pytest.fixture(scope="module")
def gq():
    import torch
    torch.cuda.init()
    import gpuq
    return gpuq.load_gpuq(0)


@pytest.fixture
def stage_mb():
    old = os.environ.get("GPUQ_STAGE_MB")

    def set_mb(mb):
        os.environ["GPUQ_STAGE_MB"] = str(mb)
    yield set_mb
    if old is None:
        os.environ.pop("GPUQ_STAGE_MB", None)
    else:
        os.environ["GPUQ_STAGE_MB"] = old


def matrices(nmat, nrow, ncol, seed):
    rng = np.random.default_rng(seed)
    sig = rng.uniform(0.01, 0.03, nmat).astype(np.float32)
    x = (rng.standard_normal((nmat, nrow, ncol)).astype(np.float32) * sig[:, None, None])
    x[:, :3] = 0                                            # all-zero rows at each matrix's start
    im = rng.lognormal(0.0, 1.5, (nmat, ncol)).astype(np.float32)
    return x, im


def source_bytes(oracle_lib, src, x):
    flat = x.reshape(-1)
    if src == F32:
        return flat.view(np.uint8)
    if src == F16:
        return flat.astype(np.float16).view(np.uint8)
    if src == BF16:
        u = flat.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).view(np.uint8)
    return oracle_lib.quantize(8, x.reshape(-1, x.shape[-1])).reshape(-1)


# (nmat, nrow, ncol, GPUQ_STAGE_MB): whole-matrix chunks after two partial ones (0.5 MiB matrices, 1 MiB budget),
# rows of one matrix (a 2.5 MiB BF16 matrix in chunks of at most 1 MiB, ending at the matrix), and an input that
# fits one chunk
SHAPES = [(5, 128, 2048, 1), (2, 640, 2048, 1), (3, 64, 2048, 64)]


@pytest.mark.parametrize("shape", SHAPES, ids=["matrix-chunks", "row-chunks", "one-chunk"])
@pytest.mark.parametrize("typ", [IQ2_XXS, Q4_K, IQ1_M], ids=["iq2_xxs", "q4_k", "iq1_m"])
def test_stream_chunks_match_oracle(gq, oracle_lib, stage_mb, shape, typ):
    nmat, nrow, ncol, mb = shape
    x, im = matrices(nmat, nrow, ncol, seed=nmat * 1000 + nrow)
    raw = np.ascontiguousarray(source_bytes(oracle_lib, BF16, x))
    f = oracle_lib.decode_src(BF16, raw, x.size).reshape(nmat, nrow, ncol)
    want = np.concatenate([oracle_lib.quantize(typ, f[m], im[m]).reshape(-1) for m in range(nmat)])
    out = np.zeros_like(want)
    stage_mb(mb)
    print("case stream %s nmat=%d nrow=%d ncol=%d stage=%d MiB" % (typ, nmat, nrow, ncol, mb), flush=True)
    got = gq.gpuq_requantize_batch(BF16, raw.ctypes.data, typ, out.ctypes.data, nmat, nrow, ncol, im.ctypes.data)
    assert got == out.nbytes
    assert np.array_equal(out, want), "%d bytes differ" % int((out != want).sum())


@pytest.mark.parametrize("src", [F32, F16, SQ8_0], ids=["f32", "f16-decoded", "q8_0-decoded"])
def test_stream_sources(gq, oracle_lib, stage_mb, src):
    """the separate decode pass (F16, Q8_0 sources) runs per chunk into the slot's float buffer"""
    nmat, nrow, ncol = 3, 256, 2048
    x, im = matrices(nmat, nrow, ncol, seed=77 + src)
    raw = np.ascontiguousarray(source_bytes(oracle_lib, src, x))
    f = oracle_lib.decode_src(src, raw, x.size).reshape(nmat, nrow, ncol)
    want = np.concatenate([oracle_lib.quantize(IQ2_XXS, f[m], im[m]).reshape(-1) for m in range(nmat)])
    out = np.zeros_like(want)
    stage_mb(1)
    print("case stream src %d" % src, flush=True)
    got = gq.gpuq_requantize_batch(src, raw.ctypes.data, IQ2_XXS, out.ctypes.data, nmat, nrow, ncol, im.ctypes.data)
    assert got == out.nbytes
    assert np.array_equal(out, want), "%d bytes differ" % int((out != want).sum())


def test_stream_q8_0_rows_and_repeat(gq, oracle_lib, stage_mb):
    """32-value blocks (Q8_0 ignores the imatrix) over row chunks; a second, smaller call reuses the grown buffers"""
    stage_mb(1)
    for nrow in (1536, 200):
        x, _ = matrices(1, nrow, 4096, seed=nrow)
        want = oracle_lib.quantize(Q8_0, x[0]).reshape(-1)
        out = np.zeros_like(want)
        print("case stream q8_0 nrow=%d" % nrow, flush=True)
        got = gq.gpuq_quantize(Q8_0, np.ascontiguousarray(x[0]).ctypes.data, out.ctypes.data, nrow, 4096, None)
        assert got == out.nbytes
        assert np.array_equal(out, want)
    assert gq.gpuq_take_error() == 0


def test_stream_rejects_bad_shapes(gq):
    """the host API's argument checks still answer 0 before anything is copied (gpuq/gpuq.hip:2160-2170)"""
    x = np.zeros((4, 256), dtype=np.float32)
    out = np.zeros(4096, dtype=np.uint8)
    assert gq.gpuq_quantize(Q4_K, x.ctypes.data, out.ctypes.data, 0, 256, None) == 0
    assert gq.gpuq_quantize(Q4_K, x.ctypes.data, out.ctypes.data, 4, 100, None) == 0
    assert gq.gpuq_quantize(IQ2_XXS, x.ctypes.data, out.ctypes.data, 4, 256, None) == 0   # needs an imatrix


def test_stream_concurrent_callers(gq, oracle_lib, stage_mb):
    """host calls from two threads at once (ctypes drops the GIL) serialize on the library's lock: each gets its
    own input's bytes (the reference's drivers hold a lock of their own, requant_experts.py:361)"""
    import threading
    stage_mb(1)
    jobs = []
    for seed in (11, 12):
        x, im = matrices(2, 256, 2048, seed=seed)
        raw = np.ascontiguousarray(source_bytes(oracle_lib, BF16, x))
        f = oracle_lib.decode_src(BF16, raw, x.size).reshape(x.shape)
        want = np.concatenate([oracle_lib.quantize(IQ2_XXS, f[m], im[m]).reshape(-1) for m in range(2)])
        jobs.append((raw, im, want, np.zeros_like(want)))
    got = [0, 0]

    def run(k):
        raw, im, _, out = jobs[k]
        for _ in range(3):
            got[k] = gq.gpuq_requantize_batch(BF16, raw.ctypes.data, IQ2_XXS, out.ctypes.data, 2, 256, 2048,
                                              im.ctypes.data)
    print("case stream concurrent callers", flush=True)
    th = [threading.Thread(target=run, args=(k,)) for k in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    for k in range(2):
        assert got[k] == jobs[k][2].size
        assert np.array_equal(jobs[k][3], jobs[k][2])
