"""Parity at the workloads' full sizes, on the exact tensors bench.py times (its workload builders, same seeds):
- F32 4096x4096, Q8_0: the whole output against the oracle;
- BF16 2048x7168 with a log-normal imatrix, every type: the whole output against the oracle, and the host entry
  point's bytes equal to the device entry point's;
- 256 BF16 experts of 2048x7168 (IQ2_XXS) and 384 MXFP4 experts (IQ1_S, IQ1_M), inputs of 3-7.5 GB: the batch
  equals the same experts quantized one call each (each expert's own source offset and imatrix row, offsets past
  2^32 bytes), and whole sampled experts equal the oracle;
- LDLQ IQ2_S over 64 experts with per-expert factors (26 GB of U): the batch equals single-expert calls, and sampled
  rows equal the oracle's loop on the same factor (the loop's rows are independent: a row's bytes depend only on
  that row, the factor and the block weights; tools/ldlq.py:71-107 of the reference).
The multi-threaded oracle (gqo_requantize_batch_mt) runs the same single-threaded restatement over row units."""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

ALL = [8, 10, 11, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29]
NAMES = {8: "q8_0", 10: "q2_k", 11: "q3_k", 12: "q4_k", 13: "q5_k", 14: "q6_k", 16: "iq2_xxs", 17: "iq2_xs",
         18: "iq3_xxs", 19: "iq1_s", 20: "iq4_nl", 21: "iq3_s", 22: "iq2_s", 23: "iq4_xs", 29: "iq1_m"}


def threads():
    try:
        return max(1, min(len(os.sched_getaffinity(0)), 16))
    except AttributeError:
        return 1


@pytest.fixture(scope="module")
def env():
    import torch
    torch.cuda.init()
    import gpuq
    import bench
    return torch, gpuq, gpuq.load_gpuq(0), bench


def free(torch):
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def out_bytes(gq, gpuq, typ, n):
    return n // gpuq.BLOCK[typ] * gq.gpuq_block_bytes(typ)


def run_dev(torch, gq, gpuq, wl, typ, raw=None, nmat=None, im=None):
    """gpuq_requantize_dev over `nmat` matrices of the workload (all by default) into a fresh device buffer"""
    raw = wl.raw if raw is None else raw
    nmat = wl.nmat if nmat is None else nmat
    n = nmat * wl.nrow * wl.ncol
    out = torch.zeros(out_bytes(gq, gpuq, typ, n), dtype=torch.uint8, device="cuda")
    if im is None and wl.imatrix is not None and typ != gpuq.Q8_0:
        im = wl.imatrix
    st = torch.cuda.current_stream().cuda_stream
    got = gq.gpuq_requantize_dev(wl.src, raw.data_ptr(), typ, out.data_ptr(), nmat, wl.nrow, wl.ncol,
                                 None if im is None else im.data_ptr(), st)
    assert got == out.numel()
    return out


def oracle_experts(torch, oracle_lib, gpuq, wl, typ, experts):
    """the oracle's bytes for whole matrices `experts` of the workload"""
    u8 = wl.raw.reshape(-1).view(torch.uint8)
    per = u8.numel() // wl.nmat
    res = []
    for e in experts:
        raw = u8[e * per:(e + 1) * per].cpu().numpy()
        im = None if (wl.imatrix is None or typ == gpuq.Q8_0) else wl.imatrix[e].cpu().numpy()
        res.append(oracle_lib.requantize_mt(wl.src, raw, typ, 1, wl.nrow, wl.ncol, im, 16, threads()))
    return res


def test_c1_q8_0_full(env, oracle_lib):
    torch, gpuq, gq, bench = env
    wl = bench.wl_c1(torch, gpuq)
    print("case full c1 q8_0", flush=True)
    got = run_dev(torch, gq, gpuq, wl, gpuq.Q8_0).cpu().numpy()
    want = oracle_experts(torch, oracle_lib, gpuq, wl, gpuq.Q8_0, [0])[0]
    assert np.array_equal(got, want), "%d bytes differ" % int((got != want).sum())
    assert gq.gpuq_take_error() == 0
    del wl
    free(torch)


@pytest.fixture(scope="module")
def c2(env):
    torch, gpuq, gq, bench = env
    wl = bench.wl_c2(torch, gpuq)
    yield wl
    del wl
    free(torch)


@pytest.mark.parametrize("typ", ALL, ids=[NAMES[t] for t in ALL])
def test_c2_full_every_type(env, oracle_lib, c2, typ):
    torch, gpuq, gq, bench = env
    print("case full c2 %s" % gpuq.TYPE_NAMES[typ], flush=True)
    dev = run_dev(torch, gq, gpuq, c2, typ)
    torch.cuda.synchronize()
    assert gq.gpuq_take_error() == 0
    got = dev.cpu().numpy()
    want = oracle_experts(torch, oracle_lib, gpuq, c2, typ, [0])[0]
    assert np.array_equal(got, want), "%d bytes differ" % int((got != want).sum())
    if typ in (gpuq.Q4_K, gpuq.IQ2_XXS, gpuq.Q8_0):
        # the streamed host entry point on the same bytes (pageable host memory in and out)
        raw = c2.raw.view(torch.uint8).cpu().numpy()
        im = None if typ == gpuq.Q8_0 else np.ascontiguousarray(c2.imatrix[0].cpu().numpy())
        host = np.zeros_like(want)
        n = gq.gpuq_requantize(c2.src, raw.ctypes.data, typ, host.ctypes.data, c2.nrow, c2.ncol,
                               None if im is None else im.ctypes.data)
        assert n == host.nbytes
        assert np.array_equal(host, want)


def experts_case(env, oracle_lib, wl, typ, sample, host_experts=0):
    """batch == one call per expert (all of them), sampled whole experts == the oracle, and optionally the host
    batch entry point over the first experts == the device bytes"""
    torch, gpuq, gq, bench = env
    per_in = wl.raw.view(torch.uint8).numel() // wl.nmat
    per_out = out_bytes(gq, gpuq, typ, wl.nrow * wl.ncol)
    batch = run_dev(torch, gq, gpuq, wl, typ)
    torch.cuda.synchronize()
    assert gq.gpuq_take_error() == 0
    u8 = wl.raw.view(torch.uint8)
    single = torch.zeros_like(batch)
    st = torch.cuda.current_stream().cuda_stream
    for e in range(wl.nmat):
        got = gq.gpuq_requantize_dev(wl.src, u8[e * per_in:].data_ptr(), typ, single[e * per_out:].data_ptr(), 1,
                                     wl.nrow, wl.ncol, wl.imatrix[e].data_ptr(), st)
        assert got == per_out
    torch.cuda.synchronize()
    same = (batch.view(wl.nmat, per_out) == single.view(wl.nmat, per_out)).all(dim=1).cpu().numpy()
    assert same.all(), "experts %s differ between the batch and single calls" % np.nonzero(~same)[0][:8]
    del single
    for e, want in zip(sample, oracle_experts(torch, oracle_lib, gpuq, wl, typ, sample)):
        got = batch[e * per_out:(e + 1) * per_out].cpu().numpy()
        assert np.array_equal(got, want), "expert %d: %d bytes differ" % (e, int((got != want).sum()))
    if host_experts:
        raw = u8[:host_experts * per_in].cpu().numpy()
        im = np.ascontiguousarray(wl.imatrix[:host_experts].cpu().numpy())
        host = np.zeros(host_experts * per_out, dtype=np.uint8)
        n = gq.gpuq_requantize_batch(wl.src, raw.ctypes.data, typ, host.ctypes.data, host_experts, wl.nrow,
                                     wl.ncol, im.ctypes.data)
        assert n == host.nbytes
        assert np.array_equal(host, batch[:host.nbytes].cpu().numpy())
    assert gq.gpuq_take_error() == 0


def test_c3_iq2_xxs_256_experts(env, oracle_lib):
    torch, gpuq, gq, bench = env
    wl = bench.wl_c3(torch, gpuq)
    print("case full c3 iq2_xxs 256 experts", flush=True)
    experts_case(env, oracle_lib, wl, gpuq.IQ2_XXS, [0, 1, 97, 146, 255], host_experts=16)
    del wl
    free(torch)


@pytest.mark.parametrize("typ", [19, 29], ids=["iq1_s", "iq1_m"])
def test_c4_iq1_384_mxfp4_experts(env, oracle_lib, typ):
    torch, gpuq, gq, bench = env
    wl = bench.wl_c4(torch, gpuq)
    print("case full c4 %s 384 experts" % gpuq.TYPE_NAMES[typ], flush=True)
    experts_case(env, oracle_lib, wl, typ, [0, 200, 383], host_experts=8 if typ == 29 else 0)
    del wl
    free(torch)


def test_c5_ldlq_64_experts(env, oracle_lib):
    torch, gpuq, gq, bench = env
    from gpuq import ldlq
    import concurrent.futures
    W, Us, perm, im = bench.wl_c5(torch, gpuq, ldlq, 64)
    nexp, ne1, ne0 = W.shape
    slots = np.ascontiguousarray(ldlq.slot_order(perm), dtype=np.int64)
    pt = torch.as_tensor(perm, device="cuda")
    Wp0 = W.index_select(2, pt).contiguous()
    del W
    qw = im.index_select(1, pt).contiguous()
    row_out = ne0 // 256 * gq.gpuq_block_bytes(gpuq.IQ2_S)
    st = torch.cuda.current_stream().cuda_stream

    def loop(e0, n):
        Wp = Wp0[e0:e0 + n].clone()
        out = torch.zeros((n, ne1, row_out), dtype=torch.uint8, device="cuda")
        got = gq.gpuq_ldlq_dev(gpuq.IQ2_S, Wp.data_ptr(), Us[e0].data_ptr(), ne0 * ne0, qw[e0].data_ptr(), n, ne1,
                               ne0, slots.ctypes.data, 1, out.data_ptr(), st)
        assert got == out.numel()
        torch.cuda.synchronize()
        return out
    print("case full c5 ldlq iq2_s 64 experts", flush=True)
    batch = loop(0, nexp)
    assert gq.gpuq_take_error() == 0
    for e in (0, 37, 63):
        assert torch.equal(loop(e, 1)[0], batch[e]), "expert %d differs between the batch and a single call" % e
    nthr = threads()
    for e in (0, 63):
        rows = np.sort(np.random.default_rng(e).choice(ne1, 2 * nthr, replace=False))
        U = Us[e].cpu().numpy()
        Wr = Wp0[e, torch.as_tensor(rows, device="cuda")].cpu().numpy()[None]
        qe = qw[e:e + 1].cpu().numpy()
        with concurrent.futures.ThreadPoolExecutor(nthr) as ex:
            parts = list(ex.map(lambda r: oracle_lib.ldlq(gpuq.IQ2_S, Wr[:, r:r + 2], U, qe, slots)[0],
                                range(0, len(rows), 2)))
        want = np.concatenate(parts, axis=1)[0]
        got = batch[e, torch.as_tensor(rows, device="cuda")].cpu().numpy()
        assert np.array_equal(got, want), "expert %d: %d bytes differ" % (e, int((got != want).sum()))
    del Us, Wp0, qw, batch
    free(torch)
