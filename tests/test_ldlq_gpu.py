"""The on-device LDLQ loop (gpuq_ldlq_dev) against the CPU oracle's fixed-order loop, byte for byte, on the recipe
of the reference's tools/test_ldlq.py:42-50 (a correlated Gaussian design, H = X^T X in f64, imatrix = diag(H)/n,
W ~ N(0, 0.05)), in sequential and act order, with a shared and with per-matrix factors, and without feedback
(where it must equal plain quantization, tools/test_ldlq.py:69-73); i-quant and k-quant targets; the three
importance modes of tools/ldlq.py:88-96 (imatrix, diag, schur); calls from two streams ordered on the device."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TYPES = {22: "iq2_s", 16: "iq2_xxs", 19: "iq1_s", 29: "iq1_m", 23: "iq4_xs", 18: "iq3_xxs", 12: "q4_k", 13: "q5_k",
         14: "q6_k"}


@pytest.fixture(scope="module")
def env():
    import torch
    torch.cuda.init()
    import gpuq
    return torch, gpuq, gpuq.load_gpuq(0)


def design(ne1=64, ne0=1024, seed=1):
    rng = np.random.default_rng(seed)
    n = 4 * ne0
    A = rng.standard_normal((ne0, ne0)).astype(np.float32) * 0.2 + np.eye(ne0, dtype=np.float32)
    X = rng.standard_normal((n, ne0)).astype(np.float32) @ A
    X *= (1 + 3 * rng.random(ne0, dtype=np.float32))[None]
    H = (X.T @ X).astype(np.float64)
    imatrix = (np.diag(H) / n).astype(np.float32)
    W = (rng.standard_normal((2, ne1, ne0)) * 0.05).astype(np.float32)
    return H, n, imatrix, W


@pytest.mark.parametrize("order", ["seq", "act"])
@pytest.mark.parametrize("typ", list(TYPES), ids=list(TYPES.values()))
def test_ldlq_matches_oracle(env, oracle_lib, typ, order):
    torch, gpuq, gq = env
    from gpuq import ldlq
    H, n, imatrix, W = design()
    U, perm, diag_n, _ = ldlq.prepare_hessian(H, n, damp=0.01, order=order)
    qw = np.stack([ldlq.block_weights("imatrix", perm=perm, imatrix=imatrix)] * 2)
    slots = ldlq.slot_order(perm)
    want, want_w = oracle_lib.ldlq(typ, W[:, :, perm], U, qw, slots, feedback=True)
    print("case ldlq %s %s" % (TYPES[typ], order), flush=True)
    Wd = torch.from_numpy(W).cuda()
    got = ldlq.quantize_matrix_dev(gq, typ, Wd, torch.from_numpy(U).cuda(), perm, torch.from_numpy(qw).cuda())
    torch.cuda.synchronize()
    g = got.cpu().numpy()
    bb = gq.gpuq_block_bytes(typ)
    same = (g.reshape(-1, bb) == want.reshape(-1, bb)).all(axis=1)
    assert same.all(), "%d of %d blocks differ" % (int((~same).sum()), len(same))
    assert gq.gpuq_take_error() == 0


def test_ldlq_per_matrix_factors(env, oracle_lib):
    torch, gpuq, gq = env
    from gpuq import ldlq
    H, n, imatrix, W = design(ne1=32, ne0=768)
    H2, n2, _, _ = design(ne1=32, ne0=768, seed=2)
    U1, perm, _, _ = ldlq.prepare_hessian(H, n)
    U2, _, _, _ = ldlq.prepare_hessian(H2, n2)
    qw = np.stack([imatrix, imatrix * 0.5]).astype(np.float32)
    slots = ldlq.slot_order(perm)
    want = np.concatenate([oracle_lib.ldlq(22, W[m:m + 1], U, qw[m:m + 1], slots)[0] for m, U in ((0, U1), (1, U2))])
    Us = torch.from_numpy(np.stack([U1, U2])).cuda()
    got = ldlq.quantize_matrix_dev(gq, 22, torch.from_numpy(W).cuda(), Us, perm, torch.from_numpy(qw).cuda(),
                                   u_per_matrix=True)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), want)


def test_ldlq_without_feedback_is_plain_quantization(env, oracle_lib):
    torch, gpuq, gq = env
    from gpuq import ldlq
    H, n, imatrix, W = design()
    U, perm, _, _ = ldlq.prepare_hessian(H, n)
    qw = np.stack([imatrix] * 2)
    got = ldlq.quantize_matrix_dev(gq, 16, torch.from_numpy(W).cuda(), torch.from_numpy(U).cuda(), perm,
                                   torch.from_numpy(qw).cuda(), feedback=False)
    torch.cuda.synchronize()
    for m in range(2):
        want = oracle_lib.quantize(16, W[m], imatrix)            # one whole-row call, tools/test_ldlq.py:69-73
        assert np.array_equal(got[m].cpu().numpy(), want)


def prepare_dev(torch, gq, H, n, order, damp=0.01):
    ne0 = H.shape[0]
    dH = torch.from_numpy(np.ascontiguousarray(H, dtype=np.float64)).cuda()
    dU = torch.empty_like(dH)
    perm = np.empty(ne0, dtype=np.int64)
    diag_n = np.empty(ne0, dtype=np.float64)
    dead = np.empty(ne0, dtype=np.uint8)
    rc = gq.gpuq_prepare_hessian_dev(dH.data_ptr(), ne0, float(n), damp, 1 if order == "act" else 0, dU.data_ptr(),
                                     perm.ctypes.data, diag_n.ctypes.data, dead.ctypes.data,
                                     torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    return dU.cpu().numpy(), perm, diag_n, dead.astype(bool)


@pytest.mark.parametrize("order", ["seq", "act"])
def test_prepare_hessian_dev_matches_host(env, order):
    """the device factor (rocSOLVER potrf / potri) against the host restatement of tools/ldlq.py:34-68: the same
    permutation, diag and dead columns exactly, the same U to rounding, and U^T U = (Hp + ridge)^-1"""
    torch, gpuq, gq = env
    from gpuq import ldlq
    H, n, _, _ = design(ne1=8, ne0=1024)
    Hd = H.copy()
    Hd[5, :] = 0                                           # a dead column (no energy), replaced by a unit row
    Hd[:, 5] = 0
    for Hx in (H, Hd):
        U, perm, diag_n, dead = ldlq.prepare_hessian(Hx, n, damp=0.01, order=order)
        print("case prepare_hessian_dev %s dead=%d" % (order, int(dead.sum())), flush=True)
        Ud, pd, dd, zd = prepare_dev(torch, gq, Hx, n, order)
        assert np.array_equal(pd, perm) and np.array_equal(zd, dead) and np.array_equal(dd, diag_n)
        assert np.array_equal(np.tril(Ud, -1), np.zeros_like(Ud))
        assert np.allclose(Ud, U, rtol=1e-6, atol=1e-9 * np.abs(U).max())
        ne0 = Hx.shape[0]
        Hn = Hx / n
        Hn[dead, :] = 0
        Hn[:, dead] = 0
        Hn[dead, dead] = 1.0
        Hp = Hn[np.ix_(perm, perm)]
        Hp[np.diag_indices(ne0)] += 0.01 * np.mean(np.diag(Hp))
        assert np.allclose(Ud.T @ Ud @ Hp, np.eye(ne0), atol=1e-8)


@pytest.mark.parametrize("shared", [True, False], ids=["shared-H", "per-matrix-H"])
@pytest.mark.parametrize("typ", [22, 16], ids=["iq2_s", "iq2_xxs"])
def test_ldlq_host_matches_oracle(env, oracle_lib, typ, shared):
    """gpuq_ldlq (host memory in and out, factor built on the device) == the oracle's loop on the same factor"""
    torch, gpuq, gq = env
    from gpuq import ldlq
    H, n, imatrix, W = design(ne1=32, ne0=768)
    H2, _, _, _ = design(ne1=32, ne0=768, seed=2)
    Hs = [H, H] if shared else [H, H2]
    ims = np.ascontiguousarray(np.stack([imatrix, imatrix * 0.5]).astype(np.float32))
    want = []
    for m in range(2):
        U, perm, _, _ = prepare_dev(torch, gq, Hs[m], n, "act")
        qw = ims[m][perm][None]
        want.append(oracle_lib.ldlq(typ, W[m:m + 1][:, :, perm], U, qw, ldlq.slot_order(perm))[0][0])
    want = np.stack(want)
    out = np.zeros_like(want)
    Hh = np.ascontiguousarray(H if shared else np.stack([H, H2]), dtype=np.float64)
    print("case ldlq host %d shared=%s" % (typ, shared), flush=True)
    got = gq.gpuq_ldlq(typ, np.ascontiguousarray(W).ctypes.data, Hh.ctypes.data, 0 if shared else 768 * 768,
                       float(n), 0.01, 1, 0, ims.ctypes.data, 2, 32, 768, out.ctypes.data)
    assert got == out.nbytes
    assert np.array_equal(out, want), "%d bytes differ" % int((out != want).sum())


def test_quantize_matrix_host_wrapper(env, oracle_lib):
    """the numpy wrapper over gpuq_ldlq: one imatrix row for all matrices, a 2-D W"""
    torch, gpuq, gq = env
    from gpuq import ldlq
    H, n, imatrix, W = design(ne1=16, ne0=512)
    got = ldlq.quantize_matrix_host(gq, 22, W[0], H, n, imatrix, order="seq")
    U, perm, _, _ = prepare_dev(torch, gq, H, n, "seq")
    want, _ = oracle_lib.ldlq(22, W[0:1][:, :, perm], U, imatrix[perm][None], ldlq.slot_order(perm))
    assert np.array_equal(got, want)


def test_hessian_accumulate_dev(env):
    """H += X^T X (tools/hessian_from_dump.py:73-79) on the f64 matrix cores: twice, onto a symmetric start, with a
    row count that is not a multiple of the 16-row chunk; the result stays exactly symmetric"""
    torch, gpuq, gq = env
    rng = np.random.default_rng(4)
    nrows, ne0 = 1000, 512
    X = (rng.standard_normal((nrows, ne0)) * (1 + rng.random(ne0))).astype(np.float32)
    A = rng.standard_normal((ne0, ne0))
    H0 = A + A.T
    dX = torch.from_numpy(X).cuda()
    dH = torch.from_numpy(H0.copy()).cuda()
    st = torch.cuda.current_stream().cuda_stream
    print("case hessian_accumulate", flush=True)
    for _ in range(2):
        assert gq.gpuq_hessian_accumulate_dev(dX.data_ptr(), nrows, ne0, dH.data_ptr(), st) == 0
    torch.cuda.synchronize()
    H = dH.cpu().numpy()
    Xd = X.astype(np.float64)
    want = H0 + 2 * (Xd.T @ Xd)
    assert np.array_equal(H, H.T)
    assert np.allclose(H, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())
    assert gq.gpuq_hessian_accumulate_dev(dX.data_ptr(), nrows, 500, dH.data_ptr(), st) == 1


def test_schur_weights_dev_matches_oracle(env, oracle_lib):
    """gpuq_schur_weights_dev == the oracle's fixed-order restatement, bit for bit, in every row it fills"""
    torch, gpuq, gq = env
    from gpuq import ldlq
    H, n, _, _ = design(ne1=8, ne0=1024)
    U, perm, diag_n, _ = ldlq.prepare_hessian(H, n, damp=0.01, order="act")
    want = oracle_lib.schur_weights(U)
    print("case schur_weights_dev", flush=True)
    got = ldlq.schur_weights_dev(gq, torch.from_numpy(U).cuda(), nrep=3)
    torch.cuda.synchronize()
    g = got.cpu().numpy()
    for r in range(3):
        assert np.array_equal(g[r].view(np.uint32), want.view(np.uint32))
    assert np.allclose(want, ldlq.block_weights("schur", U=U, perm=perm, diag_n=diag_n), rtol=2e-6)


@pytest.mark.parametrize("weights", ["diag", "schur"])
@pytest.mark.parametrize("typ", [22, 12], ids=["iq2_s", "q4_k"])
def test_ldlq_host_weight_modes(env, oracle_lib, typ, weights):
    """gpuq_ldlq with the importance from the Hessian (diag(H)/n) or the factor (schur) == the oracle's loop on the
    device-built factor with the same importances"""
    torch, gpuq, gq = env
    from gpuq import ldlq
    H, n, _, W = design(ne1=32, ne0=768)
    U, perm, diag_n, _ = prepare_dev(torch, gq, H, n, "act")
    qw = diag_n.astype(np.float32) if weights == "diag" else oracle_lib.schur_weights(U)
    want = np.stack([oracle_lib.ldlq(typ, W[m:m + 1][:, :, perm], U, qw[None], ldlq.slot_order(perm))[0][0]
                     for m in range(2)])
    print("case ldlq host %d weights=%s" % (typ, weights), flush=True)
    got = ldlq.quantize_matrix_host(gq, typ, W, H, n, None, order="act", weights=weights)
    assert np.array_equal(got, want), "%d bytes differ" % int((got != want).sum())


def test_ldlq_calls_from_two_streams_are_ordered(env, oracle_lib):
    """two gpuq_ldlq_dev calls issued back to back on different streams share the library's Es scratch: the second
    waits for the first on the device, so each equals the oracle's loop"""
    torch, gpuq, gq = env
    from gpuq import ldlq
    H, n, imatrix, W = design(ne1=256, ne0=1024)
    U, perm, _, _ = ldlq.prepare_hessian(H, n, damp=0.01, order="seq")
    slots = np.ascontiguousarray(ldlq.slot_order(perm), dtype=np.int64)
    qw = np.stack([imatrix[perm]] * 2).astype(np.float32)
    want = oracle_lib.ldlq(22, W[:, :, perm], U, qw, slots)[0]
    dU = torch.from_numpy(U).cuda()
    dqw = torch.from_numpy(qw).cuda()
    Wp = torch.from_numpy(np.ascontiguousarray(W[:, :, perm])).cuda()
    parts = [Wp[m:m + 1].clone() for m in range(2)]
    outs = [torch.empty((1, 256, 4 * 82), dtype=torch.uint8, device="cuda") for _ in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    print("case ldlq two streams", flush=True)
    for m in range(2):
        got = gq.gpuq_ldlq_dev(22, parts[m].data_ptr(), dU.data_ptr(), 0, dqw[m].data_ptr(), 1, 256, 1024,
                               slots.ctypes.data, 1, outs[m].data_ptr(), streams[m].cuda_stream)
        assert got == outs[m].numel()
    torch.cuda.synchronize()
    for m in range(2):
        assert np.array_equal(outs[m].cpu().numpy()[0], want[m])
    assert gq.gpuq_take_error() == 0
