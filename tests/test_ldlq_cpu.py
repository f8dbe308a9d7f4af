"""LDLQ on the CPU: the host's prepare_hessian against its defining equations, and the oracle's fixed-order loop
against the properties that pin it: no feedback is plain quantization; a diagonal factor feeds nothing forward; the
first update equals E U_BB^-1 U_B,rest computed independently in float64 (to f32 rounding); and on the reference's
correlated design (tools/test_ldlq.py:42-50) the feedback lowers the proxy loss (tools/ldlq.py:110-113) that it
exists to lower, in sequential order with imatrix weights and in act order with Schur weights."""
import numpy as np
import pytest

from gpuq import ldlq


def small_design(ne1=8, ne0=512, seed=3):
    rng = np.random.default_rng(seed)
    n = 2 * ne0
    X = rng.standard_normal((n, ne0)) @ (np.eye(ne0) + 0.1 * rng.standard_normal((ne0, ne0)))
    H = X.T @ X
    W = (rng.standard_normal((1, ne1, ne0)) * 0.05).astype(np.float32)
    imatrix = (np.diag(H) / n).astype(np.float32)
    return H, n, W, imatrix


@pytest.mark.parametrize("order", ["seq", "act"])
def test_prepare_hessian(order):
    H, n, _, _ = small_design()
    U, perm, diag_n, dead = ldlq.prepare_hessian(H, n, damp=0.01, order=order)
    ne0 = H.shape[0]
    assert sorted(perm.tolist()) == list(range(ne0))
    assert (perm.reshape(-1, 256) - perm.reshape(-1, 256)[:, :1] == np.arange(256)).all()   # whole blocks
    assert np.allclose(np.tril(U, -1), 0)
    Hp = (H / n)[np.ix_(perm, perm)]
    Hp[np.diag_indices(ne0)] += 0.01 * np.mean(np.diag(Hp))
    assert np.allclose(U.T @ U @ Hp, np.eye(ne0), atol=1e-8)
    if order == "act":
        e = np.diag(H / n)[perm].reshape(-1, 256).sum(1)
        assert (np.diff(e) <= 0).all()
    assert np.array_equal(diag_n, np.diag(H / n)[perm]) and not dead.any()


def test_no_feedback_is_plain_quantization(oracle_lib):
    H, n, W, im = small_design()
    U, perm, _, _ = ldlq.prepare_hessian(H, n, order="act")
    qw = ldlq.block_weights("imatrix", perm=perm, imatrix=im)[None]
    got, _ = oracle_lib.ldlq(22, W[:, :, perm], U, qw, ldlq.slot_order(perm), feedback=False)
    want = oracle_lib.quantize(22, W[0], im)            # super-blocks are independent: whole-row bytes
    assert np.array_equal(got[0], want)


def test_diagonal_factor_feeds_nothing_forward(oracle_lib):
    _, _, W, im = small_design()
    ne0 = W.shape[2]
    U = np.diag(np.linspace(0.5, 2.0, ne0))
    got, Wout = oracle_lib.ldlq(16, W, U, im[None], np.arange(ne0 // 256), feedback=True)
    assert np.array_equal(Wout, W)
    assert np.array_equal(got[0], oracle_lib.quantize(16, W[0], im))


def test_first_update_is_the_block_solve(oracle_lib):
    H, n, W, im = small_design(ne0=512)
    U, perm, _, _ = ldlq.prepare_hessian(H, n)
    Wp = W[:, :, perm]
    _, Wout = oracle_lib.ldlq(22, Wp, U, im[perm][None], np.arange(2), feedback=True)
    q = oracle_lib.dequantize(22, oracle_lib.quantize(22, Wp[0][:, :256], im[perm][:256]), Wp.shape[1] * 256)
    E = (Wp[0][:, :256] - q.reshape(-1, 256)).astype(np.float64)
    Es = np.linalg.solve(U[:256, :256].T, E.T).T
    upd = (Es @ U[:256, 256:]).astype(np.float32)
    want = Wp[0][:, 256:] - upd
    assert np.allclose(Wout[0][:, 256:], want, rtol=0, atol=4 * np.spacing(np.abs(want).max()))
    assert not np.array_equal(Wout[0][:, 256:], Wp[0][:, 256:])


def correlated_design(ne1=32, ne0=1024, seed=1):
    rng = np.random.default_rng(seed)
    n = 4 * ne0
    A = rng.standard_normal((ne0, ne0)).astype(np.float32) * 0.2 + np.eye(ne0, dtype=np.float32)
    X = rng.standard_normal((n, ne0)).astype(np.float32) @ A
    X *= (1 + 3 * rng.random(ne0, dtype=np.float32))[None]
    H = (X.T @ X).astype(np.float64)
    imatrix = (np.diag(H) / n).astype(np.float32)
    W = (rng.standard_normal((ne1, ne0)) * 0.05).astype(np.float32)
    return H, n, imatrix, W


def test_proxy_loss_closed_form():
    rng = np.random.default_rng(0)
    W = rng.standard_normal((3, 4))
    Q = rng.standard_normal((3, 4))
    X = rng.standard_normal((10, 4))
    H = X.T @ X
    # tr((W-Q) H (W-Q)^T) / n = ||X (W-Q)^T||_F^2 / n
    assert np.isclose(ldlq.proxy_loss(W, Q, H, 10), np.sum((X @ (W - Q).T) ** 2) / 10, rtol=1e-12)
    assert ldlq.proxy_loss(W, W, H, 10) == 0.0


@pytest.mark.parametrize("typ", [22, 16], ids=["iq2_s", "iq2_xxs"])
def test_feedback_lowers_the_proxy_loss(oracle_lib, typ):
    H, n, im, W = correlated_design()
    ne1, ne0 = W.shape
    plain = oracle_lib.dequantize(typ, oracle_lib.quantize(typ, W, im), W.size).reshape(ne1, ne0)
    lp = ldlq.proxy_loss(W, plain, H, n)
    for order, mode in (("seq", "imatrix"), ("act", "schur")):
        U, perm, diag_n, _ = ldlq.prepare_hessian(H, n, damp=0.01, order=order)
        qw = ldlq.block_weights(mode, U=U, perm=perm, diag_n=diag_n, imatrix=im)[None]
        q, _ = oracle_lib.ldlq(typ, W[None][:, :, perm], U, qw, ldlq.slot_order(perm), feedback=True)
        fb = oracle_lib.dequantize(typ, q[0], W.size).reshape(ne1, ne0)
        lf = ldlq.proxy_loss(W, fb, H, n)
        assert lf < 0.95 * lp, (order, mode, lf, lp)
