"""LDLQ on the CPU, pinned over every block: the oracle's fixed-order loop (oracle/gq_oracle.c gqo_ldlq) against an
independent restatement of the reference's loop in numpy's LAPACK / BLAS order (tools/ldlq.py:71-107: np.linalg.solve
for E U_BB^-1, a matrix product for the update, the f32 cast and subtraction), driven by the oracle's own
quantizer and dequantizer.

- Every block: replaying the updates in numpy from the oracle's own quantized blocks reproduces the weights each
  later block was quantized from, to f32 rounding. A slipped row or column offset in any block's solve or update
  (not only the first) breaks this.
- Whole loop: the numpy loop, run on its own (its feedback from its own rounding), gives the same bytes as the
  fixed-order loop for the share of super-blocks the reference's own test reports between its two loops
  (tools/test_ldlq.py:122-127); f64 sums that differ in the last bits move a result only at rounding boundaries.
- The 'schur' importance (tools/ldlq.py:90-93) of the fixed-order restatement against numpy's inverse.
- The k-quant readers (ggml's to_float) round-trip the quantizers' output, and the loop takes the k-quants."""
import numpy as np
import pytest

from gpuq import ldlq


def design(ne1=16, ne0=768, seed=7):
    """the reference test's correlated Hessian (tools/test_ldlq.py:42-50) at a small size"""
    rng = np.random.default_rng(seed)
    n = 4 * ne0
    A = rng.standard_normal((ne0, ne0)).astype(np.float32) * 0.2 + np.eye(ne0, dtype=np.float32)
    X = rng.standard_normal((n, ne0)).astype(np.float32) @ A
    X *= (1 + 3 * rng.random(ne0, dtype=np.float32))[None]
    H = (X.T @ X).astype(np.float64)
    im = (np.diag(H) / n).astype(np.float32)
    W = (rng.standard_normal((ne1, ne0)) * 0.05).astype(np.float32)
    return H, n, im, W


def blas_loop(orc, typ, Wp, U, qw, feedback=True):
    """the reference's quantize_matrix loop in numpy's order, on permuted weights Wp [ne1, ne0] and per-column
    importances qw [ne0] (permuted): returns the bytes of each permuted block [nblk][ne1][block bytes]"""
    Wp = Wp.copy()
    ne1, ne0 = Wp.shape
    nblk = ne0 // 256
    out = []
    for k in range(nblk):
        cols = slice(256 * k, 256 * (k + 1))
        blk = np.ascontiguousarray(Wp[:, cols])
        raw = orc.quantize(typ, blk, qw[cols])
        out.append(raw)
        if feedback and k + 1 < nblk:
            q = orc.dequantize(typ, raw, ne1 * 256).reshape(ne1, 256)
            E = blk - q
            Es = np.linalg.solve(U[cols, cols].T, E.T).T
            Wp[:, 256 * (k + 1):] -= (Es @ U[cols, 256 * (k + 1):]).astype(np.float32)
    return out


def oracle_loop(orc, typ, W, U, perm, qw):
    """the oracle's fixed-order loop on W [ne1, ne0] (original order): (bytes [ne1, row bytes], the permuted weights
    each block was quantized from [ne1, ne0])"""
    q, Wout = orc.ldlq(typ, W[None][:, :, perm], U, qw[None], ldlq.slot_order(perm))
    return q[0], Wout[0]


CASES = [(22, "seq", 768), (16, "act", 1024), (12, "seq", 768), (14, "act", 768)]


@pytest.mark.parametrize("typ,order,ne0", CASES, ids=["iq2_s-seq", "iq2_xxs-act", "q4_k-seq", "q6_k-act"])
def test_every_block_update_matches_the_blas_order(oracle_lib, typ, order, ne0):
    H, n, im, W = design(ne0=ne0)
    ne1 = W.shape[0]
    U, perm, _, _ = ldlq.prepare_hessian(H, n, damp=0.01, order=order)
    qw = im[perm]
    got, Wout = oracle_loop(oracle_lib, typ, W, U, perm, qw)
    nblk = ne0 // 256
    bb = oracle_lib.block_bytes(typ)
    slots = ldlq.slot_order(perm)
    rows = got.reshape(ne1, nblk, bb)
    Wr = W[:, perm].copy()                                 # the numpy replay, from the oracle's own blocks
    tol = 8 * np.spacing(np.float32(np.abs(Wout).max()))
    worst = []
    for k in range(nblk - 1):
        cols = slice(256 * k, 256 * (k + 1))
        # the weights block k was quantized from: equal to the replay's (to f32 rounding; exactly for k = 0)
        d = np.abs(Wr[:, cols] - Wout[:, cols]).max()
        assert d <= tol, (k, d, tol)
        worst.append(d)
        raw = np.ascontiguousarray(rows[:, slots[k]])
        q = oracle_lib.dequantize(typ, raw, ne1 * 256).reshape(ne1, 256)
        E = Wout[:, cols] - q
        Es = np.linalg.solve(U[cols, cols].T, E.T).T
        Wr[:, 256 * (k + 1):] -= (Es @ U[cols, 256 * (k + 1):]).astype(np.float32)
    last = slice(256 * (nblk - 1), ne0)
    assert np.abs(Wr[:, last] - Wout[:, last]).max() <= tol
    assert not np.array_equal(Wout, W[:, perm])             # the feedback did move the later blocks
    assert worst[0] == 0.0                                  # block 0 is quantized from the input as is


@pytest.mark.parametrize("typ,order,ne0", CASES, ids=["iq2_s-seq", "iq2_xxs-act", "q4_k-seq", "q6_k-act"])
def test_blas_order_loop_agreement(oracle_lib, typ, order, ne0):
    """the share of identical super-blocks between the fixed-order loop and the numpy-order loop run on their own"""
    H, n, im, W = design(ne0=ne0, seed=11)
    ne1 = W.shape[0]
    U, perm, _, _ = ldlq.prepare_hessian(H, n, damp=0.01, order=order)
    qw = im[perm]
    got, _ = oracle_loop(oracle_lib, typ, W, U, perm, qw)
    bb = oracle_lib.block_bytes(typ)
    nblk = ne0 // 256
    blocks = blas_loop(oracle_lib, typ, W[:, perm], U, qw)
    slots = ldlq.slot_order(perm)
    mine = got.reshape(ne1, nblk, bb)
    same = np.array([[np.array_equal(mine[r, slots[k]], blocks[k][r]) for k in range(nblk)] for r in range(ne1)])
    share = same.mean()
    print("identical super-blocks, fixed order vs numpy order: %.1f%% (%s)" % (100 * share, order))
    assert same[:, 0].all()                                 # block 0 sees no feedback
    assert share >= 0.75, share


def test_schur_weights_against_numpy(oracle_lib):
    H, n, _, _ = design(ne0=512)
    U, perm, diag_n, _ = ldlq.prepare_hessian(H, n, damp=0.01, order="act")
    got = oracle_lib.schur_weights(U)
    want = ldlq.block_weights("schur", U=U, perm=perm, diag_n=diag_n)
    assert np.allclose(got, want, rtol=2e-6, atol=0)
    assert (got == want).mean() > 0.9
    # a diagonal factor: (U_BB^T U_BB)^-1 = diag(1 / u^2), exactly for powers of two
    u = 2.0 ** np.arange(-4, 4)[np.arange(512) % 8]
    assert np.array_equal(oracle_lib.schur_weights(np.diag(u)), (1 / u ** 2).astype(np.float32))


KQ_BOUND = {10: 0.45, 11: 0.3, 12: 0.15, 13: 0.08, 14: 0.04}


@pytest.mark.parametrize("typ", sorted(KQ_BOUND), ids=["q2_k", "q3_k", "q4_k", "q5_k", "q6_k"])
def test_kquant_reader_round_trip(oracle_lib, typ):
    """to_float of the quantizer's bytes: close to the input (a misplaced field, scale or bit would not be), zero
    blocks give zeros, and the quantizer's own choice is a fixed point of quantize(to_float(.))"""
    rng = np.random.default_rng(typ)
    x = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    x[0] = 0
    im = rng.gamma(1.0, 1.0, 1024).astype(np.float32)
    for imat in (None, im):
        q = oracle_lib.quantize(typ, x, imat)
        y = oracle_lib.dequantize(typ, q, x.size).reshape(x.shape)
        rel = np.sqrt(((y[1:] - x[1:]) ** 2).mean() / (x[1:] ** 2).mean())
        assert rel < KQ_BOUND[typ], rel
        assert (y[0] == 0).all()
    # a constant block of one sign: every value comes back within its sub-block's step of the input
    c = np.full((1, 256), 0.01, dtype=np.float32)
    yc = oracle_lib.dequantize(typ, oracle_lib.quantize(typ, c, None), 256)
    assert np.abs(yc - 0.01).max() < 0.01 * 0.1


@pytest.mark.parametrize("typ", [12, 13, 14], ids=["q4_k", "q5_k", "q6_k"])
def test_kquant_feedback_lowers_the_proxy_loss(oracle_lib, typ):
    H, n, im, W = design(ne1=32, ne0=1024, seed=1)
    ne1, ne0 = W.shape
    plain = oracle_lib.dequantize(typ, oracle_lib.quantize(typ, W, im), W.size).reshape(ne1, ne0)
    lp = ldlq.proxy_loss(W, plain, H, n)
    U, perm, _, _ = ldlq.prepare_hessian(H, n, damp=0.01, order="seq")
    q, _ = oracle_loop(oracle_lib, typ, W, U, perm, im[perm])
    fb = oracle_lib.dequantize(typ, q, W.size).reshape(ne1, ne0)
    assert ldlq.proxy_loss(W, fb, H, n) < 0.95 * lp
