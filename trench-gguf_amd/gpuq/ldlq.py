"""LDLQ (GPTQ-style block error feedback) around the GPU quantizer, on the device.

The host half of the reference's tools/ldlq.py, restated: `prepare_hessian` (tools/ldlq.py:34-68) builds the upper
Cholesky factor U of the inverse of the damped, normalized, block-permuted Hessian; `quantize_matrix_dev`
(tools/ldlq.py:391-431, quantize_matrix_torch) quantizes a batch of matrices that share U one 256-column block at a
time, feeding each block's rounding error forward. Unlike the reference's loop, which calls gpuq_quantize_dev /
gpuq_dequantize_dev from Python and does the solve and the GEMM in torch, the whole loop runs inside one C-ABI call,
gpuq_ldlq_dev, with a fixed summation order for the f64 solve and update (see trench-gguf_amd/csrc/ldlq.cuh), so its
bytes equal the CPU oracle's exactly. torch is used only to hold device memory.

Importance weights of a block (the reference's `weights`): 'imatrix' (the imatrix row, permuted), 'diag'
(diag(H)/n, permuted), 'schur' (diag((U_BB^T U_BB)^-1) of each block).
"""
import numpy as np

QK_K = 256


def prepare_hessian(H, n, damp=0.01, order="seq", bs=QK_K):
    """H [ne0, ne0] (sum of x x^T), n rows it summed -> (U f64 upper, perm, diag_n, dead): U^T U = inverse of
    Hn[perm][:, perm] + damp * mean(diag) * I, Hn = H / n with dead (zero-energy) columns replaced by unit rows;
    perm keeps bs-column blocks together ('seq': in order; 'act': by descending block energy, ties in order)."""
    ne0 = H.shape[0]
    Hn = np.asarray(H, dtype=np.float64) / max(float(n), 1.0)
    d = np.diag(Hn).copy()
    dead = d <= 0
    if dead.any():
        Hn = Hn.copy()
        Hn[dead, :] = 0
        Hn[:, dead] = 0
        Hn[dead, dead] = 1.0
        d = np.diag(Hn).copy()
    nblk = ne0 // bs
    if order == "act":
        blk_order = np.argsort(-d.reshape(nblk, bs).sum(1), kind="stable")
    elif order == "seq":
        blk_order = np.arange(nblk)
    else:
        raise ValueError(order)
    perm = (blk_order[:, None] * bs + np.arange(bs)[None]).reshape(-1)
    Hp = Hn[np.ix_(perm, perm)]
    mean_d = float(np.mean(np.diag(Hp)))
    Hp[np.diag_indices(ne0)] += damp * mean_d
    try:
        Lc = np.linalg.cholesky(Hp)
    except np.linalg.LinAlgError:      # more ridge until it factors
        Hp[np.diag_indices(ne0)] += 10 * damp * mean_d
        Lc = np.linalg.cholesky(Hp)
    Linv = np.linalg.solve(Lc, np.eye(ne0))
    Hinv = Linv.T @ Linv
    Hinv = 0.5 * (Hinv + Hinv.T)
    U = np.linalg.cholesky(Hinv).T
    return np.ascontiguousarray(U), perm, d[perm], dead


def prepare_hessian_torch(H, n, damp=0.01, order="seq", bs=QK_K):
    """prepare_hessian for a torch f64 Hessian on the device (tools/ldlq.py:275-323), f64 throughout:
    -> (U f64 upper on the device, perm numpy, diag_n numpy, dead numpy)"""
    import torch
    ne0 = H.shape[0]
    Hn = H.to(torch.float64) / max(float(n), 1.0)
    d = torch.diagonal(Hn).clone()
    dead = d <= 0
    if bool(dead.any()):
        Hn = Hn.clone()
        Hn[dead, :] = 0
        Hn[:, dead] = 0
        Hn[dead, dead] = 1.0
        d = torch.diagonal(Hn).clone()
    nblk = ne0 // bs
    dn = d.cpu().numpy()
    if order == "act":
        blk_order = np.argsort(-dn.reshape(nblk, bs).sum(1), kind="stable")
    else:
        blk_order = np.arange(nblk)
    perm = (blk_order[:, None] * bs + np.arange(bs)[None]).reshape(-1)
    pt = torch.as_tensor(perm, device=H.device)
    Hp = Hn[pt][:, pt]
    mean_d = float(torch.diagonal(Hp).mean())
    for extra in (0.0, 10 * damp, 100 * damp):
        try:
            A = Hp.clone()
            A.diagonal().add_((damp + extra) * mean_d)
            Lc = torch.linalg.cholesky(A)
            Hinv = torch.cholesky_inverse(Lc)
            Hinv = 0.5 * (Hinv + Hinv.T)
            return torch.linalg.cholesky(Hinv, upper=True).contiguous(), perm, dn[perm], dead.cpu().numpy()
        except RuntimeError:
            continue
    raise RuntimeError("Hessian could not be factored")


def slot_order(perm, bs=QK_K):
    """the output slot of permuted block k: its original block index"""
    return (np.asarray(perm).reshape(-1, bs)[:, 0] // bs).astype(np.int64)


def block_weights(mode, U=None, perm=None, diag_n=None, imatrix=None, bs=QK_K):
    """the importance the quantizer gets for every permuted column: [..., ne0] f32"""
    if mode == "imatrix":
        return np.ascontiguousarray(np.asarray(imatrix, dtype=np.float32)[..., perm])
    if mode == "diag":
        return np.ascontiguousarray(np.asarray(diag_n, dtype=np.float32))
    if mode == "schur":
        ne0 = U.shape[0]
        out = np.empty(ne0, dtype=np.float32)
        for c0 in range(0, ne0, bs):
            Ubb = U[c0:c0 + bs, c0:c0 + bs]
            out[c0:c0 + bs] = np.diag(np.linalg.inv(Ubb.T @ Ubb))
        return out
    raise ValueError(mode)


def schur_weights_dev(gq, U, nrep=1, stream=None):
    """the 'schur' importance of every block of a device factor U (torch f64 [ne0, ne0]) on the device, in the
    library's fixed order (gpuq_schur_weights_dev): torch f32 [nrep, ne0], one row a matrix that shares U"""
    import torch
    U = U.to(torch.float64).contiguous()
    ne0 = U.shape[0]
    w = torch.empty((nrep, ne0), dtype=torch.float32, device=U.device)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    rc = gq.gpuq_schur_weights_dev(U.data_ptr(), ne0, w.data_ptr(), nrep, stream)
    if rc != 0:
        raise RuntimeError("gpuq_schur_weights_dev failed (%d)" % rc)
    return w


def proxy_loss(W, deq, H, n):
    """tr((W - Q) H (W - Q)^T) / n, the calibration inputs' squared output error that the feedback lowers
    (tools/ldlq.py:110-113): W and deq [ne1, ne0] in the original column order, H [ne0, ne0]"""
    D = np.asarray(W, dtype=np.float64) - np.asarray(deq, dtype=np.float64)
    return float(np.sum((D @ np.asarray(H, dtype=np.float64)) * D) / max(float(n), 1.0))


def quantize_matrix_dev(gq, typ, W, U, perm, qw, feedback=True, u_per_matrix=False, stream=None):
    """W: torch f32 [B, ne1, ne0] on the device (original column order, left unchanged); U: torch f64 [ne0, ne0]
    (or [B, ne0, ne0] with u_per_matrix); perm: [ne0] numpy/long; qw: torch f32 [B, ne0] importances in permuted
    order. Returns torch uint8 [B, ne1, nblk * block_bytes] in GGUF row layout, on the device."""
    import torch
    B, ne1, ne0 = W.shape
    perm_t = torch.as_tensor(np.asarray(perm), device=W.device, dtype=torch.long)
    Wp = W.index_select(2, perm_t).contiguous()
    U = U.to(torch.float64).contiguous()
    qw = qw.to(torch.float32).contiguous()
    tsize = gq.gpuq_block_bytes(int(typ))
    out = torch.empty((B, ne1, ne0 // QK_K * tsize), dtype=torch.uint8, device=W.device)
    order = np.ascontiguousarray(slot_order(perm), dtype=np.int64)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    got = gq.gpuq_ldlq_dev(int(typ), Wp.data_ptr(), U.data_ptr(), ne0 * ne0 if u_per_matrix else 0, qw.data_ptr(),
                           B, ne1, ne0, order.ctypes.data, 1 if feedback else 0, out.data_ptr(), stream)
    if got != out.numel():
        raise RuntimeError("gpuq_ldlq_dev failed (type %d, %d x %d x %d)" % (int(typ), B, ne1, ne0))
    return out


WEIGHTS = {"imatrix": 0, "diag": 1, "schur": 2}


def quantize_matrix_host(gq, typ, W, H, n, imatrix=None, damp=0.01, order="seq", h_per_matrix=False,
                         weights="imatrix"):
    """The whole LDLQ path from numpy, no framework: W f32 [B, ne1, ne0] (original column order), H f64 [ne0, ne0]
    (or [B, ne0, ne0] with h_per_matrix) the Hessian sum over n inputs, imatrix f32 [B, ne0] (or [ne0] for all).
    The factor is built on the device (gpuq_prepare_hessian_dev) and the loop runs there (gpuq_ldlq_dev). weights as
    tools/ldlq.py's: 'imatrix' (the imatrix in the permuted order), 'diag' (diag(H)/n) or 'schur' (diag((U_BB^T
    U_BB)^-1) of each block); imatrix is not used for the last two. Returns uint8 [B, ne1, nblk * block_bytes]."""
    if weights not in WEIGHTS:
        raise ValueError(weights)
    W = np.ascontiguousarray(W, dtype=np.float32)
    if W.ndim == 2:
        W = W[None]
    B, ne1, ne0 = W.shape
    H = np.ascontiguousarray(H, dtype=np.float64)
    im = None
    if imatrix is not None and weights == "imatrix":
        im = np.ascontiguousarray(np.broadcast_to(np.asarray(imatrix, dtype=np.float32), (B, ne0)))
    tsize = gq.gpuq_block_bytes(int(typ))
    out = np.empty((B, ne1, ne0 // QK_K * tsize), dtype=np.uint8)
    got = gq.gpuq_ldlq(int(typ), W.ctypes.data, H.ctypes.data, ne0 * ne0 if h_per_matrix else 0, float(n), float(damp),
                       1 if order == "act" else 0, WEIGHTS[weights], None if im is None else im.ctypes.data, B, ne1,
                       ne0, out.ctypes.data)
    if got != out.nbytes:
        raise RuntimeError("gpuq_ldlq failed (type %d, %d x %d x %d)" % (int(typ), B, ne1, ne0))
    return out
