"""trench-gguf_amd/bench/ldlq_loop.py - the on-device LDLQ loop (gpuq_ldlq_dev, IQ2_S, seq order) on synthetic
experts: nexp x 2048 x 7168 f32 weights N(0, 0.02), one damped Hessian from 2048 Gaussian activations factored by
prepare_hessian_torch (copied per expert, so each matrix reads its own U), a log-normal(0, 1.5) imatrix a matrix.
Times 2 loops after a warm-up with HIP events on the launch stream and prints ms and Mweights/s.
    usage: python trench-gguf_amd/bench/ldlq_loop.py [nexp=64]
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))


def main():
    nexp = int(sys.argv[1]) if len(sys.argv) > 1 else 64
    import numpy as np
    import torch
    torch.cuda.init()
    import gpuq
    from gpuq import ldlq
    gq = gpuq.load_gpuq(0)
    ne1, ne0 = 2048, 7168
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    W = (torch.randn((nexp, ne1, ne0), device="cuda", generator=g) * 0.02).contiguous()
    X = torch.randn((2048, ne0), device="cuda", generator=g)
    H = (X.T @ X).double() / 2048
    U, perm, _, _ = ldlq.prepare_hessian_torch(H, 1, damp=0.01, order="seq")
    Us = U.unsqueeze(0).expand(nexp, ne0, ne0).contiguous()
    im = torch.exp(torch.randn(nexp, ne0, device="cuda", generator=g) * 1.5).contiguous()
    slots = np.ascontiguousarray(ldlq.slot_order(perm), dtype=np.int64)
    out = torch.empty((nexp, ne1, ne0 // 256 * gq.gpuq_block_bytes(gpuq.IQ2_S)), dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream()
    ts = []
    for it in range(3):
        Wp = W.clone()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        got = gq.gpuq_ldlq_dev(gpuq.IQ2_S, Wp.data_ptr(), Us.data_ptr(), ne0 * ne0, im.data_ptr(), nexp, ne1, ne0,
                               slots.ctypes.data, 1, out.data_ptr(), st.cuda_stream)
        e1.record(st)
        torch.cuda.synchronize()
        if got != out.numel():
            raise RuntimeError("gpuq_ldlq_dev failed")
        if it:
            ts.append(e0.elapsed_time(e1))
    ms = sum(ts) / len(ts)
    print("LDLQ IQ2_S, %d experts of 2048 x 7168: %.2f ms a loop, %.1f Mweights/s" % (nexp, ms, nexp * ne1 * ne0 / ms / 1e3),
          flush=True)


if __name__ == "__main__":
    main()
