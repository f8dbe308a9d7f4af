"""gpuq_ldlq_dev_noalloc, the LDLQ entry point that allocates nothing (its Es in the library's static device array),
against gpuq_ldlq_dev on the same inputs: identical bytes and identical updated weights, on two calls in a row (the
second smaller, so the array holds the first call's contents when it starts), and the refusal of a call whose rows
exceed the array."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    torch.cuda.init()
    import gpuq
    return torch, gpuq.load_gpuq(0)


def inputs(torch, nmat, ne1, ne0, seed):
    from gpuq import ldlq
    rng = np.random.default_rng(seed)
    n = 2 * ne0
    X = rng.standard_normal((n, ne0)) @ (np.eye(ne0) + 0.1 * rng.standard_normal((ne0, ne0)))
    H = X.T @ X
    U, perm, _, _ = ldlq.prepare_hessian(H, n, damp=0.01, order="act")
    W = (rng.standard_normal((nmat, ne1, ne0)) * 0.05).astype(np.float32)
    qw = rng.lognormal(0.0, 1.5, (nmat, ne0)).astype(np.float32)
    slots = np.ascontiguousarray(ldlq.slot_order(perm), dtype=np.int64)
    return (torch.from_numpy(np.ascontiguousarray(W[:, :, perm])).cuda(), torch.from_numpy(U).cuda(),
            torch.from_numpy(qw).cuda(), slots)


@pytest.mark.parametrize("typ", [22, 12], ids=["iq2_s", "q4_k"])
def test_noalloc_matches_the_allocating_entry_point(env, typ):
    torch, gq = env
    st = torch.cuda.current_stream().cuda_stream
    bb = gq.gpuq_block_bytes(typ)
    for call, (nmat, ne1, ne0) in enumerate([(2, 1024, 1024), (1, 300, 768)]):
        Wp, U, qw, slots = inputs(torch, nmat, ne1, ne0, seed=10 * typ + call)
        outs, ws = [], []
        for fn in (gq.gpuq_ldlq_dev, gq.gpuq_ldlq_dev_noalloc):
            w = Wp.clone()
            out = torch.zeros((nmat, ne1, ne0 // 256 * bb), dtype=torch.uint8, device="cuda")
            print("case %s type %d call %d: %d x %d x %d" % (fn.__name__, typ, call, nmat, ne1, ne0), flush=True)
            got = fn(typ, w.data_ptr(), U.data_ptr(), 0, qw.data_ptr(), nmat, ne1, ne0, slots.ctypes.data, 1,
                     out.data_ptr(), st)
            assert got == out.numel()
            torch.cuda.synchronize()
            outs.append(out.cpu().numpy())
            ws.append(w.cpu().numpy())
        assert np.array_equal(outs[0], outs[1]), "%d bytes differ" % int((outs[0] != outs[1]).sum())
        assert np.array_equal(ws[0].view(np.uint32), ws[1].view(np.uint32))
    assert gq.gpuq_take_error() == 0


def test_noalloc_refuses_more_rows_than_its_scratch(env):
    torch, gq = env
    st = torch.cuda.current_stream().cuda_stream
    nmat, ne1, ne0 = 1, 8200, 512
    w = torch.zeros((nmat, ne1, ne0), dtype=torch.float32, device="cuda")
    U = torch.eye(ne0, dtype=torch.float64, device="cuda")
    qw = torch.ones((nmat, ne0), dtype=torch.float32, device="cuda")
    out = torch.zeros((nmat, ne1, 2 * 82), dtype=torch.uint8, device="cuda")
    slots = np.arange(2, dtype=np.int64)
    print("case noalloc refusal", flush=True)
    assert gq.gpuq_ldlq_dev_noalloc(22, w.data_ptr(), U.data_ptr(), 0, qw.data_ptr(), nmat, ne1, ne0,
                                    slots.ctypes.data, 1, out.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 0).all()
