"""gpuq_ldlq_dev_noalloc, the LDLQ entry point that allocates nothing (its Es in the library's static device array),
against gpuq_ldlq_dev on the same inputs: identical bytes and identical updated weights, on two calls in a row (the
second smaller, so the array holds the first call's contents when it starts), the refusal of a call whose rows
exceed the array, the entry point captured into a HIP graph and replayed on fresh inputs, and gpuq_ldlq_dev's refusal
to run under capture."""
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


def test_noalloc_captured_into_a_graph(env):
    """The use the entry point is for: captured into a HIP graph on one stream (its tile-counter resets are kernels,
    its Es the static array), then replayed on fresh inputs copied into the captured buffers; every replay gives the
    bytes and updated weights of an eager call on the same inputs."""
    torch, gq = env
    typ, nmat, ne1, ne0 = 22, 1, 512, 768
    bb = gq.gpuq_block_bytes(typ)
    _, U, _, slots = inputs(torch, nmat, ne1, ne0, seed=5)
    runs = []
    for s in (6, 7, 8):
        Wp, _, qw, _ = inputs(torch, nmat, ne1, ne0, seed=s)
        runs.append((Wp, qw))
    w = torch.empty_like(runs[0][0])
    qwb = torch.empty_like(runs[0][1])
    out = torch.zeros((nmat, ne1, ne0 // 256 * bb), dtype=torch.uint8, device="cuda")

    def call():
        return gq.gpuq_ldlq_dev_noalloc(typ, w.data_ptr(), U.data_ptr(), 0, qwb.data_ptr(), nmat, ne1, ne0,
                                        slots.ctypes.data, 1, out.data_ptr(), torch.cuda.current_stream().cuda_stream)

    def load(i):
        w.copy_(runs[i][0])
        qwb.copy_(runs[i][1])
        out.zero_()
        torch.cuda.synchronize()

    want = []
    for i in range(len(runs)):
        load(i)
        print("case noalloc graph: eager input %d" % i, flush=True)
        assert call() == out.numel()
        torch.cuda.synchronize()
        want.append((out.cpu().numpy().copy(), w.cpu().numpy().copy()))
    load(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                   # torch's capture recipe: a warm-up call on the side stream
        assert call() == out.numel()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("case noalloc graph: capture", flush=True)
    with torch.cuda.graph(g):
        assert call() == out.numel()
    torch.cuda.synchronize()
    for rep in range(2):
        for i in range(len(runs)):
            load(i)
            print("case noalloc graph: replay %d input %d" % (rep, i), flush=True)
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), want[i][0]), "replay %d input %d: bytes differ" % (rep, i)
            assert np.array_equal(w.cpu().numpy().view(np.uint32), want[i][1].view(np.uint32))
    assert gq.gpuq_take_error() == 0


def test_allocating_entry_point_refuses_capture(env):
    """gpuq_ldlq_dev shares its scratch with eager calls and forks onto a side stream: under stream capture it
    returns 0 before any launch or allocation (graphs use gpuq_ldlq_dev_noalloc)."""
    torch, gq = env
    typ, nmat, ne1, ne0 = 22, 1, 256, 512
    Wp, U, qw, slots = inputs(torch, nmat, ne1, ne0, seed=9)
    out = torch.zeros((nmat, ne1, ne0 // 256 * gq.gpuq_block_bytes(typ)), dtype=torch.uint8, device="cuda")
    mark = torch.zeros(1, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mark.add_(1)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("case ldlq_dev under capture", flush=True)
    with torch.cuda.graph(g):
        got = gq.gpuq_ldlq_dev(typ, Wp.data_ptr(), U.data_ptr(), 0, qw.data_ptr(), nmat, ne1, ne0, slots.ctypes.data,
                               1, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        mark.add_(1)                                # (a graph with one node)
    assert got == 0
    g.replay()
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 0).all()
    assert float(mark.item()) == 2.0                # (the warm-up's add and the replay's)
