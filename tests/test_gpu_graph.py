"""gpuq_requantize_dev captured into a HIP graph and replayed: each launch of a searching type zeroes its tile counter
with a kernel on the caller's stream (csrc/gpuq.hip launch_q), so a replay must give the eager call's bytes every
time. Replays alternate three inputs with eager copies and synchronizations between them, and the eager bytes are
the oracle's."""
import numpy as np
import pytest

F32 = 0
TYPES = {16: "iq2_xxs", 19: "iq1_s", 12: "q4_k"}     # two queued types (tile counter), one grid-stride type


def inputs(seed=11, nrow=16, ncol=2048):
    rng = np.random.default_rng(seed)
    xs = [(rng.standard_normal((nrow, ncol)) * s).astype(np.float32) for s in (0.02, 0.5, 3e-3)]
    im = rng.lognormal(0, 1.5, ncol).astype(np.float32)
    return xs, im


@pytest.mark.gpu
@pytest.mark.parametrize("typ", sorted(TYPES), ids=[TYPES[t] for t in sorted(TYPES)])
def test_graph_replays_match_eager(oracle_lib, typ):
    import torch
    torch.cuda.init()
    import gpuq
    gq = gpuq.load_gpuq(0)
    xs, im = inputs()
    nrow, ncol = xs[0].shape
    nb = nrow * gpuq.row_bytes(gq, typ, ncol)
    d_x = torch.empty((nrow, ncol), dtype=torch.float32, device="cuda")
    d_im = torch.from_numpy(im).cuda()
    d_out = torch.zeros(nb, dtype=torch.uint8, device="cuda")

    def launch():
        return gq.gpuq_requantize_dev(F32, d_x.data_ptr(), typ, d_out.data_ptr(), 1, nrow, ncol, d_im.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream)

    print("case graph %s: eager" % TYPES[typ], flush=True)
    want = []
    for x in xs:
        d_x.copy_(torch.from_numpy(x))
        assert launch() == nb
        torch.cuda.synchronize()
        want.append(d_out.cpu().numpy().copy())
    assert np.array_equal(want[0], oracle_lib.quantize(typ, xs[0], im).reshape(-1))
    # capture on a side stream after a warm-up call there (torch's recipe)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert launch() == nb
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("case graph %s: capture" % TYPES[typ], flush=True)
    with torch.cuda.graph(g):
        assert launch() == nb
    torch.cuda.synchronize()
    for rep in range(2):
        for i, x in enumerate(xs):
            d_x.copy_(torch.from_numpy(x))
            d_out.zero_()
            torch.cuda.synchronize()
            print("case graph %s: replay %d input %d" % (TYPES[typ], rep, i), flush=True)
            g.replay()
            torch.cuda.synchronize()
            got = d_out.cpu().numpy()
            assert np.array_equal(got, want[i]), "replay %d input %d: %d bytes differ" % (rep, i,
                                                                                          int((got != want[i]).sum()))
    assert gq.gpuq_take_error() == 0


@pytest.mark.gpu
def test_graph_replays_beside_eager_launches_on_another_stream(oracle_lib):
    """A captured launch keeps its tile counter for good, so it takes a slot that eager launches never reuse: replays
    on one stream overlap more eager launches (on a second stream) than the eager slots, and both give their own
    inputs' bytes."""
    import torch
    torch.cuda.init()
    import gpuq
    gq = gpuq.load_gpuq(0)
    typ = 16
    xs, im = inputs(seed=23, nrow=8)
    nrow, ncol = xs[0].shape
    nb = nrow * gpuq.row_bytes(gq, typ, ncol)
    d_im = torch.from_numpy(im).cuda()
    d_xg, d_xe = torch.from_numpy(xs[0]).cuda(), torch.from_numpy(xs[1]).cuda()
    d_og, d_oe = torch.zeros(nb, dtype=torch.uint8, device="cuda"), torch.zeros(nb, dtype=torch.uint8, device="cuda")

    def launch(x, out):
        return gq.gpuq_requantize_dev(F32, x.data_ptr(), typ, out.data_ptr(), 1, nrow, ncol, d_im.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream)

    want_g = oracle_lib.quantize(typ, xs[0], im).reshape(-1)
    want_e = oracle_lib.quantize(typ, xs[1], im).reshape(-1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert launch(d_xg, d_og) == nb
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("case graph beside eager: capture", flush=True)
    with torch.cuda.graph(g):
        assert launch(d_xg, d_og) == nb
    torch.cuda.synchronize()
    eager = torch.cuda.Stream()
    n_eager = 4096 + 512                              # more than the eager slots: every eager slot is reused
    print("case graph beside eager: %d eager launches, replays every 256" % n_eager, flush=True)
    for i in range(n_eager):
        with torch.cuda.stream(eager):
            assert launch(d_xe, d_oe) == nb
        if i % 256 == 0:
            g.replay()
    torch.cuda.synchronize()
    assert np.array_equal(d_og.cpu().numpy(), want_g)
    assert np.array_equal(d_oe.cpu().numpy(), want_e)
    assert gq.gpuq_take_error() == 0
