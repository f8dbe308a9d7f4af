"""The loader and the searches on tables of other shapes than the regular stand-ins.

- The extreme set (gpuq/tables.py EXTREME_SHELLS: the same grids and neighbour rule with more distance shells) has lists
  of up to 490 points and, for IQ1_S, file offsets past 2^21. gpuq_init keeps only the lists the staged maps reach
  (the trial rounding's base-3 keys) and packs their offsets; it must accept this set, and every IQ type must give the
  oracle's bytes on it (and the reference library's, where it is built).
- Tables whose reachable lists do not fit the packing (a list of 1024 points or more; reachable lists past 2^21
  entries) are refused with 6 before anything is replaced: the tables loaded before keep working.
The reference's loader takes any list length and offset (gpuq/gpuq.hip:2059-2080); the packing limits are this
library's, so the refusal is the documented difference."""
import os

import numpy as np
import pytest

from conftest import PKG, REF_LIB, TABLES, selftest_matrices

EXTREME = os.path.join(PKG, "gpuq", "gpuq_tables_extreme.bin")
IQ = [16, 17, 18, 19, 21, 22, 29]
NAMES = {16: "iq2_xxs", 17: "iq2_xs", 18: "iq3_xxs", 19: "iq1_s", 21: "iq3_s", 22: "iq2_s", 29: "iq1_m"}
OFF_LIMIT, CNT_LIMIT = 1 << 21, 1 << 10


def base3_keys():
    """the 2-bit keys of the 6561 base-3 level vectors, in base-3 order"""
    k = np.arange(6561)
    u = np.zeros(6561, dtype=np.int64)
    for i in range(8):
        u |= (k % 3) << (2 * i)
        k = k // 3
    return u


def reachable_packed(kmap, neigh, eight):
    """(entries, longest list) of the lists the staged map reaches, each once: what the loader packs"""
    keys = base3_keys() if eight else np.arange(4096)
    m = kmap[keys]
    offs = np.unique(-m[m < 0].astype(np.int64) - 1)
    cnts = neigh[offs].astype(np.int64)
    return int((cnts + 1).sum()), int(cnts.max())


@pytest.fixture(scope="module")
def tabs():
    import tables
    if not os.path.exists(EXTREME):
        pytest.skip("extreme tables not built: run __graft_entry__.build()")
    return tables


def test_extreme_tables_shape(tabs):
    t = tabs.read_tables(EXTREME)
    assert tabs.is_synthetic(EXTREME)
    for typ in (16, 17, 19, 22, 18, 21):
        grid, kmap, neigh = t[typ]
        eight = typ in (16, 17, 19, 22)
        entries, longest = reachable_packed(kmap, neigh, eight)
        assert entries < OFF_LIMIT and longest < CNT_LIMIT, (typ, entries, longest)
    assert len(t[19][2]) > OFF_LIMIT                        # IQ1_S: file offsets past 2^21
    assert max(reachable_packed(t[typ][1], t[typ][2], True)[1] for typ in (16, 17, 19, 22)) >= 240


@pytest.fixture
def oracle_extreme(oracle_lib):
    """the session oracle switched to the extreme tables for one test, then back"""
    assert oracle_lib.lib.gqo_load_tables(EXTREME.encode()) == 0
    try:
        yield oracle_lib
    finally:
        assert oracle_lib.lib.gqo_load_tables(TABLES.encode()) == 0


def fixture_matrices():
    xs, ims = selftest_matrices(ne1=96, ne0=2304, seed=77)
    return xs, ims


def test_oracle_runs_on_extreme_tables(tabs, oracle_extreme):
    xs, ims = fixture_matrices()
    for typ in IQ:
        for x, im in zip(xs, ims):
            q = oracle_extreme.quantize(typ, x, im)
            assert q.size == x.shape[0] * oracle_extreme.row_bytes(typ, x.shape[1]), NAMES[typ]


def write_variant(tabs, path, edit):
    recs = tabs.synthetic_tables()
    by = {r[0]: i for i, r in enumerate(recs)}
    edit(recs, by)
    tabs.write_tables(path, recs)
    return path


def long_list(recs, by):
    """one reachable IQ2_XXS key's list of 1100 points"""
    i = by[16]
    typ, grid, kmap, neigh = recs[i]
    kmap = kmap.copy()
    u = base3_keys()
    key = int(u[kmap[u] < 0][7])
    pts = (np.arange(1100) % len(grid)).astype(np.uint16)
    kmap[key] = -(len(neigh) + 1)
    recs[i] = (typ, grid, kmap, np.concatenate([neigh, np.array([1100], np.uint16), pts]))


def too_many(recs, by):
    """every reachable IQ1_S key with a list of its own of 500 points: 2.3M entries reached"""
    i = by[19]
    typ, grid, kmap, neigh = recs[i]
    kmap = kmap.copy()
    u = base3_keys()
    keys = u[kmap[u] < 0]
    kmap[kmap < 0] = -1                                     # (unreached keys: the first list)
    lst = np.concatenate([[500], np.arange(500) % len(grid)]).astype(np.uint16)
    base = np.concatenate([neigh[:1 + int(neigh[0])]])
    kmap[keys] = -(len(base) + 501 * np.arange(len(keys)) + 1)
    recs[i] = (typ, grid, kmap, np.concatenate([base, np.tile(lst, len(keys))]))


def test_refusal_cases_exceed_the_packing(tabs, tmp_path):
    t = tabs.read_tables(write_variant(tabs, str(tmp_path / "long.bin"), long_list))
    assert reachable_packed(t[16][1], t[16][2], True)[1] >= CNT_LIMIT
    t = tabs.read_tables(write_variant(tabs, str(tmp_path / "many.bin"), too_many))
    assert reachable_packed(t[19][1], t[19][2], True)[0] >= OFF_LIMIT


def gpu_bytes(gq, typ, x, im):
    import torch
    d_x = torch.from_numpy(x).cuda()
    d_im = torch.from_numpy(im).cuda()
    nb = x.shape[0] * (x.shape[1] // 256) * gq.gpuq_block_bytes(typ)
    d_out = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    got = gq.gpuq_requantize_dev(0, d_x.data_ptr(), typ, d_out.data_ptr(), 1, x.shape[0], x.shape[1],
                                 d_im.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert got == nb
    return d_out.cpu().numpy()


def load_gq():
    import torch
    torch.cuda.init()                                       # (torch first: it must see the device)
    import gpuq
    return gpuq.load_gpuq(0)


@pytest.fixture
def gq_extreme(tabs):
    gq = load_gq()
    assert gq.gpuq_init(EXTREME.encode(), 0) == 0
    try:
        yield gq
    finally:
        assert gq.gpuq_init(TABLES.encode(), 0) == 0


# the reference library's bytes on the extreme tables, in a process of its own: its gpuq_init appends tables and its
# lookup takes the first of a type, so a process that loaded the regular set first would keep searching that one
REF_CHILD = r"""
import ctypes, sys, numpy as np
sys.path.insert(0, sys.argv[3])
from conftest import selftest_matrices
lib = ctypes.CDLL(sys.argv[1])
lib.gpuq_init.argtypes = [ctypes.c_char_p, ctypes.c_int]
lib.gpuq_quantize.restype = ctypes.c_size_t
lib.gpuq_quantize.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                              ctypes.c_void_p]
lib.gpuq_block_bytes.restype = ctypes.c_size_t
assert lib.gpuq_init(sys.argv[2].encode(), 0) == 0
xs, ims = selftest_matrices(ne1=96, ne0=2304, seed=77)
out = {}
for typ in (16, 17, 18, 19, 21, 22, 29):
    for e, (x, im) in enumerate(zip(xs, ims)):
        q = np.zeros(x.shape[0] * (x.shape[1] // 256) * lib.gpuq_block_bytes(typ), dtype=np.uint8)
        assert lib.gpuq_quantize(typ, x.ctypes.data, q.ctypes.data, x.shape[0], x.shape[1], im.ctypes.data) == q.size
        out["%d_%d" % (typ, e)] = q
np.savez(sys.argv[4], **out)
print("reference child done", flush=True)
"""


@pytest.mark.gpu
def test_gpu_matches_oracle_on_extreme_tables(gq_extreme, oracle_extreme, tmp_path):
    import subprocess
    import sys
    xs, ims = fixture_matrices()
    refbytes = None
    if os.path.exists(REF_LIB):
        dst = str(tmp_path / "ref.npz")
        print("case extreme tables: reference library (child process)", flush=True)
        subprocess.run([sys.executable, "-c", REF_CHILD, REF_LIB, EXTREME, os.path.dirname(__file__), dst],
                       check=True, timeout=240)
        refbytes = np.load(dst)
    for typ in IQ:
        for e, (x, im) in enumerate(zip(xs, ims)):
            print("case extreme tables %s matrix %d" % (NAMES[typ], e), flush=True)
            want = oracle_extreme.quantize(typ, x, im).reshape(-1)
            got = gpu_bytes(gq_extreme, typ, x, im)
            assert np.array_equal(got, want), "%s matrix %d: %d bytes differ" % (NAMES[typ], e,
                                                                                 int((got != want).sum()))
            if refbytes is not None:
                r = refbytes["%d_%d" % (typ, e)]
                assert np.array_equal(r, want), "%s matrix %d: reference library" % (NAMES[typ], e)
    assert gq_extreme.gpuq_take_error() == 0


@pytest.mark.gpu
def test_gpu_refuses_tables_past_the_packing(tabs, oracle_lib, tmp_path):
    gq = load_gq()
    for name, edit in (("long", long_list), ("many", too_many)):
        path = write_variant(tabs, str(tmp_path / (name + ".bin")), edit)
        print("case refuse %s" % name, flush=True)
        assert gq.gpuq_init(path.encode(), 0) == 6, name
    # the tables loaded before still work
    xs, ims = fixture_matrices()
    for typ in (16, 19):
        want = oracle_lib.quantize(typ, xs[0], ims[0]).reshape(-1)
        assert np.array_equal(gpu_bytes(gq, typ, xs[0], ims[0]), want), NAMES[typ]
    assert gq.gpuq_take_error() == 0
