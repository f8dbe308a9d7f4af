"""Writes tests/golden/ref_vectors.npz: golden vectors produced by the reference implementation itself.

The reference ships no golden vectors (its tests compare against a live ggml). Its GPU library, gpuq/gpuq.hip, is
compiled from its own source by `make -C oracle ref` into oracle/_ref/libgpuq_ref.so (never shipped, never part of
the product). This script runs that library on one MI355X over a row subset of the reference's self-test fixture
(gpuq/test_gpuq.py:57-73) with the repository's search tables, and stores
  - q_<type>_<im|noim>: the quantized bytes (gpuq_quantize, one call a matrix), every type and imatrix mode;
  - dq_<type>: sha256 of to_float (gpuq_dequantize_dev) of the i-quant bytes, as hex;
  - meta: sha256 of the inputs and of the tables file.
Run on a machine with an MI355X, from the repository root:  python tests/golden/make_ref_golden.py [out.npz]
"""
import ctypes
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "trench-gguf_amd", "gpuq"))
from conftest import REF_LIB, TABLES, selftest_matrices  # noqa: E402
import tables  # noqa: E402

ROWS = [0, 1, 8, 9, 16, 17, 32, 33, 48, 49, 64, 65, 100, 101, 200, 201]
COLS = 1024
TYPES = [8, 10, 11, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29]
NO_IM = {8, 10, 11, 12, 13, 14, 20, 23}
DQ_TYPES = [16, 17, 22, 18, 21, 19, 29, 23]


def golden_inputs():
    xs, ims = selftest_matrices()
    return ([np.ascontiguousarray(x[ROWS, :COLS]) for x in xs], [np.ascontiguousarray(im[:COLS]) for im in ims])


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    import torch
    torch.cuda.init()
    lib = ctypes.CDLL(REF_LIB)
    lib.gpuq_init.argtypes = [ctypes.c_char_p, ctypes.c_int]
    lib.gpuq_block_bytes.restype = ctypes.c_size_t
    lib.gpuq_quantize.restype = ctypes.c_size_t
    lib.gpuq_quantize.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                  ctypes.c_void_p]
    lib.gpuq_dequantize_dev.restype = ctypes.c_size_t
    lib.gpuq_dequantize_dev.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    assert lib.gpuq_init(TABLES.encode(), 0) == 0
    xs, ims = golden_inputs()
    out = {"meta_inputs": np.array(sha(np.stack(xs)) + sha(np.stack(ims))),
           "meta_tables": np.array(tables.content_sha(TABLES))}
    for t in TYPES:
        bs = 32 if t in (8, 20) else 256
        for with_im in ([False] if t == 8 else [True, False] if t in NO_IM else [True]):
            rows = []
            for x, im in zip(xs, ims):
                ob = np.zeros(len(ROWS) * COLS // bs * lib.gpuq_block_bytes(t), dtype=np.uint8)
                got = lib.gpuq_quantize(t, x.ctypes.data, ob.ctypes.data, len(ROWS), COLS,
                                        im.ctypes.data if with_im else None)
                assert got == ob.nbytes, (t, with_im, got)
                rows.append(ob)
            out["q_%d_%s" % (t, "im" if with_im else "noim")] = np.stack(rows)
            print("type %d %s done" % (t, "im" if with_im else "noim"), flush=True)
    for t in DQ_TYPES:
        q = out["q_%d_im" % t]
        dq = torch.from_numpy(q.reshape(-1).copy()).cuda()
        nb = q.size // lib.gpuq_block_bytes(t)
        f = torch.empty(nb * 256, dtype=torch.float32, device="cuda")
        assert lib.gpuq_dequantize_dev(t, dq.data_ptr(), f.data_ptr(), nb, None) == nb * 1024
        torch.cuda.synchronize()
        out["dq_%d" % t] = np.array(sha(f.cpu().numpy()))
    dst = sys.argv[1] if len(sys.argv) > 1 else os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(dst, **out)
    print("wrote", dst, os.path.getsize(dst), "bytes")


if __name__ == "__main__":
    main()
