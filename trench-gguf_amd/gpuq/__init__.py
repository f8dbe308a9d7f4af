"""Host side of the MI355X GGUF quantizer: loads gpuq/libgpuq.so through ctypes, as the reference's drivers do.

`load_gpuq(device)` mirrors tools/requant_experts.py:116-159 of the reference: the library and its tables are found
through GPUQ_DIR (default: this folder) and GPUQ_LIB (default libgpuq.so), every entry point gets the reference's
argtypes, and gpuq_init must return 0. Unlike the reference's loader, which falls back to the CPU with a one-line
reason, `load_gpuq(required=True)` raises: the product path has no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))

F32, F16, Q8_0, BF16, MXFP4 = 0, 1, 8, 30, 39
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, IQ1_M = 16, 17, 18, 19, 20, 21, 22, 23, 29
Q4_0, Q5_0, Q5_1 = 2, 6, 7          # (with F16: llama-quantize's fallback types for rows of other lengths)
TYPE_NAMES = {Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
              IQ2_XXS: "IQ2_XXS", IQ2_XS: "IQ2_XS", IQ3_XXS: "IQ3_XXS", IQ1_S: "IQ1_S", IQ4_NL: "IQ4_NL",
              IQ3_S: "IQ3_S", IQ2_S: "IQ2_S", IQ4_XS: "IQ4_XS", IQ1_M: "IQ1_M",
              Q4_0: "Q4_0", Q5_0: "Q5_0", Q5_1: "Q5_1", F16: "F16"}
BLOCK = {t: (1 if t == F16 else 32 if t in (Q8_0, IQ4_NL, Q4_0, Q5_0, Q5_1) else 256) for t in TYPE_NAMES}

_i, _i64, _sz, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p

# (restype, argtypes) of every exported entry point: the reference's (tools/requant_experts.py:133-149,
# tools/ldlq.py:341-353) plus this library's additions
SIGNATURES = {
    "gpuq_init": (_i, [ctypes.c_char_p, _i]),
    "gpuq_block_bytes": (_sz, [_i]),
    "gpuq_can_quantize": (_i, [_i, _i]),
    "gpuq_quantize": (_sz, [_i, _vp, _vp, _i64, _i64, _vp]),
    "gpuq_quantize_batch": (_sz, [_i, _vp, _vp, _i64, _i64, _i64, _vp]),
    "gpuq_can_dequantize": (_i, [_i]),
    "gpuq_requantize": (_sz, [_i, _vp, _i, _vp, _i64, _i64, _vp]),
    "gpuq_requantize_batch": (_sz, [_i, _vp, _i, _vp, _i64, _i64, _i64, _vp]),
    "gpuq_quantize_dev": (_sz, [_i, _vp, _vp, _i64, _vp, _i64, _i64, _vp]),
    "gpuq_can_dequantize_type": (_i, [_i]),
    "gpuq_dequantize_dev": (_sz, [_i, _vp, _vp, _i64, _vp]),
    "gpuq_dequantize_src_dev": (_sz, [_i, _vp, _vp, _i64, _vp]),
    "gpuq_requantize_dev": (_sz, [_i, _vp, _i, _vp, _i64, _i64, _i64, _vp, _vp]),
    "gpuq_take_error": (_i, []),
    "gpuq_ldlq_dev": (_sz, [_i, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _i, _vp, _vp]),
    "gpuq_ldlq_dev_noalloc": (_sz, [_i, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _i, _vp, _vp]),
    "gpuq_hessian_accumulate_dev": (_i, [_vp, _i64, _i64, _vp, _vp]),
    "gpuq_prepare_hessian_dev": (_i, [_vp, _i64, ctypes.c_double, ctypes.c_double, _i, _vp, _vp, _vp, _vp, _vp]),
    "gpuq_schur_weights_dev": (_i, [_vp, _i64, _vp, _i64, _vp]),
    "gpuq_ldlq": (_sz, [_i, _vp, _vp, _i64, ctypes.c_double, ctypes.c_double, _i, _i, _vp, _i64, _i64, _i64, _vp]),
}
REFERENCE_SYMBOLS = list(SIGNATURES)[:12]


def lib_path():
    here = os.environ.get("GPUQ_DIR", HERE)
    return os.path.join(here, os.environ.get("GPUQ_LIB") or "libgpuq.so")


def tables_path():
    return os.path.join(os.environ.get("GPUQ_DIR", HERE), "gpuq_tables.bin")


def open_lib(path=None):
    """dlopen the library and set every signature; no device work (usable without a GPU)"""
    path = path or lib_path()
    if not os.path.exists(path):
        raise FileNotFoundError("%s is not built (run __graft_entry__.build() or make -C trench-gguf_amd)" % path)
    gq = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(gq, name)
        fn.restype = res
        fn.argtypes = args
    gq.batch = True
    gq.name = os.path.basename(path)
    return gq


def load_gpuq(device=0, required=True, quiet=False):
    """the library initialised on `device` with its tables, or (required=False) None with a printed reason"""
    try:
        gq = open_lib()
        rc = gq.gpuq_init(tables_path().encode(), int(device))
        if rc != 0:
            raise RuntimeError("gpuq_init %d (no GPU %d, or gpuq_tables.bin missing / invalid)" % (rc, int(device)))
        return gq
    except (OSError, RuntimeError) as e:
        if required:
            raise
        if not quiet:
            print("GPU quantizer not available (%s)" % e, flush=True)
        return None


def row_bytes(gq, typ, n_per_row):
    return n_per_row // BLOCK[typ] * gq.gpuq_block_bytes(typ)
