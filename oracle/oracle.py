"""ctypes wrapper of the CPU oracle (oracle/liboracle.so). TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg, never by the product library or its host module."""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

F32, F16, Q8_0, BF16, MXFP4 = 0, 1, 8, 30, 39
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, IQ1_M = 16, 17, 18, 19, 20, 21, 22, 23, 29
QUANT_TYPES = [Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS,
               IQ1_M]
TABLE_TYPES = [IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ1_M]
NO_IMATRIX_OK = [Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS]
Q4_0, Q5_0, Q5_1 = 2, 6, 7
FALLBACK_TYPES = [Q4_0, Q5_0, Q5_1, F16]     # llama-quantize's types for rows that are not whole super-blocks
NAMES = {Q8_0: "q8_0", Q2_K: "q2_k", Q3_K: "q3_k", Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k", IQ2_XXS: "iq2_xxs",
         IQ2_XS: "iq2_xs", IQ3_XXS: "iq3_xxs", IQ1_S: "iq1_s", IQ4_NL: "iq4_nl", IQ3_S: "iq3_s", IQ2_S: "iq2_s",
         IQ4_XS: "iq4_xs", IQ1_M: "iq1_m", Q4_0: "q4_0", Q5_0: "q5_0", Q5_1: "q5_1", F16: "f16"}

_vp, _i64, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t


def _ptr(a):
    return None if a is None else a.ctypes.data


class Oracle:
    def __init__(self, lib="liboracle.so", tables=None):
        self.lib = ctypes.CDLL(os.path.join(HERE, lib))
        L = self.lib
        L.gqo_load_tables.argtypes = [ctypes.c_char_p]
        L.gqo_have_tables.argtypes = [ctypes.c_int]
        L.gqo_block_bytes.restype = _sz
        L.gqo_block_bytes.argtypes = [ctypes.c_int]
        L.gqo_block_len.argtypes = [ctypes.c_int]
        L.gqo_quantize_chunk.restype = _sz
        L.gqo_quantize_chunk.argtypes = [ctypes.c_int, _vp, _vp, _i64, _i64, _i64, _vp]
        L.gqo_dequantize.restype = _sz
        L.gqo_dequantize.argtypes = [ctypes.c_int, _vp, _vp, _i64]
        L.gqo_decode_src.restype = _sz
        L.gqo_decode_src.argtypes = [ctypes.c_int, _vp, _vp, _i64]
        L.gqo_src_bytes.restype = _sz
        L.gqo_src_bytes.argtypes = [ctypes.c_int, _i64]
        L.gqo_fp32_to_fp16.restype = ctypes.c_uint16
        L.gqo_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.gqo_fp16_to_fp32.restype = ctypes.c_float
        L.gqo_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.gqo_nearest_int.argtypes = [ctypes.c_float]
        L.gqo_fp32_to_fp16_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, _vp]
        L.gqo_fp16_to_fp32_all.argtypes = [_vp]
        L.gqo_requantize_batch_mt.restype = _sz
        L.gqo_requantize_batch_mt.argtypes = [ctypes.c_int, _vp, ctypes.c_int, _vp, _i64, _i64, _i64, _vp, _i64,
                                              ctypes.c_int]
        L.gqo_ldlq.restype = _sz
        L.gqo_ldlq.argtypes = [ctypes.c_int, _vp, _vp, _vp, _i64, _i64, _i64, _vp, ctypes.c_int, _vp]
        L.gqo_schur_weights.argtypes = [_vp, _i64, _vp]
        L.gqo_ops_read_reset.restype = ctypes.c_uint64
        L.gqo_stat_read_reset.restype = ctypes.c_uint64
        L.gqo_stat_read_reset.argtypes = [ctypes.c_int]
        if tables is not None:
            rc = L.gqo_load_tables(tables.encode())
            if rc != 0:
                raise RuntimeError("oracle: cannot load tables %s (rc %d)" % (tables, rc))

    def block_bytes(self, typ):
        return self.lib.gqo_block_bytes(typ)

    def block_len(self, typ):
        return self.lib.gqo_block_len(typ)

    def row_bytes(self, typ, n_per_row):
        return n_per_row // self.block_len(typ) * self.block_bytes(typ)

    def quantize(self, typ, x, imatrix=None):
        """x: f32 [nrow, n_per_row] -> uint8 [nrow, row_bytes] (ggml_quantize_chunk)"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        nrow, npr = x.shape
        out = np.empty((nrow, self.row_bytes(typ, npr)), dtype=np.uint8)
        im = None if imatrix is None else np.ascontiguousarray(imatrix, dtype=np.float32)
        got = self.lib.gqo_quantize_chunk(typ, x.ctypes.data, out.ctypes.data, 0, nrow, npr, _ptr(im))
        if got != out.nbytes:
            raise RuntimeError("oracle quantize %s failed (%d of %d bytes)" % (NAMES.get(typ, typ), got, out.nbytes))
        return out

    def dequantize(self, typ, raw, n):
        raw = np.ascontiguousarray(raw)
        out = np.empty(n, dtype=np.float32)
        if self.lib.gqo_dequantize(typ, raw.ctypes.data, out.ctypes.data, n) != n * 4:
            raise RuntimeError("oracle dequantize %s failed" % NAMES.get(typ, typ))
        return out

    def decode_src(self, src, raw, n):
        raw = np.ascontiguousarray(raw)
        out = np.empty(n, dtype=np.float32)
        if self.lib.gqo_decode_src(src, raw.ctypes.data, out.ctypes.data, n) != n * 4:
            raise RuntimeError("oracle decode failed (src %d)" % src)
        return out

    def requantize_mt(self, src, raw, typ, nmat, nrow, n_per_row, imatrix, unit_rows, nthreads):
        raw = np.ascontiguousarray(raw)
        out = np.empty(nmat * nrow * self.row_bytes(typ, n_per_row), dtype=np.uint8)
        im = None if imatrix is None else np.ascontiguousarray(imatrix, dtype=np.float32)
        got = self.lib.gqo_requantize_batch_mt(src, raw.ctypes.data, typ, out.ctypes.data, nmat, nrow, n_per_row,
                                               _ptr(im), unit_rows, nthreads)
        if got != out.nbytes:
            raise RuntimeError("oracle requantize_mt failed")
        return out

    def ldlq(self, typ, Wp, U, qw, blk_order, feedback=True):
        """Wp [nmat, ne1, ne0] f32 (permuted; a copy is updated), U [ne0, ne0] f64, qw [nmat, ne0] f32"""
        Wp = np.array(Wp, dtype=np.float32, order="C", copy=True)
        nmat, ne1, ne0 = Wp.shape
        U = np.ascontiguousarray(U, dtype=np.float64)
        qw = np.ascontiguousarray(qw, dtype=np.float32).reshape(nmat, ne0)
        bo = np.ascontiguousarray(blk_order, dtype=np.int64)
        out = np.empty((nmat, ne1, self.row_bytes(typ, ne0)), dtype=np.uint8)
        got = self.lib.gqo_ldlq(typ, Wp.ctypes.data, U.ctypes.data, qw.ctypes.data, nmat, ne1, ne0, bo.ctypes.data,
                                1 if feedback else 0, out.ctypes.data)
        if got != out.nbytes:
            raise RuntimeError("oracle ldlq failed")
        return out, Wp

    def schur_weights(self, U):
        """U [ne0, ne0] f64 -> [ne0] f32, diag((U_BB^T U_BB)^-1) of each 256-column block (fixed order)"""
        U = np.ascontiguousarray(U, dtype=np.float64)
        w = np.empty(U.shape[0], dtype=np.float32)
        self.lib.gqo_schur_weights(U.ctypes.data, U.shape[0], w.ctypes.data)
        return w

    def fp32_to_fp16(self, f):
        return self.lib.gqo_fp32_to_fp16(f)

    def nearest_int(self, f):
        return self.lib.gqo_nearest_int(f)

    def ops_read_reset(self):
        return self.lib.gqo_ops_read_reset()

    STATS = {"nb8_searches": 0, "nb8_ties": 1, "iq2xxs_negchain": 2, "nb1_negative": 3, "iq2x16_negchain": 4}

    def stats_read_reset(self):
        """the path counters (gq_oracle.h) since the last read, as a dict"""
        return {k: self.lib.gqo_stat_read_reset(v) for k, v in self.STATS.items()}
