"""The C ABI without a GPU: the library loads, exports every entry point include/gpuq.h declares with the
signatures the host module sets (the reference's ctypes argtypes, tools/requant_experts.py:133-149), and its pure
functions answer as the reference's do (gpuq/gpuq.hip:2082-2101, 2213-2235)."""
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "gpuq.h")


def header_functions():
    with open(HEADER) as f:
        src = f.read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.findall(r"\b(?:int|size_t)\s+(gpuq_\w+)\s*\(", src)


@pytest.fixture(scope="module")
def lib():
    import gpuq
    return gpuq.open_lib()


def test_header_declares_reference_symbols():
    names = header_functions()
    ref = ["gpuq_init", "gpuq_block_bytes", "gpuq_can_quantize", "gpuq_quantize", "gpuq_quantize_batch",
           "gpuq_can_dequantize", "gpuq_requantize", "gpuq_requantize_batch", "gpuq_quantize_dev",
           "gpuq_can_dequantize_type", "gpuq_dequantize_dev", "gpuq_dequantize_src_dev"]
    assert names[:12] == ref


def test_library_exports_every_declared_symbol(lib):
    import gpuq
    for name in header_functions():
        assert hasattr(lib, name), name
        assert name in gpuq.SIGNATURES, name


def test_block_bytes(lib):
    want = {8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 16: 66, 17: 74, 18: 98, 19: 50, 20: 18, 21: 110,
            22: 82, 23: 136, 29: 56, 2: 18, 6: 22, 7: 24, 1: 2, 0: 0, 30: 0, 39: 0, 3: 0, 9: 0}
    for t, b in want.items():
        assert lib.gpuq_block_bytes(t) == b, t


def test_can_dequantize_sources(lib):
    assert [lib.gpuq_can_dequantize(s) for s in (0, 1, 8, 30, 39)] == [1, 1, 1, 1, 1]
    assert [lib.gpuq_can_dequantize(s) for s in (2, 12, 16, 40)] == [0, 0, 0, 0]


def test_nothing_quantizes_before_init(lib):
    # no device selected: every capability probe answers 0 and no call reaches the GPU
    if lib.gpuq_can_dequantize_type(23) == 1:
        pytest.skip("the library was initialized earlier in this process (GPU tests ran first)")
    assert all(lib.gpuq_can_quantize(t, 1) == 0 for t in (8, 12, 16, 19, 29))
    assert lib.gpuq_can_dequantize_type(16) == 0
    assert lib.gpuq_quantize_dev(16, None, None, 1, None, 1, 1, None) == 0
    assert lib.gpuq_prepare_hessian_dev(None, 256, 1.0, 0.01, 0, None, None, None, None, None) == 1
    assert lib.gpuq_ldlq(22, None, None, 0, 1.0, 0.01, 0, 0, None, 1, 1, 256, None) == 0
    assert lib.gpuq_schur_weights_dev(None, 256, None, 1, None) == 1
