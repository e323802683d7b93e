"""The C-ABI boundary, checked without a GPU: libmiq.so loads, exports every function
declared in include/miq.h, the ctypes table matches the header, and the product path
refuses CPU tensors instead of falling back to host code."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "miq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(miq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ("miq_w8a16_gemm", "miq_w4a16_gemm", "miq_fp8_gemm", "miq_fp8_quantize_rows",
              "miq_paged_decode", "miq_moe_align", "miq_w4a16_moe", "miq_kv_quant_write"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from kernels import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    from kernels import _lib
    assert sorted(_lib.SIGNATURES) == declared_functions()
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), name


def test_abi_version_and_error_string():
    from kernels import _lib
    lib = _lib.load()
    assert lib.miq_abi_version() == _lib.ABI_VERSION == 4
    assert lib.miq_tuning_reload() == 0
    # a shape error is reported without touching the GPU
    rc = lib.miq_w8a16_gemm(None, 0, None, None, 0, None, 0, 0, 16, 128, None, 0, None)
    assert rc == -1
    assert b"M=0" in lib.miq_last_error()


def test_workspace_sizes():
    from kernels import _lib
    lib = _lib.load()
    assert lib.miq_wo_gemm_workspace_bytes(1, 2560, 9728, 4) >= 256
    assert lib.miq_moe_workspace_bytes(64, 8, 64, 2048, 1024) >= 64 * 8 * 2048 * 4


def test_cpu_tensors_are_refused():
    from engine.quantization import get_method
    from kernels.paged_attention import paged_decode_attention
    w = torch.randn(64, 256) * 0.02
    for name in ("int8_wo", "int4_wo", "fp8"):
        with pytest.raises(RuntimeError, match="ROCm device tensors only"):
            get_method(name).quantize(w)
    q = torch.zeros(1, 4, 128, dtype=torch.bfloat16)
    kv = torch.zeros(16, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        paged_decode_attention(q, kv, kv, torch.zeros(1, 1, dtype=torch.int32),
                               torch.ones(1, dtype=torch.int32), 16, 0.1, 16)


def test_device_error_word_encoding():
    """The device error word's bits and their text (host only): a panel reducer that gives
    up waiting sets MIQ_DEVERR_PANEL_WAIT (and writes NaN), which check_device_errors
    turns into a RuntimeError naming it."""
    from kernels import _lib
    text = open(HEADER).read()
    assert re.search(r"MIQ_DEVERR_PANEL_WAIT\s*=\s*1\b", text)
    assert _lib.device_error_text(0) == "no device error"
    assert "gave up waiting" in _lib.device_error_text(1)
    assert "unknown" in _lib.device_error_text(1 << 30)
