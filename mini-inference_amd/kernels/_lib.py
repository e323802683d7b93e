"""ctypes binding of libmiq.so, the gfx950 kernels of the quantized path.

This is the only place that talks to the C ABI declared in include/miq.h. Every call
passes raw device pointers, element strides and torch's current HIP stream; the library
allocates nothing. A missing library, a CPU tensor or a failed call raises RuntimeError:
there is no host fallback on this path.
"""
import collections
import ctypes
import os
import threading

import torch

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("MIQ_LIB", os.path.join(_PKG_DIR, "libmiq.so"))

MIQ_F32, MIQ_BF16, MIQ_F16, MIQ_FP8_E4M3, MIQ_INT8, MIQ_UINT8, MIQ_INT32, MIQ_INT64 = range(8)
ABI_VERSION = 4  # miq_abi_version() of the library these signatures describe

_DTYPE_CODES = {
    torch.float32: MIQ_F32,
    torch.bfloat16: MIQ_BF16,
    torch.float16: MIQ_F16,
    torch.float8_e4m3fn: MIQ_FP8_E4M3,
    torch.int8: MIQ_INT8,
    torch.uint8: MIQ_UINT8,
    torch.int32: MIQ_INT32,
    torch.int64: MIQ_INT64,
}

_P, _I64, _I32, _F32, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/miq.h
SIGNATURES = {
    "miq_last_error": (ctypes.c_char_p, []),
    "miq_abi_version": (_I32, []),
    "miq_tuning_reload": (_I32, []),
    "miq_device_errors": (_I32, [_P, _P]),
    "miq_device_error_string": (ctypes.c_char_p, [ctypes.c_uint]),
    "miq_stream_read": (_I32, [_P, _SZ, _P, _P]),
    "miq_int8_quantize": (_I32, [_P, _I32, _I64, _I64, _I64, _P, _P, _I32, _P]),
    "miq_int8_dequantize": (_I32, [_P, _P, _I32, _I64, _I64, _P, _P]),
    "miq_int4_quantize": (_I32, [_P, _I32, _I64, _I64, _I64, _I64, _P, _P, _P, _I32, _P]),
    "miq_int4_dequantize": (_I32, [_P, _P, _P, _I32, _I64, _I64, _I64, _P, _P]),
    "miq_fp8_quantize_rows": (_I32, [_P, _I32, _I64, _I64, _I64, _P, _P, _P]),
    "miq_fp8_dequantize": (_I32, [_P, _P, _I64, _I64, _P, _P]),
    "miq_wo_gemm_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I32]),
    "miq_w8a16_gemm": (_I32, [_P, _I64, _P, _P, _I32, _P, _I64, _I64, _I64, _I64, _P, _SZ, _P]),
    "miq_w4a16_gemm": (_I32, [_P, _I64, _P, _P, _P, _I32, _I64, _P, _I64, _I64, _I64, _I64, _P, _SZ, _P]),
    "miq_w4a16_gemm_noalloc": (_I32, [_P, _I64, _P, _P, _P, _I32, _I64, _P, _I64, _I64, _I64, _I64, _P]),
    "miq_fp8_gemm": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "miq_kv_quant_write": (_I32, [_P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _P, _I32, _I64, _I64,
                                  _P, _I32, _I64, _I64, _P]),
    "miq_paged_decode": (_I32, [_P, _I64, _I64, _P, _P, _I32, _I64, _I64, _P, _P, _I32, _I64, _I64,
                                _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _F32, _I64, _I64, _P, _P,
                                _P, _I64, _I64, _P]),
    "miq_moe_align": (_I32, [_P, _I32, _I64, _I64, _I64, _P, _P, _P, _P]),
    "miq_moe_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "miq_w8a16_moe": (_I32, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I32, _P, _I32, _P, _P, _P, _P, _SZ,
                             _P, _P]),
    "miq_fp8_moe": (_I32, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _SZ, _P, _P]),
    "miq_w4a16_moe": (_I32, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I32, _I64, _P,
                             _I32, _P, _P, _P, _P, _SZ, _P, _P]),
    "miq_w4a16_moe_routed": (_I32, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I32, _I64, _P,
                                    _I32, _P, _I32, _P, _SZ, _P, _P]),
    "miq_w8a16_moe_routed": (_I32, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I32, _P, _I32, _P, _I32,
                                    _P, _SZ, _P, _P]),
    "miq_fp8_moe_routed": (_I32, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I32, _P, _I32, _P, _SZ,
                                  _P, _P]),
}

_lib = None
_lock = threading.Lock()


def load():
    """Load libmiq.so once; raise RuntimeError naming the path if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f"libmiq.so not found at {LIB_PATH}; build it with "
                                   f"`make -C mini-inference_amd/csrc` (or __graft_entry__.build())")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            version = lib.miq_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI version {version}, this binding expects {ABI_VERSION}; "
                                   f"rebuild the library")
            _lib = lib
    return _lib


def dtype_code(dtype):
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"libmiq: unsupported dtype {dtype}") from None


def require_device(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("libmiq kernels run on ROCm device tensors only "
                               f"(got a tensor on {t.device}); there is no CPU path")


def ptr(t):
    return None if t is None else t.data_ptr()


def stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def call(name, *args):
    rc = getattr(load(), name)(*args)
    if rc != 0:
        msg = load().miq_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def device_error_text(bits):
    """The library's description of device error word `bits` (host only)."""
    return load().miq_device_error_string(bits).decode(errors="replace")


def check_device_errors(device=None):
    """Wait for the current stream of `device`, then raise RuntimeError if any kernel set a
    bit of the device error word since the last check (the word is cleared). A diagnostic
    for tests and health checks: it synchronises."""
    device = torch.device("cuda") if device is None else device
    bits = ctypes.c_uint(0)
    call("miq_device_errors", ctypes.byref(bits), stream(device))
    if bits.value:
        raise RuntimeError(f"libmiq device error 0x{bits.value:x}: {device_error_text(bits.value)}")


# ---------------------------------------------------------------- workspaces
# Zero-initialised buffers for the split-K counters / partials of the weight-only GEMMs,
# one per (device, stream): kernels leave the counters at zero, so a buffer is reused as
# is by the launches of its stream, which run one after another. Two streams never share
# one (concurrent launches would race on the counters). A buffer only grows (a new zeroed
# buffer) when a larger shape comes along; the old one is released by the caching
# allocator in the stream order of its last use. At most _WO_WS_MAX buffers are kept (the
# least recently used one is dropped, and the caching allocator reuses its memory only on
# the stream it was allocated on, after the work queued there). A stream handle that HIP
# recycles finds a buffer that is still all zero: every call leaves it so.
_WO_WS_MAX = 8
_wo_ws = collections.OrderedDict()


def wo_workspace(device, nbytes):
    st = torch.cuda.current_stream(device)
    key = (device.type, device.index, st.cuda_stream)
    buf = _wo_ws.pop(key, None)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
    _wo_ws[key] = buf
    while len(_wo_ws) > _WO_WS_MAX:
        _wo_ws.popitem(last=False)
    return buf
