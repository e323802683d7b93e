"""Torch-facing wrappers of the quantize / dequantize / GEMM entry points of libmiq.

Each wrapper checks shapes on the host, allocates the outputs with torch (so the
caching allocator and HIP graph capture see them) and launches on torch's current
stream. Inputs must already be on the ROCm device.
"""
import math

import torch

from kernels import _lib as L

SKINNY_MAX_M = 64  # decode kernels up to 64 activation rows; above, the prefill kernels
# The fused weight-only GEMMs take any M whose activations stay below 2^31 elements (their
# buffer descriptors address 32-bit offsets).
MAX_X_ELEMS = 1 << 31


def _rows(t):
    return math.prod(t.shape[:-1]) if t.dim() > 1 else 1


def _contig_rows(w):
    """View w [..., K] as [rows, K] with a row stride; copies only if the last dim is strided."""
    w2 = w.reshape(-1, w.shape[-1])
    if w2.stride(-1) != 1:
        w2 = w2.contiguous()
    return w2


# ---------------------------------------------------------------- int8 weight-only
def int8_quantize(weight, scale_dtype):
    """engine/quantization/int8_wo.py:8-12 -> (q int8 [..., N, K], scale [..., N, 1])."""
    q = torch.empty(weight.shape, dtype=torch.int8, device=weight.device)
    scale = torch.empty(weight.shape[:-1] + (1,), dtype=scale_dtype, device=weight.device)
    if weight.is_meta:  # shapes only (a cache load builds the modules on "meta" first)
        return q, scale
    L.require_device(weight)
    w2 = _contig_rows(weight)
    L.call("miq_int8_quantize", L.ptr(w2), L.dtype_code(w2.dtype), w2.shape[0], w2.shape[1], w2.stride(0),
           L.ptr(q), L.ptr(scale), L.dtype_code(scale_dtype), L.stream(weight.device))
    return q, scale


def int8_dequantize(qweight, scale):
    """int8_wo.py:14-15: q.to(scale.dtype) * scale."""
    L.require_device(qweight, scale)
    q = qweight.contiguous()
    s = scale.contiguous()
    out = torch.empty(q.shape, dtype=scale.dtype, device=q.device)
    L.call("miq_int8_dequantize", L.ptr(q), L.ptr(s), L.dtype_code(s.dtype), _rows(q), q.shape[-1],
           L.ptr(out), L.stream(q.device))
    return out


def w8a16_linear(x, qweight, scale):
    """int8_wo.py:17-21: y = bf16(bf16(x @ q^T) * bf16(scale)), any number of rows."""
    L.require_device(x, qweight, scale)
    K = x.shape[-1]
    N = qweight.shape[-2]
    x2 = _contig_rows(x)
    M = x2.shape[0]
    q = qweight.contiguous()
    s = scale.reshape(-1).contiguous()
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    nbytes = L.load().miq_wo_gemm_workspace_bytes(M, N, K, 8)
    ws = L.wo_workspace(x.device, nbytes)
    L.call("miq_w8a16_gemm", L.ptr(x2), x2.stride(0), L.ptr(q), L.ptr(s), L.dtype_code(s.dtype), L.ptr(y), N,
           M, N, K, L.ptr(ws), ws.numel(), L.stream(x.device))
    return y.reshape(*x.shape[:-1], N)


def w8a16_supported(x, qweight):
    M = _rows(x)
    return (x.dtype == torch.bfloat16 and M >= 1 and M * x.shape[-1] < MAX_X_ELEMS and x.shape[-1] % 128 == 0
            and qweight.shape[-2] % 16 == 0 and qweight.dim() == 2)


# ---------------------------------------------------------------- int4 weight-only
def int4_quantize(weight, group_size, sz_dtype, symmetric=False):
    """int4_wo.py:15-31 -> (packed uint8 [..., N, K/2], scale [..., N, K/g], zero or None)."""
    K = weight.shape[-1]
    lead = weight.shape[:-1]
    q = torch.empty(lead + (K // 2,), dtype=torch.uint8, device=weight.device)
    scale = torch.empty(lead + (K // group_size,), dtype=sz_dtype, device=weight.device)
    zero = None if symmetric else torch.empty_like(scale)
    if weight.is_meta:  # shapes only
        return q, scale, zero
    L.require_device(weight)
    w2 = _contig_rows(weight)
    L.call("miq_int4_quantize", L.ptr(w2), L.dtype_code(w2.dtype), w2.shape[0], K, w2.stride(0), group_size,
           L.ptr(q), L.ptr(scale), L.ptr(zero), L.dtype_code(sz_dtype), L.stream(weight.device))
    return q, scale, zero


def int4_dequantize(qweight, scale, zero):
    """int4_wo.py:33-42: (q * scale) + zero, rounded to scale.dtype after each op."""
    L.require_device(qweight, scale, zero)
    q = qweight.contiguous()
    s = scale.contiguous()
    z = None if zero is None else zero.contiguous()
    K = q.shape[-1] * 2
    group = K // s.shape[-1]
    out = torch.empty(q.shape[:-1] + (K,), dtype=s.dtype, device=q.device)
    L.call("miq_int4_dequantize", L.ptr(q), L.ptr(s), L.ptr(z), L.dtype_code(s.dtype), _rows(q), K, group,
           L.ptr(out), L.stream(q.device))
    return out


def w4a16_linear(x, qweight, scale, zero):
    """QuantMethod.linear over Int4WeightOnly (base.py:20-24), any number of rows."""
    L.require_device(x, qweight, scale, zero)
    K = x.shape[-1]
    N = qweight.shape[-2]
    group = K // scale.shape[-1]
    x2 = _contig_rows(x)
    M = x2.shape[0]
    q = qweight.contiguous()
    s = scale.contiguous()
    z = None if zero is None else zero.contiguous()
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    nbytes = L.load().miq_wo_gemm_workspace_bytes(M, N, K, 4)
    ws = L.wo_workspace(x.device, nbytes)
    L.call("miq_w4a16_gemm", L.ptr(x2), x2.stride(0), L.ptr(q), L.ptr(s), L.ptr(z), L.dtype_code(s.dtype), group,
           L.ptr(y), N, M, N, K, L.ptr(ws), ws.numel(), L.stream(x.device))
    return y.reshape(*x.shape[:-1], N)


def w4a16_supported(x, qweight, scale):
    M = _rows(x)
    K = x.shape[-1]
    if scale.shape[-1] == 0 or K % scale.shape[-1]:
        return False
    group = K // scale.shape[-1]
    return (x.dtype == torch.bfloat16 and M >= 1 and M * K < MAX_X_ELEMS and group % 128 == 0
            and qweight.shape[-2] % 16 == 0 and qweight.dim() == 2)


# ---------------------------------------------------------------- fp8 weight + activation
def fp8_quantize_rows(x):
    """fp8.py:32-36 / 41-46 -> (e4m3fn [..., K], fp32 scale [...])."""
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    scale = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    if x.is_meta:  # shapes only
        return q, scale
    L.require_device(x)
    x2 = _contig_rows(x)
    L.call("miq_fp8_quantize_rows", L.ptr(x2), L.dtype_code(x2.dtype), x2.shape[0], x2.shape[1], x2.stride(0),
           L.ptr(q), L.ptr(scale), L.stream(x.device))
    return q, scale


def fp8_dequantize(qweight, scale):
    """fp8.py:38-39: q.float() * scale[..., None]."""
    L.require_device(qweight, scale)
    q = qweight.contiguous()
    s = scale.contiguous().float()
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    L.call("miq_fp8_dequantize", L.ptr(q), L.ptr(s), _rows(q), q.shape[-1], L.ptr(out), L.stream(q.device))
    return out


def fp8_gemm(x_fp8, x_scale, w_fp8, w_scale):
    """The torch._scaled_mm call of fp8.py:55-61: bf16 (x_fp8 @ w_fp8^T) * x_scale * w_scale."""
    L.require_device(x_fp8, x_scale, w_fp8, w_scale)
    M, K = x_fp8.shape
    N = w_fp8.shape[0]
    if K % 128:
        raise RuntimeError(f"fp8_gemm: K={K} must be a multiple of 128")
    xq = x_fp8.contiguous()
    wq = w_fp8.contiguous()
    xs = x_scale.reshape(-1).float().contiguous()
    wsc = w_scale.reshape(-1).float().contiguous()
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x_fp8.device)
    L.call("miq_fp8_gemm", L.ptr(xq), L.ptr(xs), L.ptr(wq), L.ptr(wsc), L.ptr(y), N, M, N, K,
           L.stream(x_fp8.device))
    return y
