"""CPU restatement of the reference's quantization formulas (test infrastructure only).

All functions take and return CPU tensors and use PyTorch's CPU arithmetic, which is what
the reference runs on CPU: fp32 math for quantization, the storage dtype (bf16) for
dequantization and for the weight-only linears.
"""
import torch

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0


# ---------------------------------------------------------------- int8 weight-only
def int8_quantize(weight, compute_dtype=torch.bfloat16):
    """engine/quantization/int8_wo.py:8-12."""
    w = weight.float()
    scale = w.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8) / 127.0
    q = torch.round(w / scale).clamp(-127, 127).to(torch.int8)
    return {"qweight": q, "scale": scale.to(compute_dtype)}


def int8_dequantize(qweight, scale):
    """int8_wo.py:14-15."""
    return qweight.to(scale.dtype) * scale


def int8_linear(x, qweight, scale):
    """int8_wo.py:17-21: bf16 matmul of x with the int8 codes, then * scale (two roundings)."""
    y = torch.nn.functional.linear(x, qweight.to(x.dtype))
    return y * scale.squeeze(-1).to(x.dtype)


def int8_linear_fp32(x, qweight, scale):
    """fp32-accumulated product on the dequantized weights (the tolerance reference)."""
    return torch.nn.functional.linear(x.float(), qweight.float() * scale.float())


# ---------------------------------------------------------------- int4 weight-only
def int4_quantize(weight, group_size=128, compute_dtype=torch.bfloat16):
    """engine/quantization/int4_wo.py:15-31 (asymmetric, zero = group min)."""
    *lead, out_f, in_f = weight.shape
    g = group_size
    w = weight.float().reshape(*lead, out_f, in_f // g, g)
    w_min = w.amin(dim=-1, keepdim=True)
    w_max = w.amax(dim=-1, keepdim=True)
    scale = ((w_max - w_min) / 15.0).clamp(min=1e-8)
    q = torch.round((w - w_min) / scale).clamp(0, 15).to(torch.uint8)
    q = q.reshape(*lead, out_f, in_f)
    packed = q[..., 0::2] | (q[..., 1::2] << 4)
    return {"qweight": packed, "scale": scale.squeeze(-1).to(compute_dtype),
            "zero": w_min.squeeze(-1).to(compute_dtype)}


def int4_quantize_symmetric(weight, group_size=128, compute_dtype=torch.bfloat16):
    """Symmetric group-wise INT4 of the benchmark configuration (no reference counterpart):
    s = max|w| / 7 (clamped to 1e-8), code = clamp(round(w / s), -8, 7) + 8, same packing
    as int4_wo.py:26."""
    *lead, out_f, in_f = weight.shape
    g = group_size
    w = weight.float().reshape(*lead, out_f, in_f // g, g)
    scale = (w.abs().amax(dim=-1, keepdim=True) / 7.0).clamp(min=1e-8)
    q = (torch.round(w / scale).clamp(-8, 7) + 8).to(torch.uint8).reshape(*lead, out_f, in_f)
    packed = q[..., 0::2] | (q[..., 1::2] << 4)
    return {"qweight": packed, "scale": scale.squeeze(-1).to(compute_dtype)}


def int4_unpack(qweight):
    """int4_wo.py:34-36: low nibble = even k."""
    low = qweight & 0x0F
    high = qweight >> 4
    return torch.stack((low, high), dim=-1).reshape(*qweight.shape[:-1], qweight.shape[-1] * 2)


def int4_dequantize(qweight, scale, zero=None):
    """int4_wo.py:33-42: q * scale + zero in the scale dtype (two roundings);
    zero None: the symmetric format, (q - 8) * scale (one rounding)."""
    q = int4_unpack(qweight)
    *lead, out_f, in_f = q.shape
    g = in_f // scale.shape[-1]
    q = q.reshape(*lead, out_f, in_f // g, g)
    if zero is None:
        w = ((q.float() - 8.0) * scale.float().unsqueeze(-1)).to(scale.dtype)
    else:
        q = q.to(scale.dtype)
        w = q * scale.unsqueeze(-1) + zero.unsqueeze(-1)
    return w.reshape(*lead, out_f, in_f)


def int4_linear(x, qweight, scale, zero=None):
    """engine/quantization/base.py:20-24 with int4_dequantize."""
    return torch.nn.functional.linear(x, int4_dequantize(qweight, scale, zero).to(x.dtype))


def int4_linear_fp32(x, qweight, scale, zero=None):
    """fp32-accumulated product on the exactly dequantized weights (q * s + z in fp32)."""
    q = int4_unpack(qweight).float()
    *lead, out_f, in_f = q.shape
    g = in_f // scale.shape[-1]
    q = q.reshape(*lead, out_f, in_f // g, g)
    s = scale.float().unsqueeze(-1)
    w = (q - 8.0) * s if zero is None else q * s + zero.float().unsqueeze(-1)
    return torch.nn.functional.linear(x.float(), w.reshape(*lead, out_f, in_f))


# ---------------------------------------------------------------- fp8 weight + activation
def fp8_quantize(weight):
    """engine/quantization/fp8.py:32-36."""
    w = weight.float()
    scale = w.abs().amax(dim=-1, keepdim=True).clamp(min=1e-12) / FP8_MAX
    q = (w / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8)
    return {"qweight": q, "scale": scale.squeeze(-1)}


def fp8_dequantize(qweight, scale):
    """fp8.py:38-39."""
    return qweight.float() * scale.unsqueeze(-1)


def fp8_quantize_activation(x2d):
    """fp8.py:41-46."""
    scale = x2d.float().abs().amax(dim=-1, keepdim=True).clamp(min=1e-12) / FP8_MAX
    x_fp8 = (x2d.float() / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8)
    return x_fp8, scale


def fp8_linear_emulated(x, qweight, scale):
    """fp8.py:48-73, the emulation branch (what the reference runs without native FP8)."""
    out_dtype = x.dtype
    x2d = x.reshape(-1, x.shape[-1])
    x_fp8, x_scale = fp8_quantize_activation(x2d)
    x_deq = x_fp8.to(out_dtype) * x_scale.to(out_dtype)
    y = torch.nn.functional.linear(x_deq, qweight.to(out_dtype))
    y = y * scale.to(out_dtype)
    return y.reshape(*x.shape[:-1], -1)


def fp8_scaled_mm(x_fp8, x_scale, qweight, scale):
    """What torch._scaled_mm computes in fp8.py:55-61: fp32 (x_fp8 @ w_fp8^T) * sa * sb."""
    acc = x_fp8.float() @ qweight.float().t()
    return acc * x_scale.reshape(-1, 1).float() * scale.reshape(1, -1).float()


# ---------------------------------------------------------------- KV cache quantize-on-write
KV_QMAX = {"int8": 127.0, "fp8": 448.0}


def kv_quantize(x, kind, model_dtype=torch.bfloat16):
    """engine/core/kv_cache.py:359-369: x [T, heads, D] -> (codes, scale [T, heads])."""
    qmax = KV_QMAX[kind]
    x = x.float()
    scale = (x.abs().amax(dim=-1) / qmax).clamp(min=1e-8).to(model_dtype)
    q = x / scale.float()[..., None]
    if kind == "int8":
        q = q.round().clamp(-127, 127).to(torch.int8)
    else:
        q = q.clamp(-qmax, qmax).to(FP8)
    return q, scale


def kv_dequantize(q, scale):
    """kv_cache.py:396-400 in fp32."""
    return q.float() * scale.float()[..., None]
