"""INT4 group-wise weight-only quantization (W4A16).

Reference: engine/quantization/int4_wo.py:5-44. Asymmetric codes 0..15 with a bf16
scale and zero (= group min) per (row, group); two codes per byte, the even k in the
low nibble. `symmetric=True` (no counterpart in the reference) stores codes
clamp(round(w / s), -8, 7) + 8 with s = max|w| / 7 and no zero tensor; it is the format
of the INT4 benchmark configuration.
"""
import torch

from engine.quantization.base import QuantMethod
from kernels import quant_ops as ops


class Int4WeightOnly(QuantMethod):
    name = "int4_wo"

    def __init__(self, group_size: int = 128, symmetric: bool = False, **kwargs):
        super().__init__(**kwargs)
        self.group_size = group_size
        self.symmetric = symmetric

    def supports(self, weight):
        """int4_wo.py:12-13."""
        return weight.shape[-1] % self.group_size == 0 and self.group_size % 2 == 0

    def quantize(self, weight):
        """int4_wo.py:15-31."""
        q, scale, zero = ops.int4_quantize(weight, self.group_size, self.compute_dtype, self.symmetric)
        out = {"qweight": q, "scale": scale}
        if zero is not None:
            out["zero"] = zero
        return out

    def dequantize(self, qweight, scale, zero=None):
        """int4_wo.py:33-42 (bit-exact: two roundings to the scale dtype)."""
        return ops.int4_dequantize(qweight, scale, zero)

    def linear(self, x, qweight, scale, zero=None):
        """base.py:20-24 with the int4 dequantize.

        The fused GEMM runs for every M (the decode kernels up to 64 rows, the prefill and
        wide kernels above: the weights are unpacked inside the K loop and never written out
        as bf16); shapes outside its contract (see ops.w4a16_supported) dequantize with the
        HIP kernel and use the device GEMM."""
        if ops.w4a16_supported(x, qweight, scale):
            return ops.w4a16_linear(x, qweight, scale, zero)
        w = self.dequantize(qweight, scale, zero).to(x.dtype)
        return torch.nn.functional.linear(x, w)

    def describe(self):
        d = {"method": self.name, "group_size": self.group_size}
        if self.symmetric:
            d["symmetric"] = True
        return d
