"""INT8 per-output-channel weight-only quantization (W8A16).

Reference: engine/quantization/int8_wo.py:5-21. Buffers `qweight` int8 [..., N, K] and
`scale` [..., N, 1] in compute_dtype, exactly as the reference stores them.
"""
import torch

from engine.quantization.base import QuantMethod
from kernels import quant_ops as ops


class Int8WeightOnly(QuantMethod):
    name = "int8_wo"

    def quantize(self, weight: torch.Tensor) -> dict:
        """int8_wo.py:8-12: s = max|w_row| / 127, q = round(w / s) in [-127, 127]."""
        q, scale = ops.int8_quantize(weight, self.compute_dtype)
        return {"qweight": q, "scale": scale}

    def dequantize(self, qweight, scale) -> torch.Tensor:
        """int8_wo.py:14-15."""
        return ops.int8_dequantize(qweight, scale)

    def linear(self, x, qweight, scale):
        """int8_wo.py:17-21: (x @ q^T) * scale.

        The fused GEMM runs for every M (the int8 codes are read once, no bf16 weight is
        written); shapes outside its contract (see ops.w8a16_supported) use the reference's
        own formula with the device GEMM."""
        if ops.w8a16_supported(x, qweight):
            return ops.w8a16_linear(x, qweight, scale)
        y = torch.nn.functional.linear(x, qweight.to(x.dtype))
        return y * scale.squeeze(-1).to(x.dtype)
