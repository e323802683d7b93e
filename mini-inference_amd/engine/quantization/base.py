"""QuantMethod interface (reference: engine/quantization/base.py:3-26).

Same names and contract as the reference: `quantize(w) -> dict`, `dequantize(**q)`,
`linear(x, **q)`, `supports(w)`, `describe()`. The default `linear` is the reference's
"dequantize then matmul" path (base.py:20-24); here the dequantize step is the HIP kernel
and the matmul is the device GEMM of torch.
"""
import torch


class QuantMethod:
    name = "base"

    def __init__(self, compute_dtype=torch.bfloat16):
        # dtype of activations and outputs
        self.compute_dtype = compute_dtype

    def supports(self, weight: torch.Tensor) -> bool:
        """Whether this weight's shape can be quantized (otherwise it stays in bf16)."""
        return True

    def quantize(self, weight: torch.Tensor) -> dict:
        raise NotImplementedError

    def dequantize(self, **q) -> torch.Tensor:
        raise NotImplementedError

    def linear(self, x: torch.Tensor, **q) -> torch.Tensor:
        """Rebuild the weight in x's dtype, then an ordinary matmul (base.py:20-24)."""
        w = self.dequantize(**q).to(x.dtype)
        return torch.nn.functional.linear(x, w)

    def describe(self) -> dict:
        return {"method": self.name}
