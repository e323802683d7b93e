"""The quantization-method interface (reference: engine/quantization/base.py:3-26).

A method turns a float weight into a dict of tensors (`quantize`), back into a float
weight (`dequantize`), and multiplies activations by the stored form (`linear`).
`supports` says whether a weight's shape fits the format; rejected weights stay in the
model dtype. The generic `linear` rebuilds the float weight and calls an ordinary
matmul (base.py:20-24); the subclasses replace it with the fused HIP kernels where the
shapes allow.
"""
import torch


class QuantMethod:
    name = "base"

    def __init__(self, compute_dtype=torch.bfloat16):
        self.compute_dtype = compute_dtype  # activations in, outputs out

    def supports(self, weight: torch.Tensor) -> bool:
        return True

    def quantize(self, weight: torch.Tensor) -> dict:
        raise NotImplementedError

    def dequantize(self, **q) -> torch.Tensor:
        raise NotImplementedError

    def linear(self, x: torch.Tensor, **q) -> torch.Tensor:
        """x @ dequantize(**q)^T with the weight cast to x's dtype first."""
        return torch.nn.functional.linear(x, self.dequantize(**q).to(x.dtype))

    def describe(self) -> dict:
        return {"method": self.name}
