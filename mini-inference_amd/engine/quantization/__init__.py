"""Quantization methods registry (reference: engine/quantization/__init__.py:1-20)."""
import torch

from engine.quantization.fp8 import FP8WeightAct
from engine.quantization.int4_wo import Int4WeightOnly
from engine.quantization.int8_wo import Int8WeightOnly

METHODS = {
    "int8_wo": Int8WeightOnly,
    "int4_wo": Int4WeightOnly,
    "fp8": FP8WeightAct,
}


def get_method(name: str, device="cpu", compute_dtype=torch.bfloat16, group_size=128, fp8_backend="auto"):
    """Method object by registry name, with the reference factory's arguments and error
    message (__init__.py:13-20): group_size goes to INT4, device and fp8_backend to FP8."""
    try:
        cls = METHODS[name]
    except KeyError:
        raise ValueError(f"Unknown quantization '{name}'. Options: none, {', '.join(METHODS)}") from None
    extra = {"int4_wo": {"group_size": group_size},
             "fp8": {"backend": fp8_backend, "device": device}}.get(name, {})
    return cls(compute_dtype=compute_dtype, **extra)
