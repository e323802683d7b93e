"""FP8 (e4m3fn) weight + per-token dynamic activation quantization (W8A8).

Reference: engine/quantization/fp8.py:1-75. Buffers `qweight` float8_e4m3fn [..., N, K]
and `scale` fp32 [..., N]. The reference calls torch._scaled_mm when the device has
native FP8 and otherwise emulates it; on gfx950 FP8 is native and `linear` runs the
activation-quantize kernel and the FP8 MFMA GEMM of libmiq. `backend` is accepted for
API compatibility; "emulate" keeps the reference's emulation formula (fp8.py:69-73) on
the device.
"""
import torch

from engine.quantization.base import QuantMethod
from kernels import quant_ops as ops

FP8 = torch.float8_e4m3fn
FP8_MAX = torch.finfo(FP8).max   # 448.0


def native_fp8_available(device) -> bool:
    """fp8.py:8-12: every ROCm device this library targets (gfx950) computes FP8."""
    return torch.device(device).type == "cuda"


class FP8WeightAct(QuantMethod):
    name = "fp8"

    def __init__(self, backend: str = "auto", device="cpu", **kwargs):
        super().__init__(**kwargs)
        if backend == "auto":
            self.native = native_fp8_available(device)
        else:
            self.native = backend == "native"

    def _padded_weight(self, qweight, pad):
        """qweight with `pad` zero columns, made once per weight tensor instead of on every
        call. The entry holds the source tensor, so its address cannot be reused by another
        weight while the entry exists; an in-place update of the weight makes a new entry."""
        key = (qweight.data_ptr(), qweight._version, tuple(qweight.shape))
        cache = self.__dict__.setdefault("_pads", {})
        hit = cache.get(key)
        if hit is None or hit[0] is not qweight:
            hit = (qweight, torch.nn.functional.pad(qweight.view(torch.uint8), (0, pad)).view(FP8))
            cache[key] = hit
        return hit[1]

    def supports(self, weight):
        """fp8.py:28-30."""
        return weight.shape[-1] % 16 == 0 and weight.shape[-2] % 16 == 0

    def quantize(self, weight):
        """fp8.py:32-36: per-row s = amax / 448, q = e4m3fn(clamp(w / s))."""
        q, scale = ops.fp8_quantize_rows(weight)
        return {"qweight": q, "scale": scale}

    def dequantize(self, qweight, scale):
        """fp8.py:38-39."""
        return ops.fp8_dequantize(qweight, scale)

    @staticmethod
    def quantize_activation(x2d):
        """fp8.py:41-46: per-token dynamic quantization -> (x_fp8 [M, K], scale fp32 [M, 1])."""
        q, s = ops.fp8_quantize_rows(x2d)
        return q, s.unsqueeze(-1)

    def linear(self, x, qweight, scale):
        """fp8.py:48-73."""
        out_dtype = x.dtype
        x2d = x.reshape(-1, x.shape[-1])
        x_fp8, x_scale = self.quantize_activation(x2d)
        if self.native:
            K = x2d.shape[-1]
            w = qweight
            if K % 128:  # the MFMA kernel takes K in steps of 128: zero padding adds nothing
                pad = 128 - K % 128
                x_fp8 = torch.nn.functional.pad(x_fp8.view(torch.uint8), (0, pad)).view(FP8)
                w = self._padded_weight(qweight, pad)
            y = ops.fp8_gemm(x_fp8, x_scale, w, scale)
            return y.to(out_dtype).reshape(*x.shape[:-1], -1)
        # emulation (fp8.py:69-73): same FP8 rounding, matmul in the compute dtype
        x_deq = x_fp8.to(out_dtype) * x_scale.to(out_dtype)
        y = torch.nn.functional.linear(x_deq, qweight.to(out_dtype))
        y = y * scale.to(out_dtype)
        return y.reshape(*x.shape[:-1], -1)

    def describe(self):
        return {"method": self.name, "fp8_backend": "native" if self.native else "emulated"}
