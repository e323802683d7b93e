"""Quantized drop-in modules: `QuantLinear` and `QuantExperts`.

Interface of the reference's engine/quantization/modules.py:15-85: the method's tensors
are buffers named after the method's dict keys (`qweight`, `scale` and, for asymmetric
INT4, `zero`), prefixed `gate_up_` / `down_` for experts, so state dicts and cache files
are interchangeable; `forward` signatures are the reference's.

`QuantExperts.forward` (modules.py:55-75) takes the fused MoE kernels when the experts
are INT4, INT8 or native FP8 with a SiLU gate on a ROCm device. Otherwise (other gates,
emulated FP8, FP8 layers wider than 4096, the CPU) it groups the (token, slot)
pairs by expert with one sort and runs every hit expert through `method.linear`. The
numerics are the reference loop's: gate/up and down in the compute dtype, the product
with the routing weight in the weights' own dtype, and the results added in ascending
expert order into a zeroed output of the hidden dtype.
"""
import torch
from torch import nn

from engine.quantization.fp8 import FP8WeightAct
from engine.quantization.int4_wo import Int4WeightOnly
from engine.quantization.int8_wo import Int8WeightOnly
from kernels.fused_moe import fused_moe_fp8, fused_moe_int4, fused_moe_int8


class _QuantTensors:
    """Mixin: stores a method's tensor dict as buffers `<prefix><key>` and gives it back."""

    def _store(self, prefix, tensors):
        self._qkeys = tuple(tensors)
        for key in self._qkeys:
            self.register_buffer(prefix + key, tensors[key])

    def _tensors(self, prefix, index=None):
        out = {}
        for key in self._qkeys:
            t = getattr(self, prefix + key)
            out[key] = t if index is None else t[index]
        return out


class QuantLinear(_QuantTensors, nn.Module):
    """nn.Linear with a quantized weight (reference modules.py:15-33); the bias, if any,
    stays a frozen parameter and is added after the quantized product."""

    def __init__(self, linear: nn.Linear, method):
        nn.Module.__init__(self)
        self.method = method
        self.in_features, self.out_features = linear.in_features, linear.out_features
        self._store("", method.quantize(linear.weight.data))
        bias = linear.bias
        self.bias = nn.Parameter(bias.data, requires_grad=False) if bias is not None else None

    def forward(self, x):
        y = self.method.linear(x, **self._tensors(""))
        return y if self.bias is None else y + self.bias

    def extra_repr(self):
        return f"in={self.in_features}, out={self.out_features}, method={self.method.name}"


class QuantExperts(_QuantTensors, nn.Module):
    """OLMoE-style fused experts (3-D `gate_up_proj` [E, 2I, H], `down_proj` [E, H, I])
    with quantized weights (reference modules.py:36-78)."""

    def __init__(self, experts: nn.Module, method):
        nn.Module.__init__(self)
        self.method = method
        self.act_fn = experts.act_fn
        self.num_experts = int(experts.gate_up_proj.shape[0])
        gate_up = method.quantize(experts.gate_up_proj.data)
        down = method.quantize(experts.down_proj.data)
        self._store("gate_up_", gate_up)
        self._store("down_", down)

    def _fused_ok(self, hidden_states):
        """The fused kernels' contract: bf16 activations on the device, a SiLU gate, and INT4
        codes in groups that are whole multiples of 128 dividing H and I, INT8 codes with
        H and I multiples of 128, or native FP8 codes with H and I multiples of 128 of at
        most 4096 (a whole activation row is quantized in one staging)."""
        m = self.method
        if hidden_states.device.type != "cuda" or hidden_states.dtype != torch.bfloat16:
            return False
        if not isinstance(self.act_fn, nn.SiLU) or hidden_states.dim() != 2:
            return False
        hidden = hidden_states.shape[-1]
        if isinstance(m, Int4WeightOnly):
            inter = self.down_qweight.shape[-1] * 2
            return m.group_size % 128 == 0 and hidden % m.group_size == 0 and inter % m.group_size == 0
        if isinstance(m, Int8WeightOnly):
            inter = self.down_qweight.shape[-1]
            return hidden % 128 == 0 and inter % 128 == 0
        if isinstance(m, FP8WeightAct):
            inter = self.down_qweight.shape[-1]
            return m.native and hidden % 128 == 0 and inter % 128 == 0 and hidden <= 4096 and inter <= 4096
        return False

    def forward(self, hidden_states, top_k_index, top_k_weights):
        if self._fused_ok(hidden_states):
            if isinstance(self.method, Int8WeightOnly):
                return fused_moe_int8(hidden_states, top_k_index, top_k_weights, self.gate_up_qweight,
                                      self.gate_up_scale, self.down_qweight, self.down_scale)
            if isinstance(self.method, FP8WeightAct):
                return fused_moe_fp8(hidden_states, top_k_index, top_k_weights, self.gate_up_qweight,
                                     self.gate_up_scale, self.down_qweight, self.down_scale)
            return fused_moe_int4(hidden_states, top_k_index, top_k_weights,
                                  self.gate_up_qweight, self.gate_up_scale, getattr(self, "gate_up_zero", None),
                                  self.down_qweight, self.down_scale, getattr(self, "down_zero", None))
        return self._grouped(hidden_states, top_k_index, top_k_weights)

    def _grouped(self, hidden_states, top_k_index, top_k_weights):
        out = torch.zeros_like(hidden_states)
        k = top_k_index.shape[-1]
        flat = top_k_index.reshape(-1)
        with torch.no_grad():
            # pairs sorted by expert (stable: ascending pair index inside an expert)
            order = torch.sort(flat, stable=True).indices
            experts, counts = torch.unique_consecutive(flat[order], return_counts=True)
        start = 0
        for e, n in zip(experts.tolist(), counts.tolist()):
            pairs = order[start:start + n]
            start += n
            if not 0 <= e < self.num_experts:
                continue  # an out-of-range id (e.g. a padding slot) routes nowhere
            tok, slot = pairs // k, pairs % k
            gu = self.method.linear(hidden_states[tok], **self._tensors("gate_up_", e))
            half = gu.shape[-1] // 2
            h = self.act_fn(gu[..., :half]) * gu[..., half:]
            y = self.method.linear(h, **self._tensors("down_", e)) * top_k_weights[tok, slot, None]
            out.index_add_(0, tok, y.to(out.dtype))
        return out

    def extra_repr(self):
        return f"num_experts={self.num_experts}, method={self.method.name}"


def is_fused_experts(module: nn.Module) -> bool:
    """True for a module holding 3-D `gate_up_proj` and `down_proj` parameters, expert
    dimension first (reference modules.py:81-85)."""
    params = [getattr(module, name, None) for name in ("gate_up_proj", "down_proj")]
    return all(isinstance(p, nn.Parameter) and p.dim() == 3 for p in params)
