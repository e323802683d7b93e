"""Drop-in quantized modules (reference: engine/quantization/modules.py:1-85).

`QuantLinear` registers the method's tensors as buffers under the method's own keys
(`qweight`, `scale`, [`zero`]) and calls `method.linear`; `QuantExperts` holds 3-D
expert weights (`gate_up_*` [E, 2I, H], `down_*` [E, H, I]) with the same buffer names
as the reference, so state dicts and quantized-weight caches load unchanged.

For INT4 experts with a SiLU gate, `QuantExperts.forward` runs the fused MoE kernels
(moe_align + grouped W4A16 GEMMs) instead of the reference's per-expert host loop; the
loop (modules.py:55-75) remains for the other methods.
"""
import torch
from torch import nn

from engine.quantization.int4_wo import Int4WeightOnly
from kernels.fused_moe import fused_moe_int4


def _register(module: nn.Module, prefix: str, tensors: dict):
    for key, tensor in tensors.items():
        module.register_buffer(f"{prefix}{key}", tensor)


def _collect(module: nn.Module, prefix: str, keys) -> dict:
    return {key: getattr(module, f"{prefix}{key}") for key in keys}


class QuantLinear(nn.Module):
    """modules.py:15-33."""

    def __init__(self, linear: nn.Linear, method):
        super().__init__()
        self.method = method
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        q = method.quantize(linear.weight.data)
        self._keys = list(q)
        _register(self, "", q)
        self.bias = None if linear.bias is None else nn.Parameter(linear.bias.data, requires_grad=False)

    def forward(self, x):
        y = self.method.linear(x, **_collect(self, "", self._keys))
        if self.bias is not None:
            y = y + self.bias
        return y

    def extra_repr(self):
        return f"in={self.in_features}, out={self.out_features}, method={self.method.name}"


class QuantExperts(nn.Module):
    """modules.py:36-78: same routing contract as transformers' OlmoeExperts.forward."""

    def __init__(self, experts: nn.Module, method):
        super().__init__()
        self.method = method
        self.num_experts = experts.gate_up_proj.shape[0]
        self.act_fn = experts.act_fn

        gate_up = method.quantize(experts.gate_up_proj.data)
        down = method.quantize(experts.down_proj.data)
        self._keys = list(gate_up)
        _register(self, "gate_up_", gate_up)
        _register(self, "down_", down)

    def _expert_weights(self, prefix, e):
        # Every quantized tensor has the expert dimension first, so [e] picks one expert
        return {k: v[e] for k, v in _collect(self, prefix, self._keys).items()}

    def _fused_ok(self, hidden_states):
        if not isinstance(self.method, Int4WeightOnly) or hidden_states.device.type != "cuda":
            return False
        if hidden_states.dtype != torch.bfloat16 or not isinstance(self.act_fn, nn.SiLU):
            return False
        gs = self.method.group_size
        H = hidden_states.shape[-1]
        inter = self.down_qweight.shape[-1] * 2
        return gs % 128 == 0 and H % gs == 0 and inter % gs == 0 and H % 64 == 0 and inter % 32 == 0

    def forward(self, hidden_states, top_k_index, top_k_weights):
        if self._fused_ok(hidden_states):
            return fused_moe_int4(hidden_states, top_k_index, top_k_weights,
                                  self.gate_up_qweight, self.gate_up_scale, getattr(self, "gate_up_zero", None),
                                  self.down_qweight, self.down_scale, getattr(self, "down_zero", None))
        final_hidden_states = torch.zeros_like(hidden_states)
        with torch.no_grad():
            expert_mask = nn.functional.one_hot(top_k_index, num_classes=self.num_experts + 1)
            expert_mask = expert_mask.permute(2, 1, 0)
            expert_hit = torch.greater(expert_mask.sum(dim=(-1, -2)), 0).nonzero()
        for expert_idx in expert_hit:
            e = int(expert_idx[0])
            if e == self.num_experts:
                continue
            top_k_pos, token_idx = torch.where(expert_mask[e])
            current = hidden_states[token_idx]
            gate, up = self.method.linear(current, **self._expert_weights("gate_up_", e)).chunk(2, dim=-1)
            current = self.act_fn(gate) * up
            current = self.method.linear(current, **self._expert_weights("down_", e))
            current = current * top_k_weights[token_idx, top_k_pos, None]
            final_hidden_states.index_add_(0, token_idx, current.to(final_hidden_states.dtype))
        return final_hidden_states

    def extra_repr(self):
        return f"num_experts={self.num_experts}, method={self.method.name}"


def is_fused_experts(module: nn.Module) -> bool:
    """modules.py:81-85: OLMoE-style experts, two 3-D weights with the expert dim first."""
    gu = getattr(module, "gate_up_proj", None)
    dn = getattr(module, "down_proj", None)
    return (isinstance(gu, nn.Parameter) and isinstance(dn, nn.Parameter)
            and gu.dim() == 3 and dn.dim() == 3)
