"""CPU restatement of a quantized model for end-to-end checks: TEST INFRASTRUCTURE ONLY.

`oracle_model(model)` copies a model whose linears / experts were swapped by
quantize_model (QuantLinear / QuantExperts, any device) to an fp32 CPU model in which
every quantized module computes the reference's formula on the same stored codes in fp32:

  int8_wo   y = (x @ q^T) * s                                    int8_wo.py:17-21
  int4_wo   y = x @ (q * s + z)^T   (symmetric codes: (q - 8) s) int4_wo.py:33-42, base.py:20-24
  fp8       per-token e4m3 x, y = (x_fp8 @ w_fp8^T) * s_x * s_w  fp8.py:41-73
  experts   per-expert dequantized INT4 MoE                      fused_moe/reference.py:5-15

`OracleKVCache` stores keys / values like engine/core/kv_cache.py (8-bit codes and one
bf16-rounded scale per (token, head), kv_cache.py:359-388) with the restated quantizer,
and `oracle_decode_attention` is the fp32 per-request paged attention
(kernels/paged_attention/reference.py:10-28). With these, the build's ModelRunner
(engine/core/model_runner.py) runs entirely on the CPU in fp32.
"""
import copy

import torch
from torch import nn

from engine.core.kv_cache import CacheBookkeeping, make_allocator
from oracle import quant as Q
from oracle.attention import paged_decode_reference
from oracle.moe import int4_experts_reference, quant_experts_loop


def quant_linear_fp32(name, x2, q):
    """The method's linear on 2-D x, in fp32 on the stored codes."""
    x2 = x2.float()
    if name == "int8_wo":
        return (x2 @ q["qweight"].float().t()) * q["scale"].float().reshape(1, -1)
    if name == "int4_wo":
        return Q.int4_linear_fp32(x2, q["qweight"], q["scale"], q.get("zero"))
    if name == "fp8":
        xq, xs = Q.fp8_quantize_activation(x2)
        return Q.fp8_scaled_mm(xq, xs, q["qweight"], q["scale"])
    raise ValueError(f"no oracle for method {name}")


def quant_linear(name, x2, q, dtype):
    """quant_linear_fp32 with the output in `dtype`. In bf16 the roundings are the ones of
    the reference's bf16 formulas: int8 y = bf16(bf16(x @ q^T) * bf16(s)) (int8_wo.py:20-21),
    the others one rounding of the fp32 result."""
    if dtype == torch.float32:
        return quant_linear_fp32(name, x2, q)
    if name == "int8_wo":
        acc = (x2.float() @ q["qweight"].float().t()).to(dtype).float()
        return (acc * q["scale"].to(dtype).float().reshape(1, -1)).to(dtype)
    return quant_linear_fp32(name, x2, q).to(dtype)


class OracleLinear(nn.Module):
    def __init__(self, qlinear, dtype=torch.float32):
        super().__init__()
        self.name = qlinear.method.name
        self.dtype = dtype
        # the method's tensors are the module's buffers, named after the method's dict keys
        self.q = {k: t.detach().cpu() for k, t in qlinear.named_buffers(recurse=False)}
        self.bias = None if qlinear.bias is None else qlinear.bias.detach().cpu().to(dtype)

    def forward(self, x):
        shape = x.shape
        y = quant_linear(self.name, x.reshape(-1, shape[-1]), self.q, self.dtype)
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*shape[:-1], -1)


class OracleExperts(nn.Module):
    """QuantExperts.forward's contract (hidden [T, H], top_k_index, top_k_weights)."""

    def __init__(self, qexperts, dtype=torch.float32):
        super().__init__()
        self.name = qexperts.method.name
        self.dtype = dtype
        self.num_experts = qexperts.num_experts
        bufs = dict(qexperts.named_buffers(recurse=False))
        self.gu = {k[len("gate_up_"):]: t.detach().cpu() for k, t in bufs.items() if k.startswith("gate_up_")}
        self.dn = {k[len("down_"):]: t.detach().cpu() for k, t in bufs.items() if k.startswith("down_")}

    def forward(self, hidden_states, top_k_index, top_k_weights):
        if self.dtype != torch.float32:
            # the reference's per-expert loop (modules.py:55-75) with its roundings
            lin = lambda x, **q: quant_linear(self.name, x, q, self.dtype)  # noqa: E731
            return quant_experts_loop(hidden_states.to(self.dtype), lin, self.gu, self.dn, top_k_index,
                                      top_k_weights.to(self.dtype), self.num_experts)
        if self.name == "int4_wo":
            return int4_experts_reference(hidden_states.float(), self.gu, self.dn, top_k_weights.float(),
                                          top_k_index)
        # fused_moe/reference.py:5-15 with each expert's linear restated for the method
        x = hidden_states.float()
        out = torch.zeros_like(x)
        for e in top_k_index.unique().tolist():
            token, slot = torch.where(top_k_index == e)
            gu = quant_linear_fp32(self.name, x[token], {k: v[e] for k, v in self.gu.items()})
            inter = gu.shape[-1] // 2
            h = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
            y = quant_linear_fp32(self.name, h, {k: v[e] for k, v in self.dn.items()})
            out.index_add_(0, token, y * top_k_weights[token, slot].float()[:, None])
        return out


def oracle_model(model, dtype=torch.float32):
    """A CPU copy of `model` in `dtype` with every QuantLinear / QuantExperts replaced by
    the restated formula on the same codes. fp32: everything in fp32 (the rest of the
    model: the same bf16 values widened). bf16: the model's own modules in bf16 on the
    CPU, the quantized ones accumulating in fp32 and rounding their outputs to bf16."""
    from engine.quantization.modules import QuantExperts, QuantLinear

    swaps = {}
    for name, module in model.named_modules():
        if isinstance(module, QuantLinear):
            swaps[name] = OracleLinear(module, dtype)
        elif isinstance(module, QuantExperts):
            swaps[name] = OracleExperts(module, dtype)
    # copy without the quantized modules (their buffers may live on the GPU)
    saved = {}
    for name in swaps:
        parent, _, child = name.rpartition(".")
        owner = model.get_submodule(parent) if parent else model
        saved[name] = getattr(owner, child)
        setattr(owner, child, nn.Identity())
    try:
        cpu = copy.deepcopy(model).to("cpu").to(dtype)
    finally:
        for name, module in saved.items():
            parent, _, child = name.rpartition(".")
            setattr(model.get_submodule(parent) if parent else model, child, module)
    for name, module in swaps.items():
        parent, _, child = name.rpartition(".")
        setattr(cpu.get_submodule(parent) if parent else cpu, child, module)
    return cpu.eval()


class OracleKVCache(CacheBookkeeping):
    """engine/core/kv_cache.py:305-420 storage on the CPU with the restated quantizer. Slot
    bookkeeping (which slots a request owns, its block table) is the product's host-side
    allocator: it decides where values go, not what they are."""

    def __init__(self, num_layers, num_kv_heads, head_dim, capacity_tokens, dtype=torch.float32, kv_dtype=None,
                 scale_dtype=torch.bfloat16, mode="paged", block_size=16):
        self.mode = mode
        self.allocator = make_allocator(mode, capacity_tokens, block_size)
        self.kv_dtype = kv_dtype
        self.model_dtype = dtype
        self.scale_dtype = scale_dtype
        shape = (num_layers, capacity_tokens, num_kv_heads, head_dim)
        if kv_dtype is None:
            self.k = torch.zeros(shape, dtype=dtype)
            self.v = torch.zeros(shape, dtype=dtype)
            self.k_scale = self.v_scale = None
        else:
            store = torch.int8 if kv_dtype == "int8" else Q.FP8
            self.k = torch.zeros(shape, dtype=store)
            self.v = torch.zeros(shape, dtype=store)
            self.k_scale = torch.ones(shape[:3], dtype=scale_dtype)
            self.v_scale = torch.ones(shape[:3], dtype=scale_dtype)

    def write(self, layer, slots, k, v):
        slots = slots.long()
        if self.kv_dtype is None:
            self.k[layer][slots] = k.to(self.model_dtype)
            self.v[layer][slots] = v.to(self.model_dtype)
            return
        for cache, scale, x in ((self.k, self.k_scale, k), (self.v, self.v_scale, v)):
            q, s = Q.kv_quantize(x, self.kv_dtype, self.scale_dtype)
            if q.dtype == Q.FP8:
                cache[layer].view(torch.uint8)[slots] = q.view(torch.uint8)
            else:
                cache[layer][slots] = q
            scale[layer][slots] = s

    def gather(self, layer, idx):
        idx = idx.long()
        if self.kv_dtype is None:
            return self.k[layer][idx], self.v[layer][idx]
        out = []
        for cache, scale in ((self.k, self.k_scale), (self.v, self.v_scale)):
            c = cache[layer]
            q = c.view(torch.uint8)[idx].view(Q.FP8) if c.dtype == Q.FP8 else c[idx]
            out.append(Q.kv_dequantize(q, scale[layer][idx]).to(self.model_dtype))
        return tuple(out)


def oracle_decode_attention(q, k_cache, v_cache, block_table, seq_lens, page_size, scale, max_len=None,
                            k_scale=None, v_scale=None, **_):
    """paged_decode_attention's contract, computed by the fp32 per-request reference."""
    return paged_decode_reference(q, k_cache, v_cache, block_table, seq_lens, page_size, scale,
                                  k_scale, v_scale).to(q.dtype)
