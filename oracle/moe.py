"""CPU restatement of moe_align and the INT4 MoE references (test infrastructure only)."""
import torch
import torch.nn.functional as F

from oracle import quant


def moe_align(topk_ids, num_experts, block_m):
    """kernels/fused_moe/fused_moe_triton.py:8-39 (stable order inside each expert)."""
    flat = topk_ids.reshape(-1).to(torch.int64)
    num_pairs = flat.numel()
    max_padded = num_pairs + num_experts * (block_m - 1)
    max_blocks = -(-max_padded // block_m)
    counts = torch.bincount(flat, minlength=num_experts)
    padded = (counts + block_m - 1) // block_m * block_m
    ends = torch.cumsum(padded, 0)
    starts = ends - padded
    order = torch.argsort(flat, stable=True)
    sorted_experts = flat[order]
    first = torch.cumsum(counts, 0) - counts
    rank = torch.arange(num_pairs) - first[sorted_experts]
    dest = starts[sorted_experts] + rank
    sorted_ids = torch.full((max_padded,), num_pairs, dtype=torch.int32)
    sorted_ids[dest] = order.to(torch.int32)
    block_starts = torch.arange(max_blocks) * block_m
    expert_ids = torch.searchsorted(ends, block_starts, right=True).clamp_(max=num_experts - 1)
    return sorted_ids, expert_ids.to(torch.int32), ends[-1:].to(torch.int32)


def moe_reference(hidden, w_gate_up, w_down, topk_weights, topk_ids):
    """kernels/fused_moe/reference.py:5-15, fp32 (returned in fp32)."""
    T, H = hidden.shape
    inter = w_down.shape[2]
    out = torch.zeros(T, H, dtype=torch.float32)
    for e in topk_ids.unique().tolist():
        token, slot = torch.where(topk_ids == e)
        x = hidden[token].float()
        gate_up = x @ w_gate_up[e].float().t()
        h = F.silu(gate_up[:, :inter]) * gate_up[:, inter:]
        y = h @ w_down[e].float().t()
        out.index_add_(0, token, y * topk_weights[token, slot].float()[:, None])
    return out


def int4_experts_reference(hidden, gu, dn, topk_weights, topk_ids):
    """The per-expert dequant + matmul reference of the INT4 MoE configuration: the
    experts dequantized exactly (fp32) and fed to moe_reference.
    gu / dn: dicts with qweight, scale, [zero] of [E, rows, ...]."""
    w_gu = _dequant_fp32(gu)
    w_dn = _dequant_fp32(dn)
    return moe_reference(hidden, w_gu, w_dn, topk_weights, topk_ids)


def _dequant_fp32(d):
    q = quant.int4_unpack(d["qweight"]).float()
    *lead, rows, k = q.shape
    g = k // d["scale"].shape[-1]
    q = q.reshape(*lead, rows, k // g, g)
    s = d["scale"].float().unsqueeze(-1)
    z = d.get("zero")
    w = (q - 8.0) * s if z is None else q * s + z.float().unsqueeze(-1)
    return w.reshape(*lead, rows, k)


def quant_experts_loop(hidden, method_linear, gate_up_q, down_q, top_k_index, top_k_weights, num_experts):
    """engine/quantization/modules.py:55-75 on CPU with a given linear(x, **q)."""
    final = torch.zeros_like(hidden)
    mask = F.one_hot(top_k_index, num_classes=num_experts + 1).permute(2, 1, 0)
    hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero()
    for idx in hit:
        e = int(idx[0])
        if e == num_experts:
            continue
        pos, tok = torch.where(mask[e])
        cur = hidden[tok]
        gate, up = method_linear(cur, **{k: v[e] for k, v in gate_up_q.items()}).chunk(2, dim=-1)
        cur = F.silu(gate) * up
        cur = method_linear(cur, **{k: v[e] for k, v in down_q.items()})
        cur = cur * top_k_weights[tok, pos, None]
        final.index_add_(0, tok, cur.to(final.dtype))
    return final
