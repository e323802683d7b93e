"""Torch-facing wrappers of miq_moe_align, miq_w4a16_moe, miq_w8a16_moe and miq_fp8_moe.

The layer wrappers take topk_ids as the reference's fused_moe does. By default they call
the routed entry points, whose expert GEMMs align the pairs themselves (no align launch;
the library falls back to moe_align internally past its LDS tables); routed=False runs
moe_align and passes its layout explicitly (the same results).

moe_align keeps the contract of the reference (kernels/fused_moe/fused_moe_triton.py:8-39
and csrc/moe_align.cu:5-88): (sorted_ids, expert_ids, num_padded) with the pairs of each
expert padded to block_m by the sentinel T*k. fused_moe_int4 replaces the per-expert loop
of QuantExperts.forward (engine/quantization/modules.py:55-75) for INT4 experts.
"""
import torch

from kernels import _lib as L

BLOCK_M = 16  # rows per expert tile of the grouped GEMMs


def moe_align(topk_ids, num_experts, block_m):
    L.require_device(topk_ids)
    flat = topk_ids.reshape(-1)
    if flat.dtype not in (torch.int32, torch.int64):
        raise RuntimeError("moe_align: topk_ids must be int32 or int64")
    flat = flat.contiguous()
    num_pairs = flat.numel()
    max_padded = num_pairs + num_experts * (block_m - 1)
    max_blocks = (max_padded + block_m - 1) // block_m
    dev = flat.device
    sorted_ids = torch.empty(max_padded, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(max_blocks, dtype=torch.int32, device=dev)
    num_padded = torch.empty(1, dtype=torch.int32, device=dev)
    L.call("miq_moe_align", L.ptr(flat), L.dtype_code(flat.dtype), num_pairs, num_experts, block_m,
           L.ptr(sorted_ids), L.ptr(expert_ids), L.ptr(num_padded), L.stream(dev))
    return sorted_ids, expert_ids, num_padded


def _ids(topk_ids):
    flat = topk_ids.reshape(-1)
    if flat.dtype not in (torch.int32, torch.int64):
        raise RuntimeError("fused moe: topk_ids must be int32 or int64")
    return flat.contiguous()


def fused_moe_int4(hidden, topk_ids, topk_weights, gu_q, gu_scale, gu_zero, dn_q, dn_scale, dn_zero, routed=True):
    """out[t] = sum_j w[t, j] * down_e(silu(gate_e(x_t)) * up_e(x_t)), e = topk_ids[t, j].

    hidden bf16 [T, H]; gu_q uint8 [E, 2I, H/2]; dn_q uint8 [E, H, I/2]; scale/zero
    [E, rows, K/group] (zero may be None: symmetric codes)."""
    L.require_device(hidden, topk_ids, topk_weights, gu_q, dn_q)
    T, H = hidden.shape
    E, two_i, _ = gu_q.shape
    inter = two_i // 2
    k = topk_ids.shape[-1]
    group = H // gu_scale.shape[-1]
    if dn_scale.shape[-1] * group != inter:
        raise RuntimeError("fused_moe_int4: gate_up and down must share one group size")
    h = hidden.contiguous()
    w = topk_weights.contiguous()  # used in its own dtype, as the reference multiplies by it
    nbytes = L.load().miq_moe_workspace_bytes(T, k, E, H, inter)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=hidden.device)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=hidden.device)
    sdt = gu_scale.dtype
    weights = (L.ptr(gu_q.contiguous()), L.ptr(gu_scale.contiguous()),
               L.ptr(None if gu_zero is None else gu_zero.contiguous()),
               L.ptr(dn_q.contiguous()), L.ptr(dn_scale.contiguous()),
               L.ptr(None if dn_zero is None else dn_zero.contiguous()),
               L.dtype_code(sdt), group, L.ptr(w), L.dtype_code(w.dtype))
    if routed:
        ids = _ids(topk_ids)
        L.call("miq_w4a16_moe_routed", L.ptr(h), T, H, inter, E, k, *weights, L.ptr(ids), L.dtype_code(ids.dtype),
               L.ptr(ws), nbytes, L.ptr(out), L.stream(hidden.device))
        return out
    sorted_ids, expert_ids, num_padded = moe_align(topk_ids, E, BLOCK_M)
    L.call("miq_w4a16_moe", L.ptr(h), T, H, inter, E, k, *weights,
           L.ptr(sorted_ids), L.ptr(expert_ids), L.ptr(num_padded), L.ptr(ws), nbytes, L.ptr(out), L.stream(hidden.device))
    return out


def fused_moe_int8(hidden, topk_ids, topk_weights, gu_q, gu_scale, dn_q, dn_scale, routed=True):
    """The INT8 twin of fused_moe_int4: every expert linear is int8_wo.linear
    (bf16(bf16(x @ q^T) * bf16(scale)), int8_wo.py:17-21) and the rest of the layer is the
    reference loop's (modules.py:55-75). gu_q int8 [E, 2I, H], gu_scale [E, 2I(, 1)];
    dn_q int8 [E, H, I], dn_scale [E, H(, 1)]; both scales of one dtype."""
    L.require_device(hidden, topk_ids, topk_weights, gu_q, dn_q, gu_scale, dn_scale)
    T, H = hidden.shape
    E, two_i, _ = gu_q.shape
    inter = two_i // 2
    k = topk_ids.shape[-1]
    if dn_scale.dtype != gu_scale.dtype:
        raise RuntimeError("fused_moe_int8: gate_up and down scales must share a dtype")
    h = hidden.contiguous()
    w = topk_weights.contiguous()
    nbytes = L.load().miq_moe_workspace_bytes(T, k, E, H, inter)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=hidden.device)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=hidden.device)
    gs, ds = gu_scale.contiguous(), dn_scale.contiguous()
    weights = (L.ptr(gu_q.contiguous()), L.ptr(gs), L.ptr(dn_q.contiguous()), L.ptr(ds), L.dtype_code(gs.dtype),
               L.ptr(w), L.dtype_code(w.dtype))
    if routed:
        ids = _ids(topk_ids)
        L.call("miq_w8a16_moe_routed", L.ptr(h), T, H, inter, E, k, *weights, L.ptr(ids), L.dtype_code(ids.dtype),
               L.ptr(ws), nbytes, L.ptr(out), L.stream(hidden.device))
        return out
    sorted_ids, expert_ids, num_padded = moe_align(topk_ids, E, BLOCK_M)
    L.call("miq_w8a16_moe", L.ptr(h), T, H, inter, E, k, *weights,
           L.ptr(sorted_ids), L.ptr(expert_ids), L.ptr(num_padded), L.ptr(ws), nbytes, L.ptr(out),
           L.stream(hidden.device))
    return out


def fused_moe_fp8(hidden, topk_ids, topk_weights, gu_q, gu_scale, dn_q, dn_scale, routed=True):
    """The FP8 twin of fused_moe_int4: every expert linear is FP8WeightAct.linear on a
    native device (fp8.py:48-61): the activation rows quantized per row to e4m3 with
    s = amax / 448, then bf16(sum(x_q w_q) * s_x * s_w). gu_q float8_e4m3fn [E, 2I, H],
    gu_scale fp32 [E, 2I]; dn_q float8_e4m3fn [E, H, I], dn_scale fp32 [E, H]; H and I
    multiples of 128 and at most 4096."""
    L.require_device(hidden, topk_ids, topk_weights, gu_q, dn_q, gu_scale, dn_scale)
    T, H = hidden.shape
    E, two_i, _ = gu_q.shape
    inter = two_i // 2
    k = topk_ids.shape[-1]
    if gu_scale.dtype != torch.float32 or dn_scale.dtype != torch.float32:
        raise RuntimeError("fused_moe_fp8: scales must be float32")
    h = hidden.contiguous()
    w = topk_weights.contiguous()
    nbytes = L.load().miq_moe_workspace_bytes(T, k, E, H, inter)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=hidden.device)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=hidden.device)
    weights = (L.ptr(gu_q.contiguous()), L.ptr(gu_scale.contiguous()), L.ptr(dn_q.contiguous()),
               L.ptr(dn_scale.contiguous()), L.ptr(w), L.dtype_code(w.dtype))
    if routed:
        ids = _ids(topk_ids)
        L.call("miq_fp8_moe_routed", L.ptr(h), T, H, inter, E, k, *weights, L.ptr(ids), L.dtype_code(ids.dtype),
               L.ptr(ws), nbytes, L.ptr(out), L.stream(hidden.device))
        return out
    sorted_ids, expert_ids, num_padded = moe_align(topk_ids, E, BLOCK_M)
    L.call("miq_fp8_moe", L.ptr(h), T, H, inter, E, k, *weights,
           L.ptr(sorted_ids), L.ptr(expert_ids), L.ptr(num_padded), L.ptr(ws), nbytes, L.ptr(out),
           L.stream(hidden.device))
    return out
