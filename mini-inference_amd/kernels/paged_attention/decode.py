"""paged_decode_attention with the reference's signature and contract
(kernels/paged_attention/decode_triton.py:123-180), on the HIP kernels of libmiq.

Differences in mechanism, not in results:
  * one workgroup handles all query heads of a kv head (the K/V bytes are read once);
  * the context of each request is cut into fixed partitions of `partition` tokens
    (multiple of 128; 256 by default) instead of a
    per-request count of splits. Passing
    num_splits keeps the reference's meaning of "about that many pieces for the longest
    request": the partition becomes cdiv(max_len, num_splits) rounded up to 128.
The workspace (per-partition outputs and log-sum-exps) comes from torch's allocator, so
the call needs no host synchronisation and can be captured in a HIP graph when max_len
(or the block table width) is fixed.
"""
import math

import torch

from kernels import _lib as L

# Default partitions by cache dtype. Config 4 on MI355X (B = 64, 271.5k context tokens),
# with the K / V pages addressed from scalar page bases: FP8 128 / 256 / 512 / 1024 took
# 141.5 / 135.1 / 137.9 / 139.8 us per step, INT8 149.1 / 145.2 / 156.0 / 161.2 us (one
# run each, same box)
DEFAULT_PARTITION = 256
_DEFAULT_PARTITION_BY_DTYPE = {}
_KV_DTYPES = (torch.bfloat16, torch.float8_e4m3fn, torch.int8)


def choose_partition(max_len, num_splits=None, kv_dtype=None):
    if num_splits is None or num_splits < 1:
        return _DEFAULT_PARTITION_BY_DTYPE.get(kv_dtype, DEFAULT_PARTITION)
    per = -(-max_len // num_splits)
    return max(128, -(-per // 128) * 128)


def paged_decode_attention(q, k_cache, v_cache, block_table, seq_lens, page_size, scale, max_len=None,
                           k_scale=None, v_scale=None, num_splits=None, block_n=64, num_warps=4,
                           partition=None):
    """
    q           [B, H, D] bf16      one query token per request (D = 128)
    k_cache     [slots, KV, D]      one layer of the cache (bf16, fp8 e4m3fn or int8)
    v_cache     [slots, KV, D]
    block_table [B, max_pages] int32 page ids per request (PAGE = page_size tokens each)
    seq_lens    [B] int32            context length per request (including the new token)
    max_len     int                  max(seq_lens) from the host; None -> the table's capacity
    k_scale / v_scale [slots, KV]    per-(token, head) scales for 8-bit caches (any strides,
                                     e.g. an expand()ed per-tensor scale), else None
    block_n, num_warps               accepted for signature compatibility (Triton tuning knobs)
    returns     [B, H, D] in q's dtype
    """
    L.require_device(q, k_cache, v_cache, block_table, seq_lens, k_scale, v_scale)
    B, H, D = q.shape
    KV = k_cache.shape[1]
    if H % KV:
        raise ValueError("query heads must be a multiple of kv heads")
    if q.dtype != torch.bfloat16:
        raise RuntimeError(f"paged_decode_attention: q must be bf16 (got {q.dtype})")
    if k_cache.dtype not in _KV_DTYPES or v_cache.dtype != k_cache.dtype:
        raise RuntimeError(f"paged_decode_attention: unsupported cache dtype {k_cache.dtype}")
    if k_cache.stride(2) != 1 or v_cache.stride(2) != 1 or q.stride(2) != 1:
        raise ValueError("the head dimension must be contiguous")
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share strides")
    if (k_scale is None) != (v_scale is None):
        raise ValueError("give both k_scale and v_scale or neither")
    if k_scale is not None and k_scale.stride() != v_scale.stride():
        raise ValueError("k_scale and v_scale must share strides")
    if block_table.dtype != torch.int32:
        block_table = block_table.to(torch.int32)
    if not block_table.is_contiguous():
        # the kernel reads page ids ahead of need, anywhere in B * stride(0) entries: an
        # expanded (stride 0) or column-sliced table is copied to a dense one first
        block_table = block_table.contiguous()
    if seq_lens.dtype != torch.int32:
        seq_lens = seq_lens.to(torch.int32)
    if max_len is None:
        max_len = block_table.shape[1] * page_size
    if partition is None:
        partition = choose_partition(max_len, num_splits, k_cache.dtype)
    max_parts = max(1, math.ceil(max_len / partition))
    out = torch.empty_like(q)
    o_part = torch.empty((B, H, max_parts, D), dtype=torch.float32, device=q.device)
    lse_part = torch.empty((B, H, max_parts), dtype=torch.float32, device=q.device)
    kv_code = L.dtype_code(k_cache.dtype)
    if k_scale is not None:
        s_code, s_st, s_sh = L.dtype_code(k_scale.dtype), k_scale.stride(0), k_scale.stride(1)
    else:
        s_code, s_st, s_sh = L.MIQ_F32, 0, 0
    L.call("miq_paged_decode",
           L.ptr(q), q.stride(0), q.stride(1),
           L.ptr(k_cache), L.ptr(v_cache), kv_code, k_cache.stride(0), k_cache.stride(1),
           L.ptr(k_scale), L.ptr(v_scale), s_code, s_st, s_sh,
           L.ptr(block_table), block_table.stride(0), L.ptr(seq_lens),
           B, H, KV, D, page_size, float(scale), partition, max_parts,
           L.ptr(o_part), L.ptr(lse_part),
           L.ptr(out), out.stride(0), out.stride(1), L.stream(q.device))
    return out
