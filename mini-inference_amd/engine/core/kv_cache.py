"""8-bit KV-cache storage and its quantize-on-write.

Interface of the reference's engine/core/kv_cache.py (the storage half, :6-35 and
:305-425): the format names "fp8" / "int8", `resolve_kv_dtype`, `kv_bytes_per_token`,
`tokens_for_budget`, and `KVCache` with `write`, `gather`, `decode_tables`, `memory_mb`.

Layout (the reference's, so the paged-attention kernels read it as is):
  k, v                [layers, slots, kv_heads, head_dim] in the storage dtype
  k_scale, v_scale    [layers, slots, kv_heads] in the model dtype, 8-bit formats only
  slot                page_id * block_size + position in the page

`write` is one fused kernel per tensor (amax, bf16 scale, encode, scatter by slot).
The reference's page allocators (free lists, prefix caching) belong to its serving
engine and are not rebuilt here: callers hand in slots and page lists.
"""
from typing import NamedTuple

import torch

from kernels import _lib as L


class KVFormat(NamedTuple):
    dtype: torch.dtype   # storage dtype of the codes
    qmax: float          # largest code magnitude; scale = amax / qmax


KV_FORMATS = {
    "fp8": KVFormat(torch.float8_e4m3fn, float(torch.finfo(torch.float8_e4m3fn).max)),
    "int8": KVFormat(torch.int8, 127.0),
}

_UNQUANTIZED = frozenset({None, "", "auto", "bf16", "fp16", "none"})


def resolve_kv_dtype(kv_dtype):
    """Format name of an 8-bit cache, or None for a cache in the model dtype."""
    if kv_dtype in _UNQUANTIZED:
        return None
    if kv_dtype in KV_FORMATS:
        return kv_dtype
    raise ValueError(f"Unknown KV_CACHE_DTYPE '{kv_dtype}' (use auto, fp8 or int8)")


def _itemsize(dtype):
    return torch.empty((), dtype=dtype).element_size()


def kv_bytes_per_token(num_layers, num_kv_heads, head_dim, model_dtype, kv_dtype=None):
    """Cache bytes one token occupies: K and V of every layer and kv head, plus one scale
    per (layer, kv head, K/V) in the model dtype for 8-bit formats."""
    fmt = resolve_kv_dtype(kv_dtype)
    if fmt is None:
        per_head = head_dim * _itemsize(model_dtype)
    else:
        per_head = head_dim * _itemsize(KV_FORMATS[fmt].dtype) + _itemsize(model_dtype)
    return 2 * num_layers * num_kv_heads * per_head


def tokens_for_budget(budget_bytes, num_layers, num_kv_heads, head_dim, dtype, kv_dtype=None):
    """Whole tokens that fit in `budget_bytes` of cache."""
    return int(budget_bytes // kv_bytes_per_token(num_layers, num_kv_heads, head_dim, dtype, kv_dtype))


def kv_quant_write(cache, scale, slots, x):
    """Quantize x [T, heads, D] per (token, head) into the 8-bit `cache` [slots, heads, D]
    at rows `slots` (int64), scales into `scale` [slots, heads] (reference
    kv_cache.py:359-388: s = bf16(max(amax / qmax, 1e-8)), code = x / s, int8 rounded
    half-to-even and clamped to 127, fp8 clamped to 448 then encoded)."""
    L.require_device(x, slots, cache, scale)
    if x.stride(-1) != 1:
        x = x.contiguous()
    per_launch = 65535  # tokens one launch takes
    for a in range(0, x.shape[0], per_launch):
        xa, sa = x[a:a + per_launch], slots[a:a + per_launch]
        L.call("miq_kv_quant_write", L.ptr(xa), L.dtype_code(xa.dtype), xa.shape[0], xa.shape[1], xa.shape[2],
               xa.stride(0), xa.stride(1), L.ptr(sa), L.ptr(cache), L.dtype_code(cache.dtype),
               cache.stride(0), cache.stride(1), L.ptr(scale), L.dtype_code(scale.dtype),
               scale.stride(0), scale.stride(1), L.stream(x.device))


class KVCache:
    """Paged KV storage for all layers (reference kv_cache.py:305-425, storage part).

    Only mode="paged" exists here; capacity is rounded down to whole blocks. The
    `watermark` and `prefix_caching` arguments belong to the reference's allocator and
    are accepted for signature compatibility."""

    def __init__(self, mode, num_layers, num_kv_heads, head_dim, capacity_tokens, dtype, device,
                 block_size=16, watermark=0.01, kv_dtype=None, prefix_caching=False):
        if mode != "paged":
            raise ValueError("only the paged storage layout is provided (mode='paged')")
        self.mode, self.block_size, self.model_dtype = mode, block_size, dtype
        self.capacity = capacity_tokens - capacity_tokens % block_size
        self.kv_dtype = resolve_kv_dtype(kv_dtype)
        dims = (num_layers, self.capacity, num_kv_heads, head_dim)
        fmt = KV_FORMATS.get(self.kv_dtype)
        store = dtype if fmt is None else fmt.dtype
        self.k, self.v = (torch.zeros(dims, dtype=store, device=device) for _ in range(2))
        if fmt is None:
            self.k_scale = self.v_scale = None
        else:
            self.qmax = fmt.qmax
            self.k_scale, self.v_scale = (torch.ones(dims[:3], dtype=dtype, device=device) for _ in range(2))
        self.bytes_per_token = kv_bytes_per_token(num_layers, num_kv_heads, head_dim, dtype, self.kv_dtype)

    def write(self, layer, slots, k, v):
        """Store k, v [T, heads, D] of `layer` at `slots`, quantizing on the way for 8-bit
        formats (reference kv_cache.py:378-388)."""
        if self.kv_dtype is None:
            for dst, src in ((self.k, k), (self.v, v)):
                dst[layer].index_copy_(0, slots, src)
            return
        slots = slots.to(torch.int64).contiguous()
        kv_quant_write(self.k[layer], self.k_scale[layer], slots, k)
        kv_quant_write(self.v[layer], self.v_scale[layer], slots, v)

    def _codes(self, t, layer, idx):
        if t.dtype == torch.float8_e4m3fn:  # advanced indexing of fp8 goes through the raw bytes
            return t[layer].view(torch.uint8)[idx].view(t.dtype)
        return t[layer][idx]

    def gather(self, layer, idx):
        """Keys and values of `layer` at slots `idx` (any index shape), dequantized to the
        model dtype as codes.to(dtype) * scale (reference kv_cache.py:390-401)."""
        if self.kv_dtype is None:
            return self.k[layer][idx], self.v[layer][idx]
        out = []
        for codes, scale in ((self.k, self.k_scale), (self.v, self.v_scale)):
            out.append(self._codes(codes, layer, idx).to(self.model_dtype) * scale[layer][idx].unsqueeze(-1))
        return tuple(out)

    @staticmethod
    def decode_tables(pages, lens, block_size, device):
        """Kernel tables for a decode batch (reference kv_cache.py:403-420, paged case):
        page lists and context lengths -> (block_table int32 [B, width] zero-padded,
        seq_lens int32 [B], page_size, max_len)."""
        used = [list(p)[: (n + block_size - 1) // block_size] for p, n in zip(pages, lens)]
        table = torch.zeros(len(used), max(map(len, used)), dtype=torch.int32)
        for row, ids in enumerate(used):
            table[row, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
        return table.to(device), torch.tensor(list(lens), dtype=torch.int32).to(device), block_size, max(lens)

    def memory_mb(self):
        """MiB of device memory the cache tensors hold."""
        held = [t for t in (self.k, self.v, self.k_scale, self.v_scale) if t is not None]
        return round(sum(t.numel() * t.element_size() for t in held) / (1 << 20), 1)
