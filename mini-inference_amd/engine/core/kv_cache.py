"""8-bit KV-cache storage formats and quantize-on-write
(reference: engine/core/kv_cache.py:6-33, 305-437, storage part only).

Layout, as in the reference: k / v [layers, slots, kv_heads, head_dim] in the storage
dtype, and for 8-bit formats one scale per (token, kv head) in the model dtype,
k_scale / v_scale [layers, slots, kv_heads]. Slot = page_id * block_size + offset.
`write` runs the fused quantize + scatter kernel; `gather` dequantizes on the device
for the non-paged attention path. The reference's allocators (contiguous / paged with
prefix caching) belong to the serving engine and are not part of this package: callers
pass slots and block tables directly (`decode_tables` builds the kernel's tables from
page lists).
"""
import torch

from kernels import _lib as L

KV_FORMATS = {
    # name: (storage dtype, largest representable magnitude)
    "fp8": (torch.float8_e4m3fn, torch.finfo(torch.float8_e4m3fn).max),   # 448
    "int8": (torch.int8, 127.0),
}


def resolve_kv_dtype(kv_dtype):
    """kv_cache.py:13-19."""
    if kv_dtype in (None, "", "auto", "bf16", "fp16", "none"):
        return None
    if kv_dtype not in KV_FORMATS:
        raise ValueError(f"Unknown KV_CACHE_DTYPE '{kv_dtype}' (use auto, fp8 or int8)")
    return kv_dtype


def kv_bytes_per_token(num_layers, num_kv_heads, head_dim, model_dtype, kv_dtype=None):
    """kv_cache.py:22-30: K + V bytes per token over all layers, scales included."""
    kv_dtype = resolve_kv_dtype(kv_dtype)
    scale_bytes = torch.tensor([], dtype=model_dtype).element_size()
    if kv_dtype is None:
        per_head = head_dim * scale_bytes
    else:
        per_head = head_dim * torch.tensor([], dtype=KV_FORMATS[kv_dtype][0]).element_size() + scale_bytes
    return 2 * num_layers * num_kv_heads * per_head


def tokens_for_budget(budget_bytes, num_layers, num_kv_heads, head_dim, dtype, kv_dtype=None):
    return int(budget_bytes // kv_bytes_per_token(num_layers, num_kv_heads, head_dim, dtype, kv_dtype))


def kv_quant_write(cache, scale, slots, x):
    """Quantize x [T, heads, D] per (token, head) into the 8-bit `cache` [slots, heads, D]
    at rows `slots` (int64), scales into `scale` [slots, heads] (kv_cache.py:359-388)."""
    L.require_device(x, slots, cache, scale)
    x = x if x.stride(-1) == 1 else x.contiguous()
    T = x.shape[0]
    for a in range(0, T, 65535):  # the kernel takes at most 65535 tokens per launch
        xa, sa = x[a:a + 65535], slots[a:a + 65535]
        L.call("miq_kv_quant_write", L.ptr(xa), L.dtype_code(xa.dtype), xa.shape[0], xa.shape[1], xa.shape[2],
               xa.stride(0), xa.stride(1), L.ptr(sa), L.ptr(cache), L.dtype_code(cache.dtype),
               cache.stride(0), cache.stride(1), L.ptr(scale), L.dtype_code(scale.dtype),
               scale.stride(0), scale.stride(1), L.stream(x.device))


class KVCache:
    """Storage of a paged KV cache (kv_cache.py:305-333). `mode` must be "paged"."""

    def __init__(self, mode, num_layers, num_kv_heads, head_dim, capacity_tokens, dtype, device,
                 block_size=16, watermark=0.01, kv_dtype=None, prefix_caching=False):
        if mode != "paged":
            raise ValueError("only the paged storage layout is provided (mode='paged')")
        capacity_tokens = (capacity_tokens // block_size) * block_size
        self.mode = mode
        self.block_size = block_size
        self.capacity = capacity_tokens
        self.model_dtype = dtype
        self.kv_dtype = resolve_kv_dtype(kv_dtype)
        shape = (num_layers, capacity_tokens, num_kv_heads, head_dim)
        if self.kv_dtype is None:
            self.k = torch.zeros(shape, dtype=dtype, device=device)
            self.v = torch.zeros(shape, dtype=dtype, device=device)
            self.k_scale = self.v_scale = None
        else:
            store, self.qmax = KV_FORMATS[self.kv_dtype]
            self.k = torch.zeros(shape, dtype=store, device=device)
            self.v = torch.zeros(shape, dtype=store, device=device)
            self.k_scale = torch.ones(shape[:3], dtype=dtype, device=device)   # one per (token, head)
            self.v_scale = torch.ones(shape[:3], dtype=dtype, device=device)
        self.bytes_per_token = kv_bytes_per_token(num_layers, num_kv_heads, head_dim, dtype, self.kv_dtype)

    def write(self, layer, slots, k, v):
        """kv_cache.py:378-388: quantize k, v [T, heads, D] and store them at `slots`."""
        if self.kv_dtype is None:
            self.k[layer].index_copy_(0, slots, k)
            self.v[layer].index_copy_(0, slots, v)
            return
        slots = slots.to(torch.int64).contiguous()
        kv_quant_write(self.k[layer], self.k_scale[layer], slots, k)
        kv_quant_write(self.v[layer], self.v_scale[layer], slots, v)

    def gather(self, layer, idx):
        """kv_cache.py:390-401: keys and values at the given slots, in the model dtype."""
        if self.kv_dtype is None:
            return self.k[layer][idx], self.v[layer][idx]
        if self.k.dtype == torch.float8_e4m3fn:
            k = self.k[layer].view(torch.uint8)[idx].view(torch.float8_e4m3fn)
            v = self.v[layer].view(torch.uint8)[idx].view(torch.float8_e4m3fn)
        else:
            k, v = self.k[layer][idx], self.v[layer][idx]
        k = k.to(self.model_dtype) * self.k_scale[layer][idx][..., None]
        v = v.to(self.model_dtype) * self.v_scale[layer][idx][..., None]
        return k, v

    @staticmethod
    def decode_tables(pages, lens, block_size, device):
        """kv_cache.py:403-420 (paged branch): page lists -> (block_table int32 [B, pages],
        seq_lens int32 [B], page_size, max_len), zero-padded rows."""
        tables = [list(p[: -(-n // block_size)]) for p, n in zip(pages, lens)]
        width = max(len(t) for t in tables)
        table = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.int32)
        return table.to(device), torch.tensor(lens, dtype=torch.int32).to(device), block_size, max(lens)

    def memory_mb(self):
        total = sum(t.numel() * t.element_size() for t in (self.k, self.v, self.k_scale, self.v_scale)
                    if t is not None)
        return round(total / 1024 ** 2, 1)
