"""8-bit KV-cache storage and its quantize-on-write.

Interface of the reference's engine/core/kv_cache.py (the storage half, :6-35 and
:305-425): the format names "fp8" / "int8", `resolve_kv_dtype`, `kv_bytes_per_token`,
`tokens_for_budget`, the two allocators (`PagedAllocator`, `ContiguousAllocator`), and
`KVCache` with the allocator wrappers, `write`, `gather`, `decode_tables`, `memory_mb`.

Layout (the reference's, so the paged-attention kernels read it as is):
  k, v                [layers, slots, kv_heads, head_dim] in the storage dtype
  k_scale, v_scale    [layers, slots, kv_heads] in the model dtype, 8-bit formats only
  slot                page_id * block_size + position in the page

`write` is one fused kernel per tensor (amax, bf16 scale, encode, scatter by slot).
The allocators keep the reference's bookkeeping contract (`tables[request id]` = the
block table of a paged cache, `ranges[request id]` = (base, size) of a contiguous one,
`slots`, `admit` / `reserve` / `ensure` / `free`), which is what `decode_tables` and the
runner read. Prefix caching and the admission watermark belong to the reference's
scheduler and are not rebuilt: `register` is a no-op and `admit` reports 0 cached tokens.
"""
import bisect
from collections import deque
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


def _cdiv(a, b):
    return -(-a // b)


class PagedAllocator:
    """Fixed-size blocks handed out from a free list (reference kv_cache.py:124-300, without
    prefix caching). `tables[request id]` is the request's block table: block i holds
    positions i * block_size .. (i + 1) * block_size - 1."""

    name = "paged"

    def __init__(self, capacity, block_size):
        self.block_size = block_size
        self.num_blocks = capacity // block_size
        self.capacity = self.num_blocks * block_size
        self._free = deque(range(self.num_blocks))
        self.tables = {}
        self.length = {}

    def blocks_for(self, num_tokens):
        return _cdiv(num_tokens, self.block_size)

    def can_admit(self, req, max_len):
        return self.blocks_for(min(_total_len(req), max_len)) <= len(self._free)

    def admit(self, req, max_len, size=None):
        """Registers the request with an empty table; 0 tokens are cached already (None
        when its current length does not fit)."""
        if not self.can_admit(req, max_len):
            return None
        self.tables[req.id], self.length[req.id] = [], 0
        return 0

    def reserve(self, req, num_tokens):
        table = self.tables.setdefault(req.id, [])
        need = self.blocks_for(num_tokens) - len(table)
        if need > len(self._free):
            return False
        table.extend(self._free.popleft() for _ in range(max(need, 0)))
        return True

    def ensure(self, req, num_tokens):
        if not self.reserve(req, num_tokens):
            return False
        self.length[req.id] = num_tokens
        return True

    def free(self, req):
        self._free.extend(self.tables.pop(req.id, ()))
        self.length.pop(req.id, None)

    def slots(self, req, start, end):
        pos = torch.arange(start, end)
        blocks = torch.tensor(self.tables[req.id], dtype=torch.long)
        return blocks[pos // self.block_size] * self.block_size + pos % self.block_size

    def stored_tokens(self):
        return sum(self.length.values())


class ContiguousAllocator:
    """One first-fit range of slots per request, sized at admission (reference
    kv_cache.py:50-121). `ranges[request id]` = (first slot, size)."""

    name = "contiguous"

    def __init__(self, capacity):
        self.capacity = capacity
        self._holes = [(0, capacity)]  # sorted (start, size) of free ranges
        self.ranges = {}
        self.length = {}

    def _hole_for(self, size):
        return next((i for i, (_, n) in enumerate(self._holes) if n >= size), None)

    def can_admit(self, req, max_len):
        return self._hole_for(min(_max_total_len(req), max_len)) is not None

    def admit(self, req, max_len, size=None):
        size = size or min(_max_total_len(req), max_len)
        i = self._hole_for(size)
        if i is None:
            return None
        start, n = self._holes.pop(i)
        if n > size:
            self._holes.insert(i, (start + size, n - size))
        self.ranges[req.id], self.length[req.id] = (start, size), 0
        return 0

    def reserve(self, req, num_tokens):
        return num_tokens <= self.ranges[req.id][1]

    def ensure(self, req, num_tokens):
        if not self.reserve(req, num_tokens):
            return False
        self.length[req.id] = num_tokens
        return True

    def free(self, req):
        if req.id not in self.ranges:
            return
        start, size = self.ranges.pop(req.id)
        self.length.pop(req.id, None)
        # merge with the free range that ends at `start` and the one that begins at its end
        holes, lo, hi = self._holes, start, start + size
        i = bisect.bisect(holes, (start, size))
        if i < len(holes) and holes[i][0] == hi:
            hi += holes.pop(i)[1]
        if i > 0 and sum(holes[i - 1]) == lo:
            i -= 1
            lo = holes.pop(i)[0]
        holes.insert(i, (lo, hi - lo))

    def slots(self, req, start, end):
        base = self.ranges[req.id][0]
        return torch.arange(base + start, base + end)

    def stored_tokens(self):
        return sum(self.length.values())


def _total_len(req):
    return getattr(req, "total_len", None) or len(req.all_ids)


def _max_total_len(req):
    return getattr(req, "max_total_len", None) or _total_len(req)


def make_allocator(mode, capacity_tokens, block_size=16):
    if mode == "paged":
        return PagedAllocator(capacity_tokens, block_size)
    if mode == "contiguous":
        return ContiguousAllocator(capacity_tokens)
    raise ValueError(f"Unknown KV_CACHE '{mode}' (use 'contiguous' or 'paged')")


def pack_block_tables(tables, lens, device):
    """Per-request page lists and context lengths -> (block_table int32 [B, width], zero
    padded, seq_lens int32 [B]) on `device`, the paged-attention kernel's operands."""
    width = max(1, max(len(t) for t in tables))
    table = torch.zeros(len(tables), width, dtype=torch.int32)
    for row, ids in enumerate(tables):
        if ids:
            table[row, : len(ids)] = torch.as_tensor(ids, dtype=torch.int32)
    return table.to(device), torch.tensor(list(lens), dtype=torch.int32).to(device)


class CacheBookkeeping:
    """The allocator half of KVCache: thin wrappers (reference kv_cache.py:337-356) and the
    kernel tables of a decode batch. Needs `self.allocator` and `self.mode`."""

    def can_admit(self, req, max_len):
        return self.allocator.can_admit(req, max_len)

    def admit(self, req, max_len, size=None):
        return self.allocator.admit(req, max_len, size)

    def reserve(self, req, num_tokens):
        return self.allocator.reserve(req, num_tokens)

    def ensure(self, req, num_tokens):
        return self.allocator.ensure(req, num_tokens)

    def free(self, req):
        self.allocator.free(req)

    def register(self, req):
        """After a step (prefix caching in the reference; nothing to publish here)."""

    def slots(self, req, start, end):
        return self.allocator.slots(req, start, end)

    def decode_tables(self, entries, device):
        """Page tables for the paged decode-attention kernel (reference kv_cache.py:403-420).
        entries: (request, context_length) pairs. Returns (block_table int32 [B, pages],
        seq_lens int32 [B], page_size, max_len). A paged cache hands over each request's
        block table cut to its context (page = block size); a contiguous one describes its
        range token by token (page = 1)."""
        lens = [n for _, n in entries]
        if self.mode == "paged":
            a = self.allocator
            tables = [a.tables[r.id][: a.blocks_for(n)] for r, n in entries]
            page = a.block_size
        else:
            span = max(lens)
            tables = [list(range(self.allocator.ranges[r.id][0], self.allocator.ranges[r.id][0] + span))
                      for r, _ in entries]
            page = 1
        table, seq_lens = pack_block_tables(tables, lens, device)
        return table, seq_lens, page, max(lens)

class KVCache(CacheBookkeeping):
    """KV storage for all layers with its allocator (reference kv_cache.py:305-425).

    mode "paged": blocks of `block_size` slots (capacity rounded down to whole blocks);
    "contiguous": one range per request. `watermark` and `prefix_caching` belong to the
    reference's scheduler policy and are accepted for signature compatibility."""

    def __init__(self, mode, num_layers, num_kv_heads, head_dim, capacity_tokens, dtype, device,
                 block_size=16, watermark=0.01, kv_dtype=None, prefix_caching=False):
        self.allocator = make_allocator(mode, capacity_tokens, block_size)
        self.mode, self.block_size, self.model_dtype = mode, block_size, dtype
        self.capacity = self.allocator.capacity
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

    def memory_mb(self):
        """MiB of device memory the cache tensors hold."""
        held = [t for t in (self.k, self.v, self.k_scale, self.v_scale) if t is not None]
        return round(sum(t.numel() * t.element_size() for t in held) / (1 << 20), 1)
