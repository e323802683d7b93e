"""CPU restatement of the paged decode attention contract (test infrastructure only)."""
import numpy as np
import torch


def _rows(t, slots):
    """reference.py:3-7: t[slots], also for FP8 tensors (indexed as raw bytes)."""
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8)[slots].view(torch.float8_e4m3fn)
    return t[slots]


def paged_decode_reference(q, k_cache, v_cache, block_table, seq_lens, page_size, scale,
                           k_scale=None, v_scale=None):
    """kernels/paged_attention/reference.py:10-28: one request at a time, in float32."""
    B, H, D = q.shape
    group = H // k_cache.shape[1]
    out = torch.empty(B, H, D, dtype=torch.float32)
    for b in range(B):
        n = int(seq_lens[b])
        pos = torch.arange(n)
        slots = block_table[b, pos // page_size].long() * page_size + pos % page_size
        k = _rows(k_cache, slots).float()
        v = _rows(v_cache, slots).float()
        if k_scale is not None:
            k = k * k_scale[slots].float()[..., None]
            v = v * v_scale[slots].float()[..., None]
        k = k.repeat_interleave(group, dim=1)
        v = v.repeat_interleave(group, dim=1)
        scores = torch.einsum("hd,nhd->hn", q[b].float(), k) * scale
        out[b] = torch.einsum("hn,nhd->hd", scores.softmax(dim=-1), v)
    return out


def paged_decode_numpy64(q, k, v, block_table, seq_lens, page_size, scale):
    """Independent float64 textbook softmax attention over dequantized float K/V
    (k, v: float arrays [slots, KV, D]), used to pin paged_decode_reference."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    bt = np.asarray(block_table)
    B, H, D = q.shape
    KV = k.shape[1]
    out = np.zeros((B, H, D))
    for b in range(B):
        n = int(seq_lens[b])
        for h in range(H):
            kvh = h // (H // KV)
            s = np.empty(n)
            rows = []
            for i in range(n):
                slot = int(bt[b, i // page_size]) * page_size + i % page_size
                rows.append(slot)
                s[i] = q[b, h] @ k[slot, kvh] * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            out[b, h] = p @ v[rows, kvh]
    return out
