"""A minimal prefill + decode runner over the quantized modules and the paged KV cache.

Reference: engine/core/model_runner.py:11-195 (BatchMetadata, ModelRunner.forward_meta,
ModelRunner._attention with the paged decode kernel), engine/models.py:9-36 (what the
runner needs to know about an architecture) and engine/core/sampler.py (greedy = argmax).
The reference's scheduler and KV allocators belong to the serving engine and are not
rebuilt: `generate` below runs a fixed set of prompts to completion with a plain page
list per request, which is all an end-to-end parity check needs.

One step takes "chunks" (request, start, end) exactly as the reference does:
  * every layer projects q, k, v through the model's own modules (QuantLinear after
    quantize_model), applies the q/k norm of the architecture and RoPE;
  * this step's keys and values are written to the cache (`KVCache.write`, the fused
    HIP quantize-and-scatter kernel for 8-bit caches);
  * prefill chunks attend over their context read back through the cache (dequantized),
    with torch's SDPA, as the reference does;
  * decode rows run `paged_decode_attention` on the cache in place (the HIP kernel);
  * the MLP is the model's own block (QuantExperts' fused INT4 MoE path for OLMoE).
`decode_attention` can be replaced (tests run the runner on the CPU with a restatement);
the default is the HIP kernel, which raises when libmiq is not loaded.
"""
import torch
import torch.nn.functional as F

SUPPORTED = ("OlmoeForCausalLM", "Qwen3ForCausalLM", "Qwen3MoeForCausalLM", "Qwen2ForCausalLM")


def rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def describe(model):
    """engine/models.py:9-36: architecture, q/k norm kind ("none", "per_head", "full"),
    whether the MLP is a mixture of experts, and the attention shape."""
    cfg = model.config
    arch = (getattr(cfg, "architectures", None) or [type(model).__name__])[0]
    if arch not in SUPPORTED:
        raise ValueError(f"unsupported architecture {arch} (supported: {', '.join(SUPPORTED)})")
    heads = cfg.num_attention_heads
    head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // heads
    attn = model.model.layers[0].self_attn
    qk_norm = "none"
    if getattr(attn, "q_norm", None) is not None:
        size = attn.q_norm.weight.numel()
        qk_norm = "per_head" if size == head_dim else "full"
        if qk_norm == "full" and size != heads * head_dim:
            raise ValueError(f"{arch}: q_norm has {size} weights, expected {head_dim} or {heads * head_dim}")
    moe = any(getattr(cfg, k, None) for k in ("num_experts", "num_local_experts", "n_routed_experts"))
    return {"architecture": arch, "qk_norm": qk_norm, "moe": bool(moe), "heads": heads,
            "kv_heads": getattr(cfg, "num_key_value_heads", None) or heads, "head_dim": head_dim}


class Request:
    """A prompt and its generated tokens, with the cache pages it owns."""

    def __init__(self, rid, prompt_ids, max_new_tokens):
        self.id = rid
        self.all_ids = list(prompt_ids)
        self.prompt_len = len(prompt_ids)
        self.max_new_tokens = max_new_tokens
        self.pages = []
        self.done = False

    @property
    def output_ids(self):
        return self.all_ids[self.prompt_len:]


class PagePool:
    """Pages of `block_size` slots handed out in order (kv_cache.py:124-300 keeps free lists,
    watermarks and prefix hashes; none of that changes what attention reads)."""

    def __init__(self, num_pages, block_size):
        self.block_size = block_size
        self.free = list(range(num_pages))

    def ensure(self, req, num_tokens):
        need = -(-num_tokens // self.block_size) - len(req.pages)
        if need > len(self.free):
            raise RuntimeError(f"KV cache full: {need} more pages needed, {len(self.free)} free")
        for _ in range(max(0, need)):
            req.pages.append(self.free.pop(0))

    def slots(self, req, start, end):
        pos = torch.arange(start, end)
        pages = torch.tensor(req.pages, dtype=torch.long)
        return pages[pos // self.block_size] * self.block_size + pos % self.block_size

    def release(self, req):
        self.free.extend(req.pages)
        req.pages = []


class BatchMetadata:
    """model_runner.py:11-61: token ids, positions, cache slots to write, the prefill
    chunks with their context slots, the decode rows and their block tables."""

    def __init__(self, chunks, cache, pool, device):
        ids, positions, write_slots = [], [], []
        self.prefill, decode_rows, decode_pages, decode_lens, last_rows = [], [], [], [], []
        offset = 0
        for req, start, end in chunks:
            n = end - start
            ids.extend(req.all_ids[start:end])
            positions.append(torch.arange(start, end))
            write_slots.append(pool.slots(req, start, end))
            if n == 1 and start > 0:
                decode_rows.append(offset)
                decode_pages.append(req.pages)
                decode_lens.append(end)
            else:
                self.prefill.append((offset, n, start, pool.slots(req, 0, end).to(device)))
            offset += n
            last_rows.append(offset - 1)
        self.num_tokens = offset
        self.input_ids = torch.tensor(ids, dtype=torch.long, device=device)
        self.positions = torch.cat(positions).to(device)
        self.write_slots = torch.cat(write_slots).to(device)
        self.last_rows = torch.tensor(last_rows, dtype=torch.long, device=device)
        self.decode_rows = torch.tensor(decode_rows, dtype=torch.long, device=device)
        self.all_decode = not self.prefill
        self.decode_tables = (cache.decode_tables(decode_pages, decode_lens, pool.block_size, device)
                              if decode_rows else None)


class ModelRunner:
    """model_runner.py:64-195 with the paged decode backend."""

    def __init__(self, model, cache, decode_attention=None):
        self.model = model
        self.cache = cache
        self.arch = describe(model)
        cfg = model.config
        self.num_heads = self.arch["heads"]
        self.num_kv_heads = self.arch["kv_heads"]
        self.head_dim = self.arch["head_dim"]
        self.clip_qkv = getattr(cfg, "clip_qkv", None)
        if decode_attention is None:
            from kernels.paged_attention import paged_decode_attention
            decode_attention = paged_decode_attention
        self.decode_attention = decode_attention
        inner = model.model
        self.embed, self.layers, self.norm, self.rotary = inner.embed_tokens, inner.layers, inner.norm, inner.rotary_emb
        self.device = next(model.parameters()).device

    @torch.inference_mode()
    def forward(self, meta, all_logits=False):
        """model_runner.py:113-137: logits [chunks, vocab] (fp32) for each chunk's last token,
        or for every token with all_logits."""
        x = self.embed(meta.input_ids)
        cos, sin = self.rotary(x, meta.positions[None])
        cos, sin = cos[0][:, None, :], sin[0][:, None, :]
        for i, layer in enumerate(self.layers):
            x = x + self._attention(i, layer.self_attn, layer.input_layernorm(x), cos, sin, meta)
            out = layer.mlp(layer.post_attention_layernorm(x)[None])
            if isinstance(out, tuple):  # some MoE blocks also return router logits
                out = out[0]
            x = x + out[0]
        x = self.norm(x if all_logits else x[meta.last_rows])
        return self.model.lm_head(x).float()

    def _attention(self, layer_idx, attn, h, cos, sin, meta):
        """model_runner.py:139-195."""
        T, H, KV, D = meta.num_tokens, self.num_heads, self.num_kv_heads, self.head_dim
        q, k, v = attn.q_proj(h), attn.k_proj(h), attn.v_proj(h)
        if self.arch["qk_norm"] == "full":
            q, k = attn.q_norm(q), attn.k_norm(k)
        if self.clip_qkv is not None:
            q, k, v = (t.clamp(-self.clip_qkv, self.clip_qkv) for t in (q, k, v))
        q, k, v = q.view(T, H, D), k.view(T, KV, D), v.view(T, KV, D)
        if self.arch["qk_norm"] == "per_head":
            q, k = attn.q_norm(q), attn.k_norm(k)
        q = q * cos + rotate_half(q) * sin
        k = k * cos + rotate_half(k) * sin

        self.cache.write(layer_idx, meta.write_slots, k, v)
        out = torch.empty_like(q)
        gqa = KV != H
        for offset, n, start, ctx in meta.prefill:
            qi = q[offset:offset + n].transpose(0, 1)[None]
            kc, vc = self.cache.gather(layer_idx, ctx)
            ki, vi = kc.transpose(0, 1)[None], vc.transpose(0, 1)[None]
            if start == 0:
                o = F.scaled_dot_product_attention(qi, ki, vi, is_causal=True, scale=attn.scaling, enable_gqa=gqa)
            else:  # tokens after a cached prefix: position p sees keys 0..p
                qpos = torch.arange(start, start + n, device=q.device)
                mask = torch.arange(ctx.numel(), device=q.device)[None, :] <= qpos[:, None]
                o = F.scaled_dot_product_attention(qi, ki, vi, attn_mask=mask[None, None], scale=attn.scaling,
                                                   enable_gqa=gqa)
            out[offset:offset + n] = o[0].transpose(0, 1)
        if meta.decode_tables is not None:
            table, lens, page, max_len = meta.decode_tables
            c = self.cache
            o = self.decode_attention(
                q if meta.all_decode else q[meta.decode_rows], c.k[layer_idx], c.v[layer_idx], table, lens, page,
                attn.scaling, max_len, k_scale=None if c.k_scale is None else c.k_scale[layer_idx],
                v_scale=None if c.v_scale is None else c.v_scale[layer_idx])
            if meta.all_decode:
                out = o
            else:
                out[meta.decode_rows] = o
        return attn.o_proj(out.reshape(T, H * D))


@torch.inference_mode()
def generate(runner, pool, prompts, max_new_tokens, eos_token_id=None, logits_out=None):
    """Greedy generation for a fixed set of prompts (token id lists): one prefill step for
    all of them, then decode steps over every unfinished request (engine/core/sampler.py:
    argmax when the temperature is 0). Returns the generated ids per prompt; with
    `logits_out` (a list) it also collects, per prompt, the fp32 logits of every step
    on the CPU."""
    if isinstance(max_new_tokens, int):
        max_new_tokens = [max_new_tokens] * len(prompts)
    reqs = [Request(i, p, n) for i, (p, n) in enumerate(zip(prompts, max_new_tokens))]
    if logits_out is not None:
        logits_out[:] = [[] for _ in reqs]

    def step(chunks):
        for req, _, end in chunks:
            pool.ensure(req, end)
        meta = BatchMetadata(chunks, runner.cache, pool, runner.device)
        logits = runner.forward(meta)
        ids = logits.argmax(dim=-1).tolist()
        if logits_out is not None:
            rows = logits.cpu()
            for j, (req, _, _) in enumerate(chunks):
                logits_out[req.id].append(rows[j])
        for (req, _, _), t in zip(chunks, ids):
            req.all_ids.append(t)
            if len(req.output_ids) >= req.max_new_tokens or (eos_token_id is not None and t == eos_token_id):
                req.done = True
                pool.release(req)

    step([(r, 0, len(r.all_ids)) for r in reqs if r.max_new_tokens > 0])
    while True:
        live = [r for r in reqs if not r.done and r.max_new_tokens > 0]
        if not live:
            break
        step([(r, len(r.all_ids) - 1, len(r.all_ids)) for r in live])
    return [r.output_ids for r in reqs]
