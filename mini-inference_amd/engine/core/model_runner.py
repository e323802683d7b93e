"""The step runner over the quantized modules and the KV cache.

Contract of the reference's engine/core/model_runner.py (:11-61 BatchMetadata, :64-137
ModelRunner.forward / forward_meta, :139-195 ModelRunner._attention) and
engine/models.py:9-36 (what the runner must know about an architecture):

  * a step is a list of chunks (request, start, end): tokens start..end-1 of each request;
    a chunk of one token after position 0 is a decode row, anything else a prefill;
  * `BatchMetadata(chunks, cache, device, attn_backend)` is built once per step and read by
    every layer; its `decode_tables` is the 5-tuple (block_table, seq_lens, page_size,
    max_len, num_splits) that `KVCache.decode_tables` plus the split choice give;
  * `ModelRunner(model, cache, attn_backend, arch)`: `forward(chunks)` returns fp32 logits of
    each chunk's last token (every token with all_logits), `forward_meta(meta)` the same
    from prepared metadata.

How a layer runs here:
  * q, k, v come from the model's own projections (QuantLinear after quantize_model), then
    the architecture's q/k norm (over the whole projection for OLMoE, per head for
    Qwen3), the optional clip and RoPE;
  * the step's keys and values go into the cache first (`KVCache.write`: the fused HIP
    quantize-and-scatter kernel for 8-bit caches), and attention reads them back from
    there, so prefill and decode see the same (quantized) context;
  * prefill chunks: torch SDPA over their context gathered (dequantized) from the cache;
  * decode rows, backend "triton" (the reference's name for its paged kernel; "paged" is
    accepted too): `paged_decode_attention` on the cache in place, the HIP kernel. Backend
    "sdpa": the context gathered per row and one masked SDPA call;
  * the MLP is the model's own block (QuantExperts' fused MoE for OLMoE).
`decode_attention` replaces the decode kernel (the tests run the runner on the CPU with a
restatement); by default the HIP kernel runs, which raises when libmiq is not loaded.
The reference's scheduler, CUDA-graph capture and fused projections are serving-engine
features outside this path; `generate` below runs a fixed set of prompts greedily.
"""
import itertools

import torch
import torch.nn.functional as F

SUPPORTED = ("OlmoeForCausalLM", "Qwen3ForCausalLM", "Qwen3MoeForCausalLM", "Qwen2ForCausalLM")
_PAGED_BACKENDS = ("triton", "paged")


def rotate_half(x):
    lo, hi = x.chunk(2, dim=-1)
    return torch.cat((-hi, lo), dim=-1)


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
    """A prompt and its generated tokens (the fields of the reference's
    engine/core/request.py that the cache and the runner read)."""

    _ids = itertools.count()

    def __init__(self, prompt_ids, max_new_tokens, rid=None):
        self.id = next(Request._ids) if rid is None else rid
        self.prompt_ids = list(prompt_ids)
        self.output_ids = []
        self.max_new_tokens = max_new_tokens
        self.num_computed = 0

    @property
    def all_ids(self):
        return self.prompt_ids + self.output_ids

    @property
    def total_len(self):
        return len(self.prompt_ids) + len(self.output_ids)

    @property
    def max_total_len(self):
        return len(self.prompt_ids) + self.max_new_tokens


class BatchMetadata:
    """What every layer of one step needs (reference model_runner.py:11-61):

      input_ids, positions, write_slots   [T] per token of the step
      last_rows        [chunks] row of each chunk's last token
      prefill          [(first row, tokens, start position, context slots [end])]
      decode_rows      [B] rows of the decode tokens; all_decode when every row is one
      decode_tables    paged backends: (block_table, seq_lens, page_size, max_len,
                       num_splits=None, chosen by the kernel wrapper)
      decode_idx, decode_mask   "sdpa" backend: context slots [B, L] and validity mask
      context_tokens   keys and values attention reads this step
    """

    def __init__(self, chunks, cache, device, attn_backend="triton"):
        lengths = [end - start for _, start, end in chunks]
        ends = list(itertools.accumulate(lengths))       # row after each chunk
        firsts = [e - n for e, n in zip(ends, lengths)]  # first row of each chunk
        is_decode = [n == 1 and start > 0 for n, (_, start, _) in zip(lengths, chunks)]

        token_ids = [t for req, start, end in chunks for t in req.all_ids[start:end]]
        self.num_tokens = ends[-1] if ends else 0
        self.input_ids = torch.tensor(token_ids, dtype=torch.long, device=device)
        self.positions = torch.cat([torch.arange(s, e) for _, s, e in chunks]).to(device)
        self.write_slots = torch.cat([cache.slots(r, s, e) for r, s, e in chunks]).to(device)
        self.last_rows = torch.tensor([e - 1 for e in ends], dtype=torch.long, device=device)
        self.context_tokens = sum(end for _, _, end in chunks)

        self.prefill = [(first, end - start, start, cache.slots(req, 0, end).to(device))
                        for first, dec, (req, start, end) in zip(firsts, is_decode, chunks) if not dec]
        decodes = [(first, req, end) for first, dec, (req, _, end) in zip(firsts, is_decode, chunks) if dec]
        self.decode_rows = torch.tensor([row for row, _, _ in decodes], dtype=torch.long, device=device)
        self.all_decode = not self.prefill
        self.decode_tables = None
        if decodes and attn_backend in _PAGED_BACKENDS:
            tables = cache.decode_tables([(req, end) for _, req, end in decodes], device)
            self.decode_tables = (*tables, None)
        elif decodes:
            slots = [cache.slots(req, 0, end) for _, req, end in decodes]
            width = max(len(s) for s in slots)
            idx = torch.zeros(len(slots), width, dtype=torch.long)
            for i, s in enumerate(slots):
                idx[i, : len(s)] = s
            lens = torch.tensor([len(s) for s in slots])
            self.decode_idx = idx.to(device)
            self.decode_mask = (torch.arange(width)[None, :] < lens[:, None]).to(device)[:, None, None, :]


class ModelRunner:
    """Runs steps of a Hugging Face decoder (reference model_runner.py:64-195)."""

    def __init__(self, model, cache, attn_backend="triton", arch=None, decode_attention=None):
        if attn_backend not in _PAGED_BACKENDS + ("sdpa",):
            raise ValueError(f"Unknown ATTN_BACKEND '{attn_backend}' (use sdpa or triton)")
        self.model, self.cache, self.attn_backend = model, cache, attn_backend
        self.arch = arch or describe(model)
        self.num_heads = self.arch["heads"]
        self.num_kv_heads = self.arch["kv_heads"]
        self.head_dim = self.arch["head_dim"]
        self.clip_qkv = getattr(model.config, "clip_qkv", None)
        if decode_attention is None and attn_backend in _PAGED_BACKENDS:
            from kernels.paged_attention import paged_decode_attention
            decode_attention = paged_decode_attention
        self.decode_attention = decode_attention
        inner = model.model
        self.embed, self.layers, self.norm, self.rotary = inner.embed_tokens, inner.layers, inner.norm, inner.rotary_emb
        self.device = next(model.parameters()).device

    @torch.inference_mode()
    def forward(self, chunks, all_logits=False):
        """Logits (fp32) of each chunk's last token, or of every token with all_logits."""
        meta = BatchMetadata(chunks, self.cache, self.device, self.attn_backend)
        return self.forward_meta(meta, all_logits)

    @torch.inference_mode()
    def forward_meta(self, meta, all_logits=False):
        x = self.embed(meta.input_ids)
        cos, sin = self.rotary(x, meta.positions[None])
        rope = (cos[0].unsqueeze(1), sin[0].unsqueeze(1))  # [T, 1, D], broadcast over heads
        for i, layer in enumerate(self.layers):
            x = x + self._attention(i, layer.self_attn, layer.input_layernorm(x), *rope, meta)
            mlp = layer.mlp(layer.post_attention_layernorm(x).unsqueeze(0))
            x = x + (mlp[0] if isinstance(mlp, tuple) else mlp).squeeze(0)  # MoE blocks may add router logits
        rows = x if all_logits else x.index_select(0, meta.last_rows)
        return self.model.lm_head(self.norm(rows)).float()

    # ------------------------------------------------------------------ attention
    def _project(self, attn, h, T):
        """q [T, H, D], k and v [T, KV, D] after the architecture's norms, clip and RoPE
        inputs (RoPE is applied by the caller)."""
        q, k, v = attn.q_proj(h), attn.k_proj(h), attn.v_proj(h)
        norm = self.arch["qk_norm"]
        if norm == "full":
            q, k = attn.q_norm(q), attn.k_norm(k)
        if self.clip_qkv is not None:
            c = self.clip_qkv
            q, k, v = q.clamp(-c, c), k.clamp(-c, c), v.clamp(-c, c)
        D = self.head_dim
        q, k, v = q.view(T, -1, D), k.view(T, -1, D), v.view(T, -1, D)
        if norm == "per_head":
            q, k = attn.q_norm(q), attn.k_norm(k)
        return q, k, v

    def _attention(self, layer_idx, attn, h, cos, sin, meta):
        q, k, v = self._project(attn, h, meta.num_tokens)
        q = q * cos + rotate_half(q) * sin
        k = k * cos + rotate_half(k) * sin
        self.cache.write(layer_idx, meta.write_slots, k, v)

        if meta.all_decode and meta.decode_tables is not None:
            out = self._paged_decode(layer_idx, attn, q, meta)
        else:
            out = torch.empty_like(q)
            for first, n, start, ctx in meta.prefill:
                out[first:first + n] = self._prefill(layer_idx, attn, q[first:first + n], start, ctx)
            if len(meta.decode_rows):
                qd = q.index_select(0, meta.decode_rows)
                if meta.decode_tables is not None:
                    out[meta.decode_rows] = self._paged_decode(layer_idx, attn, qd, meta)
                else:
                    out[meta.decode_rows] = self._gathered_decode(layer_idx, attn, qd, meta)
        return attn.o_proj(out.flatten(1))

    def _prefill(self, layer_idx, attn, q, start, ctx):
        """Tokens start .. start + n - 1 of one request over its cached context `ctx`
        (slots of positions 0 .. start + n - 1): position p sees keys 0 .. p."""
        keys, values = self.cache.gather(layer_idx, ctx)           # [ctx, KV, D]
        # one batch of heads: [1, heads, tokens, D] (the 4-D form selects the same SDPA
        # kernels on the GPU as a batched call would)
        qh, kh, vh = (t.transpose(0, 1).unsqueeze(0) for t in (q, keys, values))
        gqa = self.num_kv_heads != self.num_heads
        if start == 0:
            o = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=attn.scaling, enable_gqa=gqa)
        else:
            visible = torch.arange(ctx.numel(), device=q.device) <= torch.arange(
                start, start + q.shape[0], device=q.device).unsqueeze(1)
            o = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=visible, scale=attn.scaling, enable_gqa=gqa)
        return o.squeeze(0).transpose(0, 1)

    def _paged_decode(self, layer_idx, attn, q, meta):
        table, lens, page, max_len, splits = meta.decode_tables
        c = self.cache
        scales = {} if c.k_scale is None else {"k_scale": c.k_scale[layer_idx], "v_scale": c.v_scale[layer_idx]}
        return self.decode_attention(q, c.k[layer_idx], c.v[layer_idx], table, lens, page, attn.scaling, max_len,
                                     num_splits=splits, **scales)

    def _gathered_decode(self, layer_idx, attn, q, meta):
        keys, values = self.cache.gather(layer_idx, meta.decode_idx)  # [B, L, KV, D]
        o = F.scaled_dot_product_attention(q.unsqueeze(2), keys.transpose(1, 2), values.transpose(1, 2),
                                           attn_mask=meta.decode_mask, scale=attn.scaling,
                                           enable_gqa=self.num_kv_heads != self.num_heads)
        return o.squeeze(2)


@torch.inference_mode()
def generate(runner, prompts, max_new_tokens, eos_token_id=None, logits_out=None):
    """Greedy generation for a fixed set of prompts (token id lists) through the runner's
    cache: one prefill step for all of them, then decode steps over every unfinished
    request (engine/core/sampler.py: argmax when the temperature is 0). Returns the
    generated ids per prompt; with `logits_out` (a list) it also collects, per prompt, the
    fp32 logits of every step on the CPU."""
    cache = runner.cache
    if isinstance(max_new_tokens, int):
        max_new_tokens = [max_new_tokens] * len(prompts)
    reqs = [Request(p, n, rid=i) for i, (p, n) in enumerate(zip(prompts, max_new_tokens))]
    if logits_out is not None:
        logits_out[:] = [[] for _ in reqs]
    live = [r for r in reqs if r.max_new_tokens > 0]
    for r in live:
        if cache.admit(r, r.max_total_len) is None:
            raise RuntimeError(f"KV cache full: request {r.id} does not fit")
    while live:
        chunks = [(r, r.num_computed, r.total_len) for r in live]
        for r, _, end in chunks:
            if not cache.ensure(r, end):
                raise RuntimeError(f"KV cache full at request {r.id}, {end} tokens")
        logits = runner.forward(chunks)
        picks = logits.argmax(dim=-1).tolist()
        rows = logits.cpu() if logits_out is not None else None
        for j, (r, _, end) in enumerate(chunks):
            r.num_computed = end
            r.output_ids.append(picks[j])
            if rows is not None:
                logits_out[r.id].append(rows[j])
        finished = [r for r in live if len(r.output_ids) >= r.max_new_tokens
                    or (eos_token_id is not None and r.output_ids[-1] == eos_token_id)]
        for r in finished:
            cache.free(r)
        live = [r for r in live if r not in finished]
    return [r.output_ids for r in reqs]
