"""Quantized model loading and the quantized-weight cache file.

Reference: engine/quantization/loader.py:1-180. The public functions keep the reference's
names, arguments and return values, and the cache file keeps its format, so a cache
written by either implementation loads in the other:

  * file name  <cache_dir>/<model name with "/" -> "__">__<method>[_g<group>]__<targets
               sorted, "-"-joined>.safetensors                       (loader.py:77-80)
  * tensors    the quantized model's state_dict on the CPU, contiguous; a tensor that is
               shared under several names (tied embeddings / lm_head) is stored once
  * metadata   "info"    JSON of {"model", **method.describe(), "targets"}
               "aliases" JSON of {alias name: stored name}            (loader.py:83-100)

Quantization runs the HIP kernels of this package, so `device` must be a ROCm device for
real weights; "meta" builds the quantized modules with shapes only (the first half of a
cache load).
"""
import gc
import json
import os
import time

import torch
from torch import nn

from engine.quantization.modules import QuantExperts, QuantLinear, is_fused_experts


def _set_module(root: nn.Module, name: str, new: nn.Module):
    parent, _, child = name.rpartition(".")
    setattr(root.get_submodule(parent) if parent else root, child, new)


def _decoder_layers(model):
    layers = getattr(getattr(model, "model", None), "layers", None)
    if layers is None:
        raise RuntimeError("Expected the decoder layers at model.model.layers")
    return layers


def _release(device):
    gc.collect()
    if torch.device(device).type == "cuda":
        torch.cuda.empty_cache()


def quantize_model(model, method, targets, device):
    """Swap eligible modules for quantized ones, one decoder layer at a time on `device`
    (loader.py:38-74). targets: any of "experts" (fused 3-D expert weights), "linear"
    (nn.Linear inside the decoder layers), "lm_head". Returns counts and skipped names."""
    stats = {"experts": 0, "linear": 0, "lm_head": 0, "skipped": [], "quantized_params": 0}
    for i, layer in enumerate(_decoder_layers(model)):
        layer.to(device)
        for name, module in list(layer.named_modules()):
            qualified = f"model.layers.{i}.{name}"
            if "experts" in targets and is_fused_experts(module):
                if method.supports(module.gate_up_proj) and method.supports(module.down_proj):
                    stats["quantized_params"] += module.gate_up_proj.numel() + module.down_proj.numel()
                    _set_module(layer, name, QuantExperts(module, method))
                    stats["experts"] += 1
                else:
                    stats["skipped"].append(qualified)
            elif "linear" in targets and isinstance(module, nn.Linear):
                if method.supports(module.weight):
                    stats["quantized_params"] += module.weight.numel()
                    _set_module(layer, name, QuantLinear(module, method))
                    stats["linear"] += 1
                else:
                    stats["skipped"].append(qualified)
        if device != "meta":
            _release(device)
    head = getattr(model, "lm_head", None)
    if "lm_head" in targets and isinstance(head, nn.Linear):
        if method.supports(head.weight):
            stats["quantized_params"] += head.weight.numel()
            model.lm_head = QuantLinear(head.to(device), method)
            stats["lm_head"] = 1
        else:
            stats["skipped"].append("lm_head")
    model.to(device)  # the rest (embeddings, norms, router, rotary) in the original dtype
    return stats


def cache_path(cache_dir, model_name, method, targets):
    """loader.py:77-80."""
    stem = model_name.strip("/").replace("/", "__")
    tag = method.name + (f"_g{method.group_size}" if hasattr(method, "group_size") else "")
    return os.path.join(cache_dir, f"{stem}__{tag}__{'-'.join(sorted(targets))}.safetensors")


def save_cache(model, path, info):
    """Write the quantized state dict (loader.py:83-100); tensors that share storage are
    stored once and recorded in the "aliases" metadata. Written to a temporary name first
    and renamed, so a cache file is never seen half written."""
    from safetensors.torch import save_file

    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    tensors, aliases, first = {}, {}, {}
    for name, t in model.state_dict().items():
        ident = (t.data_ptr(), tuple(t.shape), t.dtype, t.device)
        if ident in first:
            aliases[name] = first[ident]
            continue
        first[ident] = name
        tensors[name] = t.detach().to("cpu").contiguous()
    tmp = path + ".tmp"
    save_file(tensors, tmp, metadata={"info": json.dumps(info), "aliases": json.dumps(aliases)})
    os.replace(tmp, path)


def _rebuild_meta_buffers(model, device):
    """Non-persistent buffers (rotary frequencies) are not in the file; rebuild the modules
    that still hold meta buffers from the model config (loader.py:103-118)."""
    for name, module in list(model.named_modules()):
        if any(b.is_meta for b in module.buffers(recurse=False)):
            try:
                _set_module(model, name, type(module)(config=model.config).to(device))
            except TypeError as err:
                raise RuntimeError(f"cannot rebuild {name} ({type(module).__name__}) after a cache load: {err}; "
                                   f"set QUANT_USE_CACHE=0") from err
    left = [n for n, t in list(model.named_parameters()) + list(model.named_buffers()) if t.is_meta]
    if left:
        raise RuntimeError(f"weights missing after the cache load (e.g. {left[:3]}); delete the cache file or "
                           f"set QUANT_USE_CACHE=0")


def load_from_cache(path, model_name, method, targets, device, dtype):
    """Build the model on "meta", put quantized modules in place, then assign the cached
    tensors (loader.py:121-145). Returns (model in eval mode, stats)."""
    from safetensors import safe_open
    from safetensors.torch import load_file
    from transformers import AutoConfig, AutoModelForCausalLM, GenerationConfig

    config = AutoConfig.from_pretrained(model_name)
    with torch.device("meta"):
        model = AutoModelForCausalLM.from_config(config, dtype=dtype)
    stats = quantize_model(model, method, targets, "meta")
    with safe_open(path, framework="pt") as f:
        aliases = json.loads((f.metadata() or {}).get("aliases", "{}"))
    state = load_file(path, device=str(device))
    missing, unexpected = model.load_state_dict(state, strict=False, assign=True)
    for name, source in aliases.items():
        parent, _, attr = name.rpartition(".")
        setattr(model.get_submodule(parent), attr, model.get_parameter(source))
    missing = [m for m in missing if m not in aliases]
    if missing or unexpected:
        raise RuntimeError(f"cache {path} does not match the model (missing {missing[:3]}, unexpected "
                           f"{unexpected[:3]}); delete it and restart")
    del state
    _rebuild_meta_buffers(model, device)
    try:
        model.generation_config = GenerationConfig.from_pretrained(model_name)
    except OSError:
        pass
    return model.eval(), stats


def load_quantized_model(model_name, method, targets, device, dtype, cache_dir=None, use_cache=True):
    """loader.py:148-168: the cache when present, else load bf16 weights, quantize and save
    the cache. stats gains "load_source" ("cache" / "fresh"), "cache_path", "load_time_s"."""
    from transformers import AutoModelForCausalLM

    start = time.perf_counter()
    path = cache_path(cache_dir, model_name, method, targets) if cache_dir else None
    if use_cache and path and os.path.exists(path):
        model, stats = load_from_cache(path, model_name, method, targets, device, dtype)
        source = "cache"
    else:
        model = AutoModelForCausalLM.from_pretrained(model_name, dtype=dtype).eval()
        stats = quantize_model(model, method, targets, device)
        source = "fresh"
        if use_cache and path:
            save_cache(model, path, {"model": model_name, **method.describe(), "targets": targets})
    stats["load_source"] = source
    stats["cache_path"] = path
    stats["load_time_s"] = round(time.perf_counter() - start, 1)
    return model, stats


def weight_memory(model) -> dict:
    """Bytes of parameters and buffers, split into quantized modules and the rest
    (loader.py:171-186), in MiB."""
    quant = other = 0
    seen = set()
    for m in model.modules():
        if isinstance(m, (QuantLinear, QuantExperts)):
            for t in list(m.parameters()) + list(m.buffers()):
                seen.add(id(t))
                quant += t.numel() * t.element_size()
    for t in list(model.parameters()) + list(model.buffers()):
        if id(t) not in seen:
            other += t.numel() * t.element_size()
    mib = 1024 ** 2
    return {"weights_total_mb": round((quant + other) / mib, 1),
            "weights_quantized_layers_mb": round(quant / mib, 1),
            "weights_other_mb": round(other / mib, 1)}
