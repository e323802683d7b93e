"""Quantizing a transformers model in place, and the quantized-weight cache file.

Public functions and their contracts are those of the reference's
engine/quantization/loader.py:38-186 (`quantize_model`, `cache_path`, `save_cache`,
`load_from_cache`, `load_quantized_model`, `weight_memory`). The cache file format is an
interface shared with the reference, so a file written by either loads in the other:

  * name      <cache_dir>/<model name, "/" -> "__">__<method>[_g<group>]__<targets sorted,
              "-"-joined>.safetensors                                   (loader.py:77-80)
  * tensors   the quantized model's state dict, on the CPU, contiguous; a tensor reachable
              under several names (tied embedding / lm_head) is stored under one of them
  * metadata  "info": JSON of {"model", **method.describe(), "targets"};
              "aliases": JSON of {other name: stored name}              (loader.py:83-100)

Design: the swap is planned first (a list of (parent, attribute, replacement kind)) and
then carried out one decoder layer at a time, so device memory holds one unquantized
layer at most. Quantization runs this package's HIP kernels; on device "meta" the
quantized modules are built with shapes only, which is how a cache load starts.
"""
import gc
import json
import os
import time

import torch
from torch import nn

from engine.quantization.modules import QuantExperts, QuantLinear, is_fused_experts


def _layers_of(model):
    inner = getattr(model, "model", None)
    layers = getattr(inner, "layers", None)
    if layers is None:
        raise RuntimeError("quantize_model expects the decoder layers at model.model.layers")
    return layers


def _plan(root, prefix, targets):
    """(parent module, child attribute, qualified name, kind) for every swap candidate
    under `root`; kind is "experts" or "linear". Children of a candidate are not visited."""
    found = []
    for attr, child in root.named_children():
        qualified = f"{prefix}.{attr}" if prefix else attr
        if "experts" in targets and is_fused_experts(child):
            found.append((root, attr, qualified, "experts"))
        elif "linear" in targets and isinstance(child, nn.Linear):
            found.append((root, attr, qualified, "linear"))
        else:
            found.extend(_plan(child, qualified, targets))
    return found


def _tidy(device):
    gc.collect()
    if torch.device(device).type == "cuda":
        torch.cuda.empty_cache()


def quantize_model(model, method, targets, device):
    """Replace eligible modules by quantized ones on `device`, layer by layer.

    targets: any of "experts" (3-D fused expert weights), "linear" (nn.Linear inside the
    decoder layers) and "lm_head". Modules `method.supports` rejects stay as they are and
    are listed under "skipped". Returns {"experts", "linear", "lm_head", "skipped",
    "quantized_params"} (reference loader.py:38-74)."""
    stats = dict(experts=0, linear=0, lm_head=0, skipped=[], quantized_params=0)
    for index, layer in enumerate(_layers_of(model)):
        layer.to(device)
        for parent, attr, name, kind in _plan(layer, f"model.layers.{index}", targets):
            module = getattr(parent, attr)
            weights = [module.gate_up_proj, module.down_proj] if kind == "experts" else [module.weight]
            if not all(method.supports(w) for w in weights):
                stats["skipped"].append(name)
                continue
            stats["quantized_params"] += sum(w.numel() for w in weights)
            setattr(parent, attr, QuantExperts(module, method) if kind == "experts" else QuantLinear(module, method))
            stats[kind] += 1
        if device != "meta":
            _tidy(device)
    head = getattr(model, "lm_head", None)
    if "lm_head" in targets and isinstance(head, nn.Linear):
        if method.supports(head.weight):
            stats["quantized_params"] += head.weight.numel()
            model.lm_head = QuantLinear(head.to(device), method)
            stats["lm_head"] = 1
        else:
            stats["skipped"].append("lm_head")
    model.to(device)  # what stays unquantized: embeddings, norms, router, rotary tables
    return stats


def cache_path(cache_dir, model_name, method, targets):
    """The cache file's path (format above; reference loader.py:77-80)."""
    tag = method.name
    if hasattr(method, "group_size"):
        tag += f"_g{method.group_size}"
    stem = "__".join([model_name.strip("/").replace("/", "__"), tag, "-".join(sorted(targets))])
    return os.path.join(cache_dir, stem + ".safetensors")


def _storage_key(t):
    """Two state-dict entries are the same tensor when they view the same bytes the same way."""
    return (t.device, t.untyped_storage().data_ptr(), t.storage_offset(), tuple(t.shape), tuple(t.stride()), t.dtype)


def save_cache(model, path, info):
    """Write the model's state dict to `path` in the cache format (reference
    loader.py:83-100). The file appears under its name only once complete."""
    from safetensors.torch import save_file

    stored_as = {}
    tensors, aliases = {}, {}
    for name, t in model.state_dict().items():
        key = _storage_key(t)
        if key in stored_as:
            aliases[name] = stored_as[key]
        else:
            stored_as[key] = name
            tensors[name] = t.detach().cpu().contiguous()
    folder = os.path.dirname(path)
    if folder:
        os.makedirs(folder, exist_ok=True)
    partial = f"{path}.tmp"
    save_file(tensors, partial, metadata={"info": json.dumps(info), "aliases": json.dumps(aliases)})
    os.replace(partial, path)


def _restore_meta_modules(model, device):
    """Buffers that are not saved (rotary frequencies) are still on "meta" after the load:
    rebuild the modules holding them from the model config."""
    stale = [name for name, m in model.named_modules() if any(b.is_meta for b in m.buffers(recurse=False))]
    for name in stale:
        module = model.get_submodule(name)
        try:
            fresh = type(module)(config=model.config).to(device)
        except TypeError as err:
            raise RuntimeError(f"cannot rebuild {name} ({type(module).__name__}) after a cache load ({err}); "
                               "set QUANT_USE_CACHE=0") from err
        parent, _, attr = name.rpartition(".")
        setattr(model.get_submodule(parent) if parent else model, attr, fresh)
    for name, t in list(model.named_parameters()) + list(model.named_buffers()):
        if t.is_meta:
            raise RuntimeError(f"{name} is missing after the cache load; delete the cache file or set "
                               "QUANT_USE_CACHE=0")


def load_from_cache(path, model_name, method, targets, device, dtype):
    """Model skeleton on "meta" with the quantized modules in place, then the cached
    tensors assigned and shared names re-tied (reference loader.py:121-145).
    Returns (model in eval mode, stats of the skeleton's quantize_model)."""
    from safetensors import safe_open
    from safetensors.torch import load_file
    from transformers import AutoConfig, AutoModelForCausalLM, GenerationConfig

    with torch.device("meta"):
        model = AutoModelForCausalLM.from_config(AutoConfig.from_pretrained(model_name), dtype=dtype)
    stats = quantize_model(model, method, targets, "meta")
    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
    aliases = json.loads(meta.get("aliases", "{}"))
    result = model.load_state_dict(load_file(path, device=str(device)), strict=False, assign=True)
    for name, source in aliases.items():
        owner, _, attr = name.rpartition(".")
        setattr(model.get_submodule(owner), attr, model.get_parameter(source))
    missing = [n for n in result.missing_keys if n not in aliases]
    if missing or result.unexpected_keys:
        raise RuntimeError(f"cache {path} does not match the model (missing {missing[:3]}, unexpected "
                           f"{result.unexpected_keys[:3]}); delete it and restart")
    _restore_meta_modules(model, device)
    try:
        model.generation_config = GenerationConfig.from_pretrained(model_name)
    except OSError:
        pass
    return model.eval(), stats


def load_quantized_model(model_name, method, targets, device, dtype, cache_dir=None, use_cache=True):
    """Load from the cache file when it exists; otherwise load the bf16 checkpoint,
    quantize it and write the cache (reference loader.py:148-168). stats gains
    "load_source" ("cache" / "fresh"), "cache_path" and "load_time_s"."""
    from transformers import AutoModelForCausalLM

    t0 = time.perf_counter()
    path = cache_path(cache_dir, model_name, method, targets) if cache_dir else None
    cached = bool(use_cache and path and os.path.exists(path))
    if cached:
        model, stats = load_from_cache(path, model_name, method, targets, device, dtype)
    else:
        model = AutoModelForCausalLM.from_pretrained(model_name, dtype=dtype).eval()
        stats = quantize_model(model, method, targets, device)
        if use_cache and path:
            save_cache(model, path, {"model": model_name, **method.describe(), "targets": targets})
    stats.update(load_source="cache" if cached else "fresh", cache_path=path,
                 load_time_s=round(time.perf_counter() - t0, 1))
    return model, stats


def weight_memory(model) -> dict:
    """MiB held by parameters and buffers: inside quantized modules, and everywhere else
    (reference loader.py:171-186). A tensor reachable twice is counted once."""
    def nbytes(tensors):
        return sum(t.numel() * t.element_size() for t in tensors)

    quantized = {}
    for m in model.modules():
        if isinstance(m, (QuantLinear, QuantExperts)):
            for t in [*m.parameters(), *m.buffers()]:
                quantized[id(t)] = t
    rest = {id(t): t for t in [*model.parameters(), *model.buffers()] if id(t) not in quantized}
    q, o = nbytes(quantized.values()), nbytes(rest.values())
    mib = float(1 << 20)
    return {"weights_total_mb": round((q + o) / mib, 1), "weights_quantized_layers_mb": round(q / mib, 1),
            "weights_other_mb": round(o / mib, 1)}
