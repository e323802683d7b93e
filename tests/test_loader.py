"""The quantized-weight cache file and the model loader (reference: engine/quantization/
loader.py:1-186, tests/test_quantizaton.py:134-149).

CPU tests pin the file name scheme, the "meta" build of quantized modules (shapes and
dtypes of every buffer), and the tied-weight "aliases" metadata through a full
save / load round trip of an unquantized tiny model. The GPU test is the reference's cache
round trip: a fresh quantization and a load from the saved file give bit-identical
logits, for every method, and the quantized logits stay close to the bf16 ones
(MIN_LOGIT_COSINE of test_quantizaton.py:16).
"""
import json
import os
import tempfile

import pytest
import torch

DTYPE = torch.bfloat16
MIN_LOGIT_COSINE = {"int8_wo": 0.995, "int4_wo": 0.95, "fp8": 0.99}  # test_quantizaton.py:16


def olmoe_config():
    from transformers import OlmoeConfig
    # the reference test's tiny OLMoE (test_quantizaton.py:19-22)
    return OlmoeConfig(hidden_size=256, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                       num_key_value_heads=4, num_experts=8, num_experts_per_tok=2, vocab_size=512,
                       max_position_embeddings=512, eos_token_id=1, pad_token_id=0, bos_token_id=2)


def tiny_olmoe():
    from transformers import OlmoeForCausalLM
    torch.manual_seed(0)
    return OlmoeForCausalLM(olmoe_config()).to(DTYPE).eval()


def methods(group_size=64):
    from engine.quantization import METHODS, get_method
    return {n: get_method(n, device="cuda", compute_dtype=DTYPE, group_size=group_size) for n in METHODS}


def test_cache_path_scheme():
    from engine.quantization import get_method
    from engine.quantization.loader import cache_path
    m4 = get_method("int4_wo", group_size=128)
    assert cache_path("/c", "Qwen/Qwen3-4B", m4, ["linear", "experts"]) == \
        "/c/Qwen__Qwen3-4B__int4_wo_g128__experts-linear.safetensors"
    assert cache_path("/c", "/abs/model/", get_method("fp8"), ["linear"]) == "/c/abs__model__fp8__linear.safetensors"
    assert cache_path("c", "m", get_method("int8_wo"), ["linear", "lm_head"]) == "c/m__int8_wo__linear-lm_head.safetensors"


def test_meta_build_has_the_stored_layout():
    """quantize_model on "meta" (the first half of a cache load) runs no kernel and gives
    every buffer the name, shape and dtype the quantizers write."""
    from transformers import OlmoeForCausalLM
    from engine.quantization import get_method
    from engine.quantization.loader import quantize_model
    cfg = olmoe_config()
    H, inter, E = cfg.hidden_size, cfg.intermediate_size, cfg.num_experts
    expect = {
        "int8_wo": {"q_proj.qweight": ((H, H), torch.int8), "q_proj.scale": ((H, 1), DTYPE),
                    "experts.gate_up_qweight": ((E, 2 * inter, H), torch.int8),
                    "experts.down_scale": ((E, H, 1), DTYPE)},
        "int4_wo": {"q_proj.qweight": ((H, H // 2), torch.uint8), "q_proj.scale": ((H, H // 64), DTYPE),
                    "q_proj.zero": ((H, H // 64), DTYPE),
                    "experts.gate_up_qweight": ((E, 2 * inter, H // 2), torch.uint8),
                    "experts.down_zero": ((E, H, inter // 64), DTYPE)},
        "fp8": {"q_proj.qweight": ((H, H), torch.float8_e4m3fn), "q_proj.scale": ((H,), torch.float32),
                "experts.down_qweight": ((E, H, inter), torch.float8_e4m3fn)},
    }
    for name, want in expect.items():
        with torch.device("meta"):
            model = OlmoeForCausalLM(cfg).to(DTYPE)
        stats = quantize_model(model, get_method(name, group_size=64), ["experts", "linear"], "meta")
        assert stats["experts"] == cfg.num_hidden_layers and stats["linear"] == 4 * cfg.num_hidden_layers
        assert stats["skipped"] == []
        sd = model.state_dict()
        for suffix, (shape, dtype) in want.items():
            key = next(k for k in sd if k.startswith("model.layers.0.") and k.endswith(suffix))
            assert tuple(sd[key].shape) == shape and sd[key].dtype == dtype, (name, key, sd[key].shape, sd[key].dtype)


def test_tied_weights_saved_once_and_retied():
    """save_cache stores a shared tensor once with an "aliases" entry; load_from_cache
    re-ties it (loader.py:86-94, 134-137). No quantized targets: runs on the CPU."""
    from safetensors import safe_open
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from engine.quantization import get_method
    from engine.quantization.loader import cache_path, load_from_cache, save_cache
    cfg = Qwen3Config(hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, head_dim=16, vocab_size=256, max_position_embeddings=128,
                      tie_word_embeddings=True)
    torch.manual_seed(3)
    model = Qwen3ForCausalLM(cfg).to(DTYPE).eval()
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    method = get_method("int8_wo")
    with tempfile.TemporaryDirectory() as tmp:
        model_dir = os.path.join(tmp, "tiny")
        model.save_pretrained(model_dir)
        path = cache_path(os.path.join(tmp, "cache"), model_dir, method, [])
        save_cache(model, path, {"model": model_dir, **method.describe(), "targets": []})
        with safe_open(path, framework="pt") as f:
            meta = f.metadata()
            keys = set(f.keys())
        aliases = json.loads(meta["aliases"])
        assert aliases == {"lm_head.weight": "model.embed_tokens.weight"}
        assert "lm_head.weight" not in keys and "model.embed_tokens.weight" in keys
        assert json.loads(meta["info"])["method"] == "int8_wo"
        loaded, _ = load_from_cache(path, model_dir, method, [], "cpu", DTYPE)
        assert loaded.lm_head.weight.data_ptr() == loaded.model.embed_tokens.weight.data_ptr()
        # against the same checkpoint loaded by transformers (same rebuilt rotary buffers)
        from transformers import AutoModelForCausalLM
        fresh = AutoModelForCausalLM.from_pretrained(model_dir, dtype=DTYPE).eval()
        ids = torch.randint(3, 256, (1, 12), generator=torch.Generator().manual_seed(4))
        with torch.no_grad():
            assert torch.equal(fresh(ids).logits, loaded(ids).logits)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["int8_wo", "int4_wo", "fp8"])
def test_cache_roundtrip(name):
    """test_quantizaton.py:134-149 on the GPU: fresh == cached logits, bit for bit."""
    from engine.quantization.loader import load_quantized_model
    print(f"[case] cache roundtrip {name}", flush=True)
    base = tiny_olmoe()
    ids = torch.randint(3, 512, (1, 16), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        ref = base.to("cuda")(ids.to("cuda")).logits.float().cpu()
    m = methods()[name]
    with tempfile.TemporaryDirectory() as tmp:
        model_dir = os.path.join(tmp, "tiny")
        base.to("cpu").save_pretrained(model_dir)
        cache_dir = os.path.join(tmp, "cache")
        fresh, s1 = load_quantized_model(model_dir, m, ["experts", "linear"], "cuda", DTYPE, cache_dir=cache_dir)
        cached, s2 = load_quantized_model(model_dir, m, ["experts", "linear"], "cuda", DTYPE, cache_dir=cache_dir)
        assert s1["load_source"] == "fresh" and s2["load_source"] == "cache"
        assert os.path.exists(s1["cache_path"])
        with torch.no_grad():
            a = fresh(ids.to("cuda")).logits.float().cpu()
            b = cached(ids.to("cuda")).logits.float().cpu()
    assert torch.equal(a, b), f"{name}: cache mismatch"
    cos = torch.nn.functional.cosine_similarity(a.flatten(), ref.flatten(), dim=0).item()
    assert cos > MIN_LOGIT_COSINE[name], f"{name}: logit cosine {cos:.4f}"
