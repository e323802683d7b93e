"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP kernels.

Every oracle function is checked here against something it was not written from:
hand-derived known answers (tests/golden/known_answers.json), independent numpy codecs,
a float64 numpy attention, closed forms and invariants, and the reference tests' own
error bounds (tests/test_quantizaton.py:14-16 of the reference).
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import attention, codecs, moe, quant

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))

# reference tests/test_quantizaton.py:14
MAX_WEIGHT_ERROR = {"int8_wo": 0.01, "int4_wo": 0.12, "fp8": 0.05}


def rel_error(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


# ---------------------------------------------------------------- codecs pin torch's casts
def test_bf16_cast_matches_rne_definition():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(100000, generator=g) * torch.exp(torch.randn(100000, generator=g) * 8)
    # exact ties: low 16 bits = 0x8000 with both parities of bit 16
    ties = torch.tensor([0x3F808000, 0x3F818000, 0xBF808000, 0x40490000 | 0x8000], dtype=torch.int64)
    x = torch.cat([x, ties.to(torch.int32).view(torch.float32)])
    want = codecs.bf16_round(x.numpy())
    got = x.to(torch.bfloat16).float().numpy()
    assert np.array_equal(want.view(np.uint32), got.view(np.uint32))


def test_e4m3_decode_table_matches_definition():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = codes.view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    want = codecs.e4m3_table()
    nan = np.isnan(want)
    assert np.array_equal(nan, np.isnan(got))
    assert np.array_equal(want[~nan], got[~nan])
    assert want[0x7E] == 448.0 and want[0x01] == 2.0 ** -9


def test_e4m3_encode_matches_nearest_even():
    g = torch.Generator().manual_seed(1)
    mags = torch.exp(torch.rand(3000, generator=g) * 16 - 11)  # 2^-16 .. 2^7 roughly
    x = torch.cat([mags, -mags]).clamp(-448, 448)
    table = torch.tensor(codecs.e4m3_table())
    finite = table[:127]
    mid = ((finite[1:] + finite[:-1]) / 2).float()  # every tie point between codes
    x = torch.cat([x, mid, -mid])
    want = codecs.e4m3_encode(x.double().numpy())
    got = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(want, got)


def test_e4m3_known_answers():
    v = torch.tensor(GOLD["e4m3"]["value"], dtype=torch.float32)
    got = v.to(torch.float8_e4m3fn).view(torch.uint8).tolist()
    assert got == GOLD["e4m3"]["code"]
    assert codecs.e4m3_encode(np.array(GOLD["e4m3"]["value"])).tolist() == GOLD["e4m3"]["code"]


# ---------------------------------------------------------------- quantizers: known answers
def test_int8_known_answer():
    w = torch.tensor(GOLD["int8"]["w"], dtype=torch.float32)
    q = quant.int8_quantize(w)
    assert q["qweight"].tolist() == GOLD["int8"]["q"]
    assert q["scale"].float().flatten().tolist() == GOLD["int8"]["scale"]
    assert q["scale"].dtype == torch.bfloat16 and q["scale"].shape == (1, 1)


def test_int4_known_answer_and_unpack_order():
    w = torch.tensor(GOLD["int4"]["w"], dtype=torch.float32)
    q = quant.int4_quantize(w, group_size=128)
    assert q["qweight"].tolist() == GOLD["int4"]["q"]
    assert q["scale"].float().tolist() == GOLD["int4"]["scale"]
    assert q["zero"].float().tolist() == GOLD["int4"]["zero"]
    assert quant.int4_dequantize(**q).float().tolist() == GOLD["int4"]["dequant"]
    b = GOLD["int4_unpack"]
    u = quant.int4_unpack(torch.tensor([[b["byte"]]], dtype=torch.uint8))
    assert u.tolist() == [[b["k0"], b["k1"]]]


def test_fp8_rows_known_answer():
    x = torch.tensor(GOLD["fp8_rows"]["x"], dtype=torch.float32)
    q, s = quant.fp8_quantize_activation(x)
    assert s.flatten().tolist() == GOLD["fp8_rows"]["scale"]
    assert q.float().tolist() == GOLD["fp8_rows"]["q_values"]


def test_kv_int8_known_answer():
    x = torch.tensor(GOLD["kv_int8"]["x"], dtype=torch.float32)
    q, s = quant.kv_quantize(x, "int8")
    assert q.tolist() == GOLD["kv_int8"]["q"]
    assert s.float().tolist() == GOLD["kv_int8"]["scale"]


def test_moe_align_known_answer():
    c = GOLD["moe_align"]
    s, e, n = moe.moe_align(torch.tensor(c["topk_ids"]), c["E"], c["block_m"])
    assert s.tolist() == c["sorted_ids"] and e.tolist() == c["expert_ids"] and n.item() == c["num_padded"]


# ---------------------------------------------------------------- quantizers: properties
def test_roundtrip_error_bounds_with_expert_dim():
    """reference tests/test_quantizaton.py:47-57 bounds; leading expert dimension kept."""
    torch.manual_seed(1)
    w = (torch.randn(3, 64, 256) * 0.02).to(torch.bfloat16)
    q8 = quant.int8_quantize(w)
    assert rel_error(quant.int8_dequantize(**q8), w) < MAX_WEIGHT_ERROR["int8_wo"]
    q4 = quant.int4_quantize(w, 64)
    assert q4["qweight"].shape == (3, 64, 128) and q4["scale"].shape == (3, 64, 4)
    assert rel_error(quant.int4_dequantize(**q4), w) < MAX_WEIGHT_ERROR["int4_wo"]
    q4s = quant.int4_quantize_symmetric(w, 64)
    assert rel_error(quant.int4_dequantize(**q4s), w) < MAX_WEIGHT_ERROR["int4_wo"]
    qf = quant.fp8_quantize(w)
    assert rel_error(quant.fp8_dequantize(**qf), w) < MAX_WEIGHT_ERROR["fp8"]


def test_int8_codes_are_exact_rounding():
    """Brute-force restatement: each code is the nearest integer (ties even) to w / s."""
    g = torch.Generator().manual_seed(3)
    w = torch.randn(8, 512, generator=g) * 0.02
    q = quant.int8_quantize(w)
    s = w.abs().amax(-1, keepdim=True) / 127
    d = (w / s).double()
    assert (q["qweight"].double() - d).abs().max() <= 0.5 + 1e-9
    assert q["qweight"].abs().max() == 127


def test_int4_symmetric_range_and_dequant():
    g = torch.Generator().manual_seed(4)
    w = torch.randn(16, 256, generator=g) * 0.02
    q = quant.int4_quantize_symmetric(w, 128)
    u = quant.int4_unpack(q["qweight"])
    assert int(u.min()) >= 1 and int(u.max()) <= 15  # |round(w / s)| <= 7
    d = quant.int4_dequantize(q["qweight"], q["scale"])
    # symmetric: the group's largest magnitude is reproduced up to bf16 scale rounding
    err = (d.float() - w).abs().reshape(16, 2, 128).amax(-1)
    assert (err <= q["scale"].float() * 0.5 + w.abs().reshape(16, 2, 128).amax(-1) * 2 ** -8).all()


def test_linear_matches_dequantized_matmul():
    """reference tests/test_quantizaton.py:60-72."""
    torch.manual_seed(2)
    w = (torch.randn(64, 256) * 0.02).to(torch.bfloat16)
    x = torch.randn(2, 5, 256).to(torch.bfloat16)
    q8 = quant.int8_quantize(w)
    exp8 = torch.nn.functional.linear(x.float(), quant.int8_dequantize(**q8).float())
    assert rel_error(quant.int8_linear(x, **q8), exp8) < 0.01
    q4 = quant.int4_quantize(w, 64)
    exp4 = torch.nn.functional.linear(x.float(), quant.int4_dequantize(**q4).float())
    assert rel_error(quant.int4_linear(x, **q4), exp4) < 0.01
    assert rel_error(quant.int4_linear_fp32(x, **q4), exp4) < 0.01
    qf = quant.fp8_quantize(w)
    expf = torch.nn.functional.linear(x.float(), quant.fp8_dequantize(**qf))
    assert rel_error(quant.fp8_linear_emulated(x, **qf), expf) < 0.05
    xf, xs = quant.fp8_quantize_activation(x.reshape(-1, 256))
    assert rel_error(quant.fp8_scaled_mm(xf, xs, **qf), expf.reshape(-1, 64)) < 0.05


# ---------------------------------------------------------------- attention
def random_paged(lens, H, KV, D, page, seed=0):
    """reference tests/test_paged_attention.py:27-41 (CPU, fp32)."""
    g = torch.Generator().manual_seed(seed)
    pages = [-(-n // page) for n in lens]
    total = sum(pages) + 3
    k = torch.randn(total * page, KV, D, generator=g)
    v = torch.randn(total * page, KV, D, generator=g)
    perm = torch.randperm(total, generator=g).tolist()
    table = torch.zeros(len(lens), max(pages), dtype=torch.int32)
    i = 0
    for b, n in enumerate(pages):
        table[b, :n] = torch.tensor(perm[i:i + n])
        i += n
    q = torch.randn(len(lens), H, D, generator=g)
    return q, k, v, table, torch.tensor(lens, dtype=torch.int32)


@pytest.mark.parametrize("lens,H,KV,D,page", [
    ([1, 17, 40], 4, 4, 32, 16), ([33, 5], 8, 2, 32, 16), ([9, 30], 4, 4, 32, 1), ([50], 4, 4, 24, 16)])
def test_attention_reference_matches_float64(lens, H, KV, D, page):
    q, k, v, t, sl = random_paged(lens, H, KV, D, page)
    got = attention.paged_decode_reference(q, k, v, t, sl, page, D ** -0.5)
    want = attention.paged_decode_numpy64(q.numpy(), k.numpy(), v.numpy(), t.numpy(), sl.numpy(), page, D ** -0.5)
    assert np.abs(got.numpy() - want).max() < 1e-5


def test_attention_closed_forms():
    q, k, v, t, sl = random_paged([1, 24], 4, 2, 16, 8, seed=5)
    out = attention.paged_decode_reference(q, k, v, t, sl, 8, 0.25)
    slot0 = int(t[0, 0]) * 8
    assert torch.allclose(out[0], v[slot0].repeat_interleave(2, 0), atol=1e-6)   # one token -> its value
    # equal keys for request 1 -> the mean of its values
    slots = torch.tensor([int(t[1, i // 8]) * 8 + i % 8 for i in range(24)])
    k2 = k.clone()
    k2[slots] = k[slots[0]].clone()
    out2 = attention.paged_decode_reference(q, k2, v, t, sl, 8, 0.25)
    assert torch.allclose(out2[1], v[slots].mean(0).repeat_interleave(2, 0), atol=1e-5)


def test_attention_gqa_equals_repeated_heads_and_page_invariance():
    q, k, v, t, sl = random_paged([37, 12], 8, 2, 32, 16, seed=6)
    gqa = attention.paged_decode_reference(q, k, v, t, sl, 16, 0.2)
    mha = attention.paged_decode_reference(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), t, sl, 16, 0.2)
    assert torch.allclose(gqa, mha, atol=1e-6)
    # the same logical tokens described with page size 1
    slots = [[int(t[b, i // 16]) * 16 + i % 16 for i in range(int(sl[b]))] for b in range(2)]
    width = max(len(s) for s in slots)
    t1 = torch.tensor([s + [0] * (width - len(s)) for s in slots], dtype=torch.int32)
    tok = attention.paged_decode_reference(q, k, v, t1, sl, 1, 0.2)
    assert torch.allclose(gqa, tok, atol=1e-6)


def test_attention_quantized_cache_close_to_unquantized():
    """reference tests/test_paged_attention.py:73-89 bound (< 0.1 vs the unquantized cache)."""
    q, k, v, t, sl = random_paged([40, 7, 90], 4, 4, 32, 16, seed=2)
    full = attention.paged_decode_reference(q, k, v, t, sl, 16, 32 ** -0.5)
    for kind in ("int8", "fp8"):
        qk, sk = quant.kv_quantize(k, kind)
        qv, sv = quant.kv_quantize(v, kind)
        got = attention.paged_decode_reference(q, qk, qv, t, sl, 16, 32 ** -0.5, k_scale=sk, v_scale=sv)
        assert rel_error(got, full) < 0.1


# ---------------------------------------------------------------- moe
def test_moe_align_invariants():
    """reference tests/test_fused_moe.py:39-53."""
    torch.manual_seed(1)
    for T, k, E, bm in ((13, 3, 8, 4), (64, 8, 64, 16), (1, 8, 64, 16)):
        ids = torch.stack([torch.randperm(E)[:k] for _ in range(T)])
        s, e, n = moe.moe_align(ids, E, bm)
        n = int(n)
        rows = s[:n]
        real = rows[rows < T * k]
        assert sorted(real.tolist()) == list(range(T * k))
        flat = ids.reshape(-1)
        for b in range(n // bm):
            tile = rows[b * bm:(b + 1) * bm]
            tile = tile[tile < T * k]
            assert all(int(flat[p]) == int(e[b]) for p in tile.tolist())
        assert n % bm == 0 and n <= T * k + E * (bm - 1)
        assert (s[n:] == T * k).all() and (rows[rows >= T * k] == T * k).all()


def test_moe_reference_single_expert_is_dense_mlp():
    g = torch.Generator().manual_seed(7)
    T, H, inter, E = 5, 32, 16, 3
    hidden = torch.randn(T, H, generator=g)
    wgu = torch.randn(E, 2 * inter, H, generator=g) * 0.1
    wdn = torch.randn(E, H, inter, generator=g) * 0.1
    ids = torch.full((T, 1), 2)
    w = torch.ones(T, 1)
    got = moe.moe_reference(hidden, wgu, wdn, w, ids)
    gu = hidden @ wgu[2].t()
    want = (torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]) @ wdn[2].t()
    assert torch.allclose(got, want, atol=1e-5)


def test_int4_experts_reference_matches_quant_loop():
    """The dequantized-expert reference equals the QuantExperts loop (modules.py:55-75)
    run with the oracle's int4 linear, up to bf16 rounding of the loop."""
    g = torch.Generator().manual_seed(8)
    T, H, inter, E, k = 6, 256, 128, 4, 2
    hidden = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gu = quant.int4_quantize((torch.randn(E, 2 * inter, H, generator=g) * 0.02).to(torch.bfloat16), 128)
    dn = quant.int4_quantize((torch.randn(E, H, inter, generator=g) * 0.02).to(torch.bfloat16), 128)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.softmax(torch.randn(T, k, generator=g), -1).to(torch.bfloat16)
    ref = moe.int4_experts_reference(hidden, gu, dn, w, ids)
    loop = moe.quant_experts_loop(hidden, quant.int4_linear, gu, dn, ids, w, E)
    assert rel_error(loop, ref) < 0.02
