"""Quantize / dequantize kernels vs the CPU oracle: bit-exact (integer codes, bf16 and
e4m3 bytes, fp32 scales)."""
import json
import os

import pytest
import torch

from oracle import quant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def case(msg):
    print(f"[case] {msg}", flush=True)


def weights(shape, seed, dtype=torch.bfloat16, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(dtype)


def same_bytes(a, b):
    a = a.detach().cpu().contiguous()
    b = b.detach().cpu().contiguous()
    assert a.shape == b.shape and a.dtype == b.dtype, (a.shape, b.shape, a.dtype, b.dtype)
    return torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("shape,dtype", [((64, 256), torch.bfloat16), ((3, 64, 256), torch.bfloat16),
                                         ((96, 2560), torch.float32), ((2048, 2560), torch.bfloat16)])
def test_int8_quantize_dequantize_bit_exact(shape, dtype):
    from kernels import quant_ops as ops
    case(f"int8 quantize {shape} {dtype}")
    w = weights(shape, 1, dtype)
    want = O.int8_quantize(w)
    q, s = ops.int8_quantize(w.to(DEV), torch.bfloat16)
    assert same_bytes(q, want["qweight"]) and same_bytes(s, want["scale"])
    assert same_bytes(ops.int8_dequantize(q, s), O.int8_dequantize(**want))


@pytest.mark.parametrize("shape,group", [((64, 256), 64), ((3, 64, 256), 128), ((2560, 9728), 128),
                                         ((40, 384), 32)])
def test_int4_quantize_dequantize_bit_exact(shape, group):
    from kernels import quant_ops as ops
    case(f"int4 quantize {shape} g={group}")
    w = weights(shape, 2)
    want = O.int4_quantize(w, group)
    q, s, z = ops.int4_quantize(w.to(DEV), group, torch.bfloat16)
    assert same_bytes(q, want["qweight"]) and same_bytes(s, want["scale"]) and same_bytes(z, want["zero"])
    assert same_bytes(ops.int4_dequantize(q, s, z), O.int4_dequantize(**want))


@pytest.mark.parametrize("shape,group", [((64, 256), 128), ((2560, 9728), 128)])
def test_int4_symmetric_quantize_dequantize_bit_exact(shape, group):
    from kernels import quant_ops as ops
    case(f"int4 symmetric {shape}")
    w = weights(shape, 3)
    want = O.int4_quantize_symmetric(w, group)
    q, s, z = ops.int4_quantize(w.to(DEV), group, torch.bfloat16, symmetric=True)
    assert z is None
    assert same_bytes(q, want["qweight"]) and same_bytes(s, want["scale"])
    assert same_bytes(ops.int4_dequantize(q, s, None), O.int4_dequantize(**want))


# bf16 rows of at most 4096 (multiples of 8) take the wavefront-per-row kernel, the others
# the workgroup-per-row kernel; "wg" forces the latter everywhere (MIQ_FP8_QUANT_ROWS_WG)
@pytest.mark.parametrize("shape,dtype,std", [((64, 256), torch.bfloat16, 0.02), ((2048, 2560), torch.bfloat16, 1.0),
                                             ((6144, 2560), torch.float32, 0.02), ((7, 200), torch.bfloat16, 3.0),
                                             ((5, 8192), torch.bfloat16, 1.0), ((3, 8200), torch.bfloat16, 1.0),
                                             ((9, 4096), torch.bfloat16, 1.0), ((6, 4104), torch.bfloat16, 1.0),
                                             ((1, 8), torch.bfloat16, 1.0)])
@pytest.mark.parametrize("kernel", ["auto", "wg"])
def test_fp8_quantize_rows_bit_exact(shape, dtype, std, kernel, miq_env):
    from kernels import quant_ops as ops
    case(f"fp8 rows {shape} {dtype} {kernel}")
    if kernel == "wg":
        miq_env("MIQ_FP8_QUANT_ROWS_WG", "1")
    x = weights(shape, 4, dtype, std)
    wq = O.fp8_quantize(x)
    q, s = ops.fp8_quantize_rows(x.to(DEV))
    assert same_bytes(q, wq["qweight"]) and same_bytes(s, wq["scale"])
    assert same_bytes(ops.fp8_dequantize(q, s), O.fp8_dequantize(**wq))


def test_fp8_codec_known_answers_and_all_codes():
    from kernels import quant_ops as ops
    case("fp8 known answers")
    c = GOLD["fp8_rows"]
    q, s = ops.fp8_quantize_rows(torch.tensor(c["x"], device=DEV))
    assert s.cpu().tolist() == c["scale"] and q.float().cpu().tolist() == c["q_values"]
    # every finite e4m3 value and every midpoint between neighbours, scaled so amax = 448
    vals = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float()
    vals = vals[~torch.isnan(vals)]
    pos = vals[vals > 0].sort().values
    mids = (pos[1:] + pos[:-1]) / 2
    row = torch.cat([vals, mids, -mids, torch.tensor([448.0])])
    row = torch.cat([row, torch.zeros((-row.numel()) % 8)]).reshape(1, -1)
    q, s = ops.fp8_quantize_rows(row.to(DEV))
    assert s.item() == 1.0
    assert same_bytes(q, row.to(torch.float8_e4m3fn))


def test_fp8_quantize_rows_every_bf16_value():
    """The bf16 path's e4m3 encode on every bf16 value in [-448, 448] (a row with amax 448,
    so the scale is 1 and each code is the encode of the value itself): every normal and
    subnormal e4m3 code, every tie between neighbours, against the oracle's restated
    encode and torch's float8_e4m3fn conversion."""
    from kernels import quant_ops as ops
    case("fp8 rows every bf16 value")
    bits = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    vals = bits[~torch.isnan(bits.float())]
    vals = vals[vals.float().abs() <= 448.0]
    row = torch.cat([vals, torch.tensor([448.0], dtype=torch.bfloat16)])
    row = torch.cat([row, torch.zeros((-row.numel()) % 8, dtype=torch.bfloat16)]).reshape(1, -1)
    q, s = ops.fp8_quantize_rows(row.to(DEV))
    assert s.item() == 1.0
    want = O.fp8_quantize(row)
    assert same_bytes(q, want["qweight"])
    # the same values in rows of 4096 (the wavefront-per-row kernel), each row with 448 so
    # that every scale is 1
    flat = torch.cat([vals, torch.zeros((-vals.numel()) % 4095, dtype=torch.bfloat16)]).reshape(-1, 4095)
    rows = torch.cat([flat, torch.full((flat.shape[0], 1), 448.0, dtype=torch.bfloat16)], dim=1)
    q2, s2 = ops.fp8_quantize_rows(rows.to(DEV))
    assert (s2 == 1.0).all()
    assert same_bytes(q2, O.fp8_quantize(rows)["qweight"])
    assert same_bytes(q, row.float().to(torch.float8_e4m3fn))


@pytest.mark.parametrize("kind", ["int8", "fp8"])
def test_kv_quant_write_bit_exact(kind):
    from engine.core.kv_cache import KVCache
    case(f"kv quant write {kind}")
    g = torch.Generator().manual_seed(5)
    T, KV, D = 37, 8, 128
    k = (torch.randn(T, KV, D, generator=g) * torch.rand(T, KV, 1, generator=g) * 4).to(torch.bfloat16)
    v = (torch.randn(T, KV, D, generator=g)).to(torch.bfloat16)
    cache = KVCache("paged", 2, KV, D, 128, torch.bfloat16, DEV, block_size=16, kv_dtype=kind)
    slots = torch.randperm(128, generator=g)[:T]
    cache.write(1, slots.to(DEV), k.to(DEV), v.to(DEV))
    for x, store, sc in ((k, cache.k, cache.k_scale), (v, cache.v, cache.v_scale)):
        qw, sw = O.kv_quantize(x, kind)
        assert same_bytes(store[1][slots.to(DEV)], qw)
        assert same_bytes(sc[1][slots.to(DEV)], sw)
    assert (cache.k_scale[0] == 1).all()  # other layer untouched


def test_kv_int8_known_answer():
    from engine.core.kv_cache import KVCache
    case("kv int8 known answer")
    c = GOLD["kv_int8"]
    cache = KVCache("paged", 1, 1, 128, 16, torch.bfloat16, DEV, block_size=16, kv_dtype="int8")
    x = torch.tensor(c["x"], dtype=torch.bfloat16, device=DEV)
    cache.write(0, torch.tensor([3], device=DEV), x, x)
    assert cache.k[0][3].cpu().tolist() == c["q"][0]
    assert cache.k_scale[0][3].float().cpu().tolist() == c["scale"][0]
