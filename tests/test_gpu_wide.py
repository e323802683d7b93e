"""The wide weight-only GEMM (long prefill chunks) vs the CPU oracle.

The wide kernel dequantizes each weight once per workgroup into bf16 and multiplies on the
bf16 MFMA, as the reference's own path does (int4_wo.py:33-42 / int8_wo.py:14-21, then
base.py:20-24). Its int4 weights are the reference's bit for bit (each op rounded to the
scale dtype, then bf16), so it is held to |got - want| <= 1e-2 + 2e-2 |want| elementwise
against the fp32-accumulated product on the reference's own bf16 weights
(oracle.quant.int4_dequantize, pinned bit-exact against the dequantize kernel and the
reference's known answers), and to the reference test's norm-wise bound (rel < 0.01,
tests/test_quantizaton.py:60-72) against the product on the exactly dequantized fp32
weights. (The exact fp32 product is not an elementwise bound for bf16 weights: at
K = 9728 the weights' rounding alone moves outputs by up to about 0.04, the reference's
own formula included.) INT8 codes are exact in bf16, so INT8 keeps the exact oracle.

Every shape runs with each tile height forced (MIQ_WO_WIDE_MT = 1, 2, 3), with K splits
forced (MIQ_WO_WIDE_S: 1 to 16 splits, fp32 partial outputs added in split order by the
reduce kernel), with the planned choice, and with the wide kernel off (the prefill kernel,
held to the exact oracle as in test_gpu_gemm), and the shared workspace must be all zeros
afterwards (the packed activations and the partials are cleared again).
"""
import pytest
import torch

from oracle import quant as O
from test_gpu_gemm import DEV, case, make_w, make_x, rel, within, workspace_is_zero
from wide_plan import wide_plan, wide_planned  # noqa: F401 (re-exported for the other GPU tests)

pytestmark = pytest.mark.gpu

# (M, N, K, group): ragged M (not a multiple of any tile height), N with a partial
# 128-row weight block (2576 = 20 * 128 + 16), one and three k-steps, groups of 1 to 4 steps
WIDE_SHAPES = [(1300, 2560, 512, 128), (520, 2576, 1536, 256), (777, 1024, 128, 128), (300, 4096, 384, 128),
               (2048, 2560, 2560, 512), (1024, 2560, 9728, 128)]
# MIQ_WO_WIDE_MT, MIQ_WO_WIDE_S: forced tile heights, forced K splits (fp32 partial outputs
# added by the reduce kernel), the planned choice, the wide kernel off
TILES = {"mt1": ("1", None), "mt2": ("2", None), "mt3": ("3", None), "mt1s3": ("1", "3"), "mt2s2": ("2", "2"),
         "mt3s16": ("3", "16"), "planned": (None, None), "off": ("0", None)}


def set_tiles(miq_env, tiles):
    mt, s = TILES[tiles]
    if mt is not None:
        miq_env("MIQ_WO_WIDE_MT", mt)
    if s is not None:
        miq_env("MIQ_WO_WIDE_S", s)


def int4_ref_weights_product(x, q):
    """fp32-accumulated product on the reference's bf16 weights (base.py:20-24)."""
    w = O.int4_dequantize(q["qweight"], q["scale"], q.get("zero")).to(torch.bfloat16)
    return torch.nn.functional.linear(x.float(), w.float())


_CACHE = {}


def int4_case(M, N, K, group, symmetric, sdt):
    """Inputs and both oracles of a shape, computed once for all tile settings."""
    key = ("int4", M, N, K, group, symmetric, sdt)
    if key not in _CACHE:
        w = make_w(N, K, 90)
        x = make_x(M, K, 91)
        q = O.int4_quantize_symmetric(w, group, sdt) if symmetric else O.int4_quantize(w, group, sdt)
        _CACHE.clear()
        _CACHE[key] = (x, q, int4_ref_weights_product(x, q), O.int4_linear_fp32(x, **q))
    return _CACHE[key]


def int8_case(M, N, K, sdt):
    key = ("int8", M, N, K, sdt)
    if key not in _CACHE:
        w = make_w(N, K, 92)
        x = make_x(M, K, 93)
        q = O.int8_quantize(w, sdt)
        _CACHE.clear()
        _CACHE[key] = (x, q, O.int8_linear_fp32(x, **q), O.int8_linear(x, **q))
    return _CACHE[key]


@pytest.mark.parametrize("M,N,K,group", WIDE_SHAPES)
@pytest.mark.parametrize("symmetric,sdt", [(False, torch.bfloat16), (True, torch.bfloat16), (False, torch.float16),
                                           (False, torch.float32)])
@pytest.mark.parametrize("tiles", list(TILES))
def test_w4a16_wide(M, N, K, group, symmetric, sdt, tiles, miq_env):
    from kernels import quant_ops as ops
    case(f"w4a16 wide M={M} N={N} K={K} g={group} sym={symmetric} {sdt} tiles={tiles}")
    set_tiles(miq_env, tiles)
    x, q, ref_w, exact = int4_case(M, N, K, group, symmetric, sdt)
    y = ops.w4a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV),
                         None if symmetric else q["zero"].to(DEV))
    assert y.shape == (M, N)
    if tiles == "off" or (tiles == "planned" and not wide_planned(M, N, K)):
        within(y, exact)  # the prefill kernel: exact weights, as in test_gpu_gemm
    else:
        within(y, ref_w)
    assert rel(y, exact) < 0.01
    assert workspace_is_zero()


@pytest.mark.parametrize("M,N,K", [(1300, 2560, 512), (520, 2576, 1536), (777, 1024, 128), (2048, 2560, 2560)])
@pytest.mark.parametrize("sdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tiles", list(TILES))
def test_w8a16_wide(M, N, K, sdt, tiles, miq_env):
    from kernels import quant_ops as ops
    case(f"w8a16 wide M={M} N={N} K={K} {sdt} tiles={tiles}")
    set_tiles(miq_env, tiles)
    x, q, want, ref = int8_case(M, N, K, sdt)
    y = ops.w8a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV))
    within(y, want)
    assert rel(y, ref) < 0.01
    assert workspace_is_zero()


def test_wide_strided_rows_and_output():
    """Activation rows with a row stride above K and an output written into a wider buffer
    (row stride above N, so the 8-byte output stores fall back to 2-byte ones)."""
    from kernels import _lib as L
    from kernels import quant_ops as ops
    M, N, K = 1100, 2560, 1024
    case(f"wide strided M={M} N={N} K={K}")
    w = make_w(N, K, 94)
    xbig = make_x(M, K + 64, 95)
    x = xbig[:, :K]
    q = O.int4_quantize(w, 128)
    want = int4_ref_weights_product(x, q)
    xd = xbig.to(DEV)[:, :K]
    qd, sd, zd = (q[k].to(DEV) for k in ("qweight", "scale", "zero"))
    buf = torch.full((M, N + 6), 7.0, dtype=torch.bfloat16, device=DEV)
    nbytes = L.load().miq_wo_gemm_workspace_bytes(M, N, K, 4)
    ws = L.wo_workspace(xd.device, nbytes)
    L.call("miq_w4a16_gemm", L.ptr(xd), xd.stride(0), L.ptr(qd), L.ptr(sd), L.ptr(zd), L.dtype_code(sd.dtype), 128,
           L.ptr(buf), buf.stride(0), M, N, K, L.ptr(ws), ws.numel(), L.stream(xd.device))
    within(buf[:, :N], want)
    assert bool((buf[:, N:].float() == 7.0).all())
    assert workspace_is_zero()
    torch.testing.assert_close(buf[:, :N], ops.w4a16_linear(xd, qd, sd, zd), rtol=0, atol=0)


@pytest.mark.parametrize("K", [1024, 9728])
def test_wide_graph_replays_match_eager(K):
    """Pack, multiply and clear under HIP graph capture (K = 9728: the planned K splits, with
    the reduce kernel adding and clearing the partials): every replay (with eager work and a
    synchronization between replays) matches the eager result bit for bit."""
    from kernels import quant_ops as ops
    M, N = 1024, 2560
    case(f"wide graph replays M={M} N={N} K={K} plan={wide_plan(M, N, K)}")
    assert wide_plan(M, N, K)[1] == (1 if K == 1024 else 3)
    w = make_w(N, K, 96)
    q = O.int4_quantize(w, 128)
    qd, sd, zd = (q[k].to(DEV) for k in ("qweight", "scale", "zero"))
    x = make_x(M, K, 97).to(DEV)
    eager = ops.w4a16_linear(x, qd, sd, zd)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.w4a16_linear(x, qd, sd, zd)  # workspace for this stream exists before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            y = ops.w4a16_linear(x, qd, sd, zd)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(y, eager, rtol=0, atol=0)
        _ = (x * 2).sum().item()  # eager work between replays
    with torch.cuda.stream(s):
        assert workspace_is_zero()


@pytest.mark.parametrize("symmetric,sdt", [(False, torch.bfloat16), (True, torch.bfloat16), (False, torch.float16),
                                           (True, torch.float16), (False, torch.float32), (True, torch.float32)])
def test_wide_weights_are_the_references_bit_for_bit(symmetric, sdt):
    """With one-hot activation rows (x = the first M rows of the identity) every output is one
    dequantized weight times 1, so y = W^T exactly: the wide kernel's bf16 weights must equal
    the reference's dequantize (int4_wo.py:33-42, in the scale dtype's arithmetic) rounded
    to bf16 for the matmul (base.py:20-24), bit for bit."""
    from kernels import quant_ops as ops
    M, N, K, group = 1024, 2560, 1024, 128
    case(f"wide weights bit-exact sym={symmetric} {sdt}")
    w = make_w(N, K, 98)
    q = O.int4_quantize_symmetric(w, group, sdt) if symmetric else O.int4_quantize(w, group, sdt)
    w_ref = O.int4_dequantize(q["qweight"], q["scale"], q.get("zero")).to(torch.bfloat16)
    x = torch.eye(K, dtype=torch.bfloat16)[:M]
    y = ops.w4a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV),
                         None if symmetric else q["zero"].to(DEV)).cpu()
    assert torch.equal(y.view(torch.int16), w_ref.t()[:M].contiguous().view(torch.int16))
