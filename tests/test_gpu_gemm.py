"""Weight-only skinny GEMMs and the FP8 GEMM vs the fp32-accumulated CPU oracle.

Tolerance: |got - want| <= 1e-2 + 2e-2 * |want| elementwise,
want = the fp32-accumulated product on the dequantized weights evaluated in fp32
(q * s + z exactly, as the kernels do). The reference's own bf16 formula
(int4_wo.py:33-42 + base.py:20-24) rounds every dequantized weight to bf16 twice; at
K = 9728 that alone moves outputs by up to ~0.04, so it is held to the norm-wise bound of
the reference's test (tests/test_quantizaton.py:60-72, rel < 0.01), and the kernel output
is checked against the reference formula to that same bound.
"""
import pytest
import torch

from oracle import quant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL, RTOL = 1e-2, 2e-2


def case(msg):
    print(f"[case] {msg}", flush=True)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def within(got, want, atol=ATOL, rtol=RTOL):
    got = got.float().cpu()
    want = want.float().cpu()
    err = (got - want).abs()
    bound = atol + rtol * want.abs()
    worst = (err - bound).max().item()
    assert worst <= 0, f"max excess {worst:.3e}, max abs err {err.max().item():.3e}"


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm()).item()


def make_x(M, K, seed):
    return torch.randn(M, K, generator=gen(seed)).to(torch.bfloat16)


def make_w(N, K, seed, std=0.02):
    return (torch.randn(N, K, generator=gen(seed)) * std).to(torch.bfloat16)


INT8_SHAPES = [(1, 64, 256), (3, 128, 512), (8, 192, 384), (16, 64, 1024), (17, 64, 256), (32, 512, 2560),
               (64, 256, 640), (1, 19456, 2560), (8, 19456, 2560), (32, 19456, 2560), (64, 19456, 2560)]


@pytest.mark.parametrize("M,N,K", INT8_SHAPES)
def test_w8a16_gemm(M, N, K):
    from kernels import quant_ops as ops
    case(f"w8a16 M={M} N={N} K={K}")
    w = make_w(N, K, 10)
    x = make_x(M, K, 11)
    q = O.int8_quantize(w)
    want = O.int8_linear_fp32(x, **q)
    y = ops.w8a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV))
    assert y.dtype == torch.bfloat16 and y.shape == (M, N)
    within(y, want)
    within(O.int8_linear(x, **q), want)  # the reference's bf16 formula meets the same bound
    assert rel(y, O.int8_linear(x, **q)) < 0.01


def test_w8a16_fp32_scale_and_strided_x():
    from kernels import quant_ops as ops
    case("w8a16 fp32 scale, strided x")
    M, N, K = 5, 256, 1024
    w = make_w(N, K, 12)
    xb = make_x(M, 2 * K, 13)
    x = xb[:, K:]
    q = O.int8_quantize(w, torch.float32)
    want = O.int8_linear_fp32(x, **q)
    y = ops.w8a16_linear(xb.to(DEV)[:, K:], q["qweight"].to(DEV), q["scale"].to(DEV))
    within(y, want)


@pytest.mark.parametrize("M", [1, 8, 32, 64])
def test_w8a16_config1_fp32_scales(M):
    """BASELINE config 1 exactly: fused gate/up N = 19456, K = 2560, fp32 per-row scales
    (the form bench.py times), every M of the configuration."""
    from kernels import quant_ops as ops
    case(f"w8a16 config 1 fp32 scales M={M}")
    N, K = 19456, 2560
    w = (torch.randn(N, K, generator=gen(20)) * 0.02)
    x = make_x(M, K, 21)
    q = O.int8_quantize(w, torch.float32)
    assert q["scale"].dtype == torch.float32
    want = O.int8_linear_fp32(x, **q)
    y = ops.w8a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV))
    assert y.dtype == torch.bfloat16 and y.shape == (M, N)
    within(y, want)
    assert rel(y, O.int8_linear(x, **q)) < 0.01


INT4_SHAPES = [(1, 64, 256, 128), (5, 128, 512, 128), (8, 64, 1024, 256), (16, 192, 384, 128),
               (33, 64, 512, 128), (64, 128, 768, 128), (1, 2560, 9728, 128), (8, 2560, 9728, 128),
               (32, 2560, 9728, 128), (64, 2560, 9728, 128),
               # large groups (a group spans several chunks / the whole split range), ragged N
               (64, 256, 4096, 1024), (20, 144, 2048, 2048), (1, 512, 8192, 4096), (40, 80, 1024, 256),
               # odd k-step counts and 3-step groups, every activation-tile count, a ragged row block
               (17, 256, 1152, 384), (48, 1280, 9728, 128), (2, 2560, 9728, 128), (3, 2512, 1152, 128)]


PLANS = {"default": {}, "panel": {"MIQ_WO_PANEL": "1"},
         "panel_s3": {"MIQ_WO_PANEL": "1", "MIQ_WO_PANEL_S": "3"},
         "panel_s16": {"MIQ_WO_PANEL": "1", "MIQ_WO_PANEL_S": "16"},
         "panel_mt2": {"MIQ_WO_PANEL": "1", "MIQ_WO_PANEL_MT": "2"},
         "panel_mt4": {"MIQ_WO_PANEL": "1", "MIQ_WO_PANEL_MT": "4"},
         "nopanel": {"MIQ_WO_PANEL": "0"}, "tile_m1": {"MIQ_WO_GEMV_MAX_M": "0"},
         "msplit_4_3": {"MIQ_WO_PANEL": "0"}, "msplit_off": {"MIQ_WO_PANEL": "0"}}


@pytest.mark.parametrize("M,N,K,group", INT4_SHAPES)
@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("plan", list(PLANS))
def test_w4a16_gemm(M, N, K, group, symmetric, plan, miq_env):
    """plan: the default; the panel kernel forced (split-K panels with a cross-workgroup
    reduction), with 3 or 16 K splits, or 2 / 4 activation tiles per workgroup; the panel
    kernel off (the tile / streamed kernels' plan), with the streamed kernel's M split
    forced to 4 weight tiles per wavefront and 3 splits, or turned off."""
    from kernels import quant_ops as ops
    for k, v in PLANS[plan].items():
        miq_env(k, v)
    if plan.startswith("msplit"):
        if M <= 16:
            pytest.skip("the M split applies to more than 16 rows")
        miq_env("MIQ_WO_MSPLIT", "4,3" if plan == "msplit_4_3" else "0,0")
    case(f"w4a16 M={M} N={N} K={K} g={group} sym={symmetric} plan={plan}")
    w = make_w(N, K, 20)
    x = make_x(M, K, 21)
    q = O.int4_quantize_symmetric(w, group) if symmetric else O.int4_quantize(w, group)
    want = O.int4_linear_fp32(x, **q)
    y = ops.w4a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV),
                         None if symmetric else q["zero"].to(DEV))
    assert y.dtype == torch.bfloat16 and y.shape == (M, N)
    within(y, want)
    ref = O.int4_linear(x, **q)
    assert rel(ref, want) < 0.01 and rel(y, ref) < 0.01


@pytest.mark.parametrize("sdt", [torch.float16, torch.float32])
def test_w4a16_scale_dtypes(sdt):
    """Scales / zeros stored as f16 or f32 (the kernels read them at storage precision)."""
    from kernels import quant_ops as ops
    case(f"w4a16 scale dtype {sdt}")
    M, N, K, group = 8, 320, 2048, 256
    w = make_w(N, K, 40)
    x = make_x(M, K, 41)
    q = O.int4_quantize(w, group)
    q["scale"], q["zero"] = q["scale"].to(sdt), q["zero"].to(sdt)
    want = O.int4_linear_fp32(x, **q)
    y = ops.w4a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV), q["zero"].to(DEV))
    within(y, want)


# Up to 16 rows whose activations fit LDS run the one-tile-per-workgroup kernel; the
# streamed split-K kernel (forced with MIQ_WO_STREAM) must give the same results there.
# Cases: multi-wavefront slices (K = 9728), an odd number of k-steps (K = 1152), groups of
# 3 k-steps, long groups, f32 scales.
# The two-half plan (32-row workgroups over half of K, from 2 rows on by default) adds: 16
# rows at the configuration's K (the largest LDS staging), N an odd number of 16-row tiles
# (the last pair holds one tile), 3 units of K (halves of 1 and 2 units).
TILE_CASES = [(1, 320, 9728, 128), (4, 320, 9728, 128), (3, 160, 1152, 128), (2, 96, 1152, 384),
              (8, 64, 4096, 512), (16, 64, 1024, 128), (7, 48, 2560, 256), (1, 2560, 9728, 128),
              (5, 3008, 2048, 128), (16, 2560, 9728, 128), (8, 2576, 9728, 128), (12, 48, 9728, 128)]
# kernel choice: the default plan (INT4: the panel kernel), the plan without the panel
# kernel, the streamed kernel, the tile kernel with a forced number of weight rows per
# tile (16, and 7: a tile whose 128-byte loads are partly empty) on one workgroup per tile,
# and the two-half plan forced from one row on
# The GEMV kernel (M = 1 by default) is switched off in the plans that test the tile
# kernel, and forced up to M = 2 in "gemv2".
_NOGEMV = {"MIQ_WO_GEMV_MAX_M": "0"}
KERNELS = {"auto": {}, "gemv2": {"MIQ_WO_GEMV_MAX_M": "2"}, "nopanel": {"MIQ_WO_PANEL": "0", **_NOGEMV},
           "stream": {"MIQ_WO_STREAM": "1"},
           "rows16": {"MIQ_WO_ROWS": "16", "MIQ_WO_PANEL": "0", "MIQ_WO_PAIR_MIN_M": "-1", **_NOGEMV},
           "rows7": {"MIQ_WO_ROWS": "7", "MIQ_WO_PANEL": "0", "MIQ_WO_PAIR_MIN_M": "-1", **_NOGEMV},
           "pair": {"MIQ_WO_PANEL": "0", "MIQ_WO_PAIR_MIN_M": "1", **_NOGEMV}}


@pytest.mark.parametrize("kernel", list(KERNELS))
@pytest.mark.parametrize("M,N,K,group", TILE_CASES)
@pytest.mark.parametrize("sdt,symmetric", [(torch.bfloat16, True), (torch.float32, False), (torch.float16, False)])
def test_w4a16_tile_and_stream(kernel, M, N, K, group, sdt, symmetric, miq_env):
    from kernels import quant_ops as ops
    case(f"w4a16 {kernel} M={M} N={N} K={K} g={group} {sdt} sym={symmetric}")
    for k, v in KERNELS[kernel].items():
        miq_env(k, v)
    w = make_w(N, K, 50)
    x = make_x(M, K, 51)
    q = O.int4_quantize_symmetric(w, group) if symmetric else O.int4_quantize(w, group)
    q["scale"] = q["scale"].to(sdt)
    if not symmetric:
        q["zero"] = q["zero"].to(sdt)
    want = O.int4_linear_fp32(x, **q)
    y = ops.w4a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV),
                         None if symmetric else q["zero"].to(DEV))
    within(y, want)


# int8 kernels: as above, plus workgroups of two row tiles over all of K (at 4 and 5 rows by
# default, forced from one row): N an odd number of 16-row tiles (2512, 1008), K = 4096
# (eight wavefronts of 4 k-steps, the most that plan holds)
KERNELS8 = dict(KERNELS, tile2={"MIQ_WO_INT8_TILE2_MIN_M": "1", **_NOGEMV},
                one_tile={"MIQ_WO_INT8_TILE2_MIN_M": "-1", **_NOGEMV})


@pytest.mark.parametrize("kernel", list(KERNELS8))
@pytest.mark.parametrize("M,N,K", [(1, 19456, 2560), (2, 4096, 2560), (3, 160, 1152), (4, 64, 9728), (1, 2512, 2560),
                                   (8, 19456, 2560), (16, 1008, 2560), (13, 2512, 1152), (5, 2512, 2560),
                                   (4, 1008, 4096)])
def test_w8a16_tile_and_stream(kernel, M, N, K, miq_env):
    from kernels import quant_ops as ops
    case(f"w8a16 {kernel} M={M} N={N} K={K}")
    for k, v in KERNELS8[kernel].items():
        miq_env(k, v)
    w = make_w(N, K, 52)
    x = make_x(M, K, 53)
    q = O.int8_quantize(w, torch.float32)
    want = O.int8_linear_fp32(x, **q)
    y = ops.w8a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV))
    within(y, want)


def test_split_k_repeated_calls_are_identical():
    """The split-K counters and the two-half plan's exchange words are left at zero:
    back-to-back calls give identical bytes."""
    from kernels import quant_ops as ops
    case("w4a16 repeated split-K calls")
    w = make_w(2560, 9728, 30)
    q = O.int4_quantize(w, 128)
    qd = {k: v.to(DEV) for k, v in q.items()}
    outs = []
    for M in (1, 8, 64, 16, 1, 8, 64, 16, 33, 33):
        x = make_x(M, 9728, 31).to(DEV)
        outs.append(ops.w4a16_linear(x, qd["qweight"], qd["scale"], qd["zero"]).cpu())
    assert all(torch.equal(outs[i], outs[i + 4]) for i in range(4)) and torch.equal(outs[8], outs[9])


@pytest.mark.parametrize("name", ["int8_wo", "int4_wo", "fp8"])
def test_methods_linear_matches_dequantized_matmul(name):
    """reference tests/test_quantizaton.py:60-72 on the device, incl. the prefill branch."""
    from engine.quantization import get_method
    case(f"method {name}.linear")
    m = get_method(name, device=DEV, compute_dtype=torch.bfloat16, group_size=128)
    w = make_w(256, 512, 40).to(DEV)
    for shape in ((2, 5, 512), (1, 512), (96, 512)):
        x = torch.randn(*shape, generator=gen(41)).to(torch.bfloat16).to(DEV)
        q = m.quantize(w)
        expected = torch.nn.functional.linear(x.float(), m.dequantize(**q).float())
        got = m.linear(x, **q)
        assert got.shape == shape[:-1] + (256,) and got.dtype == torch.bfloat16
        err = ((got.float() - expected).norm() / expected.norm()).item()
        assert err < (0.05 if name == "fp8" else 0.01), (shape, err)


@pytest.mark.parametrize("M,N,K", [(128, 128, 128), (256, 384, 512), (200, 136, 384), (2048, 6144, 2560),
                                   (1024, 1920, 2560), (7, 64, 256)])
def test_fp8_gemm(M, N, K):
    from kernels import quant_ops as ops
    case(f"fp8 gemm M={M} N={N} K={K}")
    x = torch.randn(M, K, generator=gen(50)).to(torch.bfloat16)
    w = make_w(N, K, 51)
    xq, xs = O.fp8_quantize_activation(x)
    wq = O.fp8_quantize(w)
    want = O.fp8_scaled_mm(xq, xs, **wq)
    y = ops.fp8_gemm(xq.to(DEV), xs.to(DEV), wq["qweight"].to(DEV), wq["scale"].to(DEV))
    within(y, want)


def test_fp8_linear_end_to_end():
    """FP8WeightAct.linear (activation quant kernel + MFMA GEMM) vs the oracle's formula
    (fp8.py:48-61) and the emulation bound of reference tests/test_quantizaton.py:75-88."""
    from engine.quantization import get_method
    case("fp8 linear end to end")
    m = get_method("fp8", device=DEV)
    w = make_w(6144, 2560, 52)
    x = torch.randn(64, 2560, generator=gen(53)).to(torch.bfloat16)
    q = m.quantize(w.to(DEV))
    y = m.linear(x.to(DEV), **q)
    wq = O.fp8_quantize(w)
    xq, xs = O.fp8_quantize_activation(x)
    within(y, O.fp8_scaled_mm(xq, xs, **wq))
    emu = O.fp8_linear_emulated(x, **wq)
    assert ((y.float().cpu() - emu.float()).norm() / emu.float().norm()).item() < 0.02


@pytest.mark.parametrize("M", [1, 8, 32, 64])
@pytest.mark.parametrize("symmetric", [True, False])
def test_w4a16_elementwise_vs_reference_formula(M, symmetric):
    """Config 2 (N = 2560, K = 9728, group 128): the fused kernel against the reference's
    own formula, dequantize to bf16 then F.linear (int4_wo.py:33-42, base.py:20-24),
    element by element. The kernel multiplies the exactly dequantized weights (q * s + z
    in fp32); the reference rounds each one to bf16 (twice with zero points). The two
    results therefore differ by at most |x| @ |w_ref - w_exact|^T (the weight rounding,
    computed here exactly) plus one bf16 rounding of each output and fp32 accumulation
    noise; every element must lie within that bound."""
    from kernels import quant_ops as ops
    case(f"w4a16 vs reference formula M={M} sym={symmetric}")
    N, K = 2560, 9728
    w = make_w(N, K, 60)
    x = make_x(M, K, 61)
    q = O.int4_quantize_symmetric(w, 128) if symmetric else O.int4_quantize(w, 128)
    got = ops.w4a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV),
                           None if symmetric else q["zero"].to(DEV)).float().cpu()
    ref = O.int4_linear(x, **q).float()                          # the reference's bf16 formula
    w_ref = O.int4_dequantize(**q).double()
    qs = O.int4_unpack(q["qweight"]).double().reshape(N, K // 128, 128)
    s = q["scale"].double().unsqueeze(-1)
    w_exact = ((qs - 8) * s if symmetric else qs * s + q["zero"].double().unsqueeze(-1)).reshape(N, K)
    xd = x.double()
    explained = xd.abs() @ (w_ref - w_exact).abs().t()
    bound = explained + 2.0 ** -8 * (got.abs() + ref.abs()).double() + 1e-3
    diff = (got.double() - ref.double()).abs()
    print(f"[bound] M={M} sym={symmetric}: max |kernel - reference| {diff.max().item():.4f}, "
          f"max of diff / bound {(diff / bound).max().item():.3f}", flush=True)
    assert (diff <= bound).all()


@pytest.mark.parametrize("variant", ["default", "four_waves", "previous_family", "strided_y"])
def test_fp8_gemm_kernel_variants(variant, miq_env):
    """Every FP8 kernel the dispatcher can reach at the large-tile shapes: the 8-wavefront
    256x192 kernel (default), its 4-wavefront layout (MIQ_FP8_WAVES=4), the previous
    256x192 family (MIQ_FP8_OLD, also taken for an output whose row stride is not a
    multiple of 8), and a strided output through the C ABI (ldy = N + 4)."""
    from kernels import _lib as L
    from kernels import quant_ops as ops
    case(f"fp8 gemm variant {variant}")
    if variant == "four_waves":
        miq_env("MIQ_FP8_WAVES", "4")
    if variant == "previous_family":
        miq_env("MIQ_FP8_OLD", "1")
    M, N, K = 1024, 1920, 2560
    x = torch.randn(M, K, generator=gen(54)).to(torch.bfloat16)
    w = make_w(N, K, 55)
    xq, xs = O.fp8_quantize_activation(x)
    wq = O.fp8_quantize(w)
    want = O.fp8_scaled_mm(xq, xs, **wq)
    if variant != "strided_y":
        y = ops.fp8_gemm(xq.to(DEV), xs.to(DEV), wq["qweight"].to(DEV), wq["scale"].to(DEV))
    else:
        ldy = N + 4
        buf = torch.full((M, ldy), -7.0, dtype=torch.bfloat16, device=DEV)
        xd, wd = xq.to(DEV).contiguous(), wq["qweight"].to(DEV).contiguous()
        xsd, wsd = xs.reshape(-1).float().to(DEV), wq["scale"].reshape(-1).float().to(DEV)
        L.call("miq_fp8_gemm", L.ptr(xd), L.ptr(xsd), L.ptr(wd), L.ptr(wsd), L.ptr(buf), ldy, M, N, K,
               L.stream(buf.device))
        torch.cuda.synchronize()
        assert (buf[:, N:] == -7.0).all()  # the padding columns are not written
        y = buf[:, :N]
    within(y, want)


PREFILL_SHAPES = [(65, 256, 512, 128), (96, 320, 1152, 384), (200, 2560, 9728, 128), (130, 144, 2048, 1024),
                  (257, 512, 1024, 256), (1300, 2560, 512, 128)]


def workspace_is_zero():
    """The split-K workspace is all zeros between calls (the decode kernels that share it
    read a non-zero partial word as pending)."""
    from kernels import _lib as L
    torch.cuda.synchronize()
    ws = L.wo_workspace(torch.device("cuda", torch.cuda.current_device()), 0)
    return int(ws.count_nonzero().item()) == 0


@pytest.mark.parametrize("M,N,K,group", PREFILL_SHAPES)
@pytest.mark.parametrize("symmetric", [False, True])
def test_w4a16_prefill(M, N, K, group, symmetric):
    """M > 64 (prefill): the dequantize-in-the-K-loop MFMA GEMM, ragged M and N, groups of
    1 to 8 k-steps, odd k-step counts."""
    from kernels import quant_ops as ops
    case(f"w4a16 prefill M={M} N={N} K={K} g={group} sym={symmetric}")
    w = make_w(N, K, 80)
    x = make_x(M, K, 81)
    q = O.int4_quantize_symmetric(w, group) if symmetric else O.int4_quantize(w, group)
    want = O.int4_linear_fp32(x, **q)
    y = ops.w4a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV), None if symmetric else q["zero"].to(DEV))
    assert y.shape == (M, N)
    from test_gpu_wide import int4_ref_weights_product, wide_planned
    if wide_planned(M, N, K):  # the wide kernel multiplies the reference's bf16 weights
        within(y, int4_ref_weights_product(x, q))
        assert rel(y, want) < 0.01
    else:
        within(y, want)
    assert workspace_is_zero()


@pytest.mark.parametrize("M,N,K", [(65, 256, 512), (200, 19456, 2560), (129, 144, 1152), (300, 512, 2560),
                                   (96, 2560, 9728)])
@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float32])
def test_w8a16_prefill(M, N, K, sdt):
    from kernels import quant_ops as ops
    case(f"w8a16 prefill M={M} N={N} K={K} {sdt}")
    w = make_w(N, K, 82)
    x = make_x(M, K, 83)
    q = O.int8_quantize(w, sdt)
    want = O.int8_linear_fp32(x, **q)
    y = ops.w8a16_linear(x.to(DEV), q["qweight"].to(DEV), q["scale"].to(DEV))
    within(y, want)
    assert rel(y, O.int8_linear(x, **q)) < 0.01
    assert workspace_is_zero()
