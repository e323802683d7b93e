"""moe_align (HIP) and the fused INT4 MoE layer vs the CPU oracle."""
import pytest
import torch

from oracle import moe as MO
from oracle import quant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


def rel_error(a, b):
    return ((a.float().cpu() - b.float().cpu()).norm() / b.float().cpu().norm().clamp(min=1e-12)).item()


@pytest.mark.parametrize("T,k,E,bm", [(1, 8, 64, 16), (13, 3, 8, 4), (16, 8, 64, 16), (300, 8, 64, 32),
                                       (4096, 8, 64, 64), (64, 8, 64, 16)])
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("path", ["auto", "scan"])
def test_moe_align_matches_oracle_exactly(T, k, E, bm, dtype, path, miq_env):
    """The HIP kernel places pairs in ascending order inside each expert, so its output
    equals the oracle's stable restatement element for element (a stronger check than the
    grouping equality of reference tests/test_fused_moe.py:56-88). "auto" takes the
    per-chunk kernel where its tables fit in LDS (all but T=4096 here), "scan" forces the
    one-wavefront-per-expert kernel."""
    from kernels.fused_moe import moe_align
    if path == "scan":
        miq_env("MIQ_MOE_ALIGN_SCAN", "1")
    case(f"moe_align T={T} k={k} E={E} bm={bm} {dtype} {path}")
    g = torch.Generator().manual_seed(T)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(dtype)
    s, e, n = moe_align(ids.to(DEV), E, bm)
    ws, we, wn = MO.moe_align(ids, E, bm)
    assert torch.equal(s.cpu(), ws) and torch.equal(e.cpu(), we) and torch.equal(n.cpu(), wn)


def routed(T, H, E, k, seed):
    """bench/micro/bench_moe.py:113-117: softmax over a bf16 router, top-k, no renorm."""
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(T, H, generator=g).to(torch.bfloat16)
    router = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    probs = torch.softmax(hidden.float() @ router.float().t(), dim=-1)
    w, idx = torch.topk(probs, k, dim=-1)
    return hidden, w.to(torch.bfloat16), idx


@pytest.mark.parametrize("T,H,I,E,k,sym,group", [(64, 2048, 1024, 64, 8, False, 128), (64, 2048, 1024, 64, 8, True, 128),
                                                   (1, 2048, 1024, 64, 8, False, 128), (5, 256, 128, 8, 2, False, 128),
                                                   (33, 512, 256, 6, 3, True, 128), (40, 2048, 1024, 16, 4, False, 256),
                                                   (24, 4096, 512, 8, 2, True, 128), (24, 1024, 512, 8, 2, False, 512)])
def test_fused_int4_moe_matches_reference(T, H, I, E, k, sym, group):
    """Scales of the streaming kernels come from LDS where a row has 4, 8, 12 or 16 groups
    (the first six shapes' gate/up; H = 4096 with 32 groups, 2-group rows and group 512
    take the per-step scale loads)."""
    from kernels.fused_moe import fused_moe_int4
    case(f"fused int4 moe T={T} H={H} I={I} E={E} k={k} sym={sym} group={group}")
    g = torch.Generator().manual_seed(7)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    qf = O.int4_quantize_symmetric if sym else O.int4_quantize
    gu, dn = qf(wgu, group), qf(wdn, group)
    hidden, w, idx = routed(T, H, E, k, seed=8)
    want = MO.int4_experts_reference(hidden, gu, dn, w, idx)
    got = fused_moe_int4(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                         None if sym else gu["zero"].to(DEV), dn["qweight"].to(DEV), dn["scale"].to(DEV),
                         None if sym else dn["zero"].to(DEV))
    assert got.dtype == torch.bfloat16 and got.shape == (T, H)
    assert rel_error(got, want) < 2e-2
    err = (got.float().cpu() - want).abs()
    assert (err <= 1e-2 + 2e-2 * want.abs()).all(), err.max().item()


def test_quant_experts_module_uses_fused_path():
    """QuantExperts (modules.py:36-78) on the device: fused INT4 path vs the module's own
    per-expert loop with the int4 method, and vs the oracle."""
    from engine.quantization import get_method
    from engine.quantization.modules import QuantExperts
    case("QuantExperts fused vs loop")

    class Experts(torch.nn.Module):
        def __init__(self, E, H, I):
            super().__init__()
            g = torch.Generator().manual_seed(9)
            self.gate_up_proj = torch.nn.Parameter((torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16))
            self.down_proj = torch.nn.Parameter((torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16))
            self.act_fn = torch.nn.SiLU()

    E, H, I, T, k = 16, 512, 256, 24, 4
    ex = Experts(E, H, I).to(DEV)
    qe = QuantExperts(ex, get_method("int4_wo", device=DEV, group_size=128))
    hidden, w, idx = routed(T, H, E, k, seed=10)
    hd, wd, idd = hidden.to(DEV), w.to(DEV), idx.to(DEV)
    assert qe._fused_ok(hd)
    fused = qe(hd, idd, wd)
    class Silu(torch.nn.Module):  # not an nn.SiLU instance -> the reference loop runs
        def forward(self, t):
            return torch.nn.functional.silu(t)

    qe.act_fn = Silu()
    assert not qe._fused_ok(hd)
    loop = qe(hd, idd, wd)
    assert rel_error(fused, loop) < 2e-2
    gu = {kk: getattr(qe, f"gate_up_{kk}").cpu() for kk in ("qweight", "scale", "zero")}
    dn = {kk: getattr(qe, f"down_{kk}").cpu() for kk in ("qweight", "scale", "zero")}
    want = MO.int4_experts_reference(hidden, gu, dn, w, idx)
    assert rel_error(fused, want) < 2e-2


@pytest.mark.parametrize("sym", [False, True])
def test_fused_moe_fp32_routing_weights_vs_reference_loop(sym):
    """Routing weights in fp32 (a router that keeps fp32 probabilities): the fused layer uses
    them in their own dtype, as the reference loop multiplies by them (modules.py:55-75),
    and adds each token's expert contributions in ascending expert order with a bf16
    rounding after each addition (index_add_ into a bf16 output). Against the reference
    loop with the reference's own INT4 formula (dequantize to bf16, then F.linear), every
    element lies within the loop's own distance to the exact fp32 experts plus the
    north-star tolerance; the distance of each to the exact reference is printed."""
    from kernels.fused_moe import fused_moe_int4
    case(f"fused int4 moe fp32 weights sym={sym}")
    T, H, I, E, k = 64, 2048, 1024, 64, 8
    g = torch.Generator().manual_seed(11)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    qf = O.int4_quantize_symmetric if sym else O.int4_quantize
    gu, dn = qf(wgu, 128), qf(wdn, 128)
    hidden, _, idx = routed(T, H, E, k, seed=12)
    router = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    w32 = torch.softmax(hidden.float() @ router.float().t(), dim=-1).gather(1, idx)  # fp32 weights
    loop = MO.quant_experts_loop(hidden, O.int4_linear, gu, dn, idx, w32, E).float()
    exact = MO.int4_experts_reference(hidden, gu, dn, w32, idx)
    got = fused_moe_int4(hidden.to(DEV), idx.to(DEV), w32.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                         None if sym else gu["zero"].to(DEV), dn["qweight"].to(DEV), dn["scale"].to(DEV),
                         None if sym else dn["zero"].to(DEV)).float().cpu()
    d_got, d_loop = (got - exact).abs(), (loop - exact).abs()
    print(f"[bound] moe sym={sym}: max |fused - exact| {d_got.max().item():.4f}, max |loop - exact| "
          f"{d_loop.max().item():.4f}, max |fused - loop| {(got - loop).abs().max().item():.4f}", flush=True)
    assert ((got - loop).abs() <= d_loop + 1e-2 + 2e-2 * loop.abs()).all()
    assert rel_error(got, exact) < 2e-2


@pytest.mark.parametrize("T,H,I,E,k,sym", [(64, 2048, 1024, 64, 8, True), (5, 256, 128, 8, 2, False),
                                             (33, 512, 256, 6, 3, True)])
def test_fused_int4_moe_tiled_kernels(T, H, I, E, k, sym, miq_env):
    """The tiled expert kernels (one workgroup per (tile, column block), taken for shapes
    the streaming kernels do not cover; MIQ_MOE_TILED forces them) against the same
    reference as the default path."""
    from kernels.fused_moe import fused_moe_int4
    miq_env("MIQ_MOE_TILED", "1")
    case(f"fused int4 moe tiled T={T} H={H} I={I} E={E} k={k} sym={sym}")
    g = torch.Generator().manual_seed(13)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    qf = O.int4_quantize_symmetric if sym else O.int4_quantize
    gu, dn = qf(wgu, 128), qf(wdn, 128)
    hidden, w, idx = routed(T, H, E, k, seed=14)
    want = MO.int4_experts_reference(hidden, gu, dn, w, idx)
    got = fused_moe_int4(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                         None if sym else gu["zero"].to(DEV), dn["qweight"].to(DEV), dn["scale"].to(DEV),
                         None if sym else dn["zero"].to(DEV))
    assert rel_error(got, want) < 2e-2
    err = (got.float().cpu() - want).abs()
    assert (err <= 1e-2 + 2e-2 * want.abs()).all(), err.max().item()


@pytest.mark.parametrize("T,H,I,E,k", [(64, 2048, 1024, 64, 8), (5, 256, 128, 8, 2), (33, 512, 256, 6, 3),
                                       (1, 2048, 1024, 64, 8)])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_fused_int8_moe_matches_reference_loop(T, H, I, E, k, wdtype):
    """INT8 experts (Int8WeightOnly, per-row scales [E, rows, 1] in bf16): the fused layer
    against the reference loop (modules.py:55-75) with the reference's own int8 linear
    (int8_wo.py:17-21) on the same codes. Both round every expert linear, the SiLU gate,
    the routing product and each addition to bf16 at the same points; they differ only in
    fp32 summation order, so the elementwise bound is the north star's."""
    from kernels.fused_moe import fused_moe_int8
    case(f"fused int8 moe T={T} H={H} I={I} E={E} k={k} weights {wdtype}")
    g = torch.Generator().manual_seed(15)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    gu, dn = O.int8_quantize(wgu), O.int8_quantize(wdn)
    hidden, w, idx = routed(T, H, E, k, seed=16)
    if wdtype == torch.float32:
        router = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
        w = torch.softmax(hidden.float() @ router.float().t(), dim=-1).gather(1, idx)
    loop = MO.quant_experts_loop(hidden, O.int8_linear, gu, dn, idx, w, E).float()
    got = fused_moe_int8(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                         dn["qweight"].to(DEV), dn["scale"].to(DEV)).float().cpu()
    err = (got - loop).abs()
    print(f"[bound] int8 moe T={T} {wdtype}: max |fused - reference loop| {err.max().item():.4f}", flush=True)
    assert rel_error(got, loop) < 1e-2
    assert (err <= 1e-2 + 2e-2 * loop.abs()).all(), err.max().item()


def _fp8_native_linear(x, qweight, scale):
    """FP8WeightAct.linear on a native device (fp8.py:48-61): per-row activation quantize,
    then torch._scaled_mm's fp32 product times both scales, rounded to the input dtype."""
    x2d = x.reshape(-1, x.shape[-1])
    x_fp8, x_scale = O.fp8_quantize_activation(x2d)
    return O.fp8_scaled_mm(x_fp8, x_scale, qweight, scale).to(x.dtype).reshape(*x.shape[:-1], -1)


@pytest.mark.parametrize("T,H,I,E,k", [(64, 2048, 1024, 64, 8), (5, 256, 128, 8, 2), (33, 512, 256, 6, 3),
                                       (1, 2048, 1024, 64, 8), (40, 1024, 2048, 16, 4), (12, 4096, 1536, 8, 2),
                                       (9, 1152, 4096, 4, 2), (7, 384, 256, 4, 2)])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_fused_fp8_moe_matches_reference_loop(T, H, I, E, k, wdtype):
    """FP8 experts (FP8WeightAct: e4m3fn codes, fp32 per-row scales): the fused layer
    against the reference loop (modules.py:55-75) with the native FP8 linear on the same
    codes. The activation codes and scales are the reference's exactly; the products
    differ in fp32 summation order, and a gate/up output one bf16 step apart can move a
    down-projection activation code, so the bound is the INT8 layer's."""
    from kernels.fused_moe import fused_moe_fp8
    case(f"fused fp8 moe T={T} H={H} I={I} E={E} k={k} weights {wdtype}")
    g = torch.Generator().manual_seed(25)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    gu, dn = O.fp8_quantize(wgu), O.fp8_quantize(wdn)
    hidden, w, idx = routed(T, H, E, k, seed=26)
    if wdtype == torch.float32:
        router = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
        w = torch.softmax(hidden.float() @ router.float().t(), dim=-1).gather(1, idx)
    loop = MO.quant_experts_loop(hidden, _fp8_native_linear, gu, dn, idx, w, E).float()
    got = fused_moe_fp8(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                        dn["qweight"].to(DEV), dn["scale"].to(DEV)).float().cpu()
    err = (got - loop).abs()
    print(f"[bound] fp8 moe T={T} {wdtype}: max |fused - reference loop| {err.max().item():.4f}, "
          f"rel {rel_error(got, loop):.2e}", flush=True)
    assert rel_error(got, loop) < 1e-2
    assert (err <= 1e-2 + 2e-2 * loop.abs()).all(), err.max().item()


def test_fused_fp8_moe_padding_ids_and_empty_tokens():
    """Slots routed to expert id E add nothing; a token with every slot padded gets zeros."""
    from kernels.fused_moe import fused_moe_fp8
    case("fused fp8 moe padding ids")
    T, H, I, E, k = 48, 512, 256, 8, 4
    g = torch.Generator().manual_seed(27)
    gu = O.fp8_quantize((torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16))
    dn = O.fp8_quantize((torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16))
    hidden, w, idx = routed(T, H, E, k, seed=28)
    idx = idx.clone()
    idx[::3, 0] = E
    idx[1::7, :] = E
    loop = MO.quant_experts_loop(hidden, _fp8_native_linear, gu, dn, idx, w, E).float()
    got = fused_moe_fp8(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                        dn["qweight"].to(DEV), dn["scale"].to(DEV)).float().cpu()
    assert (got[1::7] == 0).all()
    assert rel_error(got, loop) < 1e-2


def test_quant_experts_int8_takes_the_fused_path():
    """QuantExperts with Int8WeightOnly on the device runs the fused kernels (no host loop)
    and matches its own grouped per-expert path."""
    from engine.quantization import get_method
    from engine.quantization.modules import QuantExperts
    case("QuantExperts int8 fused vs grouped")

    class Experts(torch.nn.Module):
        def __init__(self, E, H, I):
            super().__init__()
            g = torch.Generator().manual_seed(17)
            self.gate_up_proj = torch.nn.Parameter((torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16))
            self.down_proj = torch.nn.Parameter((torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16))
            self.act_fn = torch.nn.SiLU()

    E, H, I, T, k = 16, 512, 256, 24, 4
    qe = QuantExperts(Experts(E, H, I).to(DEV), get_method("int8_wo", device=DEV))
    hidden, w, idx = routed(T, H, E, k, seed=18)
    hd, wd, idd = hidden.to(DEV), w.to(DEV), idx.to(DEV)
    assert qe._fused_ok(hd)
    fused = qe(hd, idd, wd)
    grouped = qe._grouped(hd, idd, wd)
    assert rel_error(fused, grouped) < 1e-2


def test_quant_experts_fp8_takes_the_fused_path():
    """QuantExperts with native FP8WeightAct on the device runs the fused kernels (no host
    loop) and matches its own grouped per-expert path (method.linear per expert)."""
    from engine.quantization import get_method
    from engine.quantization.modules import QuantExperts
    case("QuantExperts fp8 fused vs grouped")

    class Experts(torch.nn.Module):
        def __init__(self, E, H, I):
            super().__init__()
            g = torch.Generator().manual_seed(29)
            self.gate_up_proj = torch.nn.Parameter((torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16))
            self.down_proj = torch.nn.Parameter((torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16))
            self.act_fn = torch.nn.SiLU()

    E, H, I, T, k = 16, 512, 256, 24, 4
    qe = QuantExperts(Experts(E, H, I).to(DEV), get_method("fp8", device=DEV))
    hidden, w, idx = routed(T, H, E, k, seed=30)
    hd, wd, idd = hidden.to(DEV), w.to(DEV), idx.to(DEV)
    assert qe._fused_ok(hd)
    fused = qe(hd, idd, wd)
    grouped = qe._grouped(hd, idd, wd)
    assert rel_error(fused, grouped) < 1e-2


@pytest.mark.parametrize("kind,k,tiled", [("int4", 8, False), ("int4", 8, True), ("int4", 12, False),
                                          ("int8", 8, False)])
def test_fused_moe_padding_expert_id(kind, k, tiled, miq_env):
    """Slots routed to expert id E (the reference loop's padding class, one_hot with E + 1
    classes, modules.py:55-75) contribute nothing; the other slots of the same token are
    still added in ascending expert order. k = 12 takes the combine's 16-slot variant."""
    from kernels.fused_moe import fused_moe_int4, fused_moe_int8
    if tiled:
        miq_env("MIQ_MOE_TILED", "1")
    case(f"fused {kind} moe with padding ids k={k} tiled={tiled}")
    T, H, I, E = 40, 512, 256, 16
    g = torch.Generator().manual_seed(17)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    hidden, w, idx = routed(T, H, E, k, seed=18)
    idx = idx.clone()
    idx[::3, 0] = E       # one padding slot in every third token
    idx[1::7, :] = E      # tokens with every slot padded: output zero
    if kind == "int4":
        gu, dn = O.int4_quantize(wgu, 128), O.int4_quantize(wdn, 128)
        loop = MO.quant_experts_loop(hidden, O.int4_linear, gu, dn, idx, w, E).float()
        got = fused_moe_int4(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                             gu["zero"].to(DEV), dn["qweight"].to(DEV), dn["scale"].to(DEV), dn["zero"].to(DEV))
    else:
        gu, dn = O.int8_quantize(wgu), O.int8_quantize(wdn)
        loop = MO.quant_experts_loop(hidden, O.int8_linear, gu, dn, idx, w, E).float()
        got = fused_moe_int8(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                             dn["qweight"].to(DEV), dn["scale"].to(DEV))
    got = got.float().cpu()
    assert (got[1::7] == 0).all()
    err = (got - loop).abs()
    print(f"[bound] {kind} moe padding ids: max |fused - reference loop| {err.max().item():.4f}", flush=True)
    assert rel_error(got, loop) < 2e-2
    assert (err <= 2e-2 + 3e-2 * loop.abs()).all(), err.max().item()


@pytest.mark.parametrize("T,H,I,E,k,sym,env", [(64, 2048, 1024, 64, 8, True, "MIQ_MOE_WAVES"),
                                               (33, 512, 256, 6, 3, False, "MIQ_MOE_WAVES"),
                                               (64, 2048, 1024, 64, 8, False, "MIQ_MOE_LDS_SCALES"),
                                               (24, 384, 256, 8, 2, True, None)])
def test_fused_int4_moe_streaming_variants(T, H, I, E, k, sym, env, miq_env):
    """The streaming expert kernels' other layouts: four wavefronts per workgroup
    (MIQ_MOE_WAVES=4; also taken without the switch by the down GEMM when H is not a
    multiple of 256, as in the last shape, H = 384) and per-k-step scale loads
    (MIQ_MOE_LDS_SCALES=0)."""
    from kernels.fused_moe import fused_moe_int4
    if env == "MIQ_MOE_WAVES":
        miq_env(env, "4")
    elif env:
        miq_env(env, "0")
    case(f"fused int4 moe variant {env} T={T} H={H} I={I} E={E} k={k} sym={sym}")
    g = torch.Generator().manual_seed(19)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    qf = O.int4_quantize_symmetric if sym else O.int4_quantize
    gu, dn = qf(wgu, 128), qf(wdn, 128)
    hidden, w, idx = routed(T, H, E, k, seed=20)
    want = MO.int4_experts_reference(hidden, gu, dn, w, idx)
    got = fused_moe_int4(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                         None if sym else gu["zero"].to(DEV), dn["qweight"].to(DEV), dn["scale"].to(DEV),
                         None if sym else dn["zero"].to(DEV))
    assert rel_error(got, want) < 2e-2
    err = (got.float().cpu() - want).abs()
    assert (err <= 1e-2 + 2e-2 * want.abs()).all(), err.max().item()


@pytest.mark.parametrize("kind,sdt", [("int4", torch.float32), ("int4", torch.float16), ("int8", torch.float32),
                                      ("int8", torch.float16)])
def test_fused_moe_scale_dtypes(kind, sdt):
    """Scales (and zero points) in fp32 (INT4: the per-k-step scale loads; 16-bit scales take
    the LDS slots) and fp16, against the same references as the bf16 tests."""
    from kernels.fused_moe import fused_moe_int4, fused_moe_int8
    case(f"fused {kind} moe with {sdt} scales")
    T, H, I, E, k = 24, 1024, 512, 8, 2
    g = torch.Generator().manual_seed(21)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    hidden, w, idx = routed(T, H, E, k, seed=22)
    if kind == "int4":
        gu, dn = O.int4_quantize(wgu, 128, sdt), O.int4_quantize(wdn, 128, sdt)
        want = MO.int4_experts_reference(hidden, gu, dn, w, idx)
        got = fused_moe_int4(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                             gu["zero"].to(DEV), dn["qweight"].to(DEV), dn["scale"].to(DEV), dn["zero"].to(DEV))
        err = (got.float().cpu() - want).abs()
        assert (err <= 1e-2 + 2e-2 * want.abs()).all(), err.max().item()
    else:
        gu, dn = O.int8_quantize(wgu, sdt), O.int8_quantize(wdn, sdt)
        loop = MO.quant_experts_loop(hidden, O.int8_linear, gu, dn, idx, w, E).float()
        got = fused_moe_int8(hidden.to(DEV), idx.to(DEV), w.to(DEV), gu["qweight"].to(DEV), gu["scale"].to(DEV),
                             dn["qweight"].to(DEV), dn["scale"].to(DEV)).float().cpu()
        err = (got - loop).abs()
        assert (err <= 1e-2 + 2e-2 * loop.abs()).all(), err.max().item()


@pytest.mark.parametrize("kind", ["int4", "int8", "fp8"])
@pytest.mark.parametrize("T,H,I,E,k,pad", [(64, 2048, 1024, 64, 8, False), (5, 256, 128, 8, 2, True),
                                           (33, 512, 256, 6, 3, True), (160, 256, 128, 64, 8, False),
                                           (3, 256, 128, 300, 4, False), (128, 256, 128, 256, 8, True)])
@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_routed_layer_equals_align_then_layer(kind, T, H, I, E, k, pad, ids_dtype, miq_env):
    """The routed entry points (the expert GEMMs align the pairs in LDS, no align launch)
    give the same bytes as moe_align followed by the layer: 1024 pairs and 256 experts (the
    LDS tables' limits, (128, .., 256, 8)) and beyond them (160 tokens of 8 slots, 300
    experts: moe_align runs inside the call), with padding ids, and with the in-LDS path
    switched off (MIQ_MOE_ALIGN_LAUNCH)."""
    from kernels.fused_moe import fused_moe_fp8, fused_moe_int4, fused_moe_int8
    case(f"routed {kind} moe T={T} H={H} I={I} E={E} k={k} pad={pad} ids {ids_dtype}")
    g = torch.Generator().manual_seed(41)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    wdn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    hidden, w, idx = routed(T, H, E, k, seed=42)
    idx = idx.clone()
    if pad:
        idx[::3, 0] = E
        idx[1::7, :] = E
    idx = idx.to(ids_dtype)
    if kind == "int4":
        gu, dn = O.int4_quantize(wgu, 128), O.int4_quantize(wdn, 128)
        args = [gu["qweight"], gu["scale"], gu["zero"], dn["qweight"], dn["scale"], dn["zero"]]
        fn = fused_moe_int4
    elif kind == "int8":
        gu, dn = O.int8_quantize(wgu), O.int8_quantize(wdn)
        args = [gu["qweight"], gu["scale"], dn["qweight"], dn["scale"]]
        fn = fused_moe_int8
    else:
        gu, dn = O.fp8_quantize(wgu), O.fp8_quantize(wdn)
        args = [gu["qweight"], gu["scale"], dn["qweight"], dn["scale"]]
        fn = fused_moe_fp8
    dev_args = [hidden.to(DEV), idx.to(DEV), w.to(DEV)] + [a.to(DEV) for a in args]
    want = fn(*dev_args, routed=False)
    got = fn(*dev_args)
    again = fn(*dev_args)
    miq_env("MIQ_MOE_ALIGN_LAUNCH", "1")
    launched = fn(*dev_args)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(again, want) and torch.equal(launched, want)
