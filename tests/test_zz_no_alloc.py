"""miq_w4a16_gemm_noalloc (the entry point that allocates nothing: its split-K scratch is a
static device array) against miq_w4a16_gemm with a caller workspace, through the C ABI.
Both run the same kernels with the same plans, so the outputs must be identical bytes;
two calls in a row, the second smaller, then the first again (the scratch is left clean)."""
import ctypes

import pytest
import torch

from oracle import quant as O
from test_gpu_wide import int4_ref_weights_product, wide_planned

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


def operands(M, N, K, group, symmetric, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    q = O.int4_quantize_symmetric(w, group) if symmetric else O.int4_quantize(w, group)
    return x.to(DEV), {k: v.to(DEV) for k, v in q.items()}


def noalloc(x, q, group):
    from kernels import _lib as L
    M, K = x.shape
    N = q["qweight"].shape[0]
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    z = q.get("zero")
    rc = L.load().miq_w4a16_gemm_noalloc(
        L.ptr(x), x.stride(0), L.ptr(q["qweight"]), L.ptr(q["scale"]), L.ptr(z), L.dtype_code(q["scale"].dtype),
        group, L.ptr(y), y.stride(0), M, N, K, L.stream(x.device))
    return rc, y


def with_workspace(x, q):
    from kernels import quant_ops as ops
    return ops.w4a16_linear(x, q["qweight"], q["scale"], q.get("zero"))


def test_noalloc_matches_workspace_entry_point():
    # (M, N, K, group, symmetric): the panel kernel with its largest scratch at config 2, the
    # wide kernel with 10 K splits (200 rows: packed activations and fp32 partials, 24.3 MiB,
    # in the scratch and cleared again), the wide kernel unsplit (1024 rows, 2 MiB), a
    # smaller panel launch, two tile-kernel launches of the two-half plan (exchange words in
    # the scratch), then the first shape again
    shapes = [(64, 2560, 9728, 128, True), (200, 2560, 9728, 128, False), (1024, 2560, 1024, 128, False),
              (40, 1280, 4096, 256, False), (16, 2560, 9728, 128, True), (8, 512, 1024, 128, False),
              (64, 2560, 9728, 128, True)]
    for i, (M, N, K, group, sym) in enumerate(shapes):
        case(f"noalloc call {i}: M={M} N={N} K={K} g={group} sym={sym}")
        x, q = operands(M, N, K, group, sym, seed=70 + (i % 3))
        rc, y = noalloc(x, q, group)
        assert rc == 0
        want = with_workspace(x, q)
        torch.cuda.synchronize()
        assert torch.equal(y, want), (y.float() - want.float()).abs().max().item()
        # and within the north-star tolerance of the fp32 oracle: the exactly dequantized
        # weights, or for the wide kernel the reference's own bf16 weights (test_gpu_wide)
        qc = {k: v.cpu() for k, v in q.items()}
        ref = (int4_ref_weights_product(x.cpu(), qc) if M > 64 and wide_planned(M, N, K)
               else O.int4_linear_fp32(x.cpu(), **qc))
        err = (y.float().cpu() - ref).abs()
        assert (err <= 1e-2 + 2e-2 * ref.abs()).all()


def test_noalloc_large_prefill_takes_the_prefill_kernel():
    """2048 x 9728 activations: the wide kernel's plan (a 40 MiB packed copy and two K
    splits' fp32 partials, 83 MiB in all) would not fit the 32 MiB scratch, so the entry point runs the prefill kernel (split-K partials within the
    scratch) where the workspace entry point runs the wide kernel: both within the
    north-star tolerance of the fp32 oracle, and the scratch left clean for the next call."""
    M, N, K, group = 2048, 2560, 9728, 128
    case(f"noalloc M={M} N={N} K={K}: prefill kernel in place of the wide one")
    x, q = operands(M, N, K, group, False, seed=75)
    rc, y = noalloc(x, q, group)
    assert rc == 0
    qc = {k: v.cpu() for k, v in q.items()}
    exact = O.int4_linear_fp32(x.cpu(), **qc)  # the prefill kernel multiplies exact weights
    ref_w = int4_ref_weights_product(x.cpu(), qc)  # the wide kernel: the reference's bf16 weights
    for got, want in ((y, exact), (with_workspace(x, q), ref_w)):
        err = (got.float().cpu() - want).abs()
        assert (err <= 1e-2 + 2e-2 * want.abs()).all()
    x, q = operands(16, 2560, 9728, 128, True, seed=76)
    rc, y = noalloc(x, q, 128)
    assert rc == 0 and torch.equal(y, with_workspace(x, q))


def test_noalloc_rejects_shapes_beyond_the_scratch():
    from kernels import _lib as L
    case("noalloc rejects a shape beyond its scratch")
    M, N, K = 64, 16384 * 8, 9728  # split-K partials well above 32 MiB
    assert L.load().miq_wo_gemm_workspace_bytes(M, N, K, 4) > 32 << 20
    rc = L.load().miq_w4a16_gemm_noalloc(None, K, None, None, None, L.MIQ_BF16, 128, None, N, M, N, K, None)
    assert rc == -1
    assert b"above the" in L.load().miq_last_error()
