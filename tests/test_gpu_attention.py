"""Paged decode attention (HIP) vs the CPU oracle (kernels/paged_attention/reference.py
restated), on the reference test's cases plus the benchmark shape.
Tolerance: relative error < 1e-2 (reference tests/test_paged_attention.py:19-20 for
bf16) and elementwise |err| <= 1e-2 + 2e-2 |want|."""
import pytest
import torch

from oracle import attention as A
from oracle import quant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2


def case(msg):
    print(f"[case] {msg}", flush=True)


def rel_error(a, b):
    return ((a.float().cpu() - b.float().cpu()).norm() / b.float().cpu().norm().clamp(min=1e-12)).item()


def within(got, want):
    err = (got.float().cpu() - want.float().cpu()).abs()
    assert (err <= 1e-2 + 2e-2 * want.float().cpu().abs()).all(), err.max().item()


def random_paged(lens, H, KV, D, page, seed=0, dtype=torch.bfloat16):
    """reference tests/test_paged_attention.py:27-41 (generated on CPU)."""
    g = torch.Generator().manual_seed(seed)
    pages = [-(-n // page) for n in lens]
    total = sum(pages) + 3
    k = torch.randn(total * page, KV, D, generator=g).to(dtype)
    v = torch.randn(total * page, KV, D, generator=g).to(dtype)
    perm = torch.randperm(total, generator=g).tolist()
    table = torch.zeros(len(lens), max(pages), dtype=torch.int32)
    i = 0
    for b, n in enumerate(pages):
        table[b, :n] = torch.tensor(perm[i:i + n])
        i += n
    q = torch.randn(len(lens), H, D, generator=g).to(dtype)
    return q, k, v, table, torch.tensor(lens, dtype=torch.int32)


def run(q, k, v, t, sl, page, scale, **kw):
    from kernels.paged_attention import paged_decode_attention
    ks, vs = kw.pop("k_scale", None), kw.pop("v_scale", None)
    def dev(x):
        if x is None:
            return None
        if x.dim() == 2 and x.stride() == (0, 0):  # keep a per-tensor scale a stride-0 view
            return x[:1, :1].contiguous().to(DEV).expand(x.shape)
        return x.to(DEV)

    return paged_decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), t.to(DEV), sl.to(DEV), page, scale,
                                  max(sl.tolist()), k_scale=dev(ks), v_scale=dev(vs), **kw)


CASES = [  # (lens, H, KV, D, page)
    ([1, 17, 40], 4, 4, 128, 16),
    ([33, 5], 8, 2, 128, 16),
    ([9, 30], 4, 4, 128, 1),
    ([1, 100, 513, 2048], 16, 16, 128, 16),
    ([4096] * 2 + [17] * 6, 16, 16, 128, 16),
    ([700, 1, 3000, 129], 32, 8, 128, 16),
]


@pytest.mark.parametrize("lens,H,KV,D,page", CASES)
def test_bf16_cache_matches_reference(lens, H, KV, D, page):
    case(f"bf16 lens={lens[:4]} H={H} KV={KV} page={page}")
    q, k, v, t, sl = random_paged(lens, H, KV, D, page)
    want = A.paged_decode_reference(q, k, v, t, sl, page, D ** -0.5)
    got = run(q, k, v, t, sl, page, D ** -0.5)
    assert got.dtype == torch.bfloat16 and got.shape == q.shape
    assert rel_error(got, want) < TOL
    within(got, want)


def test_partitions_agree():
    """reference tests/test_paged_attention.py:63-70: results do not depend on the split."""
    case("partition sizes")
    lens = [700, 3, 1290]
    q, k, v, t, sl = random_paged(lens, 8, 2, 128, 16, seed=1)
    want = A.paged_decode_reference(q, k, v, t, sl, 16, 128 ** -0.5)
    for part in (128, 256, 512, 1024, 2048):
        got = run(q, k, v, t, sl, 16, 128 ** -0.5, partition=part)
        assert rel_error(got, want) < TOL, part
    for splits in (1, 2, 3, 9):
        got = run(q, k, v, t, sl, 16, 128 ** -0.5, num_splits=splits)
        assert rel_error(got, want) < TOL, splits


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("partition,lens", [(None, [40, 7, 90]), (128, [600, 7, 1290, 300]),
                                            (256, [600, 7, 1290, 300]), (384, [600, 7, 1290]),
                                            (512, [600, 7, 1290, 1100]), (1024, [2500, 7, 1290, 1100])])
@pytest.mark.parametrize("H,KV", [(4, 4), (32, 2)])
def test_quantized_cache_written_by_kvcache(kind, partition, lens, H, KV):
    """reference tests/test_paged_attention.py:73-89 with the HIP quantize-on-write; every
    partition size with its own kernel instance (128, 256, 512, 1024) and the generic one (384),
    with requests that end inside a chunk, a partition, or after one token; one kv head per
    q head, and the largest group the kernels take (16 q heads per kv head)."""
    from engine.core.kv_cache import KVCache
    case(f"quantized cache {kind} partition {partition} lens {lens} H={H} KV={KV}")
    D, page = 128, 16
    q, k, v, t, sl = random_paged(lens, H, KV, D, page, seed=2)
    cache = KVCache("paged", 1, KV, D, k.shape[0] + 16, torch.bfloat16, DEV, block_size=page, kv_dtype=kind)
    cache.write(0, torch.arange(k.shape[0], device=DEV), k.to(DEV), v.to(DEV))
    kc, vc = cache.k[0][: k.shape[0]].cpu(), cache.v[0][: k.shape[0]].cpu()
    ks, vs = cache.k_scale[0][: k.shape[0]].cpu(), cache.v_scale[0][: k.shape[0]].cpu()
    want = A.paged_decode_reference(q, kc, vc, t, sl, page, D ** -0.5, k_scale=ks, v_scale=vs)
    got = run(q, kc, vc, t, sl, page, D ** -0.5, k_scale=ks, v_scale=vs, partition=partition)
    full = A.paged_decode_reference(q, k, v, t, sl, page, D ** -0.5)
    assert rel_error(got, want) < TOL and rel_error(got, full) < 0.1
    within(got, want)


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_benchmark_shape(kind):
    """Config 4 shape (32 q / 8 kv heads, D 128, page 16, shuffled tables) at 16 requests;
    fp8 with a per-tensor fp32 scale as a stride-0 view, int8 with per-(token, head) fp32 scales."""
    case(f"config-4 shape {kind}")
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(512, 8193, (16,), generator=g).tolist()
    q, k, v, t, sl = random_paged(lens, 32, 8, 128, 16, seed=4, dtype=torch.float32)
    if kind == "fp8":
        s = torch.tensor(0.05)
        kc = (k / s).clamp(-448, 448).to(torch.float8_e4m3fn)
        vc = (v / s).clamp(-448, 448).to(torch.float8_e4m3fn)
        ks = s.reshape(1, 1).expand(k.shape[0], 8)
        vs = ks
    else:
        kc, ks = O.kv_quantize(k, "int8", torch.float32)
        vc, vs = O.kv_quantize(v, "int8", torch.float32)
    qb = q.to(torch.bfloat16)
    want = A.paged_decode_reference(qb, kc, vc, t, sl, 16, 128 ** -0.5, k_scale=ks, v_scale=vs)
    got = run(qb, kc, vc, t, sl, 16, 128 ** -0.5, k_scale=ks, v_scale=vs)
    assert rel_error(got, want) < TOL
    within(got, want)


@pytest.mark.parametrize("kind", ["bf16", "fp8", "int8"])
@pytest.mark.parametrize("partition", [128, 256, 512, 384, 1024])
def test_max_len_below_the_longest_context(kind, partition):
    """A stale or undersized max_len never cuts a request: when a context does not fit
    max_parts partitions, its partitions grow (multiples of the partition size) so the
    whole context is attended, as the reference splits each request's own context
    (decode_triton.py:25-30, 131-132)."""
    from kernels.paged_attention import paged_decode_attention
    case(f"max_len below the context {kind} partition {partition}")
    lens = [1700, 33, 3000, 1]
    H, KV, D, page = 16, 4, 128, 16
    q, k, v, t, sl = random_paged(lens, H, KV, D, page, seed=5)
    ks = vs = None
    if kind != "bf16":
        k, ks = O.kv_quantize(k.float(), kind, torch.float32)
        v, vs = O.kv_quantize(v.float(), kind, torch.float32)
    want = A.paged_decode_reference(q, k, v, t, sl, page, D ** -0.5, k_scale=ks, v_scale=vs)
    for max_len in (partition, 700, 2999):
        got = paged_decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), t.to(DEV), sl.to(DEV), page, D ** -0.5,
                                     max_len, k_scale=None if ks is None else ks.to(DEV),
                                     v_scale=None if vs is None else vs.to(DEV), partition=partition)
        assert rel_error(got, want) < TOL, max_len
        within(got, want)


@pytest.mark.parametrize("kind", ["bf16", "fp8", "int8"])
def test_empty_context_rows(kind):
    """Requests of length 0 (padded batch rows) give zeros and do not disturb the others:
    the reference's empty split has lse -inf and output 0 (decode_triton.py:95-100)."""
    case(f"empty contexts {kind}")
    lens = [0, 300, 0, 17]
    H, KV, D, page = 8, 2, 128, 16
    q, k, v, t, sl = random_paged([max(n, 1) for n in lens], H, KV, D, page, seed=6)
    sl = torch.tensor(lens, dtype=torch.int32)
    t[0] = 0
    t[2] = 0
    ks = vs = None
    if kind != "bf16":
        k, ks = O.kv_quantize(k.float(), kind, torch.float32)
        v, vs = O.kv_quantize(v.float(), kind, torch.float32)
    got = run(q, k, v, t, sl, page, D ** -0.5, k_scale=ks, v_scale=vs)
    assert torch.count_nonzero(got[0].float()) == 0 and torch.count_nonzero(got[2].float()) == 0
    live = torch.tensor([1, 3])
    want = A.paged_decode_reference(q[live], k, v, t[live], sl[live], page, D ** -0.5, k_scale=ks, v_scale=vs)
    within(got[live], want)


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_config4_full_batch(kind):
    """BASELINE config 4 at its full size, on the benchmark's own inputs: 64 requests,
    lengths U[512, 8192] and the shuffled block table from seed 7 (bench.attention_tables),
    K/V N(0, 1) generated on the device; fp8 with the per-tensor 4/448 scale as a stride-0
    view, int8 written per (token, kv head) by the HIP quantize-on-write with fp32 scales.
    Every request of the batch against the oracle, at the default and both benchmarked
    partitions."""
    import bench
    from kernels.paged_attention import paged_decode_attention
    case(f"config 4 full batch {kind}")
    a = bench.attention_inputs(torch.device(DEV), kind, copies=1)
    kc, vc, ks, vs = a["caches"][0]
    assert a["q"].shape == (64, 32, 128) and a["tokens"] > 200_000
    if kind == "fp8":
        assert ks.stride() == (0, 0) and abs(ks[0, 0].item() - 4.0 / 448.0) < 1e-9
    else:
        assert ks.dtype == torch.float32 and ks.stride(1) == 1
    table, lens = a["table"].cpu(), a["lens"].cpu()
    kcc, vcc = kc.cpu(), vc.cpu()
    kss = ks[:1, :1].cpu().expand(ks.shape) if kind == "fp8" else ks.cpu()
    vss = kss if kind == "fp8" else vs.cpu()
    want = A.paged_decode_reference(a["q"].cpu(), kcc, vcc, table, lens, 16, 128 ** -0.5, k_scale=kss, v_scale=vss)
    for partition in (None, 256, 512):
        got = paged_decode_attention(a["q"], kc, vc, a["table"], a["lens"], 16, 128 ** -0.5, a["max_len"],
                                     k_scale=ks, v_scale=vs, partition=partition)
        assert rel_error(got, want) < TOL, partition
        within(got, want)
