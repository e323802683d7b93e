"""KVCache bookkeeping and the block-table boundary on the CPU (reference
engine/core/kv_cache.py:50-300 allocators, :403-420 decode_tables,
engine/core/model_runner.py:38-39 and :176-182 for how the runner hands the tables to the
paged kernel).

decode_tables(entries, device) takes (request, context_length) pairs and returns
(block_table int32 [B, pages], seq_lens int32 [B], page_size, max_len). These tests build
the tables from requests the allocator placed, check them against the allocator's own
slots, and feed them in the kernel's argument order to the restated paged attention,
which must equal dense attention over the request's slots."""
import torch

from engine.core.kv_cache import ContiguousAllocator, PagedAllocator, pack_block_tables
from engine.core.model_runner import Request
from oracle.attention import paged_decode_reference
from oracle.runner import OracleKVCache


def placed_requests(cache, lengths):
    reqs = [Request([1] * n, 4, rid=i) for i, n in enumerate(lengths)]
    for r, n in zip(reqs, lengths):
        assert cache.admit(r, n + 4) == 0
        assert cache.ensure(r, n)
    return reqs


def dense_attention(q, k, v, slots, scale):
    kk = k[slots].float().repeat_interleave(q.shape[0] // k.shape[1], dim=1)
    vv = v[slots].float().repeat_interleave(q.shape[0] // k.shape[1], dim=1)
    p = (torch.einsum("hd,nhd->hn", q.float(), kk) * scale).softmax(-1)
    return torch.einsum("hn,nhd->hd", p, vv)


def check_tables_feed_the_kernel_contract(mode, block):
    cache = OracleKVCache(1, 2, 16, 64 * 16, torch.float32, mode=mode, block_size=block)
    lengths = [5, 33, 16, 1, 47]
    reqs = placed_requests(cache, lengths)
    # fill the cache: the value of a slot depends on the slot
    g = torch.Generator().manual_seed(3)
    cache.k[0] = torch.randn(cache.k.shape[1:], generator=g)
    cache.v[0] = torch.randn(cache.v.shape[1:], generator=g)
    # decode entries carry the context after this step's token
    entries = [(r, n) for r, n in zip(reqs, lengths)]
    table, seq_lens, page, max_len = cache.decode_tables(entries, "cpu")
    assert table.dtype == torch.int32 and seq_lens.dtype == torch.int32
    assert seq_lens.tolist() == lengths and max_len == max(lengths)
    assert page == (block if mode == "paged" else 1)
    assert table.shape == (len(lengths), -(-max(lengths) // page))
    q = torch.randn(len(lengths), 4, 16, generator=g)
    scale = 0.25
    # the kernel's argument order: q, k, v, block_table, seq_lens, page_size, scale
    got = paged_decode_reference(q, cache.k[0], cache.v[0], table, seq_lens, page, scale)
    for b, (r, n) in enumerate(entries):
        slots = cache.slots(r, 0, n)
        pos = torch.arange(n)
        assert torch.equal(table[b, pos // page].long() * page + pos % page, slots)
        if mode == "paged":  # zero padded past the request's pages
            assert (table[b, -(-n // page):] == 0).all()
        else:  # token-level rows over max_len positions from the request's base (kv_cache.py:417-418)
            assert torch.equal(table[b].long(), cache.allocator.ranges[r.id][0] + torch.arange(max_len))
        assert torch.allclose(got[b], dense_attention(q[b], cache.k[0], cache.v[0], slots, scale), atol=1e-5)


def test_paged_decode_tables_follow_the_block_tables():
    check_tables_feed_the_kernel_contract("paged", 16)
    check_tables_feed_the_kernel_contract("paged", 8)


def test_contiguous_decode_tables_are_token_level():
    check_tables_feed_the_kernel_contract("contiguous", 16)


def test_paged_tables_are_the_allocator_tables_cut_to_the_context():
    cache = OracleKVCache(1, 1, 16, 32 * 16, torch.float32, block_size=16)
    r = placed_requests(cache, [40])[0]
    cache.ensure(r, 64)  # grown ahead: four blocks held, a 40-token context uses three
    table, lens, page, max_len = cache.decode_tables([(r, 40)], "cpu")
    assert table[0].tolist() == cache.allocator.tables[r.id][:3]
    assert (lens.tolist(), page, max_len) == ([40], 16, 40)


def test_runner_hands_the_kernel_a_five_tuple():
    """BatchMetadata.decode_tables = (block_table, seq_lens, page_size, max_len, num_splits)
    (reference model_runner.py:38-39)."""
    from engine.core.model_runner import BatchMetadata
    cache = OracleKVCache(1, 1, 16, 32 * 16, torch.float32, block_size=16)
    a, b = placed_requests(cache, [9, 20])
    for r, n in ((a, 10), (b, 21)):
        cache.ensure(r, n)
    a.prompt_ids, b.prompt_ids = [1] * 10, [1] * 21
    meta = BatchMetadata([(a, 9, 10), (b, 20, 21)], cache, "cpu")
    table, lens, page, max_len, splits = meta.decode_tables
    assert lens.tolist() == [10, 21] and page == 16 and max_len == 21 and splits is None
    assert meta.all_decode and meta.decode_rows.tolist() == [0, 1]
    assert meta.write_slots.tolist() == [cache.slots(a, 9, 10).item(), cache.slots(b, 20, 21).item()]


def test_paged_allocator_reuses_freed_blocks():
    al = PagedAllocator(10 * 4, 4)
    a, b = Request([0] * 9, 3, rid=0), Request([0] * 20, 3, rid=1)
    assert al.admit(a, 100) == 0 and al.ensure(a, 9)
    assert len(al.tables[0]) == 3
    assert al.admit(b, 100) == 0 and al.ensure(b, 20) and len(al.tables[1]) == 5
    assert not al.ensure(a, 21)  # 6 blocks: 3 more, 2 free
    assert len(al.tables[0]) == 3 and al.length[0] == 9
    assert al.ensure(a, 16) and len(al.tables[0]) == 4
    held = set(al.tables[0]) | set(al.tables[1])
    assert len(held) == 9
    al.free(b)
    assert al.ensure(a, 36) and len(al.tables[0]) == 9 and len(set(al.tables[0])) == 9
    slots = al.slots(a, 0, 36)
    assert len(set(slots.tolist())) == 36


def test_contiguous_allocator_first_fit_and_coalescing():
    al = ContiguousAllocator(100)
    rs = [Request([0] * 5, 5, rid=i) for i in range(4)]  # each reserves 10 slots
    for r in rs:
        assert al.admit(r, 1000) == 0
    assert [al.ranges[i] for i in range(4)] == [(0, 10), (10, 10), (20, 10), (30, 10)]
    al.free(rs[1])
    al.free(rs[2])  # merges with the hole left by rs[1]
    assert al._holes == [(10, 20), (40, 60)]
    big = Request([0] * 15, 5, rid=9)
    assert al.admit(big, 1000) == 0 and al.ranges[9] == (10, 20)
    assert al.slots(big, 2, 5).tolist() == [12, 13, 14]
    al.free(rs[0])
    al.free(big)
    al.free(rs[3])
    assert al._holes == [(0, 100)]


def test_pack_block_tables_pads_with_zeros():
    table, lens = pack_block_tables([[5, 7], [], [9]], [20, 0, 3], "cpu")
    assert table.tolist() == [[5, 7], [0, 0], [9, 0]] and lens.tolist() == [20, 0, 3]
