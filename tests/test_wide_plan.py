"""The tests' restatement of the wide GEMM's planner (tests/wide_plan.py) against libmiq's,
on the CPU: miq_wo_gemm_workspace_bytes is host arithmetic over the same plans, the 16 KiB
counter area plus the larger of the prefill kernel's split-K partials (at most 30 MiB) and
the wide plan's packed activations and K-split partials. A plan that differs in tile height
or split count changes the wide bytes, so for every shape where they exceed the prefill
kernel's share the two must agree exactly."""
import itertools

import pytest

from wide_plan import wide_plan

COUNTERS = 16384
PREFILL_MAX = 30 << 20


@pytest.mark.parametrize("bits", [4, 8])
def test_wide_plan_restatement_matches_the_library(bits):
    from kernels import _lib
    lib = _lib.load()
    checked = 0
    for M, N, K in itertools.product([65, 96, 128, 200, 256, 300, 512, 640, 777, 1024, 1300, 1536, 2048, 4096],
                                     [1024, 2560, 2576, 4096, 6144, 19456],
                                     [128, 512, 1536, 2560, 4096, 6144, 9728, 12288]):
        got = lib.miq_wo_gemm_workspace_bytes(M, N, K, bits)
        plan = wide_plan(M, N, K)
        if plan is None:
            assert got <= COUNTERS + PREFILL_MAX, (M, N, K, got)
            continue
        want = COUNTERS + plan[2]
        assert got >= want, (M, N, K, plan, got)
        if want > COUNTERS + PREFILL_MAX:
            assert got == want, (M, N, K, plan, got)
            checked += 1
    assert checked > 50
