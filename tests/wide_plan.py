"""libmiq's plan of the wide weight-only GEMM, restated for the tests that choose their
oracle by it (the wide kernel multiplies the reference's bf16 weights, the prefill kernel
the exact ones). tests/test_wide_plan.py pins it to the library on the CPU."""


def wide_plan(M, N, K):
    """libmiq's plan of the wide kernel (wo_wide_plan), restated: (MT, S, workspace bytes
    past the counter area) or None where the prefill kernel runs (M below 65, or fewer than
    128 workgroups in every plan). A launch of T tiles of 128 x 128 MT and S K splits runs
    ceil(T S / 256) rounds of MT 32-row tiles over ceil(steps / S) k-steps (rounded up to
    even), with relative cost 1.75 / 1.13 / 1.0 for MT = 1 / 2 / 3 and the partial outputs
    priced at 0.5 us per MB; splits only from 48 k-steps up; the least modelled time wins,
    the larger MT then the fewer splits on ties."""
    if M < 65:
        return None
    cost = {1: 1.75, 2: 1.13, 3: 1.0}
    tiles_n, steps = -(-N // 128), K // 128
    max_s = 16 if steps >= 48 else 1
    best, best_t = None, 0.0
    for mt in (1, 2, 3):
        tm = -(-M // (128 * mt))
        pack = tm * 4 * mt * 32 * K * 2
        if pack >= 0x7fff0000:
            continue
        for S in range(1, max_s + 1):
            per = -(-steps // S)
            if -(-steps // per) != S:
                continue
            part = S * ((M * N + 3) & ~3) * 4 if S > 1 else 0
            items = tm * tiles_n * S
            if items < 128:
                continue
            t = 0.8 * float(-(-items // 256)) * mt * cost[mt] * float((per + 1) & ~1) + float(part) * 0.5e-6
            if best is None or t < best_t - 1e-9 or (t <= best_t + 1e-9 and mt > best[0]):
                best, best_t = (mt, S, pack + part), t
    return best


def wide_planned(M, N, K):
    return wide_plan(M, N, K) is not None
