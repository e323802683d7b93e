"""Independent numpy codecs that pin the CPU casts the oracle relies on (test only).

bf16: round-to-nearest-even on the upper 16 bits of the fp32 pattern (the definition
of the format's RNE rounding). e4m3fn: the OCP FP8 E4M3 definition (bias 7, no
infinities, S.1111.111 = NaN, max 448, subnormals m * 2^-9); encoding by exhaustive
nearest-value search with ties to the even code.
"""
import numpy as np


def bf16_round(x):
    """fp32 -> bf16 (RNE) -> fp32, by bit manipulation."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = (r << 16).astype(np.uint32).view(np.float32)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, np.float32(np.nan), out)


def e4m3_table():
    """float64 value of each of the 256 e4m3fn codes (NaN for 0x7f / 0xff)."""
    vals = np.empty(256)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 7
        if e == 15 and m == 7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = s * m * 2.0 ** -9
        else:
            vals[c] = s * (1 + m / 8) * 2.0 ** (e - 7)
    return vals


def e4m3_encode(x):
    """Nearest e4m3fn code to each value of x (|x| <= 448), ties to the even code."""
    table = e4m3_table()
    finite = np.where(np.isnan(table), np.inf, table)
    x = np.asarray(x, dtype=np.float64).reshape(-1)
    codes = np.empty(x.shape, dtype=np.uint8)
    pos = np.array([c for c in range(128) if not np.isnan(table[c])])
    for i, v in enumerate(x):
        a = abs(v)
        d = np.abs(finite[pos] - a)
        best = d.min()
        cands = pos[d == best]
        c = cands[0] if len(cands) == 1 else [c for c in cands if c % 2 == 0][0]
        if np.signbit(v):
            c |= 0x80
        codes[i] = c
    return codes
