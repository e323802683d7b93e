"""Writes known_answers.json: small cases whose expected outputs follow from the
definitions of the formats and the reference's formulas by exact arithmetic (Python
fractions / floats that are exact powers of two), not from any implementation.

Run: python tests/golden/make_known_answers.py
"""
import json
import os
from fractions import Fraction


def rne(x):
    """round half to even of a Fraction (what torch.round / rint do)."""
    f = x.numerator // x.denominator
    rem = x - f
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and f % 2 == 1):
        f += 1
    return f


def main():
    cases = {}
    # int8_wo.py:8-12 -- s = 127 * 2^-7 / 127 = 2^-7 exactly, so w / s are exact multiples
    s = Fraction(1, 128)
    mult = [127, -127, 3, Fraction(5, 2), Fraction(3, 2), Fraction(-1, 2), Fraction(7, 2), 0, -64, Fraction(-5, 2)]
    row = [float(m * s) for m in mult] + [0.0] * 118
    cases["int8"] = {"w": [row], "q": [[rne(Fraction(m)) for m in mult] + [0] * 118], "scale": [float(s)]}

    # int4_wo.py:15-31 -- group min 0, max 15/16: s = (15/16 - 0) / 15 = 1/16 exactly
    u = [(i * 7) % 16 for i in range(128)]
    u[0], u[1] = 0, 15
    w = [x / 16 for x in u]
    ties = {5: Fraction(5, 2), 9: Fraction(7, 2), 12: Fraction(21, 2)}   # (w - min) / s = k + 1/2
    for i, t in ties.items():
        w[i] = float(t / 16)
        u[i] = rne(t)
    packed = [u[2 * j] | (u[2 * j + 1] << 4) for j in range(64)]
    cases["int4"] = {"w": [w], "q": [packed], "scale": [[1 / 16]], "zero": [[0.0]],
                     "dequant": [[x / 16 for x in u]]}
    # int4_wo.py:34-36 -- unpack order: low nibble is the even k
    cases["int4_unpack"] = {"byte": 0x7A, "k0": 10, "k1": 7}

    # e4m3fn definition: value -> code
    e4m3 = [
        (448.0, 0x7E), (-448.0, 0xFE), (1.0, 0x38), (2.0 ** -9, 0x01), (2.0 ** -10, 0x00),
        (3 * 2.0 ** -10, 0x02), (1.0625, 0x38), (1.1875, 0x3A), (0.0, 0x00), (-0.0, 0x80),
        (240.0, 0x77), (2.0 ** -6, 0x08), (7 * 2.0 ** -9, 0x07), (15 * 2.0 ** -10, 0x08),
        (-1.5, 0xBC), (0.75, 0x34), (416.0, 0x7D), (432.0, 0x7E),
    ]
    cases["e4m3"] = {"value": [v for v, _ in e4m3], "code": [c for _, c in e4m3]}

    # fp8.py:41-46 -- amax 56 -> s = 56 / 448 = 1/8 exactly; x / s exact
    x = [56.0, -56.0, 1.0, 0.5, -3.25, 0.0, 18.0, 2.0 ** -12]
    xx = x + [0.0] * (128 - len(x))
    cases["fp8_rows"] = {"x": [xx], "scale": [0.125],
                         "q_values": [[v * 8 for v in xx]]}

    # kv_cache.py:359-369 -- int8, amax 127 -> s = bf16(1.0) = 1, q = round(x)
    kv = [127.0, -126.5, 3.5, 2.5, -0.5, 0.25] + [0.0] * 122
    cases["kv_int8"] = {"x": [[kv]], "scale": [[1.0]], "q": [[[rne(Fraction(v).limit_denominator()) for v in kv]]]}

    # fused_moe_triton.py:8-39 contract on a hand-worked routing
    cases["moe_align"] = {"topk_ids": [[0, 1], [1, 2], [0, 2]], "E": 3, "block_m": 2,
                          "sorted_ids": [0, 4, 1, 2, 3, 5, 6, 6, 6], "expert_ids": [0, 1, 2, 2, 2],
                          "num_padded": 6}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")
    with open(path, "w") as f:
        json.dump(cases, f, indent=1)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
