"""Writes tests/golden/w8a8_golden.npz: small known-answer vectors for the
W8A8 path, computed WITHOUT the oracle (pure-Python integers and exact
rationals), so that they pin the oracle and the kernels independently.

The reference has no W8A8 implementation to draw vectors from (its linear
slot is bf16 F.linear, python/minisgl/layers/linear.py:31-32), so the
vectors come from the closed forms the path is defined by:

* quantizer: s = RN_f32(amax / 127) and q = clamp(RNE(RN_f32(x / s))), with
  every fp32 rounding done exactly from Fractions;
* int GEMM: exact integer dot products;
* epilogue: RN_f32(RN_f32(RN_f32(acc) * sa) * sw) then RNE to bf16, exactly;
* alignment: the worked example of the reference's moe_align_block_size
  docstring (python/minisgl/moe/fused.py:56-69), copied as data.

Run: python tests/golden/make_golden.py  (deterministic; seed fixed)
"""

from __future__ import annotations

import os
import random
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "w8a8_golden.npz")


# ------------------------------------------------------------ exact rounding
def round_to_bits(fr: Fraction, mant_bits: int, min_exp: int) -> Fraction:
    """Round a rational to the nearest binary float with ``mant_bits``
    significant bits (ties to even), subnormals below 2**min_exp."""
    if fr == 0:
        return Fraction(0)
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, min_exp)
    ulp = Fraction(2) ** (e - mant_bits + 1)
    q, r = divmod(a, ulp)
    q = int(q)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return sign * q * ulp


def rn_f32(fr: Fraction) -> Fraction:
    return round_to_bits(fr, 24, -126)


def rn_bf16(fr: Fraction) -> Fraction:
    return round_to_bits(fr, 8, -126)


def rne_int(fr: Fraction) -> int:
    fl = fr.numerator // fr.denominator
    r = fr - fl
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl


def to_f32(fr: Fraction) -> np.float32:
    return np.float32(float(fr))  # exact: fr is already an fp32 value


# ------------------------------------------------------------------ vectors
def quant_rows(rows):
    qs, ss = [], []
    for row in rows:
        row = [Fraction(v) for v in row]
        amax = max(abs(v) for v in row)
        s = rn_f32(amax / 127)
        if s == 0:
            qs.append([0] * len(row))
            ss.append(Fraction(0))
            continue
        q = [max(-127, min(127, rne_int(rn_f32(v / s)))) for v in row]
        qs.append(q)
        ss.append(s)
    return qs, ss


def bf16_values(rng: random.Random, n: int):
    """Random bf16-representable rationals (8-bit significands)."""
    out = []
    for _ in range(n):
        m = rng.randint(128, 255)
        e = rng.randint(-12, 5)
        out.append(Fraction(m * (1 if rng.random() < 0.5 else -1)) * Fraction(2) ** (e - 7))
    return out


def main() -> None:
    rng = random.Random(1234)
    # quantizer: hand-built tie rows plus seeded rows
    K = 16
    hand = [
        [127, Fraction(5, 2), Fraction(-1, 2), Fraction(253, 2), Fraction(7, 2), Fraction(-3, 2)] + [0] * 10,
        [0] * 3 + [-3] + [0] * 12,
        [0] * 16,
        [20, Fraction(-5, 64), Fraction(5, 32), Fraction(1, 1024)] + [0] * 12,
        [Fraction(1, 2 ** 130), -Fraction(1, 2 ** 133), Fraction(1, 2 ** 128)] + [0] * 13,
    ]
    seeded = [bf16_values(rng, K) for _ in range(11)]
    rows = hand + seeded
    q, s = quant_rows(rows)
    x = np.array([[float(v) for v in r] for r in rows], np.float32)
    # int GEMM + epilogue on the quantized rows
    N = 8
    w = [[rng.randint(-127, 127) for _ in range(K)] for _ in range(N)]
    sw = [rn_f32(Fraction(rng.randint(1, 2 ** 20), 2 ** 27)) for _ in range(N)]
    acc = [[sum(a * b for a, b in zip(qr, wr)) for wr in w] for qr in q]
    y = [
        [rn_bf16(rn_f32(rn_f32(rn_f32(Fraction(acc[m][n])) * s[m]) * sw[n])) for n in range(N)]
        for m in range(len(rows))
    ]
    np.savez(
        OUT,
        quant_x=x,
        quant_q=np.array(q, np.int8),
        quant_s=np.array([to_f32(v) for v in s], np.float32),
        gemm_w=np.array(w, np.int8),
        gemm_sw=np.array([to_f32(v) for v in sw], np.float32),
        gemm_acc=np.array(acc, np.int32),
        gemm_y=np.array([[float(v) for v in r] for r in y], np.float32),
        # python/minisgl/moe/fused.py:56-69 (num_experts = 4 -> 5 slots, block 4)
        align_topk_ids=np.array([[2, 3, 4], [1, 2, 4], [1, 3, 4], [1, 2, 3]], np.int32),
        align_sorted_ids=np.array([3, 6, 9, 12, 0, 4, 10, 12, 1, 7, 11, 12, 2, 5, 8, 12], np.int32),
        align_expert_ids=np.array([1, 2, 3, 4], np.int32),
        align_num_post_pad=np.array([16], np.int32),
    )
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
