"""The reference's kernel-check method (src/tools/kcheck.c), restated for the parity tests.

kcheck.c:21-22   32-bit LCG rs = rs * 1664525 + 1013904223 from rs = 12345; frand() = (rs >> 8) / 2^23 - 1.
kcheck.c:106-107 random E4M3 operand bytes: the top byte of the next LCG state, redrawn while it is a NaN code
                 (x & 0x7F == 0x7F) or its exponent field exceeds 9.
kcheck.c:117-126 97 sampled rows m = (i * 7919) mod rows, compared with fp64 loops; kcheck prints max |err| without
                 a threshold, the tests add one.
"""
import numpy as np


class Lcg:
    def __init__(self, seed=12345):
        self.rs = seed

    def next_u32(self):
        self.rs = (self.rs * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.rs

    def frand(self):
        return np.float32((self.next_u32() >> 8) / 8388608.0 - 1.0)

    def frand_n(self, n):
        return np.array([self.frand() for _ in range(n)], np.float32)

    def e4m3_bytes(self, n):
        out = np.empty(n, np.uint8)
        for i in range(n):
            while True:
                b = self.next_u32() >> 24
                if (b & 0x7F) != 0x7F and ((b >> 3) & 15) <= 9:
                    break
            out[i] = b
        return out


def sample_rows(rows, n=97):
    return np.array([(i * 7919) % rows for i in range(n)], np.int32)
