"""Seeded synthetic inputs shared by the tests (PCG-style LCG + Box-Muller, see oracle)."""
import numpy as np

import oracle


def normal(n, seed):
    return oracle.fill_normal(int(n), int(seed))


def bf16_round(x):
    """Quantise f32 values to bf16 and expand back (the 16-bit parity convention)."""
    return oracle.bf16_to_f32(oracle.f32_to_bf16(x))


def f16_round(x):
    return oracle.f16_to_f32(oracle.f32_to_f16(x))


class Lcg:
    """tests/m38_property_stress.rs:7-30 generator."""

    def __init__(self, seed=0x4D385EEDCAFEBABE):
        self.s = seed

    def next_u32(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & (2**64 - 1)
        return self.s >> 32

    def pick(self, upper):
        return self.next_u32() % upper

    def finite(self):
        return np.float32((self.next_u32() / 4294967295.0 * 2.0 - 1.0) * 3.0)

    def vec(self, n):
        return np.array([self.finite() for _ in range(n)], np.float32)
