"""Synthetic tensors for the on-GPU ternary format (test infrastructure): bf16 weights that
are exactly ternary per 32-group (zero or +-m with one bf16 magnitude m per group)."""
import numpy as np


def ternary_bf16(rng, N, K, lo=0.01, hi=0.05):
    """bf16 bits of N x K weights in {-m, 0, +m} per 32-group, m a bf16 value in [lo, hi]."""
    m = rng.uniform(lo, hi, N * K // 32).astype(np.float32)
    mb = (m.view(np.uint32) >> 16).astype(np.uint16)                # bf16 truncation of each group's m
    code = rng.integers(0, 3, N * K)                                   # 0 -> -1, 1 -> 0, 2 -> +1
    bits = np.repeat(mb, 32).astype(np.uint16)
    bits = np.where(code == 1, np.uint16(0), bits)
    bits = np.where(code == 0, bits | np.uint16(0x8000), bits)
    return bits.astype(np.uint16)


def bf16_to_f64(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32).astype(np.float64)
