"""Pins for the oracle's Gumbel-max sampler (or_gumbel_noise, or_pcg, or_seed_next:
models/qwen3.js:2713-2740).

argmax(logits + T g), g = -log(-log(u)), u uniform on (0, 1), is a sample of
softmax(logits / T). What fixes the restatement:
- the reference's own self-test (models/qwen3.js:3198-3214), restated on a larger
  sample: logits -100 except [5] = 2 and [9] = 1, so at T = 1 P(5) / P(9) = e and no
  other index is ever drawn; at T = 0.02 the draw is the greedy index;
- the Gumbel distribution's mean (Euler's gamma) and variance (pi^2 / 6), and softmax
  frequencies at T = 2 over four logits: a wrong sign, a single log, a missing T or a
  u that reaches 0 or 1 fails one of these;
- u is uniform: the hash's 24-bit outputs fill 64 equal bins evenly (chi-square).
"""
import math

import numpy as np
import pytest


def draws(orc, base, temp, n, state=None):
    """n samples with the reference's seed stream from `state` (advanced before each
    draw, as gumbelNoise does); returns the indices and the final state."""
    st = orc.SEED_INIT if state is None else state
    out = []
    for _ in range(n):
        st = orc.seed_next(st)
        out.append(orc.argmax(orc.gumbel_noise(base, st, temp)))
    return np.array(out), st


def test_reference_self_test_ratio_is_e(orc):
    base = np.full(1024, -100.0, np.float32)
    base[5], base[9] = 2.0, 1.0
    idx, _ = draws(orc, base, 1.0, 4000)
    c5, c9 = int(np.sum(idx == 5)), int(np.sum(idx == 9))
    assert c5 + c9 == idx.size                                  # nothing else is ever drawn
    p5 = c5 / idx.size                                          # e / (1 + e) = 0.7311
    assert abs(p5 - math.e / (1 + math.e)) < 4 * math.sqrt(0.7311 * 0.2689 / idx.size)


def test_cold_temperature_is_greedy(orc):
    base = np.full(1024, -100.0, np.float32)
    base[5], base[9] = 2.0, 1.0
    idx, _ = draws(orc, base, 0.02, 50)
    assert np.all(idx == 5)


def test_softmax_frequencies_at_temperature_two(orc):
    base = np.full(300, -1e4, np.float32)
    logits = np.array([0.0, 1.0, 2.0, 3.0])
    base[[17, 100, 201, 299]] = logits
    idx, _ = draws(orc, base, 2.0, 6000)
    p = np.exp(logits / 2.0)
    p /= p.sum()
    for k, i in enumerate((17, 100, 201, 299)):
        f = np.mean(idx == i)
        assert abs(f - p[k]) < 4 * math.sqrt(p[k] * (1 - p[k]) / idx.size)


def test_gumbel_mean_and_variance(orc):
    g = orc.gumbel_noise(np.zeros(1 << 20, np.float32), 0x12345678, 1.0).astype(np.float64)
    assert abs(g.mean() - 0.5772156649) < 0.005
    assert abs(g.var() - math.pi ** 2 / 6) < 0.02
    assert np.all(np.isfinite(g))


def test_hash_outputs_are_uniform(orc):
    seed = orc.seed_next(orc.SEED_INIT)
    h = np.array([orc.pcg(i ^ ((seed * 2654435761) & 0xFFFFFFFF)) >> 8 for i in range(1 << 16)], np.int64)
    counts = np.bincount(h >> 18, minlength=64)                 # 64 bins of the 24-bit value
    expect = h.size / 64
    chi2 = float(np.sum((counts - expect) ** 2 / expect))
    assert chi2 < 120                                           # 63 dof: p < 1e-5 above ~120

