"""Pins for the oracle's argmax (or_argmax), the restatement of argmaxKernel
(models/qwen3.js:2624-2690).

The oracle evaluates the reference's loops literally (per-thread strided scans with a
strict '>', then shared-memory trees where slot l takes slot l+s only if strictly
greater). It is pinned three ways:
  - known answers worked out by hand from the WGSL (which of two tied indices wins);
  - a closed form derived independently: among equal maxima the trees favour the slot
    with the smallest bit-reversed number and a scan its first index, so the winner
    minimises (bitrev6(workgroup), bitrev8(thread), i >> 14) for N >= 16384 and
    (bitrev8(thread), i >> 8) below; checked on arrays with many ties;
  - the special cases the start value (-3e38, index 0) fixes: no candidate -> 0, NaN
    and values <= -3e38 are never selected, -0.0 ties +0.0.
A plausible mistake (lowest index on ties, a tree that keeps the right slot, a scan that
keeps the last maximum) fails the known answers.
"""
import numpy as np
import pytest


def bitrev(v, bits):
    return int(format(v, "0%db" % bits)[::-1], 2)


def closed_form(x):
    x = np.asarray(x, np.float32)
    N = x.size
    cand = np.nonzero(x > np.float32(-3e38))[0]
    if cand.size == 0:
        return 0
    m = x[cand].max()
    tied = [int(i) for i in cand if x[i] == m]
    if N >= 16384:
        key = lambda i: (bitrev((i >> 8) & 63, 6), bitrev(i & 255, 8), i >> 14)
    else:
        key = lambda i: (bitrev(i & 255, 8), i >> 8)
    return min(tied, key=key)


def with_ties(N, idx, val=5.0, seed=0):
    x = np.random.default_rng(seed).standard_normal(N).astype(np.float32)
    x[list(idx)] = val
    return x


@pytest.mark.parametrize("N,idx,want", [
    (151936, (300, 16394), 16394),      # workgroup 0 (k = 1) beats workgroup 1 at stage 2's last level
    (151936, (16394, 300), 16394),
    (151936, (256, 512), 512),          # workgroups 1 and 2: bitrev6 2 = 16 < bitrev6 1 = 32
    (151936, (16384, 0), 0),            # one thread: its first index
    (151936, (1, 128), 128),            # threads 1 and 128 of workgroup 0: bitrev8 128 = 1 < bitrev8 1 = 128
    (1000, (64, 128), 128),             # one stage: slot 0 holds 128 after s = 128, keeps it at s = 64
    (1000, (5, 261), 5),                # same thread, first index
    (1000, (3, 2), 2),                  # slot 2 holds thread 2 at s = 2, slot 1 holds thread 3; 0 vs 2 at s = 2 -> 2
    (16383, (16382, 0), 0),
    (16384, (16383, 256), 256),         # N = 16384 takes the two-stage kernels
])
def test_argmax_tie_known_answers(orc, N, idx, want):
    x = with_ties(N, idx)
    assert orc.argmax(x) == want
    assert closed_form(x) == want


@pytest.mark.parametrize("N", [7, 256, 1000, 16383, 16384, 40000, 151936])
def test_argmax_matches_closed_form_on_heavy_ties(orc, N):
    rng = np.random.default_rng(N)
    for rep in range(4):
        x = rng.integers(-3, 4, N).astype(np.float32)      # about 1/7 of the entries share the maximum
        assert orc.argmax(x) == closed_form(x), rep
        x = rng.standard_normal(N).astype(np.float32)
        x[rng.integers(0, N, 5)] = 9.0
        assert orc.argmax(x) == closed_form(x), rep


def test_argmax_special_values(orc):
    N = 151936
    assert orc.argmax(np.full(N, -np.inf, np.float32)) == 0
    assert orc.argmax(np.full(1000, -3e38, np.float32)) == 0           # equal to the start value: never taken
    x = np.full(1000, -np.inf, np.float32)
    x[777] = -3.0e38
    x[778] = -2.9e38
    assert orc.argmax(x) == 778
    x = np.zeros(1000, np.float32)
    x[0] = np.nan
    x[1] = -0.0                                                         # -0.0 == +0.0: a tie
    assert orc.argmax(x) == closed_form(x)
    x = np.full(N, np.nan, np.float32)
    x[5] = 1.0
    assert orc.argmax(x) == 5
