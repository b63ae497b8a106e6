"""Pins for the oracle's Bonsai f32 glue (or_n2_*: native/crates/n2-core/src/ops.rs and the
attention of model.rs:421-447).

The reference's own tests (ops.rs:152-237) are restated: RMSNorm by hand computation,
RoPE at position 0 is the identity, the split-half pairing against the direct formula,
the table form against the direct form, softmax sums to one and survives large inputs,
per-head RMSNorm normalises each head alone. The attention and SwiGLU are checked
against f64 numpy formulas; argmax against its definition (the lowest index on ties).
A plausible mistake (interleaved RoPE pairing, a norm without the weight, a softmax
without the max shift, the wrong GQA head mapping) fails one of these.
"""
import numpy as np
import pytest


def test_rmsnorm_matches_hand_computation(orc):
    x = np.array([1, 2, 3, 4], np.float32)
    out = orc.n2_rmsnorm(x, np.ones(4, np.float32), 0.0)
    assert np.allclose(out, x / np.sqrt(7.5), atol=1e-6)
    w = np.array([0.5, 2, -1, 3], np.float32)
    out = orc.n2_rmsnorm(x, w, 1e-6)
    assert np.allclose(out, x / np.sqrt(7.5 + 1e-6) * w, rtol=1e-6)


def test_rope_at_position_zero_is_the_identity(orc):
    t = (np.arange(256) * 0.1).astype(np.float32)
    out = orc.n2_rope_with_table(t, 2, 128, orc.n2_rope_table(128, 0, 1e6))
    assert np.abs(out - t).max() < 1e-6


def test_rope_uses_the_split_half_pairing(orc):
    """ops.rs:187-204: head_dim 4, pos 3, theta 1e6 on [1, 2, 3, 4]."""
    out = orc.n2_rope_with_table(np.array([1, 2, 3, 4], np.float32), 1, 4, orc.n2_rope_table(4, 3, 1e6))
    for i, (x0, x1) in enumerate(((1.0, 3.0), (2.0, 4.0))):
        ang = 3 * 1e6 ** (-(2 * i) / 4)                       # 3 and 0.003
        c, s = np.cos(ang), np.sin(ang)
        assert abs(out[i] - (x0 * c - x1 * s)) < 1e-5
        assert abs(out[2 + i] - (x1 * c + x0 * s)) < 1e-5
    # an interleaved pairing (2i, 2i+1) would give a different vector
    assert abs(out[1] - (2 * np.cos(3) - 1 * np.sin(3))) > 0.1


def test_rope_table_agrees_with_the_direct_form(orc):
    a = np.sin(np.arange(128)).astype(np.float32)
    half = 64
    inv = 1e6 ** (-(2 * np.arange(half)) / 128)
    c, s = np.cos(17 * inv), np.sin(17 * inv)
    want = np.concatenate([a[:half] * c - a[half:] * s, a[half:] * c + a[:half] * s])
    assert np.abs(orc.n2_rope_with_table(a, 1, 128, orc.n2_rope_table(128, 17, 1e6)) - want).max() < 1e-5


def test_rmsnorm_heads_normalises_each_head_independently(orc):
    t = np.array([1, 1, 1, 1, 100, 100, 100, 100], np.float32)
    out = orc.n2_rmsnorm_heads(t, np.ones(4, np.float32), 2, 4, 0.0)
    for h in range(2):
        assert abs(np.sqrt(np.mean(out[4 * h:4 * h + 4].astype(np.float64) ** 2)) - 1) < 1e-5


def test_attention_softmax_and_gqa(orc):
    """One key: the output is that key's value (softmax of one score is 1). Large scores
    stay finite (the max shift). Random: f64 numpy with query head h reading KV head
    h // (n_heads / n_kv)."""
    rng = np.random.default_rng(0)
    nh, nkv, hd = 4, 2, 8
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k1 = rng.standard_normal(nkv * hd).astype(np.float32)
    v1 = rng.standard_normal(nkv * hd).astype(np.float32)
    out = orc.n2_attention(q, k1, v1, 1, nh, nkv, hd)
    assert np.array_equal(out.reshape(nh, hd), v1.reshape(nkv, hd)[[0, 0, 1, 1]])
    big = orc.n2_attention(q * 1000, np.tile(k1, 3) * 1000, np.tile(v1, 3), 3, nh, nkv, hd)
    assert np.all(np.isfinite(big))
    S = 37
    K = rng.standard_normal((S, nkv, hd)).astype(np.float32)
    V = rng.standard_normal((S, nkv, hd)).astype(np.float32)
    got = orc.n2_attention(q, K.ravel(), V.ravel(), S, nh, nkv, hd).reshape(nh, hd)
    for h in range(nh):
        kh = K[:, h // 2].astype(np.float64)
        sc = kh @ q.reshape(nh, hd)[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        assert np.abs(got[h] - p @ V[:, h // 2].astype(np.float64)).max() < 1e-5


def test_swiglu_and_argmax(orc):
    rng = np.random.default_rng(1)
    g, u = rng.standard_normal(100).astype(np.float32), rng.standard_normal(100).astype(np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.abs(orc.n2_swiglu(g, u) - want).max() < 1e-6
    x = np.array([0, 3, 1, 3, -np.inf], np.float32)
    assert orc.n2_argmax(x) == 1                           # the lowest index of the tie
    assert orc.n2_argmax(np.full(5, -np.inf, np.float32)) == 0
    x = np.array([np.nan, 1, np.nan, 2], np.float32)
    assert orc.n2_argmax(x) == 3
