"""Pins for the oracle's int8 KV quantizer, RoPE/QK-norm prep and decode
attention.

Independent checks: the n2 RoPE known-answer tests
(native/crates/n2-core/src/ops.rs:169-214), pair-norm preservation of a
rotation, the reference's kvQuantWrite round-trip bound
(models/qwen3.js:2939-2963), and a numpy softmax over dequantized K/V with the
reference's own fixtures (models/qwen3.js:2901-2937).
"""
import numpy as np
import pytest


def test_kv_quant_invariants(orc):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(8 * 128) * 3).astype(np.float32)
    x[32:64] = 0.0
    q, s = orc.kv_quant(x)
    codes = np.asarray(q, np.uint32).view(np.int8).astype(np.int64).reshape(-1, 32)
    g = x.reshape(-1, 32)
    assert np.array_equal(s, np.maximum(np.abs(g).max(axis=1), np.float32(1e-12)))
    nz = np.abs(g).max(axis=1) > 0
    assert np.all(np.abs(codes[nz]).max(axis=1) == 127)
    assert np.all(codes[~nz] == 0)
    deq = orc.kv_dequant(q, s).reshape(-1, 32)
    assert np.all(np.abs(deq - g) <= s[:, None] / 254.0 * (1 + 1e-6))


def test_kv_quant_round_half_up(orc):
    # pack4x8snorm: floor(0.5 + 127*clamp(e)). 127 is odd, so the only exact
    # ties are e = +/-0.5 (127*e = +/-63.5): half-up gives 64 and -63, where
    # ties-to-even or half-away-from-zero would give -64.
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1] = 63.5
    x[2] = -63.5
    x[3] = -127.0
    x[4] = 0.25        # 127*0.25/127 = 0.25 -> 0
    q, s = orc.kv_quant(x)
    c = np.asarray(q, np.uint32).view(np.int8)
    assert s[0] == 127.0 and c[0] == 127 and c[1] == 64 and c[2] == -63 and c[3] == -127 and c[4] == 0


def test_kv_roundtrip_like_reference(orc):
    # models/qwen3.js:2939-2963 fixture: T=3, nKv=2, hd=64
    n = 3 * 2 * 64
    i = np.arange(n)
    kr = (np.sin(i * 0.13) * (1 + (i % 7))).astype(np.float32)
    q, s = orc.kv_quant(kr)
    err = np.abs(orc.kv_dequant(q, s) - kr).max() / np.abs(kr).max()
    assert err < 1.2e-2


def test_rope_position_zero_is_identity(orc):
    x = (np.arange(128) * 0.1).astype(np.float32)
    out = orc.rope_norm_row(x, None, 128, 0, 1e6, 0.0, apply_norm=False)
    assert np.max(np.abs(out - x)) < 1e-6


def test_rope_split_half_pairing_known_answer(orc):
    # ops.rs:181-201: head_dim 4, theta 1e6, pos 3, t = [1,2,3,4]
    t = np.array([1, 2, 3, 4], np.float32)
    out = orc.rope_norm_row(np.concatenate([t, np.zeros(0, np.float32)]), None, 4, 3, 1e6, 0.0, False)
    for i in range(2):
        inv = 1e6 ** (-(2 * i) / 4)
        ang = 3 * inv
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = i + 1, 2 + i + 1
        assert abs(out[i] - (x0 * c - x1 * s)) < 1e-5
        assert abs(out[2 + i] - (x1 * c + x0 * s)) < 1e-5


def test_rope_preserves_pair_norms_at_32k(orc):
    rng = np.random.default_rng(10)
    x = rng.standard_normal(128).astype(np.float32)
    w = np.ones(128, np.float16).view(np.uint16)
    for pos in (1, 4095, 32767):
        normed = orc.rope_norm_row(x, w, 128, 0, 1e6, 1e-6, True)     # pos 0: norm only
        out = orc.rope_norm_row(x, w, 128, pos, 1e6, 1e-6, True)
        a = normed[:64] ** 2 + normed[64:] ** 2
        b = out[:64].astype(np.float64) ** 2 + out[64:].astype(np.float64) ** 2
        assert np.allclose(a, b, rtol=1e-5)
        # the angle of pair 0 is exactly pos radians (inv_freq[0] = 1)
        o = out.astype(np.float64)
        nr = normed.astype(np.float64)
        ang = np.arctan2(o[64], o[0]) - np.arctan2(nr[64], nr[0])
        assert abs(np.angle(np.exp(1j * (ang - pos)))) < 1e-5


@pytest.mark.parametrize("hd", [64, 128])
def test_qk_rmsnorm_against_f64(orc, hd):
    """The per-head RMSNorm of attnPrepQ8 (models/qwen3.js:2258-2262): x / sqrt(mean(x^2) + eps)
    * w in f64, with non-unit f16 weights and an eps that matters (mean x^2 ~ 2.5e-3 against
    eps 1e-3: eps outside the root, a sum in place of the mean or a dropped weight each miss
    by far more than the f32 tolerance). At pos 0 the rotation is the identity; at pos > 0
    the output is the f64 split-half rotation of the f64-normed row."""
    rng = np.random.default_rng(hd)
    theta, eps = 1e6, 1e-3
    for trial in range(4):
        x = (rng.standard_normal(hd) * 0.05).astype(np.float32)
        w = (0.5 + rng.uniform(0, 1, hd)).astype(np.float16)
        x64, w64 = x.astype(np.float64), w.astype(np.float64)
        n = x64 / np.sqrt(np.mean(x64 * x64) + eps) * w64
        got = orc.rope_norm_row(x, w.view(np.uint16), hd, 0, theta, eps, True).astype(np.float64)
        assert np.max(np.abs(got - n)) <= 1e-6 * np.max(np.abs(n))
        pos = int(rng.integers(1, 32768))
        half = hd // 2
        ang = pos * theta ** (-(2.0 * np.arange(half)) / hd)
        c, sn = np.cos(ang), np.sin(ang)
        want = np.concatenate([n[:half] * c - n[half:] * sn, n[half:] * c + n[:half] * sn])
        got = orc.rope_norm_row(x, w.view(np.uint16), hd, pos, theta, eps, True).astype(np.float64)
        # the angle pos * theta^(-2i/hd) is formed in f32 by the reference's rotary table:
        # ~pos * 2^-24 radians of phase error at most
        assert np.max(np.abs(got - want)) <= (4e-6 + pos * 2.0 ** -22) * np.max(np.abs(n))


def test_attn_prep_qk_norm_and_kv_write(orc):
    nHq, nKv, hd, pos = 4, 2, 128, 7
    i = np.arange(nHq * hd)
    q = np.sin(i * 0.11).astype(np.float32)
    k = np.cos(np.arange(nKv * hd) * 0.07).astype(np.float32)
    v = (np.sin(np.arange(nKv * hd) * 0.05 + 2) * (1 + np.arange(nKv * hd) % 3)).astype(np.float32)
    qw = (0.6 + 0.4 * np.sin(np.arange(hd) * 0.02)).astype(np.float16).view(np.uint16)
    kw = (0.7 + 0.3 * np.cos(np.arange(hd) * 0.03)).astype(np.float16).view(np.uint16)
    qr, kq, ks, vq, vs = orc.attn_prep_q8(q, k, v, qw, kw, nHq, nKv, hd, pos, 10000.0, 1e-6)
    for h in range(nHq):
        assert np.array_equal(qr[h * hd:(h + 1) * hd], orc.rope_norm_row(q[h * hd:(h + 1) * hd], qw, hd, pos, 10000.0, 1e-6, True))
    for h in range(nKv):
        kr = orc.rope_norm_row(k[h * hd:(h + 1) * hd], kw, hd, pos, 10000.0, 1e-6, True)
        q2, s2 = orc.kv_quant(kr)
        assert np.array_equal(kq[h * 32:(h + 1) * 32], q2) and np.array_equal(ks[h * 4:(h + 1) * 4], s2)
        q3, s3 = orc.kv_quant(v[h * hd:(h + 1) * hd])
        assert np.array_equal(vq[h * 32:(h + 1) * 32], q3) and np.array_equal(vs[h * 4:(h + 1) * 4], s3)


def _np_attention(Q, Kd, Vd, S, nHq, nKv, hd):
    out = np.zeros((nHq, hd))
    grp = nHq // nKv
    Kd = Kd.reshape(S, nKv, hd)
    Vd = Vd.reshape(S, nKv, hd)
    for hq in range(nHq):
        hk = hq // grp
        s = Kd[:, hk, :] @ Q[hq].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[hq] = (p[:, None] * Vd[:, hk, :]).sum(0) / p.sum()
    return out.ravel()


@pytest.mark.parametrize("S,nHq,nKv,hd", [(333, 4, 2, 128), (100, 2, 1, 64), (1, 16, 8, 128)])
def test_attn_decode_matches_numpy_softmax(orc, S, nHq, nKv, hd):
    # fixtures of models/qwen3.js:2901-2937
    Q = np.sin(np.arange(nHq * hd) * 0.017).astype(np.float32).reshape(nHq, hd)
    K = np.cos(np.arange(S * nKv * hd) * 0.009).astype(np.float32)
    V = np.sin(np.arange(S * nKv * hd) * 0.004 + 0.7).astype(np.float32)
    kq, ks = orc.kv_quant(K)
    vq, vs = orc.kv_quant(V)
    got = orc.attn_decode_q8(Q, kq, ks, vq, vs, S, nHq, nKv, hd)
    ref = _np_attention(Q, orc.kv_dequant(kq, ks), orc.kv_dequant(vq, vs), S, nHq, nKv, hd)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-12
    if S == 1:   # one key: the output is that key's dequantized V row
        assert np.allclose(got.reshape(nHq, hd)[0], orc.kv_dequant(vq, vs)[:hd])


def test_attn_causal_rows_are_prefix_decodes(orc):
    rng = np.random.default_rng(11)
    T, pos0, nHq, nKv, hd = 3, 10, 4, 2, 64
    S = pos0 + T
    K = rng.standard_normal(S * nKv * hd).astype(np.float32)
    V = rng.standard_normal(S * nKv * hd).astype(np.float32)
    kq, ks = orc.kv_quant(K)
    vq, vs = orc.kv_quant(V)
    Q = rng.standard_normal(T * nHq * hd).astype(np.float32)
    out = orc.attn_causal_q8(Q, kq, ks, vq, vs, T, pos0, nHq, nKv, hd).reshape(T, -1)
    for t in range(T):
        ref = orc.attn_decode_q8(Q[t * nHq * hd:(t + 1) * nHq * hd], kq, ks, vq, vs, pos0 + t + 1, nHq, nKv, hd)
        assert np.array_equal(out[t], ref)
