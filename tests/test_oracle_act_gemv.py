"""Pins for the oracle's int8 activation quant, fused RMSNorm+quant and
the int4 GEMV oracles.

Independent checks: invariants of the per-32 absmax quantizer
(models/qwen3.js:343-357), the ties-to-even known answer that distinguishes
WGSL round() from JS Math.round, an f64 RMSNorm, and brute-force numpy
unpacking of the nibble layout for the GEMV oracles.
"""
import numpy as np


def _codes(xq):
    return np.asarray(xq, np.uint32).view(np.int8).astype(np.int64)


def test_quant_act_q8_invariants(orc):
    rng = np.random.default_rng(4)
    K = 1024
    x = rng.standard_normal(K).astype(np.float32)
    x[100:132] = 0.0                                  # an all-zero group
    xq, xs, xsum = orc.quant_act_q8(x)
    q = _codes(xq)
    assert np.all(np.abs(q) <= 127)
    g = x.reshape(-1, 32)
    amax = np.abs(g).max(axis=1)
    assert np.array_equal(xs, amax / np.float32(127.0))
    # the group max maps to +/-127; zero group -> scale 0, codes 0
    qg = q.reshape(-1, 32)
    nz = amax > 0
    assert np.all(np.abs(qg[nz]).max(axis=1) == 127)
    assert np.all(qg[~nz] == 0)
    # dequant error <= s/2 (plus one rounding of the product)
    err = np.abs(qg * xs[:, None].astype(np.float64) - g)
    assert np.all(err <= xs[:, None] * 0.5 * (1 + 1e-6) + 1e-30)
    # xsum is the per-16 code sum
    assert np.array_equal(xsum, q.reshape(-1, 16).sum(axis=1))


def test_quant_act_q8_rounds_ties_to_even(orc):
    # group absmax 127 -> scale 1, inv 1: 2.5 -> 2 and 3.5 -> 4 (WGSL round);
    # JS Math.round would give 3 and 4.
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1], x[2], x[3] = 2.5, 3.5, -2.5
    xq, xs, _ = orc.quant_act_q8(x)
    q = _codes(xq)
    assert xs[0] == 1.0 and q[1] == 2 and q[2] == 4 and q[3] == -2


def test_rmsnorm_q8_matches_f64_norm(orc):
    rng = np.random.default_rng(5)
    for H in (256, 1024, 2048):
        x = rng.standard_normal(H).astype(np.float32)
        w = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16).view(np.uint16)
        xq, xs, xsum = orc.rmsnorm_q8(x, w, 1e-6)
        xd = x.astype(np.float64)
        y = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * orc.f16_array_to_f64(w)
        deq = _codes(xq).reshape(-1, 32) * xs[:, None]
        # per-group: |deq - y| <= s/2 + f32 rounding of the normalized value
        err = np.abs(deq.ravel() - y)
        tol = np.repeat(xs.astype(np.float64), 32) * 0.5 + np.abs(y) * 4e-7
        assert np.all(err <= tol)
        assert np.array_equal(xsum, _codes(xq).reshape(-1, 16).sum(axis=1))
        # the float path: plain RMSNorm is within 2 ulp of the f64 value
        yy = orc.rmsnorm(x, w, 1, H, 1e-6)
        assert np.max(np.abs(yy - y) / np.maximum(np.abs(y), 1e-30)) < 3e-7


def _unpack(pack, N, K):
    w = np.asarray(pack, np.uint32).reshape(N, K // 8)
    sh = np.arange(8, dtype=np.uint32) * 4
    return ((w[:, :, None] >> sh) & 0xF).reshape(N, K).astype(np.int64) - 8


def _rand_int4(rng, N, K):
    pack = rng.integers(0, 2 ** 32, N * K // 8, dtype=np.uint64).astype(np.uint32)
    sc = (rng.uniform(0.001, 0.01, N * K // 32)).astype(np.float16).view(np.uint16)
    return pack, sc


def test_group_dots_and_gemv_q4_q8_brute_force(orc):
    rng = np.random.default_rng(6)
    N, K = 37, 320
    pack, sc = _rand_int4(rng, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    xq, xs, _ = orc.quant_act_q8(x)
    Wq = _unpack(pack, N, K)
    q = _codes(xq)
    dots = (Wq * q[None, :]).reshape(N, K // 32, 32).sum(axis=2)
    assert np.array_equal(orc.group_dots_q4_q8(xq, pack, N, K).reshape(N, -1), dots)
    y = orc.gemv_q4_q8(xq, xs, pack, sc, N, K)
    s = orc.f16_array_to_f64(sc).reshape(N, -1)
    yref = (dots * s * xs[None, :].astype(np.float64)).sum(axis=1)
    assert np.allclose(y, yref, rtol=1e-12, atol=1e-12)


def test_gemv_q4_f32_and_gateup_brute_force(orc):
    rng = np.random.default_rng(7)
    N, K = 29, 256
    pack, sc = _rand_int4(rng, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    Wd = _unpack(pack, N, K) * np.repeat(orc.f16_array_to_f64(sc).reshape(N, -1), 32, axis=1)
    y = orc.gemv_q4_f32(x, pack, sc, N, K)
    assert np.allclose(y, Wd @ x.astype(np.float64), rtol=1e-12, atol=1e-12)
    # gate/up: silu(g)*u from two GEMVs of the same int8 activation
    up, us = _rand_int4(rng, N, K)
    xq, xs, _ = orc.quant_act_q8(x)
    g = orc.gemv_q4_q8(xq, xs, pack, sc, N, K)
    u = orc.gemv_q4_q8(xq, xs, up, us, N, K)
    swi = orc.gateup_silu_q4(xq, xs, pack, sc, up, us, N, K)
    assert np.allclose(swi, g * (1.0 / (1.0 + np.exp(-g))) * u, rtol=1e-12, atol=1e-14)


def test_gemm_rows_equal_gemv(orc):
    rng = np.random.default_rng(8)
    T, N, K = 5, 19, 128
    pack, sc = _rand_int4(rng, N, K)
    X = rng.standard_normal((T, K)).astype(np.float32)
    xq, xs = orc.quant_act_q8_t(X, T, K)
    Y = orc.gemm_q4_q8(xq, xs, pack, sc, T, N, K).reshape(T, N)
    for t in range(T):
        q1, s1, _ = orc.quant_act_q8(X[t])
        assert np.array_equal(q1, xq.reshape(T, -1)[t])
        assert np.array_equal(Y[t], orc.gemv_q4_q8(q1, s1, pack, sc, N, K))
