"""Pins for the ternary oracle and the int3 MoE oracle.

Ternary: the reference's own unit tests, reproduced with their generators,
shapes and seeds (native/crates/n2-kernels/src/tern.rs:351-470) and the
`n2 selftest` fixture (native/crates/n2-cli/src/main.rs:92-183).
int3 MoE: hand-built known answers for the requantizer and the router
(models/lfm25.js:833-856, 111-141) and a numpy dequant-matmul for the GEMVs.
"""
import numpy as np
import pytest


def _max_rel(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    d = np.abs(a - b)
    m = np.maximum(np.maximum(np.abs(a), np.abs(b)), np.float32(1e-3))
    return float((d / m).max())


@pytest.mark.parametrize("n,k", [(1, 64), (3, 128), (17, 256), (8, 1024)])
def test_scalar_matches_dequant_oracle(orc, n, k):
    codes, sc, act, xsum, _, _ = orc.n2_fixture(n, k, 0x2026_0805 + k)
    got = orc.tern_gemv_scalar(codes, sc, act, xsum, n, k)
    want = orc.tern_gemv_dequant(codes, sc, act, n, k)
    assert _max_rel(got, want) < 1e-5


@pytest.mark.parametrize("n,k", [(1, 64), (1, 192), (5, 192), (17, 256), (64, 2048)])
def test_avx2_matches_scalar(orc, n, k):
    if not orc.has_avx2():
        pytest.skip("no AVX2 on this host")
    codes, sc, act, xsum, _, _ = orc.n2_fixture(n, k, 0xC0FFEE + k)
    a = orc.tern_gemv_scalar(codes, sc, act, xsum, n, k)
    b = orc.tern_gemv_avx2(codes, sc, act, xsum, n, k)
    assert _max_rel(a, b) < 1e-5
    c = orc.tern_gemv_avx2(codes, sc, act, xsum, n, k, nthreads=3)
    assert np.array_equal(b, c)


@pytest.mark.parametrize("n,k", [(1, 64), (3, 192), (17, 256), (64, 2048), (128, 4096)])
def test_n2_selftest_fixture(orc, n, k):
    codes, sc, act, xsum, _, _ = orc.n2_fixture(n, k, 0x9E3779B97F4A7C15)
    got = orc.tern_gemv_scalar(codes, sc, act, xsum, n, k)
    want = orc.tern_gemv_dequant(codes, sc, act, n, k)
    assert _max_rel(got, want) < 1e-5


def test_fixture_generator_first_values(orc):
    # xorshift64 (<<13, >>7, <<17), high 32 bits, recomputed with Python ints
    s = 0x2026_0805 + 64
    ws = []
    for _ in range(64):
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        ws.append([-1.0, 1.0, 0.0, 0.2, -0.9][(s >> 32) % 5])
    _, _, _, _, w, _ = orc.n2_fixture(1, 64, 0x2026_0805 + 64)
    assert np.array_equal(w, np.array(ws, np.float32))


def test_zero_activations_are_zero_not_nan(orc):
    n, k = 4, 128
    codes, sc, _, _, _, _ = orc.n2_fixture(n, k, 7)
    act, xsum, s = orc.tern_quant_act_n2(np.zeros(k, np.float32))
    assert s == 1.0
    out = orc.tern_gemv_scalar(codes, sc, act, xsum, n, k)
    assert np.all(out == 0.0)


def test_packing_places_codes_in_the_expected_plane(orc):
    k = 64
    w = np.zeros(k, np.float32)
    w[0], w[16], w[33] = 1.0, -1.0, 1.0
    codes, sc = orc.tern_pack(w, 1, k)
    assert sc[0] == 1.0
    assert codes[0] & 3 == 2 and (codes[0] >> 2) & 3 == 0 and (codes[0] >> 4) & 3 == 1
    assert (codes[1] >> 4) & 3 == 2


def test_block_dots_brute_force(orc):
    codes, sc, act, xsum, w, x = orc.n2_fixture(9, 192, 123)
    c = np.zeros((9, 192), np.int64)
    raw = codes.reshape(9, 3, 16)
    for j in range(4):
        c.reshape(9, 3, 64)[:, :, j * 16:(j + 1) * 16] = (raw >> (2 * j)) & 3
    dots = (c * act.astype(np.int64)[None]).reshape(9, 3, 64).sum(2)
    assert np.array_equal(orc.tern_block_dots(codes, act, 9, 192).reshape(9, 3), dots)
    assert np.array_equal(xsum, act.astype(np.int64).reshape(3, 64).sum(1))


def test_quant_act_conventions(orc):
    x = np.zeros(64, np.float32)
    x[0] = 127.0
    x[1], x[2], x[3] = 2.5, -2.5, 3.5
    a, _, s = orc.tern_quant_act_n2(x)       # n2: round half away from zero
    assert s == 1.0 and a[1] == 3 and a[2] == -3 and a[3] == 4
    a, _, s = orc.tern_quant_act_wasm(x)     # WASM: nearest-even
    assert s == 1.0 and a[1] == 2 and a[2] == -2 and a[3] == 4


# ---- int3 MoE -------------------------------------------------------------------
def _pack4(q):
    """q: int array of 32-element groups in [-8,7] -> u32 words (qwen3.js layout)."""
    q = np.asarray(q).reshape(-1, 8) + 8
    sh = np.arange(8, dtype=np.uint32) * 4
    return (q.astype(np.uint32) << sh).sum(axis=1).astype(np.uint32)


def _planes_to_q3(p3):
    p = np.asarray(p3, np.uint32).reshape(-1, 3)
    i = np.arange(32, dtype=np.uint32)
    st = ((p[:, 0:1] >> i) & 1) | (((p[:, 1:2] >> i) & 1) << 1) | (((p[:, 2:3] >> i) & 1) << 2)
    return st.astype(np.int64) - 4


def test_requant43_known_answers(orc):
    q4 = np.zeros((2, 32), np.int64)
    q4[0, :8] = [-8, 7, -7, -3, 3, 6, 0, 1]          # m = 8: ratio 0.5
    sc4 = np.array([0x3C00, 0x3C00], np.uint16)      # s4 = 1.0 ; group 1 all zero
    p3, s3 = orc.requant43(_pack4(q4), sc4, 1, 64)
    q3 = _planes_to_q3(p3)
    # JS Math.round: -4, 3.5->4 clamp 3, -3.5->-3, -1.5->-1, 1.5->2, 3, 0, 0.5->1
    assert list(q3[0, :8]) == [-4, 3, -3, -1, 2, 3, 0, 1]
    assert s3[0] == 0x4000                            # 1.0*8/4 = 2.0
    assert s3[1] == 0 and list(p3[3:6]) == [0, 0, 0xFFFFFFFF]


def test_router_known_answer(orc):
    logits = np.array([[0.0, 2.0, 2.0, -1.0, 1.0, 2.0]], np.float32)
    idx, wt = orc.router(logits, np.zeros(6, np.float32), 1, 6, 4)
    assert list(idx) == [1, 2, 5, 4]                  # ties: lowest index first
    s = 1.0 / (1.0 + np.exp(-np.array([2.0, 2.0, 2.0, 1.0])))
    assert np.allclose(wt, s / (s.sum() + 1e-6), rtol=1e-6)
    idx, _ = orc.router(logits, np.array([0, 0, 0, 5.0, 0, 0], np.float32), 1, 6, 4)
    assert idx[0] == 3                                # bias changes selection only


def test_moe_gemv_and_gemm_brute_force(orc):
    rng = np.random.default_rng(12)
    nE, N, K, pairs = 4, 16, 64, 3
    p3 = rng.integers(0, 2 ** 32, nE * N * (K // 32) * 3, dtype=np.uint64).astype(np.uint32)
    s3 = rng.uniform(0.01, 0.02, nE * N * (K // 32)).astype(np.float16).view(np.uint16)
    idx = np.array([2, 0, 3], np.int32)
    Wd = (_planes_to_q3(p3).reshape(nE * N, K) *
          np.repeat(orc.f16_array_to_f64(s3).reshape(nE * N, -1), 32, axis=1))
    x = rng.standard_normal(K).astype(np.float32)
    y = orc.moe_gemv_q3(x, p3, s3, idx, pairs, N, K, K, pairs).reshape(pairs, N)
    for k in range(pairs):
        assert np.allclose(y[k], Wd[idx[k] * N:(idx[k] + 1) * N] @ x.astype(np.float64), rtol=1e-12, atol=1e-12)
    X = rng.standard_normal((pairs, K)).astype(np.float32)
    xq, xs = orc.quant_act_q8_t(X, pairs, K)
    Y = orc.moe_gemm_q3(xq, xs, p3, s3, idx, pairs, N, K, 1).reshape(pairs, N)
    Xd = np.asarray(xq, np.uint32).view(np.int8).astype(np.float64).reshape(pairs, -1, 32) * xs.reshape(pairs, -1, 1)
    for k in range(pairs):
        assert np.allclose(Y[k], Wd[idx[k] * N:(idx[k] + 1) * N] @ Xd[k].ravel(), rtol=1e-10, atol=1e-12)
