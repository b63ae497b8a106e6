"""GPU parity: int4 quantizer, int8 activation quant, fused
RMSNorm+quant bit-exact against the oracle; int4 GEMVs with
exact per-group integer dots and float outputs within max relative error 1e-3
(normwise, f64 oracle of the quantized operands — models/qwen3.js:3104)."""
import numpy as np
import pytest

from tabinfer_amd import abi

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def ctx():
    c = abi.Ctx(0)
    yield c
    c.close()


def bf16_normal(rng, n, std=0.02):
    w = (rng.standard_normal(n) * std).astype(np.float32)
    return (w.view(np.uint32) >> 16).astype(np.uint16)


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("N,K", [(64, 256), (130, 256), (2048, 1024), (1024, 3072)])
def test_quant_int4_bit_exact(ctx, orc, N, K):
    rng = np.random.default_rng(N + K)
    w = bf16_normal(rng, N * K)
    w[:32] = 0                                         # all-zero group
    w[32:64] = np.uint16(0x3000)                       # tiny group: scale underflows to 0
    w[64:96] = np.uint16(0x3F80)                       # constant 1.0
    pack, sc = orc.quant_int4_bf16(w, N, K)
    dw = ctx.upload(w)
    dp = ctx.zeros(pack.nbytes)
    ds = ctx.zeros(sc.nbytes)
    ctx.call("ti_quant_int4_bf16", dw, dp, ds, N, K)
    assert np.array_equal(ctx.download(dp, np.uint32, pack.size), pack)
    assert np.array_equal(ctx.download(ds, np.uint16, sc.size), sc)


@pytest.mark.parametrize("K", [32, 1024, 2048, 3072, 6144])
def test_quant_act_q8_bit_exact(ctx, orc, K):
    rng = np.random.default_rng(K)
    x = rng.standard_normal(K).astype(np.float32)
    x[:32] = 0
    if K >= 64:
        x[32:64] = np.float32(127.0) * (np.arange(32) % 5 - 2) / 2   # exact .5 ties after scaling
    xq, xs, xsum = orc.quant_act_q8(x)
    dx = ctx.upload(x)
    dq, ds, dsum = ctx.zeros(xq.nbytes), ctx.zeros(xs.nbytes), ctx.zeros(xsum.nbytes)
    ctx.call("ti_quant_act_q8", dx, dq, ds, dsum, K)
    assert np.array_equal(ctx.download(dq, np.uint32, xq.size), xq)
    assert np.array_equal(ctx.download(ds, np.float32, xs.size), xs)
    assert np.array_equal(ctx.download(dsum, np.int32, xsum.size), xsum)


def test_quant_act_q8_t_bit_exact(ctx, orc):
    rng = np.random.default_rng(1)
    T, K = 8, 2048
    x = rng.standard_normal(T * K).astype(np.float32)
    xq, xs = orc.quant_act_q8_t(x, T, K)
    dx = ctx.upload(x)
    dq, ds = ctx.zeros(xq.nbytes), ctx.zeros(xs.nbytes)
    ctx.call("ti_quant_act_q8_t", dx, dq, ds, T, K)
    assert np.array_equal(ctx.download(dq, np.uint32, xq.size), xq)
    assert np.array_equal(ctx.download(ds, np.float32, xs.size), xs)


@pytest.mark.parametrize("H", [256, 1024, 2048, 6144])
def test_rmsnorm_q8_bit_exact(ctx, orc, H):
    rng = np.random.default_rng(H)
    x = (rng.standard_normal(H) * 3).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16).view(np.uint16)
    xq, xs, xsum = orc.rmsnorm_q8(x, w, 1e-6)
    dx, dw = ctx.upload(x), ctx.upload(w)
    dq, ds, dsum = ctx.zeros(xq.nbytes), ctx.zeros(xs.nbytes), ctx.zeros(xsum.nbytes)
    ctx.call("ti_rmsnorm_q8", dx, dw, dq, ds, dsum, H, np.float32(1e-6))
    assert np.array_equal(ctx.download(dq, np.uint32, xq.size), xq)
    assert np.array_equal(ctx.download(ds, np.float32, xs.size), xs)
    assert np.array_equal(ctx.download(dsum, np.int32, xsum.size), xsum)
    # plain RMSNorm over 3 rows, bit-exact too
    X = (rng.standard_normal(3 * H)).astype(np.float32)
    y = orc.rmsnorm(X, w, 3, H, 1e-6)
    dX, dy = ctx.upload(X), ctx.zeros(y.nbytes)
    ctx.call("ti_rmsnorm", dX, dw, dy, 3, H, np.float32(1e-6))
    assert np.array_equal(ctx.download(dy, np.float32, y.size), y)


@pytest.mark.parametrize("T,H", [(1, 256), (5, 512), (8, 1024), (8, 2048), (16, 2048), (3, 4096)])
def test_rmsnorm_q8_t_bit_exact(ctx, orc, T, H):
    """rmsnorm + QUANTQ8T of T rows (the T-token forward's norm kernel): every code and
    scale equals the oracle's rmsnorm_q8 of that row."""
    rng = np.random.default_rng(T * 7 + H)
    X = (rng.standard_normal(T * H) * 3).astype(np.float32)
    X[:H // 2] *= 1e-3                                  # a row with small values in part
    w = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16).view(np.uint16)
    dX, dw = ctx.upload(X), ctx.upload(w)
    dq, ds = ctx.zeros(T * H), ctx.zeros(T * H // 8)
    ctx.call("ti_rmsnorm_q8_t", dX, dw, dq, ds, T, H, np.float32(1e-6))
    gq = ctx.download(dq, np.uint32, T * H // 4).reshape(T, -1)
    gs = ctx.download(ds, np.float32, T * H // 32).reshape(T, -1)
    for t in range(T):
        xq, xs, _ = orc.rmsnorm_q8(X[t * H:(t + 1) * H], w, 1e-6)
        assert np.array_equal(gq[t], xq) and np.array_equal(gs[t], xs), t
    with pytest.raises(abi.TIError):
        ctx.call("ti_rmsnorm_q8_t", dX, dw, dq, ds, T, 320, np.float32(1e-6))


def _weights(ctx, orc, rng, N, K):
    w = bf16_normal(rng, N * K)
    pack, sc = orc.quant_int4_bf16(w, N, K)
    return pack, sc, ctx.upload(pack), ctx.upload(sc)


GEMV_SHAPES = [(200, 320), (37, 32), (1, 64), (2048, 1024), (1024, 1024), (1024, 2048), (1024, 3072),
               (2048, 2048), (2048, 6144), (4096, 4096), (65, 96), (300, 1536), (17, 12288)]


@pytest.mark.parametrize("N,K", GEMV_SHAPES)
def test_gemv_q4_q8(ctx, orc, N, K):
    rng = np.random.default_rng(7 * N + K)
    pack, sc, dp, ds = _weights(ctx, orc, rng, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    xq, xs, _ = orc.quant_act_q8(x)
    dq, dxs = ctx.upload(xq), ctx.upload(xs)
    # exact integer dots
    dd = ctx.zeros(N * (K // 32) * 4)
    ctx.call("ti_group_dots_q4_q8", dq, dp, dd, N, K)
    assert np.array_equal(ctx.download(dd, np.int32, N * (K // 32)), orc.group_dots_q4_q8(xq, pack, N, K))
    ref = orc.gemv_q4_q8(xq, xs, pack, sc, N, K)
    dy = ctx.zeros(N * 4)
    ctx.call("ti_gemv_q4_q8", dq, dxs, dp, ds, dy, N, K, 0)
    y = ctx.download(dy, np.float32, N)
    assert rel_err(y, ref) < TOL
    # acc=1: y += W x (fused residual)
    ctx.call("ti_gemv_q4_q8", dq, dxs, dp, ds, dy, N, K, 1)
    assert rel_err(ctx.download(dy, np.float32, N), y.astype(np.float64) + ref) < TOL


@pytest.mark.parametrize("N,K", [(130, 256), (151936, 1024), (151936, 2048), (16384, 3072), (33, 12288)])
def test_gemv_q4_f32(ctx, orc, N, K):
    rng = np.random.default_rng(N + 3 * K)
    pack, sc, dp, ds = _weights(ctx, orc, rng, N, K)
    x = rng.standard_normal(K).astype(np.float16).astype(np.float32)
    ref = orc.gemv_q4_f32(x, pack, sc, N, K)
    dx, dy = ctx.upload(x), ctx.zeros(N * 4)
    ctx.call("ti_gemv_q4_f32", dx, dp, ds, dy, N, K, 0)
    assert rel_err(ctx.download(dy, np.float32, N), ref) < TOL


@pytest.mark.parametrize("I,H", [(130, 256), (3072, 1024), (6144, 2048), (1792, 2048), (96, 12288)])
def test_gateup_silu(ctx, orc, I, H):
    rng = np.random.default_rng(I + H)
    gp, gs, dgp, dgs = _weights(ctx, orc, rng, I, H)
    up, us, dup, dus = _weights(ctx, orc, rng, I, H)
    x = rng.standard_normal(H).astype(np.float32)
    xq, xs, _ = orc.quant_act_q8(x)
    ref = orc.gateup_silu_q4(xq, xs, gp, gs, up, us, I, H)
    dq, dxs, dy = ctx.upload(xq), ctx.upload(xs), ctx.zeros(I * 4)
    ctx.call("ti_gateup_silu_q4", dq, dxs, dgp, dgs, dup, dus, dy, I, H)
    assert rel_err(ctx.download(dy, np.float32, I), ref) < TOL


@pytest.mark.parametrize("T,N,K", [(1, 2048, 1024), (1, 151936, 1024), (8, 2048, 2048), (3, 100, 320)])
def test_linear_router(ctx, orc, T, N, K):
    rng = np.random.default_rng(T * N + K)
    pack, sc, dp, ds = _weights(ctx, orc, rng, N, K)
    X = rng.standard_normal(T * K).astype(np.float32)
    if T == 1 and N >= 16384:
        ref = orc.gemv_q4_f32(X, pack, sc, N, K)
    else:
        xq, xs = orc.quant_act_q8_t(X, T, K)
        ref = orc.gemm_q4_q8(xq, xs, pack, sc, T, N, K)
    dx, dy = ctx.upload(X), ctx.zeros(T * N * 4)
    ctx.call("ti_linear_q4", dx, dp, ds, dy, T, N, K, 0)
    assert rel_err(ctx.download(dy, np.float32, T * N), ref) < TOL


@pytest.mark.parametrize("T,N,K", [(2, 2048, 2048), (8, 6144, 2048), (8, 2048, 6144), (16, 1024, 1024),
                                   (17, 4096, 2048), (40, 96, 320), (8, 1000, 3072), (256, 256, 1024),
                                   (16, 2048, 6144), (3, 1000, 6144), (5, 2048, 2048), (7, 4096, 1024),
                                   (9, 2048, 2048)])
def test_gemm_mfma_batched_linear(ctx, orc, T, N, K):
    """linearQ at T > 1 (models/qwen3.js:1604-1607): per-token quantQ8T + the MFMA int4 x int8
    GEMM; max relative error 1e-3 against the f64 oracle of the quantized operands, with and
    without the fused residual. T <= 8 takes the pairwise-group MFMA (odd T: padding token
    rows repeat the last token), T = 9 the one-group-per-MFMA loop."""
    rng = np.random.default_rng(T * 131 + N + K)
    pack, sc, dp, ds = _weights(ctx, orc, rng, N, K)
    X = rng.standard_normal(T * K).astype(np.float32)
    X[:32] = 0                                            # a zero group in token 0
    xq, xs = orc.quant_act_q8_t(X, T, K)
    ref = orc.gemm_q4_q8(xq, xs, pack, sc, T, N, K)
    dx, dy = ctx.upload(X), ctx.zeros(T * N * 4)
    ctx.call("ti_linear_q4", dx, dp, ds, dy, T, N, K, 0)
    got = ctx.download(dy, np.float32, T * N)
    assert rel_err(got, ref) < TOL
    for t in range(T):                                    # per token as well: no row leaks into another
        assert rel_err(got[t * N:(t + 1) * N], ref[t * N:(t + 1) * N]) < TOL
    y0 = rng.standard_normal(T * N).astype(np.float32)
    ctx.write(dy, y0)
    ctx.call("ti_linear_q4", dx, dp, ds, dy, T, N, K, 1)
    assert rel_err(ctx.download(dy, np.float32, T * N), ref + y0) < TOL
    # again: the residual K = 6144 projections run as two K halves whose per-block
    # counters the second half resets for the next launch
    ctx.call("ti_linear_q4", dx, dp, ds, dy, T, N, K, 1)
    assert rel_err(ctx.download(dy, np.float32, T * N), 2 * ref + y0) < TOL


def test_shape_errors(ctx):
    d = ctx.zeros(4096)
    with pytest.raises(abi.TIError) as e:
        ctx.call("ti_gemv_q4_q8", d, d, d, d, d, 16, 33, 0)
    assert e.value.code == abi.TI_ERR_INVALID and "multiple of 32" in str(e.value)
    with pytest.raises(abi.TIError):
        ctx.call("ti_gemv_q4_q8", d, d, d.at(4), d, d, 16, 32, 0)       # misaligned pack


def test_graph_replay_matches_eager(ctx, orc):
    rng = np.random.default_rng(99)
    N, K = 2048, 1024
    pack, sc, dp, ds = _weights(ctx, orc, rng, N, K)
    w = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(K).astype(np.float32)
    dx, dw = ctx.upload(x), ctx.upload(w)
    dq, dxs, dsum, dy = ctx.zeros(K), ctx.zeros(K // 8), ctx.zeros(K // 4), ctx.zeros(N * 4)
    ctx.call("ti_rmsnorm_q8", dx, dw, dq, dxs, dsum, K, np.float32(1e-6))
    ctx.call("ti_gemv_q4_q8", dq, dxs, dp, ds, dy, N, K, 0)
    eager = ctx.download(dy, np.float32, N)
    ctx.graph_begin()
    ctx.call("ti_buf_fill_u32", dy, 0, N)
    ctx.call("ti_rmsnorm_q8", dx, dw, dq, dxs, dsum, K, np.float32(1e-6))
    ctx.call("ti_gemv_q4_q8", dq, dxs, dp, ds, dy, N, K, 0)
    g = ctx.graph_end()
    for _ in range(3):
        ctx.fill_u32(dy, 0x7FC00000, N)          # poison between replays (eager work)
        ctx.sync()
        ctx.graph_launch(g)
        ctx.sync()
        assert np.array_equal(ctx.download(dy, np.float32, N), eager)
    ctx.graph_destroy(g)
