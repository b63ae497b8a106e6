"""GPU parity of the native Qwen3 decoder (the config-4 decode step).

The reference's forward (models/qwen3.js:3938-4069) is composed from the
oracle's functions (tests/qwen3_ref.py) and stepped alongside the GPU: logits
within max relative error 1e-3 (normwise), KV rows within one int8 step (the
GEMV outputs that feed the RoPE/quantizer are float, so a code may differ by one
at a rounding boundary), and the same argmax tokens where the top-2 margin
exceeds the tolerance. Covers a T-token prefill, chained device-position decode
steps, a captured decode graph replayed token after token, and the Qwen3-1.7B
layer geometry with the full vocabulary over a 4k prefix.
"""
import numpy as np
import pytest

from tabinfer_amd import abi
import qwen3_ref as Q

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def ctx():
    c = abi.Ctx(0)
    yield c
    c.close()


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def margin_ok(logits, tol=TOL):
    s = np.sort(np.asarray(logits, np.float64))
    return (s[-1] - s[-2]) > 4 * tol * np.max(np.abs(s))


SMALL = dict(layers=2, hidden=256, intermediate=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=1000,
             rope_theta=1e6, rms_eps=1e-6, max_ctx=64, max_tokens=8)


def _logits(ctx, m, vocab):
    return ctx.download(m.logits_ptr(), np.float32, vocab)


def test_prefill_then_chained_decode(ctx):
    W = Q.make_weights(SMALL, 1)
    m = abi.Qwen3(ctx, **SMALL)
    try:
        Q.load_into(m, W)
        ref = Q.RefDecoder(SMALL, W, SMALL["max_ctx"])
        ids = np.array([11, 502, 7, 999, 123], np.int32)
        m.forward(ids, 0)
        for p, t in enumerate(ids):
            rl, rt = ref.step(int(t), p)
        got = _logits(ctx, m, SMALL["vocab"])
        assert rel_err(got, rl) < TOL
        tok = int(m.read_tokens(5, 1)[0])
        if margin_ok(rl):
            assert tok == rt
        # the device-position chain: 4 steps, each continues from the GPU's own token
        for p in range(5, 9):
            m.decode()
            rl, rt = ref.step(tok, p)
            assert rel_err(_logits(ctx, m, SMALL["vocab"]), rl) < TOL
            tok = int(m.read_tokens(p + 1, 1)[0])
            if margin_ok(rl):
                assert tok == rt
        # KV rows written by the GPU match the reference's within one int8 step
        kq, ks, vq, vs = m.kv(1)
        nkv = SMALL["n_kv_heads"] * SMALL["head_dim"]
        gk = ctx.download(kq, np.uint32, 9 * nkv // 4).view(np.int8).astype(int).reshape(9, -1)
        rk = ref.kv[1][0][:9].view(np.int8).astype(int).reshape(9, -1)
        assert np.max(np.abs(gk - rk)) <= 1
        assert np.mean(gk != rk) < 0.01
    finally:
        m.close()


def test_batched_forward_matches_sequential(ctx):
    """A T=8 forward (the batch-8 configuration) gives the same last logits as 8
    single-token forwards."""
    W = Q.make_weights(SMALL, 2)
    a, b = abi.Qwen3(ctx, **SMALL), abi.Qwen3(ctx, **SMALL)
    try:
        Q.load_into(a, W)
        Q.load_into(b, W)
        ids = np.arange(8, dtype=np.int32) * 97 + 3
        a.forward(ids, 0)
        for p in range(8):
            b.forward(ids[p:p + 1], p)
        la, lb = _logits(ctx, a, SMALL["vocab"]), _logits(ctx, b, SMALL["vocab"])
        assert rel_err(la, lb) < TOL
    finally:
        a.close()
        b.close()


def test_graph_replay_decodes_like_eager(ctx):
    W = Q.make_weights(SMALL, 3)
    m = abi.Qwen3(ctx, **SMALL)
    try:
        Q.load_into(m, W)
        m.forward(np.array([5, 6, 7], np.int32), 0)
        start = int(m.read_tokens(3, 1)[0])
        for _ in range(4):
            m.decode()
        eager = m.read_tokens(4, 4).copy()
        # rewind: same token at position 3, replay a captured step 4 times
        m.write_tokens(3, np.array([start], np.int32))
        m.set_pos(3)
        ctx.sync()
        ctx.graph_begin()
        m.decode()
        g = ctx.graph_end()
        for i in range(4):
            ctx.graph_launch(g)
            ctx.sync()
            assert int(m.read_tokens(4 + i, 1)[0]) == int(eager[i])
        ctx.graph_destroy(g)
    finally:
        m.close()


def test_qwen3_17b_geometry_over_4k_prefix(ctx, orc):
    """Qwen3-1.7B layer geometry (hidden 2048, intermediate 6144, 16/8 heads of 128,
    vocab 151936), 2 layers, one decode step at position 4096 over a seeded prefix KV
    written through the attention-prep quantizer."""
    cfg = dict(layers=2, hidden=2048, intermediate=6144, n_heads=16, n_kv_heads=8, head_dim=128, vocab=151936,
               rope_theta=1e6, rms_eps=1e-6, max_ctx=4200, max_tokens=1)
    W = Q.make_weights(cfg, 4)
    m = abi.Qwen3(ctx, **cfg)
    try:
        Q.load_into(m, W)
        ref = Q.RefDecoder(cfg, W, cfg["max_ctx"])
        rng = np.random.default_rng(9)
        P = 4096
        nkv = 8 * 128
        for l in range(cfg["layers"]):
            K = rng.standard_normal(P * nkv).astype(np.float16).astype(np.float32)
            V = rng.standard_normal(P * nkv).astype(np.float16).astype(np.float32)
            kq, ks = orc.kv_quant(K)
            vq, vs = orc.kv_quant(V)
            dk = m.kv(l)
            for dst, src in zip(dk, (kq, ks, vq, vs)):
                ctx.write(dst, src)
            ref.kv[l][0][:P], ref.kv[l][1][:P] = kq.reshape(P, -1), ks.reshape(P, -1)
            ref.kv[l][2][:P], ref.kv[l][3][:P] = vq.reshape(P, -1), vs.reshape(P, -1)
        tok = 4242
        m.write_tokens(P, np.array([tok], np.int32))
        m.set_pos(P)
        m.decode()
        rl, rt = ref.step(tok, P)
        got = _logits(ctx, m, cfg["vocab"])
        assert rel_err(got, rl) < TOL
        if margin_ok(rl):
            assert int(m.read_tokens(P + 1, 1)[0]) == rt
    finally:
        m.close()
