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
import qwen3_tf as TF

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
        gk = TF.read_kv_codes(ctx, m, kq, 0, 9, SMALL).view(np.int8).astype(int).reshape(9, -1)
        rk = ref.kv[1][0][:9].view(np.int8).astype(int).reshape(9, -1)
        assert np.max(np.abs(gk - rk)) <= 1
        assert np.mean(gk != rk) < 0.01
    finally:
        m.close()


def test_prefill_in_256_token_chunks(ctx):
    """The reference's prefill chunk (PREFILL_CHUNK = 256, models/qwen3.js:5245-5256): a
    300-token prompt as a 256-token forward and a 44-token one, with 16 query heads of 128
    (4096 query rows in one attention call, the split count cut to fit the partials), then
    chained decode steps, against the oracle decoder run token by token."""
    cfg = dict(SMALL, n_heads=16, n_kv_heads=8, head_dim=128, max_ctx=320, max_tokens=256)
    W = Q.make_weights(cfg, 6)
    m = abi.Qwen3(ctx, **cfg)
    try:
        Q.load_into(m, W)
        ref = Q.RefDecoder(cfg, W, cfg["max_ctx"])
        ids = (np.arange(300, dtype=np.int64) * 7919 % cfg["vocab"]).astype(np.int32)
        m.forward(ids[:256], 0)
        m.forward(ids[256:], 256)
        for p, t in enumerate(ids):
            rl, rt = ref.step(int(t), p)
        got = _logits(ctx, m, cfg["vocab"])
        assert rel_err(got, rl) < TOL
        tok = int(m.read_tokens(300, 1)[0])
        if margin_ok(rl):
            assert tok == rt
        for p in range(300, 304):
            m.decode()
            rl, rt = ref.step(tok, p)
            assert rel_err(_logits(ctx, m, cfg["vocab"]), rl) < TOL
            tok = int(m.read_tokens(p + 1, 1)[0])
            if margin_ok(rl):
                assert tok == rt
        # every KV row of the chunks within one int8 step of the oracle's: layer 0's K/V come
        # straight from the embeddings (flips only where the GEMM's f32 order lands on the
        # other side of a rounding boundary), layer 1's also carry layer 0's flips
        nkv = cfg["n_kv_heads"] * cfg["head_dim"]
        for layer, frac in ((0, 0.005), (1, 0.02)):
            kq, ks, vq, vs = m.kv(layer)
            gk = TF.read_kv_codes(ctx, m, kq, 0, 300, cfg).view(np.int8).astype(int).reshape(300, -1)
            rk = ref.kv[layer][0][:300].view(np.int8).astype(int).reshape(300, -1)
            print("[qwen3] 256-token chunks: layer %d K codes differing %.4f" % (layer, np.mean(gk != rk)), flush=True)
            assert np.max(np.abs(gk - rk)) <= 1
            assert np.mean(gk != rk) < frac
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


def test_decode_splits_follow_the_context(ctx):
    """The attention split count of a captured step follows the context it is captured at
    (ti_qwen3_decode_splits: 16 up to 2048 positions, 32 up to 14336, then 64); a step
    captured at a short context and replayed over a long one gives the logits
    and token of a step captured there (only the split count, hence the summation order of
    the split merge, differs)."""
    cfg = dict(SMALL, head_dim=128, max_ctx=33000)
    m = abi.Qwen3(ctx, **cfg)
    try:
        want = {0: 16, 2047: 16, 2048: 32, 8191: 32, 14335: 32, 14336: 64, 16384: 64, 32767: 64, 32999: 64}
        assert {p: m.decode_splits(p) for p in want} == want
        with pytest.raises(abi.TIError):
            m.decode_splits(33000)
        Q.load_into(m, Q.make_weights(cfg, 5))
        P, chunk, nkv = 9000, 1000, cfg["n_kv_heads"] * cfg["head_dim"]
        rng = np.random.default_rng(8)
        kx = ctx.upload(rng.standard_normal(chunk * nkv).astype(np.float32))
        vx = ctx.upload(rng.standard_normal(chunk * nkv).astype(np.float32))
        for l in range(cfg["layers"]):
            for p0 in range(0, P, chunk):
                m.kv_write(l, kx, vx, chunk, p0)
        m.write_tokens(0, rng.integers(0, cfg["vocab"], P + 2).astype(np.int32))
        m.set_pos(P)
        m.decode()                                  # eager at the long context: 32 splits
        ctx.sync()
        want_logits = _logits(ctx, m, cfg["vocab"]).copy()
        want_tok = int(m.read_tokens(P + 1, 1)[0])
        m.set_pos(100)                              # captured at a short context: 16 splits
        ctx.graph_begin()
        m.decode()
        g = ctx.graph_end()
        try:
            m.set_pos(P)
            ctx.graph_launch(g)
            ctx.sync()
            got = _logits(ctx, m, cfg["vocab"])
            assert rel_err(got, want_logits) < TOL   # (an int8 code of the output may flip at a rounding edge)
            if margin_ok(want_logits):
                assert int(m.read_tokens(P + 1, 1)[0]) == want_tok
        finally:
            ctx.graph_destroy(g)
    finally:
        m.close()


def _seed_prefix(ctx, orc, m, ref, cfg, P, seed):
    """A seeded random prefix KV of P tokens in every layer, written through the KV
    quantizer into both the model and the reference decoder."""
    rng = np.random.default_rng(seed)
    nkv = cfg["n_kv_heads"] * cfg["head_dim"]
    for l in range(cfg["layers"]):
        K = rng.standard_normal(P * nkv).astype(np.float16).astype(np.float32)
        V = rng.standard_normal(P * nkv).astype(np.float16).astype(np.float32)
        kq, ks = orc.kv_quant(K)
        vq, vs = orc.kv_quant(V)
        dk = m.kv(l)
        TF.write_kv_codes(ctx, m, dk[0], kq, P, cfg)
        ctx.write(dk[1], ks)
        TF.write_kv_codes(ctx, m, dk[2], vq, P, cfg)
        ctx.write(dk[3], vs)
        ref.kv[l][0][:P], ref.kv[l][1][:P] = kq.reshape(P, -1), ks.reshape(P, -1)
        ref.kv[l][2][:P], ref.kv[l][3][:P] = vq.reshape(P, -1), vs.reshape(P, -1)


CFG_17B = dict(layers=2, hidden=2048, intermediate=6144, n_heads=16, n_kv_heads=8, head_dim=128, vocab=151936,
               rope_theta=1e6, rms_eps=1e-6, max_ctx=4200, max_tokens=1)


def test_qwen3_17b_geometry_over_4k_prefix(ctx, orc):
    """Qwen3-1.7B layer geometry (hidden 2048, intermediate 6144, 16/8 heads of 128,
    vocab 151936), 2 layers, one decode step at position 4096 over a seeded prefix KV
    written through the attention-prep quantizer."""
    cfg = CFG_17B
    W = Q.make_weights(cfg, 4)
    m = abi.Qwen3(ctx, **cfg)
    try:
        Q.load_into(m, W)
        ref = Q.RefDecoder(cfg, W, cfg["max_ctx"])
        P = 4096
        _seed_prefix(ctx, orc, m, ref, cfg, P, 9)
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


@pytest.mark.parametrize("T", [4, 8])
def test_qwen3_17b_geometry_batch8_over_4k_prefix(ctx, orc, T):
    """The batch configuration at the Qwen3-1.7B geometry: one T-token forward at
    positions 4096.. over a seeded 4k prefix (the fused matrix-core projections:
    three-matrix q/k/v, gate/up with the SwiGLU + quantQ8 epilogue, residual o/down;
    T = 4 normalises and quantises x in the q/k/v and gate/up prologues from the partial
    sums the residual projections write, T = 8 runs the per-token norm kernel).

    Checked teacher-forced, layer by layer (tests/qwen3_tf.py): each layer's float outputs
    within 1e-3 of the oracle's value of the GPU's own quantized inputs, code flips at most
    one step and rare; the last logits within 1e-3 of the oracle's lm_head of the GPU's
    final residual. Against T single-token forwards: the same next token where the margin
    allows, and logits within 5e-3 (the T-token GEMM adds the int32 group dots in another
    f32 order than the batch-1 GEMV, so an int8 activation code can land on the other side
    of a rounding boundary, which moves the end-to-end logits by ~1e-3; the reference's
    gemmDP4A and gemvDP4 differ the same way)."""
    cfg = dict(CFG_17B, max_tokens=8)
    W = Q.make_weights(cfg, 5)
    m, one = abi.Qwen3(ctx, **cfg), abi.Qwen3(ctx, **cfg)
    try:
        Q.load_into(m, W)
        Q.load_into(one, W)
        ref = Q.RefDecoder(cfg, W, cfg["max_ctx"])
        P = 4096
        _seed_prefix(ctx, orc, m, ref, cfg, P, 10)
        _seed_prefix(ctx, orc, one, Q.RefDecoder(cfg, W, cfg["max_ctx"]), cfg, P, 10)
        ids = np.array([4242, 17, 151935, 0, 99, 1000, 77777, 5], np.int32)[:T]
        layers, x_final = TF.traced(ctx, m, cfg, lambda: m.forward(ids, P))
        for i in range(T):
            one.forward(ids[i:i + 1], P + i)
        lt, l1 = _logits(ctx, m, cfg["vocab"]), _logits(ctx, one, cfg["vocab"])
        rows = TF.new_kv_rows(ctx, m, cfg, P, T)
        R = TF.teacher_forced(orc, cfg, W, ref.kv, layers, x_final, rows, P, T)
        rl = TF.final_logits(orc, cfg, W, x_final[T - 1])
        R.e("logits", rel_err(lt, rl))
        print("[qwen3] T=%d teacher-forced: %s" % (T, R), flush=True)
        TF.check(R)
        tok = int(m.read_tokens(P + T, 1)[0])
        assert tok == orc.argmax(lt)
        if margin_ok(rl):
            assert tok == orc.argmax(rl.astype(np.float32))
        print("[qwen3] T=%d forward vs %d single-token forwards: logits rel err %.2e" % (T, T, rel_err(lt, l1)), flush=True)
        assert rel_err(lt, l1) < 5e-3
        if margin_ok(l1, 5e-3):
            assert tok == int(one.read_tokens(P + T, 1)[0])
    finally:
        m.close()
        one.close()


@pytest.mark.parametrize("T", [2, 16])
def test_batched_forward_t_sizes(ctx, T):
    """T-token forwards at the ends of the fused range (2 and 16 tokens) give the same
    last logits as T single-token forwards."""
    cfg = dict(SMALL, max_tokens=16)
    W = Q.make_weights(cfg, 6)
    a, b = abi.Qwen3(ctx, **cfg), abi.Qwen3(ctx, **cfg)
    try:
        Q.load_into(a, W)
        Q.load_into(b, W)
        ids = (np.arange(T, dtype=np.int32) * 131 + 7) % cfg["vocab"]
        pre = np.array([1, 2, 3], np.int32)
        a.forward(pre, 0)
        a.forward(ids, 3)
        b.forward(pre, 0)
        for p in range(T):
            b.forward(ids[p:p + 1], 3 + p)
        la, lb = _logits(ctx, a, cfg["vocab"]), _logits(ctx, b, cfg["vocab"])
        assert rel_err(la, lb) < TOL
    finally:
        a.close()
        b.close()

@pytest.mark.parametrize("T", [12, 16])
def test_batched_forward_two_row_tiles(ctx, T):
    """T tokens x 2 query heads per KV head = 24 / 32 query rows: the T-token attention
    serves them as two row tiles of 16 (the second partly empty at T = 12), over a
    40-token prefix (cached key blocks and the new-key block); last logits as T
    single-token forwards."""
    cfg = dict(layers=2, hidden=256, intermediate=512, n_heads=4, n_kv_heads=2, head_dim=128, vocab=1000,
               rope_theta=1e6, rms_eps=1e-6, max_ctx=128, max_tokens=64)
    W = Q.make_weights(cfg, 9)
    a, b = abi.Qwen3(ctx, **cfg), abi.Qwen3(ctx, **cfg)
    try:
        Q.load_into(a, W)
        Q.load_into(b, W)
        pre = (np.arange(40, dtype=np.int32) * 37 + 11) % cfg["vocab"]
        ids = (np.arange(T, dtype=np.int32) * 131 + 7) % cfg["vocab"]
        a.forward(pre, 0)
        a.forward(ids, 40)
        b.forward(pre, 0)
        for p in range(T):
            b.forward(ids[p:p + 1], 40 + p)
        la, lb = _logits(ctx, a, cfg["vocab"]), _logits(ctx, b, cfg["vocab"])
        assert rel_err(la, lb) < TOL
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("T", [4, 8])
def test_batched_forward_graph_replays(ctx, T):
    """The T-token forward captured in a HIP graph and replayed (the device-side counters of
    the split-K down projection and of the attention merge reset themselves; for T = 4 the
    norm partial sums flow between the projections): every replay, with eager work and a
    synchronisation in between, gives the eager forward's logits and KV rows bit for bit."""
    cfg = dict(layers=1, hidden=2048, intermediate=6144, n_heads=16, n_kv_heads=8, head_dim=128, vocab=1000,
               rope_theta=1e6, rms_eps=1e-6, max_ctx=256, max_tokens=16)
    W = Q.make_weights(cfg, 12)
    m = abi.Qwen3(ctx, **cfg)
    try:
        Q.load_into(m, W)
        pre = (np.arange(16, dtype=np.int32) * 29 + 5) % cfg["vocab"]
        m.forward(pre, 0)
        P = 16
        ids = (np.arange(T, dtype=np.int32) * 131 + 7) % cfg["vocab"]
        m.forward(ids, P)
        l0 = _logits(ctx, m, cfg["vocab"]).copy()
        nkv = cfg["n_kv_heads"] * cfg["head_dim"]
        kq = m.kv(0)[0]
        k0 = TF.read_kv_codes(ctx, m, kq, 0, P + T, cfg)
        ctx.graph_begin()
        m.forward(None, P, T=T)
        g = ctx.graph_end()
        try:
            for rep in range(3):
                ctx.graph_launch(g)
                ctx.sync()
                assert np.array_equal(_logits(ctx, m, cfg["vocab"]), l0), rep
                assert np.array_equal(TF.read_kv_codes(ctx, m, kq, 0, P + T, cfg), k0), rep
                ctx.download(m.logits_ptr(), np.float32, 16)      # eager work between replays
        finally:
            ctx.graph_destroy(g)
    finally:
        m.close()


def test_qwen3_06b_geometry_batch8_over_1k_prefix(ctx, orc):
    """The batch-8 forward at the Qwen3-0.6B geometry (hidden 1024, intermediate 3072,
    16/8 heads of 128: the K = 1024 / 2048 / 3072 projection kernels and the KU = 4 norm
    kernel) over a seeded 1k prefix (a partial last key block), against 8 reference steps.
    One layer: with two, one int8 activation code of layer 1 that flips at a rounding
    boundary (f32 sums in a different order than the oracle's f64) moves the logits by a
    few 1e-3 on either path, batch-8 or single-token, depending on the seed."""
    cfg = dict(layers=1, hidden=1024, intermediate=3072, n_heads=16, n_kv_heads=8, head_dim=128, vocab=151936,
               rope_theta=1e6, rms_eps=1e-6, max_ctx=1100, max_tokens=8)
    W = Q.make_weights(cfg, 7)
    m = abi.Qwen3(ctx, **cfg)
    try:
        Q.load_into(m, W)
        ref = Q.RefDecoder(cfg, W, cfg["max_ctx"])
        P = 1000
        _seed_prefix(ctx, orc, m, ref, cfg, P, 11)
        ids = np.array([1, 151000, 42, 4242, 7, 99999, 3, 12345], np.int32)
        m.forward(ids, P)
        for i, t in enumerate(ids):
            rl, rt = ref.step(int(t), P + i)
        assert rel_err(_logits(ctx, m, cfg["vocab"]), rl) < TOL
        if margin_ok(rl):
            assert int(m.read_tokens(P + 8, 1)[0]) == rt
    finally:
        m.close()

def test_batched_forward_g1_16_tokens(ctx):
    """T = 16 tokens with one query head per KV head (G = 1: 16 query rows per KV head, the
    attention kernel's full row tile, causal over the 16 new keys) against 16 single-token
    forwards."""
    cfg = dict(layers=2, hidden=256, intermediate=512, n_heads=2, n_kv_heads=2, head_dim=128, vocab=1000,
               rope_theta=1e6, rms_eps=1e-6, max_ctx=128, max_tokens=16)
    W = Q.make_weights(cfg, 8)
    a, b = abi.Qwen3(ctx, **cfg), abi.Qwen3(ctx, **cfg)
    try:
        Q.load_into(a, W)
        Q.load_into(b, W)
        pre = (np.arange(40, dtype=np.int32) * 37 + 5) % cfg["vocab"]
        ids = (np.arange(16, dtype=np.int32) * 53 + 11) % cfg["vocab"]
        a.forward(pre[:16], 0)
        a.forward(pre[16:32], 16)
        a.forward(pre[32:], 32)
        a.forward(ids, 40)
        for p in range(40):
            b.forward(pre[p:p + 1], p)
        for p in range(16):
            b.forward(ids[p:p + 1], 40 + p)
        assert rel_err(_logits(ctx, a, cfg["vocab"]), _logits(ctx, b, cfg["vocab"])) < TOL
    finally:
        a.close()
        b.close()
