"""GPU parity of temperature sampling (models/qwen3.js:2713-2740, 4052, 4538-4567).

- ti_gumbel_noise against the oracle's f32 restatement at the vocabulary size (the same
  PCG hash bits; the logs within f32 rounding), and the reference's own self-test
  (:3198-3214) through ti_gumbel_noise + ti_argmax with its seed stream: the same index
  as the oracle at every draw, P(5)/P(9) = e, T -> 0 greedy.
- The decoder with a temperature: the fused lm_head adds the noise before its argmax; each
  sampled token equals the oracle's argmax of (the GPU's own logits + the oracle's noise
  of that step's seed), the seed stream advances once per sampled step (and not at
  temperature 0), a captured decode step samples as the eager one, and the logits agree
  with the oracle decoder within 1e-3.
"""
import math

import numpy as np
import pytest

from tabinfer_amd import abi
import qwen3_ref as Q

pytestmark = pytest.mark.gpu

TOL = 1e-3
SMALL = dict(layers=2, hidden=256, intermediate=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=1000,
             rope_theta=1e6, rms_eps=1e-6, max_ctx=64, max_tokens=8)


@pytest.fixture(scope="module")
def ctx():
    c = abi.Ctx(0)
    yield c
    c.close()


def perturbed_margin(v):
    s = np.sort(np.asarray(v, np.float64))
    return s[-1] - s[-2]


def test_gumbel_noise_matches_oracle(ctx, orc):
    N = 151936
    rng = np.random.default_rng(1)
    base = (rng.standard_normal(N) * 3).astype(np.float32)
    for seed, temp in ((orc.seed_next(orc.SEED_INIT), 1.0), (0xDEADBEEF, 0.7), (7, 2.5)):
        buf = ctx.upload(base)
        ctx.call("ti_gumbel_noise", buf, N, seed, np.float32(temp))
        got = ctx.download(buf, np.float32, N)
        want = orc.gumbel_noise(base, seed, temp)
        err = np.abs(got.astype(np.float64) - want) / np.maximum(1.0, np.abs(want))
        assert err.max() < 2e-6, (seed, temp, err.max())
        buf.free()


def test_reference_self_test_on_the_gpu(ctx, orc):
    N = 1024
    base = np.full(N, -100.0, np.float32)
    base[5], base[9] = 2.0, 1.0
    buf, hist = ctx.upload(base), ctx.zeros(4)
    st = orc.SEED_INIT
    c5 = c9 = other = 0
    for _ in range(240):
        st = orc.seed_next(st)
        ctx.write(buf, base)
        ctx.call("ti_gumbel_noise", buf, N, st, np.float32(1.0))
        ctx.call("ti_argmax", buf, N, hist, 0)
        got = int(ctx.download(hist, np.uint32, 1)[0])
        want_v = orc.gumbel_noise(base, st, 1.0)
        if perturbed_margin(want_v) > 1e-4:
            assert got == orc.argmax(want_v)
        c5 += got == 5
        c9 += got == 9
        other += got not in (5, 9)
    assert other == 0
    assert 1.6 < c5 / max(1, c9) < 4.6                     # e, with the reference's tolerance
    for _ in range(10):
        st = orc.seed_next(st)
        ctx.write(buf, base)
        ctx.call("ti_gumbel_noise", buf, N, st, np.float32(0.02))
        ctx.call("ti_argmax", buf, N, hist, 0)
        assert int(ctx.download(hist, np.uint32, 1)[0]) == 5


def _logits(ctx, m, vocab):
    return ctx.download(m.logits_ptr(), np.float32, vocab)


def test_decoder_samples_like_the_oracle(ctx, orc):
    W = Q.make_weights(SMALL, 11)
    m = abi.Qwen3(ctx, **SMALL)
    temp = 0.8
    try:
        Q.load_into(m, W)
        ref = Q.RefDecoder(SMALL, W, SMALL["max_ctx"])
        assert m.get_seed() == orc.SEED_INIT
        st = orc.SEED_INIT
        ids = np.array([11, 502, 7, 999, 123], np.int32)
        m.sampling(temp)
        m.forward(ids, 0)                                   # the first sampled token comes from the prefill
        for p, t in enumerate(ids):
            rl, _ = ref.step(int(t), p)
        checked = 0
        tok = None
        for p in range(5, 14):
            st = orc.seed_next(st)
            got = _logits(ctx, m, SMALL["vocab"])
            assert np.max(np.abs(got - rl)) / np.max(np.abs(rl)) < TOL
            tok = int(m.read_tokens(p, 1)[0])
            noisy = orc.gumbel_noise(got, st, temp)
            if perturbed_margin(noisy) > 1e-4:
                assert tok == orc.argmax(noisy), p
                checked += 1
            if p < 13:
                m.decode()
                rl, _ = ref.step(tok, p)
        assert checked >= 7
        assert m.get_seed() == st                           # one advance per sampled step
        # temperature 0: greedy, the seed stream does not move
        m.sampling(0.0)
        m.decode()
        assert m.get_seed() == st
        rl, rt = ref.step(tok, 13)
        got = _logits(ctx, m, SMALL["vocab"])
        assert int(m.read_tokens(14, 1)[0]) == orc.argmax(got)
    finally:
        m.close()


def test_sampled_graph_replay_matches_eager(ctx, orc):
    W = Q.make_weights(SMALL, 12)
    m = abi.Qwen3(ctx, **SMALL)
    try:
        Q.load_into(m, W)
        m.sampling(1.3)
        m.forward(np.array([3, 4, 5], np.int32), 0)
        start = int(m.read_tokens(3, 1)[0])
        s0 = m.get_seed()
        for _ in range(5):
            m.decode()
        eager = m.read_tokens(4, 5).copy()
        s_end = m.get_seed()
        m.write_tokens(3, np.array([start], np.int32))
        m.set_pos(3)
        m.seed(s0)
        ctx.sync()
        ctx.graph_begin()
        m.decode()
        g = ctx.graph_end()
        try:
            for i in range(5):
                ctx.graph_launch(g)
                ctx.sync()
                assert int(m.read_tokens(4 + i, 1)[0]) == int(eager[i])
        finally:
            ctx.graph_destroy(g)
        assert m.get_seed() == s_end
    finally:
        m.close()
