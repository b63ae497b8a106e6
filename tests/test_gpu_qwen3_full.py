"""The full Qwen3-1.7B int4 / int8-KV decode step at its own size: 28 layers, hidden 2048,
intermediate 6144, 16/8 heads of 128, vocabulary 151936, over seeded prefixes of 8192 and
32768 tokens, at batch 1 (one device-position decode step) and as the T = 8 forward (the
batch configuration: 8 consecutive tokens of one sequence, models/qwen3.js:3938-4069).

Each case is checked teacher-forced, layer by layer (tests/qwen3_tf.py): every float
output of every layer (q, k, v, attention, o_proj, swi, down) within 1e-3 of the oracle's
f64 value of the GPU's own quantized inputs; quantizer outputs of identical f32 inputs
bit-exact (rmsnormQ, attention and swi quantQ8); the new KV rows, and the int8 codes where
the GPU's f32 value and the oracle's f64 value fall on two sides of a rounding boundary,
within one step and rare; the logits of the last token within 1e-3 and its token the
reference's argmax of them. An independent oracle run from the same prefix (no teacher
forcing, its own codes all through) is reported beside it, with the logits' distance and
whether the greedy token agrees."""
import time

import numpy as np
import pytest

from tabinfer_amd import abi
import qwen3_tf as TF

pytestmark = pytest.mark.gpu

CFG = dict(layers=28, hidden=2048, intermediate=6144, n_heads=16, n_kv_heads=8, head_dim=128, vocab=151936,
           rope_theta=1e6, rms_eps=1e-6)
IDS = np.array([4242, 17, 151935, 0, 99, 1000, 77777, 5], np.int32)
# End to end, the f32 path and the f64 oracle drift apart through 28 layers of int8
# re-quantization (each flipped code moves its layer's output by one quantization step),
# so the independent run is held to a looser, stated bound (normwise over the logits).
E2E_BOUND = 0.1


@pytest.fixture(scope="module")
def ctx():
    c = abi.Ctx(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def weights():
    t0 = time.time()
    W = TF.make_weights(CFG, 1717, IDS)
    print("[full] weights %.1fs" % (time.time() - t0), flush=True)
    return W


@pytest.mark.parametrize("P,T", [(8192, 1), (8192, 8), (32768, 1), (32768, 8)])
def test_qwen3_17b_28_layers(ctx, orc, weights, P, T):
    print("[full] case P=%d T=%d" % (P, T), flush=True)
    t0 = time.time()
    cfg = dict(CFG, max_ctx=P + 16, max_tokens=T)
    d = TF.dims(cfg)
    m = abi.Qwen3(ctx, **cfg)
    try:
        TF.load_into(ctx, m, weights, d["H"])
        kv_host = TF.seed_prefix(ctx, m, cfg, P, P + T, seed=P + T)
        ids = IDS[:T]

        def step():
            if T == 1:
                m.write_tokens(P, ids)
                m.set_pos(P)
                m.decode()
            else:
                m.forward(ids, P)

        layers, x_final = TF.traced(ctx, m, cfg, step)
        print("[full] gpu step + setup %.1fs" % (time.time() - t0), flush=True)
        logits = ctx.download(m.logits_ptr(), np.float32, cfg["vocab"])
        tok = int(m.read_tokens(P + T, 1)[0])
        rows = TF.new_kv_rows(ctx, m, cfg, P, T)
    finally:
        m.close()
    t1 = time.time()
    R = TF.teacher_forced(orc, cfg, weights, kv_host, layers, x_final, rows, P, T)
    ref = TF.final_logits(orc, cfg, weights, x_final[T - 1])
    R.e("logits", TF.rel(logits, ref))
    print("[full] P=%d T=%d teacher-forced (%.1fs): %s" % (P, T, time.time() - t1, R), flush=True)
    TF.check(R)
    assert tok == orc.argmax(logits)                    # the reference's argmax of the GPU's logits
    s = np.sort(ref)
    if s[-1] - s[-2] > 4 * TF.TOL * np.max(np.abs(ref)):
        assert tok == orc.argmax(ref.astype(np.float32))
    # the oracle alone from the same prefix (its own codes all through)
    t2 = time.time()
    e2e = TF.oracle_decode(orc, cfg, weights, kv_host, IDS[:T], P)
    err = TF.rel(logits, e2e)
    print("[full] P=%d T=%d end to end (%.1fs): logits rel err %.3e, greedy token gpu %d oracle %d" %
          (P, T, time.time() - t2, err, tok, orc.argmax(e2e.astype(np.float32))), flush=True)
    assert err < E2E_BOUND
