"""GPU parity of the Bonsai ternary decoder (ti_bonsai_*: native/crates/n2-core/src/model.rs
forward on the GPU) against the oracle's restatement of that forward (tests/bonsai_ref.py).

- A small geometry loaded from a `.cpu.bin` container written in the packer's layout
  (the load path, ti_cpubin_open + ti_bonsai_load): prompt prefill token by token, then
  chained decode steps; greedy tokens equal to the oracle's own decode and logits within
  1e-3 of it.
- The Bonsai-1.7B geometry (28 layers, hidden 2048, intermediate 6144,
  16/8 heads of 128, vocabulary 151936) over a seeded 1024-token f32 prefix: one decode
  step checked teacher-forced, layer by layer: the int8 codes of every quantization point,
  every ternary GEMV output, the V row, every residual and the logits bit-exact; the norms,
  the K row, the attention and SwiGLU (tree sums and expf against the reference's
  sequential f32) within 1e-3; and the oracle alone from the same prefix alongside.
- A captured decode step replayed token after token gives the eager steps' tokens.
- Loading refuses a container whose shapes disagree with the config, or lacks a tensor.
"""
import numpy as np
import pytest

from tabinfer_amd import abi
import bonsai_ref as B

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=1024, intermediate=2048, n_heads=8, n_kv_heads=4, head_dim=128, vocab=1000,
             rope_theta=1e6, rms_eps=1e-6, max_ctx=64)
FULL = dict(layers=28, hidden=2048, intermediate=6144, n_heads=16, n_kv_heads=8, head_dim=128, vocab=151936,
            rope_theta=1e6, rms_eps=1e-6)


@pytest.fixture(scope="module")
def ctx():
    c = abi.Ctx(0)
    yield c
    c.close()


def margin_ok(logits):
    s = np.sort(np.asarray(logits, np.float64))
    return s[-1] - s[-2] > 4 * B.TOL * np.abs(s).max()


def test_small_from_container_prefill_and_decode(ctx, orc, tmp_path):
    cfg = SMALL
    W = B.make_weights(cfg, 1)
    path = str(tmp_path / "small.cpu.bin")
    B.write_cpubin(path, cfg, W)
    m = abi.Bonsai(ctx, **cfg)
    try:
        with abi.CpuBin(path=path) as c:
            assert c.summary()[1] == 3 + 11 * cfg["layers"]
            m.load(c)
        d = B.dims(cfg)
        kc = [np.zeros((cfg["max_ctx"], d["nkv"]), np.float32) for _ in range(cfg["layers"])]
        vc = [np.zeros((cfg["max_ctx"], d["nkv"]), np.float32) for _ in range(cfg["layers"])]
        ids = np.array([7, 999, 0, 512, 42], np.int32)
        m.forward(ids, 0)
        for p, t in enumerate(ids):
            ref = B.oracle_step(orc, cfg, W, kc, vc, t, p)
        got = ctx.download(m.logits_ptr(), np.float32, cfg["vocab"])
        assert B.rel(got, ref) < B.TOL
        tok = int(m.read_tokens(len(ids), 1)[0])
        assert tok == orc.n2_argmax(got)
        if margin_ok(ref):
            assert tok == orc.n2_argmax(ref)
        for p in range(len(ids), len(ids) + 4):                 # chained device-position steps
            m.decode()
            ref = B.oracle_step(orc, cfg, W, kc, vc, tok, p)
            got = ctx.download(m.logits_ptr(), np.float32, cfg["vocab"])
            assert B.rel(got, ref) < B.TOL, p
            tok = int(m.read_tokens(p + 1, 1)[0])
            assert tok == orc.n2_argmax(got)
            if margin_ok(ref):
                assert tok == orc.n2_argmax(ref)
        # the GPU's f32 KV rows against the oracle's
        for l in range(cfg["layers"]):
            k, v = m.kv(l)
            n = (len(ids) + 4) * d["nkv"]
            assert B.rel(ctx.download(k, np.float32, n), kc[l][:len(ids) + 4].ravel()) < 1e-4
            assert B.rel(ctx.download(v, np.float32, n), vc[l][:len(ids) + 4].ravel()) < 1e-4
    finally:
        m.close()


def test_bonsai_17b_geometry_teacher_forced_over_1k_prefix(ctx, orc):
    P = 1024
    cfg = dict(FULL, max_ctx=P + 8)
    d = B.dims(cfg)
    tok = 4242
    print("[bonsai] weights", flush=True)
    W = B.make_weights(cfg, 2, emb_ids=[tok])
    m = abi.Bonsai(ctx, **cfg)
    try:
        B.load_into(ctx, m, W, d["H"])
        rng = np.random.default_rng(3)
        kc = [np.zeros((P + 8, d["nkv"]), np.float32) for _ in range(cfg["layers"])]
        vc = [np.zeros((P + 8, d["nkv"]), np.float32) for _ in range(cfg["layers"])]
        for l in range(cfg["layers"]):
            kc[l][:P] = rng.standard_normal((P, d["nkv"])).astype(np.float32)
            vc[l][:P] = rng.standard_normal((P, d["nkv"])).astype(np.float32)
            k, v = m.kv(l)
            ctx.write(k, kc[l][:P])
            ctx.write(v, vc[l][:P])
        tb = B.trace_bytes(cfg)
        buf = ctx.alloc(tb)
        ctx.call("ti_buf_fill_u32", buf, 0x7FC00000, tb // 4)
        m.trace(buf)
        m.write_tokens(P, np.array([tok], np.int32))
        m.set_pos(P)
        m.decode()
        ctx.sync()
        m.trace(None)
        trace, fin = B.parse_trace(ctx.download(buf, np.uint32, tb // 4), cfg)
        logits = ctx.download(m.logits_ptr(), np.float32, cfg["vocab"])
        gtok = int(m.read_tokens(P + 1, 1)[0])
        rows_k, rows_v, new_k, new_v = [], [], [], []
        for l in range(cfg["layers"]):
            k, v = m.kv(l)
            rk = ctx.download(k, np.float32, (P + 1) * d["nkv"])
            rv = ctx.download(v, np.float32, (P + 1) * d["nkv"])
            rows_k.append(rk)
            rows_v.append(rv)
            new_k.append(rk[P * d["nkv"]:])
            new_v.append(rv[P * d["nkv"]:])
    finally:
        m.close()
    print("[bonsai] teacher forcing", flush=True)
    R = B.teacher_forced(orc, cfg, W, trace, fin, rows_k, rows_v, new_k, new_v, P, logits)
    print("[bonsai] config-1 step at %d, teacher-forced: %s" % (P, R), flush=True)
    R.check()
    assert gtok == orc.n2_argmax(logits)
    ref = B.oracle_step(orc, cfg, W, kc, vc, tok, P)
    err = B.rel(logits, ref)
    print("[bonsai] oracle alone: logits rel err %.3e, greedy token gpu %d oracle %d" % (err, gtok, orc.n2_argmax(ref)),
          flush=True)
    assert err < 0.1
    if margin_ok(ref):
        assert gtok == orc.n2_argmax(ref)


def test_decode_graph_replays_like_eager(ctx):
    cfg = SMALL
    W = B.make_weights(cfg, 4)
    m = abi.Bonsai(ctx, **cfg)
    try:
        B.load_into(ctx, m, W, cfg["hidden"])
        m.forward(np.array([3, 4, 5], np.int32), 0)
        start = int(m.read_tokens(3, 1)[0])
        logits = []
        for _ in range(4):
            m.decode()
            logits.append(ctx.download(m.logits_ptr(), np.float32, cfg["vocab"]).copy())
        eager = m.read_tokens(4, 4).copy()
        m.write_tokens(3, np.array([start], np.int32))
        m.set_pos(3)
        ctx.sync()
        ctx.graph_begin()
        m.decode()
        g = ctx.graph_end()
        try:
            for i in range(4):
                ctx.graph_launch(g)
                ctx.sync()
                assert int(m.read_tokens(4 + i, 1)[0]) == int(eager[i])
                assert np.array_equal(ctx.download(m.logits_ptr(), np.float32, cfg["vocab"]), logits[i])
        finally:
            ctx.graph_destroy(g)
    finally:
        m.close()


def test_load_refuses_mismatched_containers(ctx, tmp_path):
    cfg = SMALL
    W = B.make_weights(cfg, 5)
    m = abi.Bonsai(ctx, **cfg)
    try:
        bad = dict(W)
        bad.pop("model.layers.1.mlp.up_proj.weight")
        p = str(tmp_path / "missing.cpu.bin")
        B.write_cpubin(p, cfg, bad)
        with abi.CpuBin(path=p) as c:
            with pytest.raises(abi.TIError) as e:
                m.load(c)
        assert "missing tensor `model.layers.1.mlp.up_proj.weight`" in str(e.value)
        bad = dict(W)
        bad["model.layers.0.mlp.gate_proj.weight"] = W["model.layers.0.mlp.up_proj.weight"][0][:-256], W[
            "model.layers.0.mlp.up_proj.weight"][1][:-16]             # one row (K = 1024) short
        p = str(tmp_path / "shape.cpu.bin")
        B.write_cpubin(p, cfg, bad)
        with abi.CpuBin(path=p) as c:
            with pytest.raises(abi.TIError) as e:
                m.load(c)
        assert "gate_proj" in str(e.value)
        # a transposed projection has the right byte counts: gate_proj recorded as [H, I]
        # instead of [I, H] (model.rs:288-309 compares N and K one by one)
        H, I = cfg["hidden"], cfg["intermediate"]
        p = str(tmp_path / "transposed.cpu.bin")
        B.write_cpubin(p, cfg, W, shapes={"model.layers.1.mlp.gate_proj.weight": (H, I)})
        with abi.CpuBin(path=p) as c:
            with pytest.raises(abi.TIError) as e:
                m.load(c)
        assert ("model.layers.1.mlp.gate_proj.weight: container says [%d, %d], config implies [%d, %d]"
                % (H, I, I, H)) in str(e.value)
        p = str(tmp_path / "good.cpu.bin")
        B.write_cpubin(p, cfg, W)
        with abi.CpuBin(path=p) as c:
            m.load(c)
    finally:
        m.close()
