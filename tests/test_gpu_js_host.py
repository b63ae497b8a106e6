"""GPU parity through the JavaScript host (tabinfer_amd/host/qwen3-host.js over the N-API
addon): the reference's launchers, called by their models/qwen3.js / models/lfm25.js names
and argument order, give the oracle's results; loadModel streams a bf16 safetensors
checkpoint through the GPU quantizer bit-exactly; forward/generate/runConversation produce
the same tokens as the same decoder driven from Python; generate() (greedy and with a
temperature, through the three-deep readback pipeline) follows the oracle decoder; a
conversation that reuses the prefix cache after a maxTokens stop decodes as a cold one."""
import json
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

from tabinfer_amd import abi
import qwen3_ref as Q

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_js_host import write_safetensors  # noqa: E402

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
pytestmark = [pytest.mark.gpu, pytest.mark.skipif(NODE is None, reason="node is not installed")]


def run_spec(d, spec, files):
    for name, arr in files.items():
        np.ascontiguousarray(arr).tofile(os.path.join(d, name))
    with open(os.path.join(d, "spec.json"), "w") as f:
        json.dump(spec, f)
    print("[js] run_spec", d, flush=True)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "js", "run_spec.js"), d], stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True, timeout=300)
    assert r.returncode == 0, r.stdout
    return json.load(open(os.path.join(d, "result.json")))


def load(d, name, dt):
    return np.fromfile(os.path.join(d, name), dtype=dt)


def rel(got, want):
    want = np.asarray(want, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


def bf16(rng, n, scale=0.02):
    w = (rng.standard_normal(n) * scale).astype(np.float32)
    return (w.view(np.uint32) >> 16).astype(np.uint16)


def test_qwen3_launchers(tmp_path, orc):
    d = str(tmp_path)
    rng = np.random.default_rng(21)
    N, K, I, H = 384, 1024, 512, 1024
    x = rng.standard_normal(K).astype(np.float32)
    pack, sc = orc.quant_int4_bf16(bf16(rng, N * K), N, K)
    gp, gs = orc.quant_int4_bf16(bf16(rng, I * H), I, H)
    up, us = orc.quant_int4_bf16(bf16(rng, I * H), I, H)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16).view(np.uint16)
    wbf = bf16(rng, N * K)
    logits = rng.standard_normal(5000).astype(np.float32)
    emb = rng.standard_normal(50 * H).astype(np.float16).view(np.uint16)
    ids = np.array([3, 49, 0, 17], np.int32)
    files = {"x.bin": x, "pack.bin": pack, "sc.bin": sc, "gp.bin": gp, "gs.bin": gs, "up.bin": up, "us.bin": us,
             "nw.bin": nw, "wbf.bin": wbf, "logits.bin": logits, "emb.bin": emb, "ids.bin": ids}
    B = lambda n: {"buf": n}
    spec = {
        "buffers": dict({k[:-4]: {"file": k} for k in files},
                        y={"bytes": N * 4}, yq={"bytes": N * 4}, swi={"bytes": I * 4}, qp={"bytes": N * K // 2},
                        qs={"bytes": N * K // 32 * 2}, hist={"bytes": 64}, ey={"bytes": 4 * H * 4}),
        "calls": [
            {"fn": "L.quantQ8", "args": [B("x"), K]},
            {"read_dp4": "xq", "bytes": K, "out": "xq.out"},
            {"read_dp4": "xs", "bytes": K // 8, "out": "xs.out"},
            {"fn": "L.gemvDP4_only", "args": [B("pack"), B("sc"), B("y"), N, K, False]},
            {"read": "y", "bytes": N * 4, "out": "y.out"},
            {"fn": "L.gemvQ", "args": [B("x"), B("pack"), B("sc"), B("yq"), N, K, False, 4]},
            {"read": "yq", "bytes": N * 4, "out": "yq.out"},
            {"fn": "L.rmsnormQ", "args": [B("x"), B("nw"), H, 1e-6]},
            {"read_dp4": "xq", "bytes": H, "out": "nq.out"},
            {"fn": "L.gateUpSiluDP4_only", "args": [{"rec": {"pack": "gp", "scales": "gs", "N": I, "K": H}},
                                                    {"rec": {"pack": "up", "scales": "us", "N": I, "K": H}},
                                                    B("swi"), I, H, 2]},
            {"read": "swi", "bytes": I * 4, "out": "swi.out"},
            {"fn": "L.quantizeInt4Bf16", "args": [B("wbf"), {"rec": {"pack": "qp", "scales": "qs", "N": N, "K": K}}]},
            {"read": "qp", "bytes": N * K // 2, "out": "qp.out"},
            {"read": "qs", "bytes": N * K // 32 * 2, "out": "qs.out"},
            {"fn": "L.argmaxKernel", "args": [B("logits"), B("hist"), 5000, 7]},
            {"read": "hist", "bytes": 64, "out": "hist.out"},
            {"fn": "L.embedGather", "args": [B("ids"), {"emb": {"buf": "emb", "vocab": 50}}, B("ey"), 4, H, 0]},
            {"read": "ey", "bytes": 4 * H * 4, "out": "ey.out"},
        ],
    }
    run_spec(d, spec, files)
    xq, xs, _ = orc.quant_act_q8(x)
    assert np.array_equal(load(d, "xq.out", np.uint32), xq)
    assert np.array_equal(load(d, "xs.out", np.float32), xs)
    assert rel(load(d, "y.out", np.float32), orc.gemv_q4_q8(xq, xs, pack, sc, N, K)) < 1e-5
    assert rel(load(d, "yq.out", np.float32), orc.gemv_q4_f32(x, pack, sc, N, K)) < 1e-4
    nq, ns, _ = orc.rmsnorm_q8(x, nw, 1e-6)
    assert np.array_equal(load(d, "nq.out", np.uint32), nq)
    assert rel(load(d, "swi.out", np.float32), orc.gateup_silu_q4(nq, ns, gp, gs, up, us, I, H)) < 1e-4
    qp, qs = orc.quant_int4_bf16(wbf, N, K)
    assert np.array_equal(load(d, "qp.out", np.uint32), qp) and np.array_equal(load(d, "qs.out", np.uint16), qs)
    assert load(d, "hist.out", np.uint32)[7] == orc.argmax(logits)
    assert np.array_equal(load(d, "ey.out", np.float32), orc.embed(ids, emb, 4, H))


def test_attention_ternary_moe_launchers(tmp_path, orc):
    d = str(tmp_path)
    rng = np.random.default_rng(22)
    nHq, nKv, hd, pos, cap = 4, 2, 128, 37, 64
    theta, eps = 1e6, 1e-6
    q = rng.standard_normal(nHq * hd).astype(np.float32)
    k = rng.standard_normal(nKv * hd).astype(np.float32)
    v = rng.standard_normal(nKv * hd).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float16).view(np.uint16)
    kw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float16).view(np.uint16)
    row = nKv * hd
    # a cache whose rows [0, pos) are already filled (snorm codes and scales)
    kq = rng.integers(0, 2 ** 32, cap * row // 4, dtype=np.uint64).astype(np.uint32)
    vq = rng.integers(0, 2 ** 32, cap * row // 4, dtype=np.uint64).astype(np.uint32)
    ks = rng.uniform(0.01, 0.03, cap * row // 32).astype(np.float32)
    vs = rng.uniform(0.01, 0.03, cap * row // 32).astype(np.float32)
    # ternary: rows of Q2_0_g64 codes, int8 activation
    n, kk = 256, 2048
    codes, tsc, act, xsum, _, _ = orc.n2_fixture(n, kk, 0xC0FFEE)
    # MoE: router over 8 experts, top-2, int3 experts (N=64, K=256)
    nE, topk, mN, mK = 8, 2, 64, 256
    lg = rng.standard_normal(nE).astype(np.float32)
    bias = (0.1 * rng.standard_normal(nE)).astype(np.float32)
    p3 = rng.integers(0, 2 ** 32, nE * mN * mK // 32 * 3, dtype=np.uint64).astype(np.uint32)
    s3 = rng.uniform(0.01, 0.02, nE * mN * mK // 32).astype(np.float16).view(np.uint16)
    mx = rng.standard_normal(mK).astype(np.float32)
    files = {"q.bin": q, "k.bin": k, "v.bin": v, "qw.bin": qw, "kw.bin": kw, "kq.bin": kq, "ks.bin": ks, "vq.bin": vq,
             "vs.bin": vs, "codes.bin": codes, "tsc.bin": tsc, "act.bin": act, "xsum.bin": xsum, "lg.bin": lg,
             "bias.bin": bias, "p3.bin": p3, "s3.bin": s3, "mx.bin": mx}
    B = lambda n_: {"buf": n_}
    kv = {"kv": {"kq": "kq", "ks": "ks", "vq": "vq", "vs": "vs"}}
    spec = {
        "buffers": dict({f[:-4]: {"file": f} for f in files}, qr={"bytes": nHq * hd * 4}, o={"bytes": nHq * hd * 4},
                        tout={"bytes": n * 4}, idx={"bytes": topk * 4}, wt={"bytes": topk * 4},
                        my={"bytes": topk * mN * 4}),
        "calls": [
            {"fn": "L.attnPrepQ8", "args": [B("q"), B("k"), B("v"), B("qw"), B("kw"), B("qr"), kv, nHq, nKv, hd, pos, theta, eps]},
            {"read": "qr", "bytes": nHq * hd * 4, "out": "qr.out"},
            {"read": "kq", "bytes": cap * row, "out": "kq.out"},
            {"read": "ks", "bytes": cap * row // 8, "out": "ks.out"},
            {"read": "vq", "bytes": cap * row, "out": "vq.out"},
            {"read": "vs", "bytes": cap * row // 8, "out": "vs.out"},
            {"fn": "L.attnDecodeStreamQ8", "args": [B("qr"), B("kq"), B("ks"), B("vq"), B("vs"), B("o"), pos + 1, nHq, nKv, hd, 0]},
            {"read": "o", "bytes": nHq * hd * 4, "out": "o.out"},
            {"fn": "Tern.gemv_tern", "args": [B("tout"), B("codes"), B("tsc"), B("act"), B("xsum"), n, kk]},
            {"read": "tout", "bytes": n * 4, "out": "tout.out"},
            {"fn": "Moe.router", "args": [B("lg"), B("bias"), B("idx"), B("wt"), 1, nE, topk]},
            {"read": "idx", "bytes": topk * 4, "out": "idx.out"},
            {"read": "wt", "bytes": topk * 4, "out": "wt.out"},
            {"fn": "Moe.idxGemv3", "args": [B("mx"), {"rec3": {"pack": "p3", "scales": "s3", "nE": nE}}, B("idx"), B("my"),
                                            topk, mN, mK, mK, topk]},
            {"read": "my", "bytes": topk * mN * 4, "out": "my.out"},
        ],
    }
    run_spec(d, spec, files)
    qr, k1, ks1, v1, vs1 = orc.attn_prep_q8(q, k, v, qw, kw, nHq, nKv, hd, pos, theta, eps)
    assert np.array_equal(load(d, "qr.out", np.float32), qr)
    gkq = load(d, "kq.out", np.uint32).reshape(cap, -1)
    assert np.array_equal(gkq[pos], k1) and np.array_equal(load(d, "ks.out", np.float32).reshape(cap, -1)[pos], ks1)
    assert np.array_equal(load(d, "vq.out", np.uint32).reshape(cap, -1)[pos], v1)
    assert np.array_equal(load(d, "vs.out", np.float32).reshape(cap, -1)[pos], vs1)
    kq[pos * row // 4:(pos + 1) * row // 4], vq[pos * row // 4:(pos + 1) * row // 4] = k1, v1
    ks[pos * row // 32:(pos + 1) * row // 32], vs[pos * row // 32:(pos + 1) * row // 32] = ks1, vs1
    assert rel(load(d, "o.out", np.float32), orc.attn_decode_q8(qr, kq, ks, vq, vs, pos + 1, nHq, nKv, hd)) < 1e-3
    assert np.array_equal(load(d, "tout.out", np.float32), orc.tern_gemv_scalar(codes, tsc, act, xsum, n, kk))
    oi, ow = orc.router(lg, bias, 1, nE, topk)
    assert np.array_equal(load(d, "idx.out", np.int32), oi)
    assert np.abs(load(d, "wt.out", np.float32) - ow).max() < 1e-6
    assert rel(load(d, "my.out", np.float32), orc.moe_gemv_q3(mx, p3, s3, oi, topk, mN, mK, mK, topk)) < 1e-4


def test_ternary_format_launchers(tmp_path, orc):
    """quantizeTernaryBf16 (bit-exact, and null for a continuous tensor), then gemvTern_only,
    projGemv, gateUpSiluDP4_only and linearQ (T = 1 and T = 3) routing the ternary records."""
    from tern2_data import ternary_bf16
    d = str(tmp_path)
    rng = np.random.default_rng(24)
    N, K, I = 256, 2048, 512
    w, g, u = ternary_bf16(rng, N, K), ternary_bf16(rng, I, K), ternary_bf16(rng, I, K)
    cont = bf16(rng, N * K)
    x = rng.standard_normal(3 * K).astype(np.float32)
    files = {"w.bin": w, "g.bin": g, "u.bin": u, "cont.bin": cont, "x.bin": x}
    B = lambda n: {"buf": n}
    spec = {
        "buffers": dict({k[:-4]: {"file": k} for k in files}, y={"bytes": N * 4}, yp={"bytes": N * 4},
                        swi={"bytes": I * 4}, yl={"bytes": 3 * N * 4}),
        "calls": [
            {"tern_quant": "tw", "src": "w", "N": N, "K": K},
            {"tern_quant": "tg", "src": "g", "N": I, "K": K},
            {"tern_quant": "tu", "src": "u", "N": I, "K": K},
            {"tern_quant": "tc", "src": "cont", "N": N, "K": K},
            {"fn": "L.quantQ8", "args": [B("x"), K]},
            {"fn": "L.gemvTern_only", "args": [{"trec": "tw"}, B("y"), N, K, False]},
            {"read": "y", "bytes": N * 4, "out": "y.out"},
            {"fn": "L.projGemv", "args": [{"trec": "tw"}, B("yp"), N, K, False]},
            {"read": "yp", "bytes": N * 4, "out": "yp.out"},
            {"fn": "L.gateUpSiluDP4_only", "args": [{"trec": "tg"}, {"trec": "tu"}, B("swi"), I, K]},
            {"read": "swi", "bytes": I * 4, "out": "swi.out"},
            {"fn": "L.linearQ", "args": [B("x"), {"trec": "tw"}, B("yl"), 3, N, K, False]},
            {"read": "yl", "bytes": 3 * N * 4, "out": "yl.out"},
        ],
    }
    res = run_spec(d, spec, files)
    assert res["tw"] and res["tg"] and res["tu"] and not res["tc"]
    pw, sw = orc.quant_tern_bf16(w, N, K)
    assert np.array_equal(load(d, "tw.pack", np.uint32), pw) and np.array_equal(load(d, "tw.scales", np.uint16), sw)
    pg, sg = orc.quant_tern_bf16(g, I, K)
    pu, su = orc.quant_tern_bf16(u, I, K)
    xq, xs, _ = orc.quant_act_q8(x[:K])
    want = orc.gemv_tern2(xq, xs, pw, sw, N, K)
    assert rel(load(d, "y.out", np.float32), want) < 1e-3
    assert np.array_equal(load(d, "yp.out", np.float32), load(d, "y.out", np.float32))
    assert rel(load(d, "swi.out", np.float32), orc.gateup_silu_tern2(xq, xs, pg, sg, pu, su, I, K)) < 1e-3
    yl = load(d, "yl.out", np.float32).reshape(3, N)
    for t in range(3):
        xq, xs, _ = orc.quant_act_q8(x[t * K:(t + 1) * K])
        assert rel(yl[t], orc.gemv_tern2(xq, xs, pw, sw, N, K)) < 1e-3


SMALL = dict(layers=2, hidden=256, intermediate=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=1000,
             rope_theta=1e6, rms_eps=1e-6)


def test_load_forward_generate_conversation(tmp_path, orc):
    """A bf16 checkpoint through loadModel, then forward / generate / runConversation in
    JS, against the same decoder driven through ctypes with oracle-quantized weights."""
    d = str(tmp_path)
    rng = np.random.default_rng(23)
    c = SMALL
    H, I, hd = c["hidden"], c["intermediate"], c["head_dim"]
    nq, nkv = c["n_heads"] * hd, c["n_kv_heads"] * hd
    shapes = {"self_attn.q_proj.weight": (nq, H), "self_attn.k_proj.weight": (nkv, H), "self_attn.v_proj.weight": (nkv, H),
              "self_attn.o_proj.weight": (H, nq), "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
              "mlp.down_proj.weight": (H, I)}
    T = {}
    for l in range(c["layers"]):
        p = "model.layers.%d." % l
        for nm, (N, K) in shapes.items():
            T[p + nm] = (N, K, bf16(rng, N * K))
        for nm, n in (("input_layernorm.weight", H), ("post_attention_layernorm.weight", H),
                      ("self_attn.q_norm.weight", hd), ("self_attn.k_norm.weight", hd)):
            T[p + nm] = (n, None, bf16(rng, n, 0.1))
    T["model.norm.weight"] = (H, None, bf16(rng, H, 0.1))
    T["model.embed_tokens.weight"] = (c["vocab"], H, bf16(rng, c["vocab"] * H, 0.5))   # tied lm_head
    # norms around 1: add 1.0 in f32 before the bf16 truncation
    for nm, (n, K, b) in list(T.items()):
        if K is None:
            f = (b.astype(np.uint32) << 16).view(np.float32) + np.float32(1.0)
            T[nm] = (n, None, (f.view(np.uint32) >> 16).astype(np.uint16))
    ckpt = os.path.join(d, "model.safetensors")
    write_safetensors(ckpt, {nm: ("BF16", (n,) if K is None else (n, K), b.tobytes()) for nm, (n, K, b) in T.items()})

    prompt = [11, 502, 7, 999, 123, 4, 88]
    spec = {"model": {"config": c, "nCtx": 128, "safetensors": ckpt, "prompt": prompt, "maxTokens": 20,
                      "dump": ["model.layers.1.mlp.down_proj.weight", "lm_head.weight", "model.norm.weight"],
                      "chat": {"stop": -1}}}
    res = run_spec(d, spec, {})

    # the loader's device tensors equal the oracle's quantization / conversion of the same bf16
    N, K, b = T["model.layers.1.mlp.down_proj.weight"]
    qp, qs = orc.quant_int4_bf16(b, N, K)
    assert np.array_equal(load(d, "model.layers.1.mlp.down_proj.weight.data", np.uint32), qp)
    assert np.array_equal(load(d, "model.layers.1.mlp.down_proj.weight.scales", np.uint16), qs)
    N, K, b = T["model.embed_tokens.weight"]
    lp, ls = orc.quant_int4_bf16(b, N, K)
    assert np.array_equal(load(d, "lm_head.weight.data", np.uint32), lp)
    n, _, b = T["model.norm.weight"]
    want = np.array([orc.f32_to_f16_q3(np.uint32(int(v) << 16).view(np.float32)) for v in b], np.uint16)
    assert np.array_equal(load(d, "model.norm.weight.data", np.uint16), want)

    # the same decoder through ctypes, weights prepared by the oracle
    m = abi.Qwen3(abi.Ctx(0), **c, max_ctx=128, max_tokens=8)
    try:
        for nm, (n, K, b) in T.items():
            dd, nd, s, ns = m.tensor(nm)
            if K is not None and s:
                p_, s_ = orc.quant_int4_bf16(b, n, K)
                m.ctx.write(dd, p_)
                m.ctx.write(s, s_)
            else:
                m.ctx.write(dd, np.array([orc.f32_to_f16_q3(np.uint32(int(v) << 16).view(np.float32)) for v in b], np.uint16))
        dd, nd, s, ns = m.tensor("lm_head.weight")
        m.ctx.write(dd, lp)
        m.ctx.write(s, ls)
        m.forward(np.array(prompt, np.int32), 0)
        L = len(prompt)
        toks = [int(m.read_tokens(L, 1)[0])]
        for _ in range(19):
            m.decode()
            toks.append(int(m.read_tokens(L + len(toks), 1)[0]))
    finally:
        m.close()
        m.ctx.close()
    assert res["forward"] == toks[0]
    assert res["generate"] == toks
    # runConversation: the token stream arrives as content deltas between round_start and agent_done
    ev = res["events"]
    kinds = [e["type"] for e in ev]
    assert kinds[0] == "round_start" and kinds[-1] == "agent_done" and "error" not in kinds
    text = "".join(e["delta"].get("content", "") for e in ev if e["type"] == "delta")
    assert text == "".join("<%d>" % t for t in toks)
    usage = [e for e in ev if e["type"] == "usage"][0]["usage"]
    assert usage["prompt_tokens"] == L


def _checkpoint(d, rng, c):
    """A bf16 safetensors checkpoint of geometry c (tied embeddings) and the oracle's view
    of it: int4 projections by the oracle quantizer, f16 norms / embeddings by the
    loader's own bf16 -> f16 rounding."""
    H, I, hd = c["hidden"], c["intermediate"], c["head_dim"]
    nq, nkv = c["n_heads"] * hd, c["n_kv_heads"] * hd
    shapes = {"self_attn.q_proj.weight": (nq, H), "self_attn.k_proj.weight": (nkv, H), "self_attn.v_proj.weight": (nkv, H),
              "self_attn.o_proj.weight": (H, nq), "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
              "mlp.down_proj.weight": (H, I)}
    T = {}
    for l in range(c["layers"]):
        p = "model.layers.%d." % l
        for nm, (N, K) in shapes.items():
            T[p + nm] = (N, K, bf16(rng, N * K))
        for nm, n in (("input_layernorm.weight", H), ("post_attention_layernorm.weight", H),
                      ("self_attn.q_norm.weight", hd), ("self_attn.k_norm.weight", hd)):
            T[p + nm] = (n, None, bf16(rng, n, 0.1))
    T["model.norm.weight"] = (H, None, bf16(rng, H, 0.1))
    T["model.embed_tokens.weight"] = (c["vocab"], H, bf16(rng, c["vocab"] * H, 0.5))
    for nm, (n, K, b) in list(T.items()):
        if K is None:
            f = (b.astype(np.uint32) << 16).view(np.float32) + np.float32(1.0)
            T[nm] = (n, None, (f.view(np.uint32) >> 16).astype(np.uint16))
    ckpt = os.path.join(d, "model.safetensors")
    write_safetensors(ckpt, {nm: ("BF16", (n,) if K is None else (n, K), b.tobytes()) for nm, (n, K, b) in T.items()})
    return T, ckpt


def _oracle_weights(orc, T):
    f16 = lambda b: np.array([orc.f32_to_f16_q3(np.uint32(int(v) << 16).view(np.float32)) for v in b], np.uint16)
    W = {}
    for nm, (n, K, b) in T.items():
        if nm == "model.embed_tokens.weight":
            W[nm] = f16(b)
            W["lm_head.weight"] = orc.quant_int4_bf16(b, n, K)
        elif K is None:
            W[nm] = f16(b)
        else:
            W[nm] = orc.quant_int4_bf16(b, n, K)
    return W


def test_generate_follows_the_oracle_decoder(tmp_path, orc):
    """generate() in JS (prefill, then the pipelined decodeLoop: 3 batches of 32 steps in
    flight) against the oracle decoder token by token, greedy and at temperature 0.7 with
    the reference's seed stream. The oracle is fed the GPU's tokens; a token is compared
    where the oracle's top two (perturbed) logits are apart by more than 4e-3 of their
    scale (the GPU's logits are within 1e-3), and most of them must be. Then a conversation continued after a maxTokens stop (prefix cache reused) gives
    the same tokens as the same conversation prefilled cold."""
    d = str(tmp_path)
    rng = np.random.default_rng(31)
    c = SMALL
    T, ckpt = _checkpoint(d, rng, c)
    W = _oracle_weights(orc, T)
    prompt = [11, 502, 7, 999, 123, 4, 88, 5, 600]
    n_tok, temp = 70, 0.7
    spec = {"model": {"config": c, "nCtx": 160, "safetensors": ckpt, "prompt": prompt, "maxTokens": 4,
                      "gens": [{"prompt": prompt, "maxTokens": n_tok}, {"prompt": prompt, "maxTokens": n_tok, "temperature": temp}],
                      "prefix": {"first": [{"role": "user", "content": "3 14 15 92 65"}],
                                 "second": [{"role": "user", "content": "35 89 79"}], "maxTokens": 12}}}
    res = run_spec(d, spec, {})
    for run, t in ((res["gens"][0], 0.0), (res["gens"][1], temp)):
        assert len(run) == n_tok
        ref = Q.RefDecoder(c, W, 160)
        for p, tk in enumerate(prompt):
            rl, _ = ref.step(int(tk), p)
        st, compared = orc.SEED_INIT, 0
        for j, got in enumerate(run):
            v = rl.astype(np.float32)
            if t > 0:
                st = orc.seed_next(st)
                v = orc.gumbel_noise(v, st, t)
            srt = np.sort(v.astype(np.float64))
            if srt[-1] - srt[-2] > 4e-3 * np.abs(rl).max():    # not a near tie
                assert got == orc.argmax(v), (t, j)
                compared += 1
            rl, _ = ref.step(int(got), len(prompt) + j)         # the oracle continues from the GPU's token
        print("[js] generate at T=%.1f: %d of %d tokens compared with the oracle" % (t, compared, n_tok), flush=True)
        assert compared >= 40
    pr = res["prefix"]
    assert len(pr["first"].split()) == 12
    assert pr["warm"] == pr["cold"] and len(pr["warm"].split()) == 12


def test_quant_cache_and_text_prompts(tmp_path, orc):
    """loadModel({quantCache}) (models/qwen3.js:3626-3759): a checkpoint load writes the cache,
    a load from the cache alone gives every tensor byte for byte and the same generated
    tokens, a manifest of another geometry is a miss (the checkpoint is read and the cache
    rewritten). Then text through the tokenizer.json of tests/test_js_tokenizer.py's kind:
    generate()'s prompt is the library's ChatML encoding, its streamed pieces join to its
    result, and a conversation reports the same prompt length in its usage."""
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import Regex, Tokenizer, decoders, models, pre_tokenizers, trainers
    from test_js_tokenizer import QWEN, SPECIALS
    d = str(tmp_path)
    rng = np.random.default_rng(41)
    c = dict(SMALL)
    T, ckpt = _checkpoint(d, rng, c)
    os.makedirs(os.path.join(d, "b"))
    _, ckpt_b = _checkpoint(os.path.join(d, "b"), np.random.default_rng(43), c)   # same geometry, other weights
    names = ["model.embed_tokens.weight", "lm_head.weight", "model.norm.weight", "model.layers.1.mlp.down_proj.weight",
             "model.layers.0.self_attn.q_norm.weight", "model.layers.1.self_attn.v_proj.weight"]
    prompt = [11, 502, 7, 999, 123]
    # a small byte-level BPE tokenizer (ids below the model's vocabulary)
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.Sequence([pre_tokenizers.Split(Regex(QWEN), behavior="isolated", invert=False),
                                                 pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    tok.train_from_iterator([open(os.path.join(ROOT, "DESIGN.md"), encoding="utf-8").read(), "你好 🙂 café"] * 4,
                            trainers.BpeTrainer(vocab_size=900, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                                special_tokens=SPECIALS, show_progress=False))
    assert tok.get_vocab_size() <= c["vocab"]
    tdir = os.path.join(d, "tok")
    os.makedirs(tdir)
    tok.save(os.path.join(tdir, "tokenizer.json"))
    text, system = "Summarise the decode attention in one line, please 🙂", "You are a careful assistant. " * 6
    spec = {"model": {"config": c, "nCtx": 256, "safetensors": ckpt, "prompt": prompt, "maxTokens": 2,
                      "qcache": {"dir": os.path.join(d, "qc"), "dump": names, "prompt": prompt, "maxTokens": 24,
                                 "safetensorsB": ckpt_b},
                      "tokchat": {"tokenizer": tdir, "text": text, "system": system, "maxTokens": 20}}}
    res = run_spec(d, spec, {})
    q = res["qcache"]
    assert q["fromCache"] == [False, True, False, True, False, True]
    rd = lambda tag, nm, part: open(os.path.join(d, "%s.%s.%s" % (tag, nm, part)), "rb").read()
    for nm in names:
        for part in ("data", "scales"):
            if os.path.exists(os.path.join(d, "a.%s.%s" % (nm, part))):
                assert rd("a", nm, part) == rd("b", nm, part), (nm, part)
                # checkpoint B of the same geometry: its own bytes, not A's from the cache
                assert rd("c", nm, part) != rd("a", nm, part) and rd("c", nm, part) == rd("d", nm, part), (nm, part)
    assert q["manifestB"]["source"]["files"][0]["path"] == os.path.abspath(ckpt_b)
    assert "no weights" in q["noWeights"] and q["modelAfterNoWeights"]
    assert q["gens"][0] == q["gens"][1] == q["gens"][2] and len(q["gens"][0]) == 24
    assert q["manifest"]["config"]["vocab"] == c["vocab"] and q["manifest"]["chunkSize"] == 64 << 20
    tc = res["tokchat"]
    want = tok.encode("<|im_start|>user\n%s<|im_end|>\n<|im_start|>assistant\n" % text).ids
    assert tc["prefill"] == len(want)
    assert "".join(tc["pieces"]) == tc["text"]
    usage = [e for e in tc["events"] if e["type"] == "usage"]
    chat = "<|im_start|>system\n%s<|im_end|>\n<|im_start|>user\n%s<|im_end|>\n<|im_start|>assistant\n" % (system, text)
    assert usage and usage[0]["usage"]["prompt_tokens"] == len(tok.encode(chat).ids)
    assert any(e["type"] == "agent_done" for e in tc["events"]) and not any(e["type"] == "error" for e in tc["events"])


def test_self_test_kernels(tmp_path):
    """selfTestKernels() (models/qwen3.js:2753-3219, exported at :5529): every check of the
    host's own launcher self-test passes on the GPU (each launcher against an f64
    restatement in JS, the quantizers as round trips, the argmax tie order, the Gumbel
    sampler's frequencies)."""
    res = run_spec(str(tmp_path), {"selftest": True}, {})
    st = res["selftest"]
    print("[js] selfTestKernels:", ", ".join("%s %.2e" % (c["name"], c["err"]) for c in st), flush=True)
    names = [c["name"] for c in st]
    assert len(names) >= 18 and len(set(names)) == len(names)
    assert all(c["ok"] for c in st), [c for c in st if not c["ok"]]


def test_kv_layout_and_write(tmp_path, orc):
    """qwen3_kv_layout / qwen3_kv_write from JS on a model with 8 KV heads: the code rows hold
    a spare slot, the written rows equal the oracle's kvQuantWrite of the same K/V (bit for
    bit), and the spare slot is left as it was."""
    d = str(tmp_path)
    c = dict(layers=2, hidden=256, intermediate=512, n_heads=16, n_kv_heads=8, head_dim=128, vocab=1000,
             rope_theta=1e6, rms_eps=1e-6)
    T, pos, layer, nKv, hd = 3, 37, 1, 8, 128
    n = T * nKv * hd
    i = np.arange(n)
    kr = (np.sin(i * 0.11) * (1 + (i % 5))).astype(np.float32)
    vv = (np.cos(i * 0.07) * (1 + (i % 3))).astype(np.float32)
    spec = {"buffers": {"kr": {"file": "kr.bin"}, "v": {"file": "v.bin"}},
            "kvw": {"config": c, "nCtx": 64, "layer": layer, "T": T, "pos": pos, "kr": "kr", "v": "v"}}
    res = run_spec(d, spec, {"kr.bin": kr, "v.bin": vv})
    slots = res["kvw"]["slots"]
    assert slots == nKv + 1 and res["kvw"]["kvSlots"] == slots
    for src, q, s in ((kr, "kq", "ks"), (vv, "vq", "vs")):
        want_q, want_s = orc.kv_quant(src)
        before = load(d, "kvw_before." + q, np.uint8).reshape(T, slots, hd)
        after = load(d, "kvw_after." + q, np.uint8).reshape(T, slots, hd)
        assert np.array_equal(after[:, :nKv].reshape(-1), want_q.view(np.uint8))
        assert np.array_equal(after[:, nKv:], before[:, nKv:])
        assert np.array_equal(load(d, "kvw_after." + s, np.float32), want_s)
