"""Test helpers for the Qwen3 decoder: synthetic checkpoints and a reference
decode step composed from the oracle's functions (test infrastructure)."""
import numpy as np

from oracle import oracle as orc


def bf16(rng, n, std=0.02):
    w = (rng.standard_normal(n) * std).astype(np.float32)
    return (w.view(np.uint32) >> 16).astype(np.uint16)


def make_weights(cfg, seed):
    """int4-quantized projections (oracle quantizer), f16 norms ~1, f16 embeddings."""
    rng = np.random.default_rng(seed)
    H, I, hd = cfg["hidden"], cfg["intermediate"], cfg["head_dim"]
    nq, nkv = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    W = {}
    shapes = {"self_attn.q_proj.weight": (nq, H), "self_attn.k_proj.weight": (nkv, H), "self_attn.v_proj.weight": (nkv, H),
              "self_attn.o_proj.weight": (H, nq), "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
              "mlp.down_proj.weight": (H, I)}
    norm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float16).view(np.uint16)
    for l in range(cfg["layers"]):
        p = "model.layers.%d." % l
        for name, (N, K) in shapes.items():
            W[p + name] = orc.quant_int4_bf16(bf16(rng, N * K), N, K)
        W[p + "input_layernorm.weight"] = norm(H)
        W[p + "post_attention_layernorm.weight"] = norm(H)
        W[p + "self_attn.q_norm.weight"] = norm(hd)
        W[p + "self_attn.k_norm.weight"] = norm(hd)
    W["model.embed_tokens.weight"] = (rng.standard_normal(cfg["vocab"] * H) * 0.5).astype(np.float16).view(np.uint16)
    W["model.norm.weight"] = norm(H)
    W["lm_head.weight"] = orc.quant_int4_bf16(bf16(rng, cfg["vocab"] * H), cfg["vocab"], H)
    return W


def load_into(model, W):
    ctx = model.ctx
    for name, val in W.items():
        d, nd, s, ns = model.tensor(name)
        if isinstance(val, tuple):
            assert val[0].nbytes == nd and val[1].nbytes == ns, name
            ctx.write(d, val[0])
            ctx.write(s, val[1])
        else:
            assert val.nbytes == nd, name
            ctx.write(d, val)


class RefDecoder:
    """Decode steps composed from oracle functions, in the reference's order
    (models/qwen3.js:3959-4055, T=1 path)."""

    def __init__(self, cfg, W, cap):
        self.cfg, self.W = cfg, W
        nkv = cfg["n_kv_heads"] * cfg["head_dim"]
        self.kq = np.zeros((cap, nkv // 4), np.uint32)
        self.ks = np.zeros((cap, nkv // 32), np.float32)
        self.vq = np.zeros((cap, nkv // 4), np.uint32)
        self.vs = np.zeros((cap, nkv // 32), np.float32)
        self.kv = [(self.kq.copy(), self.ks.copy(), self.vq.copy(), self.vs.copy()) for _ in range(cfg["layers"])]

    def step(self, tok, pos):
        c, W = self.cfg, self.W
        H, I, hd = c["hidden"], c["intermediate"], c["head_dim"]
        nHq, nKv = c["n_heads"], c["n_kv_heads"]
        nq, nkv = nHq * hd, nKv * hd
        eps, theta = np.float32(c["rms_eps"]), np.float32(c["rope_theta"])
        x = orc.embed(np.array([tok], np.int32), W["model.embed_tokens.weight"], 1, H)
        for l in range(c["layers"]):
            p = "model.layers.%d." % l
            xq, xs, _ = orc.rmsnorm_q8(x, W[p + "input_layernorm.weight"], eps)
            q = orc.gemv_q4_q8(xq, xs, *W[p + "self_attn.q_proj.weight"], nq, H).astype(np.float32)
            k = orc.gemv_q4_q8(xq, xs, *W[p + "self_attn.k_proj.weight"], nkv, H).astype(np.float32)
            v = orc.gemv_q4_q8(xq, xs, *W[p + "self_attn.v_proj.weight"], nkv, H).astype(np.float32)
            qr, kq, ks, vq, vs = orc.attn_prep_q8(q, k, v, W[p + "self_attn.q_norm.weight"], W[p + "self_attn.k_norm.weight"],
                                                  nHq, nKv, hd, pos, theta, eps)
            KQ, KS, VQ, VS = self.kv[l]
            KQ[pos], KS[pos], VQ[pos], VS[pos] = kq, ks, vq, vs
            attn = orc.attn_decode_q8(qr, KQ[:pos + 1], KS[:pos + 1], VQ[:pos + 1], VS[:pos + 1], pos + 1, nHq, nKv, hd)
            aq, as_, _ = orc.quant_act_q8(attn.astype(np.float32))
            x = (x + orc.gemv_q4_q8(aq, as_, *W[p + "self_attn.o_proj.weight"], H, nq).astype(np.float32)).astype(np.float32)
            xq, xs, _ = orc.rmsnorm_q8(x, W[p + "post_attention_layernorm.weight"], eps)
            swi = orc.gateup_silu_q4(xq, xs, *W[p + "mlp.gate_proj.weight"], *W[p + "mlp.up_proj.weight"], I, H).astype(np.float32)
            sq, ss, _ = orc.quant_act_q8(swi)
            x = (x + orc.gemv_q4_q8(sq, ss, *W[p + "mlp.down_proj.weight"], H, I).astype(np.float32)).astype(np.float32)
        normed = orc.rmsnorm(x, W["model.norm.weight"], 1, H, eps)
        logits = orc.gemv_q4_f32(normed, *W["lm_head.weight"], c["vocab"], H)
        return logits, orc.argmax(logits.astype(np.float32))
