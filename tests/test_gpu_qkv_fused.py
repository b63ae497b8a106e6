"""The decode step's q/k/v projection folded into its attention launch gives the same bits
as the two launches it replaces (the q/k/v GEMV, then the attention reading its rows).

The fused kernel (k_attn_fused_pv with a q/k/v prologue) computes each KV head's q, k and
v rows in the head's own workgroups and hands them over as epoch-tagged words; the
two-launch path is the one a context takes with TI_DECODE_QKV_SEPARATE set at ti_init.
Both decoders start from the same weights, tokens and seeded KV prefix and take three
chained decode steps: logits, next tokens and the new KV rows must be identical. The
cases cover both projection widths (hidden 1024: 32 lanes a row; 2048: 64) and split
counts that give both row-unit sizes (4 and 8 rows) and, with a 256-position cache
(2 splits per KV head), several rounds of units per wave. A third context is created
with TI_DECODE_QKV_POLLS=0: its waves never wait for the rows another workgroup
publishes and compute their own (the path a wave takes when its poll gives up), which
must give the same bits too."""
import os

import numpy as np
import pytest

from tabinfer_amd import abi
import qwen3_ref as Q
import qwen3_tf as TF

pytestmark = pytest.mark.gpu

GEOM = {1024: 3072, 2048: 6144}
_W = {}


def _weights(H):
    if H not in _W:
        cfg = dict(layers=2, hidden=H, intermediate=GEOM[H], n_heads=16, n_kv_heads=8, head_dim=128, vocab=4096,
                   rope_theta=1e6, rms_eps=1e-6)
        _W[H] = Q.make_weights(cfg, 31 + H)
    return _W[H]


def _ctx_with(var, value):
    old = os.environ.get(var)
    os.environ[var] = value
    try:
        return abi.Ctx(0)
    finally:
        if old is None:
            del os.environ[var]
        else:
            os.environ[var] = old


@pytest.fixture(scope="module")
def ctx_pair():
    """(fused, three launches, fused with every wave computing its own q/k/v rows)"""
    fused = abi.Ctx(0)
    sep = _ctx_with("TI_DECODE_QKV_SEPARATE", "1")
    own = _ctx_with("TI_DECODE_QKV_POLLS", "0")
    yield fused, sep, own
    own.close()
    sep.close()
    fused.close()


# (hidden, prefix P, cache capacity): splits per KV head 2, 24 (the capacity's clamp), 64, 2,
# 16, 32, 64, 64; row units of 8 rows at 16 and 24 splits, 4 at 32 and 64
CASES = [(1024, 100, 256), (1024, 2900, 3000), (1024, 20000, 20100), (2048, 100, 256), (2048, 1500, 2100),
         (2048, 12000, 12100), (2048, 20000, 20100), (2048, 32760, 32800)]


@pytest.mark.parametrize("H,P,cap", CASES)
def test_decode_fused_qkv_same_bits(ctx_pair, H, P, cap):
    print("[qkv] H=%d P=%d cap=%d" % (H, P, cap), flush=True)
    cfg = dict(layers=2, hidden=H, intermediate=GEOM[H], n_heads=16, n_kv_heads=8, head_dim=128, vocab=4096,
               rope_theta=1e6, rms_eps=1e-6, max_ctx=cap, max_tokens=1)
    W = _weights(H)
    ms = []
    try:
        for c in ctx_pair:
            m = abi.Qwen3(c, **cfg)
            ms.append(m)
            Q.load_into(m, W)
            TF.seed_prefix(c, m, cfg, P, cap, seed=P)
            m.write_tokens(P, np.array([1234], np.int32))
            m.set_pos(P)
        print("[qkv] splits per KV head: %d" % ms[0].decode_splits(P), flush=True)
        for step in range(3):
            for m in ms:
                m.decode()
            lb = ctx_pair[1].download(ms[1].logits_ptr(), np.float32, cfg["vocab"])
            assert np.isfinite(lb).all()
            for k in (0, 2):
                la = ctx_pair[k].download(ms[k].logits_ptr(), np.float32, cfg["vocab"])
                assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), "context %d step %d: logits differ" % (k, step)
        tb = ms[1].read_tokens(P + 1, 3)
        for k in (0, 2):
            assert np.array_equal(ms[k].read_tokens(P + 1, 3), tb)
        for l in range(cfg["layers"]):
            kb = ms[1].kv(l)
            for k in (0, 2):
                ka = ms[k].kv(l)
                for i in range(4):
                    if i % 2 == 0:
                        a = TF.read_kv_codes(ctx_pair[k], ms[k], ka[i], P, 3, cfg)
                        b = TF.read_kv_codes(ctx_pair[1], ms[1], kb[i], P, 3, cfg)
                    else:
                        n = 3 * cfg["n_kv_heads"] * cfg["head_dim"] // 32
                        off = P * cfg["n_kv_heads"] * cfg["head_dim"] // 32 * 4
                        a = ctx_pair[k].download(ka[i], np.float32, n, off=off)
                        b = ctx_pair[1].download(kb[i], np.float32, n, off=off)
                    assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32)), \
                        "context %d layer %d KV buffer %d differs" % (k, l, i)
    finally:
        for m in ms:
            m.close()
