"""Pins for the oracle's on-GPU ternary format (or_quant_tern_bf16, or_gemv_tern2,
or_gateup_silu_tern2: models/qwen3.js:3428-3469, 449-503, 747-810).

- Exactly ternary bf16 inputs: the GEMV oracle over the packed codes equals a dense f64
  matmul of the ORIGINAL weights (each group's weights are +-m or 0 and m is exact in f16),
  so a wrong bit position, a swapped sign map or a wrong scale conversion fails it.
- A hand-built known answer: the code words and scales of one 64-wide row.
- The acceptance edge: a magnitude 2 bf16 ULPs below its group's maximum is snapped to
  +-max, 3 ULPs is not ternary (the reference's null).
"""
import numpy as np

from tern2_data import bf16_to_f64, ternary_bf16


def test_gemv_equals_dense_matmul_of_the_original_weights(orc):
    rng = np.random.default_rng(5)
    N, K = 64, 2048
    w = ternary_bf16(rng, N, K)
    pack, sc = orc.quant_tern_bf16(w, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    xq, xs, _ = orc.quant_act_q8(x)
    codes = xq.view(np.int8).astype(np.float64)
    xd = codes * np.repeat(xs.astype(np.float64), 32)                  # the int8 activation's value
    want = bf16_to_f64(w).reshape(N, K) @ xd
    got = orc.gemv_tern2(xq, xs, pack, sc, N, K)
    assert np.abs(got - want).max() <= 1e-12 * np.abs(want).max()
    g2 = ternary_bf16(rng, N, K)
    gp, gs = orc.quant_tern_bf16(g2, N, K)
    gd = bf16_to_f64(g2).reshape(N, K) @ xd
    swi = orc.gateup_silu_tern2(xq, xs, gp, gs, pack, sc, N, K)
    assert np.abs(swi - gd / (1 + np.exp(-gd)) * want).max() <= 1e-12 * np.abs(swi).max()


def test_known_answer_of_one_row(orc):
    w = np.zeros(64, np.uint16)
    w[5] = 0x3F00                                                      # +0.5
    w[17] = 0xBF00                                                     # -0.5
    pack, sc = orc.quant_tern_bf16(w, 1, 64)
    # all zero codes are 1: 0x55555555; k = 5 (b = 1, s = 1) sits at bit 10 with code 2,
    # k = 17 (word 1, b = 1, s = 0) at bit 8 with code 0
    assert list(pack) == [0x55555955, 0x55555455, 0x55555555, 0x55555555]
    assert list(sc) == [0x3800, 0x0000]                                # f16 0.5, and an all-zero group


def test_two_ulp_wobble_is_ternary_three_is_not(orc):
    base = np.zeros(64, np.uint16)
    base[:4] = 0x3C80                                                  # 0.015625 = m
    base[4] = 0xBC80
    ok = base.copy()
    ok[7] = 0x3C80 - 2                                                 # 2 ULPs below m: snapped to +1
    packed = orc.quant_tern_bf16(ok, 1, 64)
    assert packed is not None
    pack, sc = packed
    assert (pack[0] >> (8 * (7 & 3) + 2 * ((7 >> 2) & 3))) & 3 == 2
    bad = base.copy()
    bad[7] = 0x3C80 - 3
    assert orc.quant_tern_bf16(bad, 1, 64) is None
    cont = (np.random.default_rng(1).standard_normal(4 * 64) * 0.02).astype(np.float32)
    assert orc.quant_tern_bf16((cont.view(np.uint32) >> 16).astype(np.uint16), 4, 64) is None
