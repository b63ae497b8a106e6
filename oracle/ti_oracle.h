/*
 * ti_oracle.h — CPU oracle for the quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * arithmetic (eze-paz/TabInfer), used by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg as the checker. The product library
 * (tabinfer_amd/libtabinfer.so) never links, loads or calls anything here.
 *
 * Conventions
 *  - "f16" values are IEEE binary16 bit patterns held in uint16_t.
 *  - int8 activations / KV codes are packed 4 per uint32 little-endian
 *    (byte b of word w = element 4w+b), as the reference's pack4xI8 /
 *    pack4x8snorm produce them.
 *  - int4 weights: pack[N*K/8], element k of a row lives in word k/8 at bits
 *    4*(k%8); nibble = q+8. scales[N*K/32] f16, one per 32 along K.
 *  - Functions whose outputs are integers (codes, scale bits, group dots) are
 *    bit-exact restatements; float outputs are computed in f64 from the
 *    *quantized* operands (the reference's own checking method).
 *
 * Parity pins (what checks each function; see tests/test_oracle_*.py):
 *  or_f32_to_f16_q3, or_f32_to_f16_eng, or_f16_to_f32 : exhaustive/known-answer
 *      tests from native/crates/n2-core/src/binfmt.rs:406-422 plus hand-built
 *      ties, subnormals, overflow and the engine converter's OR-carry quirk.
 *  or_quant_int4_bf16 : invariants (|q|<=8, group max -> +/-7, dequant error
 *      <= s/2), all-zero-group NaN path, hand-built nibble placement.
 *  or_quant_act_q8, or_rmsnorm_q8 : brute-force restatement at tiny K,
 *      |q|<=127, xsum = sum of codes, scale = absmax/127.
 *  or_tern_* : the n2 xorshift fixtures (tern.rs:356-389, main.rs:93-114) and
 *      known-answer tests (tern.rs:437-470); scalar vs dequant oracle rel<1e-5.
 *  or_attn_* : f64 softmax oracle, nsplit invariance, RoPE known-answer tests
 *      (native/crates/n2-core/src/ops.rs:169-214).
 *  or_argmax : a numpy emulation of the reference's two-stage tree on random ties.
 *  or_quant_tern_bf16 : exact dequantization of ternary inputs (a wrong bit layout or sign
 *      map fails it), the 2-ULP acceptance edge, a hand-placed known answer;
 *  or_gemv_tern2, or_gateup_silu_tern2 : a dense f64 matmul of the dequantized operands.
 *  or_gumbel_noise, or_pcg : the reference's own self-test (models/qwen3.js:3198-3214:
 *      P(5)/P(9) = e at T = 1 with its seed stream, T -> 0 greedy) on a larger sample,
 *      the Gumbel mean and variance (Euler's gamma, pi^2/6), u uniform on (0, 1).
 */
#ifndef TI_ORACLE_H
#define TI_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 conversions ---------------------------------------------------- */
uint16_t or_f32_to_f16_q3(float v);   /* models/qwen3.js:3357-3374 (ties away, +1 carry) */
uint16_t or_f32_to_f16_eng(float v);  /* engine/webgpu-engine.js:217-236 (+0x1000, OR)   */
double   or_f16_to_f32(uint16_t h);   /* models/qwen3.js:3397-3400 (exact)               */
float    or_bf16_to_f32(uint16_t b);  /* models/qwen3.js:3409 (u16 << 16)                */

/* ---- int4 group quantizer (models/qwen3.js:3405-3426) ---------------- */
void or_quant_int4_bf16(const uint16_t* w_bf16, int N, int K,
                        uint32_t* pack, uint16_t* scales);

/* ---- per-32 int8 activation quant (models/qwen3.js:332-358) ---------- */
void or_quant_act_q8(const float* x, int K, uint32_t* xq, float* xs, int32_t* xsum);
/* batched variant, per (token, group) (models/qwen3.js:1210-1231) */
void or_quant_act_q8_t(const float* x, int T, int K, uint32_t* xq, float* xs);

/* ---- fused RMSNorm + int8 quant (models/qwen3.js:569-612) ------------ */
void or_rmsnorm_q8(const float* x, const uint16_t* w_f16, int H, float eps,
                   uint32_t* xq, float* xs, int32_t* xsum);
/* plain RMSNorm (models/qwen3.js:60-80), y[T,H] */
void or_rmsnorm(const float* x, const uint16_t* w_f16, int T, int H, float eps, float* y);

/* ---- GEMV oracles (f64 of quantized operands) -------------------- */
/* integer per-(row, group) dots: dots[n*(K/32)+g] = sum (nib-8)*q_x  (exact) */
void or_group_dots_q4_q8(const uint32_t* xq, const uint32_t* pack, int N, int K, int32_t* dots);
void or_gemv_q4_q8(const uint32_t* xq, const float* xs, const uint32_t* pack,
                   const uint16_t* scales, int N, int K, double* y);         /* models/qwen3.js:359-400 */
void or_gemv_q4_f32(const float* x, const uint32_t* pack, const uint16_t* scales,
                    int N, int K, double* y);                                  /* models/qwen3.js:276-313 */
void or_gateup_silu_q4(const uint32_t* xq, const float* xs,
                       const uint32_t* gpack, const uint16_t* gsc,
                       const uint32_t* upack, const uint16_t* usc,
                       int I, int H, double* swi);                             /* models/qwen3.js:679-728 */
/* the on-GPU ternary format (models/qwen3.js:3428-3469): returns 1 and fills pack[N*K/16],
 * scales[N*K/32] for a ternary tensor, 0 (the reference's null) otherwise */
int  or_quant_tern_bf16(const uint16_t* w_bf16, int N, int K, uint32_t* pack, uint16_t* scales);
/* gemvTern2 (models/qwen3.js:449-503) and gateupTern2 (:747-810), f64 of the exact group sums */
void or_gemv_tern2(const uint32_t* xq, const float* xs, const uint32_t* pack, const uint16_t* scales,
                   int N, int K, double* y);
void or_gateup_silu_tern2(const uint32_t* xq, const float* xs, const uint32_t* gpack, const uint16_t* gsc,
                          const uint32_t* upack, const uint16_t* usc, int I, int H, double* swi);
/* batched: Y[T,N] from per-token int8 acts (models/qwen3.js:1326-1388) */
void or_gemm_q4_q8(const uint32_t* xq, const float* xs, const uint32_t* pack,
                   const uint16_t* scales, int T, int N, int K, double* y);

/* ---- KV snorm int8 (models/qwen3.js:2180-2210, 2280-2295) ----------------- */
/* quantize n (multiple of 32) f32 values: q[n/4] words, s[n/32] scales */
void or_kv_quant(const float* x, int n, uint32_t* q, float* s);
double or_snorm_dequant(uint32_t word, int byte, float scale);

/* ---- fused QK-norm + RoPE + KV write (models/qwen3.js:2228-2296) ------ */
/* qr[nHq*hd]; kq/vq: the position's nKv*hd/4 words; ks/vs: nKv*hd/32 scales */
void or_attn_prep_q8(const float* q, const float* k, const float* v,
                     const uint16_t* qw, const uint16_t* kw,
                     int nHq, int nKv, int hd, int pos, float theta, float eps,
                     float* qr, uint32_t* kq, float* ks, uint32_t* vq, float* vs);
/* the same RMSNorm+RoPE on one head row (exposed for the RoPE known-answer tests) */
void or_rope_norm_row(const float* x, const uint16_t* w, int hd, int pos,
                      float theta, float eps, int apply_norm, float* out);

/* ---- decode attention over the int8 KV, f64 softmax ---------------- */
/* KV layout per position: [nKv][hd] int8 (hd/4 words per head), scales [nKv][hd/32] */
void or_attn_decode_q8(const float* qr, const uint32_t* kq, const float* ks,
                       const uint32_t* vq, const float* vs,
                       int S, int nHq, int nKv, int hd, double* out);
/* causal T-token variant (batched forward attention): query t attends keys [0, pos0+t] */
void or_attn_causal_q8(const float* qr, const uint32_t* kq, const float* ks,
                       const uint32_t* vq, const float* vs,
                       int T, int pos0, int nHq, int nKv, int hd, double* out);

/* the causal variant restricted to KV heads [hk0, hk1) (and their query heads), each KV
 * head dequantized once; bit-identical to or_attn_causal_q8 on those heads. out is the
 * full [T][nHq][hd] array; only the range's heads are written. */
void or_attn_causal_q8_kvheads(const float* qr, const uint32_t* kq, const float* ks,
                               const uint32_t* vq, const float* vs,
                               int T, int pos0, int nHq, int nKv, int hd, int hk0, int hk1, double* out);

/* ---- decode-step glue ---------------------------------------------------- */
void or_embed(const int32_t* ids, const uint16_t* emb_f16, int T, int H, float* y);
int  or_argmax(const float* logits, int N);   /* the reference's one/two-stage trees, their tie order */
/* Gumbel-max temperature sampling (models/qwen3.js:2713-2740): the PCG hash, the seed
 * stream's step, and logits[i] += temp * -log(-log(u_i)) in f32 as the WGSL kernel. */
uint32_t or_pcg(uint32_t v);
uint32_t or_seed_next(uint32_t s);
void or_gumbel_noise(float* logits, int N, uint32_t seed, float temp);

/* ---- ternary (native/crates/n2-kernels/src/tern.rs) --------------- */
void or_tern_pack(const float* w, int N, int K, uint8_t* codes, float* scales); /* tern.rs:131-160 */
float or_tern_quant_act_n2(const float* x, int K, int8_t* act, int32_t* xsum);  /* tern.rs:206-222 */
float or_tern_quant_act_wasm(const float* x, int K, int8_t* act, int32_t* xsum);/* lib.rs:570-606 */
void or_tern_gemv_scalar(const uint8_t* codes, const float* scales, const int8_t* act,
                         const int32_t* xsum, int N, int K, float* out);        /* tern.rs:79-119 */
void or_tern_gemv_dequant(const uint8_t* codes, const float* scales, const int8_t* act,
                          int N, int K, float* out);                            /* tern.rs:166-189 */
void or_tern_block_dots(const uint8_t* codes, const int8_t* act, int N, int K, int32_t* dots);
/* n2 test fixture generators (tern.rs:356-389 / n2-cli main.rs:93-114).
 * flavour 0: tern.rs Rng(seed) ; flavour 1: main.rs fixture (seed fixed inside) */
void or_n2_fixture(int N, int K, uint64_t seed, uint8_t* codes, float* scales,
                   int8_t* act, int32_t* xsum, float* w_out, float* x_out);

/* ---- AVX2 restatement of n2 avx2::gemv_tern (tern.rs:246-338): the timed CPU baseline */
int  or_has_avx2(void);
void or_tern_gemv_avx2(const uint8_t* codes, const float* scales, const int8_t* act,
                       const int32_t* xsum, int N, int K, float* out);
/* static row split over nthreads (cpu/cpukern-fwd-worker.js:1-4 model), on the pool below */
void or_tern_gemv_avx2_mt(const uint8_t* codes, const float* scales, const int8_t* act,
                          const int32_t* xsum, int N, int K, float* out, int nthreads);
/* A persistent pool (threads created once) that runs a whole GEMV set: each matrix's rows
 * split statically over the workers, a barrier after each matrix (as a forward pass needs
 * between dependent GEMVs). The caller is worker 0. */
typedef struct {
    const uint8_t* codes; const float* scales; const int8_t* act; const int32_t* xsum; float* out; int N, K;
} or_tern_mat;
int  or_tern_pool_start(int nthreads);
void or_tern_pool_stop(void);
void or_tern_pool_run(const or_tern_mat* mats, int nmat);
void or_tern_set_serial(const or_tern_mat* mats, int nmat);   /* one thread, no pool */

/* ---- the Bonsai forward's f32 glue (native/crates/n2-core/src/ops.rs, model.rs:349-501) */
void or_n2_rmsnorm(const float* x, const float* w, int n, float eps, float* out);      /* ops.rs:14-22   */
void or_n2_rmsnorm_heads(float* t, const float* w, int n_heads, int head_dim, float eps); /* ops.rs:29-40 */
void or_n2_rope_table(int head_dim, int pos, float theta, float* table);               /* ops.rs:79-90   */
void or_n2_rope_with_table(float* t, int n_heads, int head_dim, const float* table);   /* ops.rs:93-107  */
void or_n2_swiglu(const float* gate, const float* up, int n, float* out);             /* ops.rs:110-117 */
void or_n2_attention(const float* q, const float* kc, const float* vc, int S, int n_heads, int n_kv,
                     int head_dim, float* out);                                        /* model.rs:421-447 */
int  or_n2_argmax(const float* x, int n);                                              /* ops.rs:138-149 */

/* ---- int3 MoE (models/lfm25.js) ----------------------------------- */
void or_requant43(const uint32_t* pack4, const uint16_t* sc4, int rows, int K,
                  uint32_t* p3, uint16_t* s3);                                  /* lfm25.js:833-856 */
void or_router(const float* logits, const float* bias, int T, int nE, int topk,
               int32_t* idx, float* wt);                                        /* lfm25.js:111-141 */
/* rows of all experts stacked expert-major (row = e*N + n); y[pairs*N] */
void or_moe_gemv_q3(const float* x, const uint32_t* p3, const uint16_t* s3,
                    const int32_t* idx, int pairs, int N, int K,
                    int in_stride, int xdiv, double* y);                        /* lfm25.js:1924-1974 */
/* T>1: per-pair int8 activation rows (quantized per token/group), y[P*N] */
void or_moe_gemm_q3(const uint32_t* xq, const float* xs, const uint32_t* p3, const uint16_t* s3,
                    const int32_t* ridx, int P, int N, int K, int src_div, double* y); /* lfm25.js:1541-1622 */
/* x[t*H+h] += sum_k wt[t*K+k]*o[(t*K+k)*H+h] (lfm25.js:1982-1995) */
void or_moe_combine(float* x, const float* o, const float* wt, int H, int K, int T);

#ifdef __cplusplus
}
#endif
#endif
