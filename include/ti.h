/*
 * ti.h — C ABI of libtabinfer: the MI355X (gfx950) implementation of TabInfer's
 * quantized decode hot path. This is the drop-in boundary: the reference's JS
 * engine calls its kernels through closure launchers over WebGPU buffers
 * (models/qwen3.js, models/lfm25.js) and the native Rust engine calls
 * n2-kernels; each entry point below replaces one of those and cites it.
 *
 * Conventions
 *  - Every function returns 0 (TI_OK) or a negative TI_ERR_* code; the message
 *    of the last failure on the calling thread is in ti_last_error().
 *  - Buffer handles are device pointers returned by ti_buf_alloc (or any other
 *    device allocation on the context's device). "f16"/"bf16" arrays are
 *    uint16_t bit patterns. int8 vectors are packed 4 per uint32 little-endian.
 *  - Compute entry points are stream-ordered on the context's stream and do not
 *    block; ti_sync waits. A context is used by one thread at a time.
 *  - Shape preconditions are validated here (K % 32 == 0 for int4/int8 paths,
 *    K % 64 == 0 for ternary, hd % 32 == 0 and hd <= 128 for attention) and
 *    fail with TI_ERR_INVALID before anything is launched.
 *
 * Data layouts are the reference's own (no re-layout is required by a caller):
 *  int4 weights  pack u32[N*K/8] (k = 8w+i at bits 4i of word w, nibble = q+8),
 *                scales f16[N*K/32]                     (models/qwen3.js:3405-3426)
 *  int8 act      xq u32[K/4], xs f32[K/32], xsum i32[K/16] (models/qwen3.js:332-358)
 *  int8 KV       per layer kq u32[cap*nKv*hd/4], ks f32[cap*nKv*hd/32], same for v
 *                (position-major, then head, then dim) (models/qwen3.js:3877-3892)
 *  ternary       codes u8[N*K/4] (Q2_0_g64 interleaved planes), scales f32[N*K/64]
 *                                                        (native/docs/FORMAT.md)
 *  int3 experts  p3 u32[rows*K/32*3] bitplanes, s3 f16[rows*K/32] (models/lfm25.js:833-856)
 */
#ifndef TI_H
#define TI_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TI_OK              0
#define TI_ERR_INVALID    -1   /* bad argument or shape precondition */
#define TI_ERR_NO_DEVICE  -2   /* no HIP device (or index out of range) */
#define TI_ERR_HIP        -3   /* HIP runtime error */
#define TI_ERR_OOM        -4   /* device allocation failed */
#define TI_ERR_STATE      -5   /* call out of order (e.g. graph end without begin) */

typedef struct ti_ctx ti_ctx;
typedef struct ti_graph ti_graph;

/* ---- context, errors ------------------------------------------------------
 * Replace E.init / E.device (engine/webgpu-engine.js:72-145). */
const char* ti_last_error(void);
int ti_version(void);                                 /* 100*major + minor */
int ti_device_count(int* n);
int ti_init(int device, ti_ctx** out);
int ti_shutdown(ti_ctx* ctx);

/* ---- buffers (engine/webgpu-engine.js:156-179, 388-393) ------------------- */
int ti_buf_alloc(ti_ctx* ctx, size_t bytes, void** dptr);
int ti_buf_free(ti_ctx* ctx, void* dptr);
int ti_buf_write(ti_ctx* ctx, void* dst, size_t off, const void* src, size_t bytes);       /* blocking H2D */
int ti_buf_read(ti_ctx* ctx, const void* src, size_t off, void* dst, size_t bytes);        /* waits, D2H   */
/* The mapAsync-style readback of the engine's staging buffers (engine/webgpu-engine.js:169-179,
 * models/qwen3.js:4423): a stream-ordered D2H copy that returns at once; it has landed when
 * an event recorded after it completes (ti_event_record + ti_event_wait). dst should be
 * page-locked (ti_host_alloc) for the copy to be asynchronous. Refused during a capture. */
int ti_buf_read_async(ti_ctx* ctx, const void* src, size_t off, void* dst, size_t bytes);
int ti_host_alloc(size_t bytes, void** host_ptr);                                           /* pinned */
int ti_host_free(void* host_ptr);   /* waits for the device first: no queued copy lands in freed memory */
int ti_buf_copy(ti_ctx* ctx, void* dst, size_t doff, const void* src, size_t soff, size_t bytes);
int ti_buf_fill_u32(ti_ctx* ctx, void* dst, uint32_t value, size_t count);                 /* kernel fill  */
int ti_sync(ti_ctx* ctx);

/* ---- batching and timing ---------------------------------------------------
 * ti_graph_begin/end capture every call in between into one HIP graph — the
 * analogue of E.beginBatch(Infinity)/E.endBatch() (engine/webgpu-engine.js:357-386).
 * Events replace the timestamp profiler (engine/webgpu-engine.js:283-306). */
int ti_graph_begin(ti_ctx* ctx);
int ti_graph_end(ti_ctx* ctx, ti_graph** out);
int ti_graph_launch(ti_ctx* ctx, ti_graph* g);
int ti_graph_destroy(ti_graph* g);
int ti_event_record(ti_ctx* ctx, int slot);                          /* slot in [0, 64); inside a
                                                                        capture: a graph node */
int ti_event_elapsed_ms(ti_ctx* ctx, int start_slot, int end_slot, float* ms);
/* Waits for the last record of one slot, not the whole stream (the readback of one
 * in-flight batch while later batches run). Callable from another thread than the
 * context's owner, provided the slot is not re-recorded until it returns. */
int ti_event_wait(ti_ctx* ctx, int slot);

/* ---- int4 weights ---------------------------------------------------------- */
/* quantizeInt4Bf16 (models/qwen3.js:3405-3426), run on the GPU, bit-exact. */
int ti_quant_int4_bf16(ti_ctx* ctx, const uint16_t* w_bf16, uint32_t* pack, uint16_t* scales,
                       int N, int K);

/* ---- the on-GPU ternary format (models/qwen3.js:3428-3469) ---------------------
 * quantizeTernaryBf16, run on the GPU, bit-exact: pack u32[N*K/16] holds c = w + 1 in {0, 1, 2}
 * for weight k of a row at bits 8(k&3) + 2((k>>2)&3) of word k/16; scales f16[N*K/32] are
 * each 32-group's largest bf16 magnitude. A nonzero magnitude more than 2 bf16 ULPs below its
 * group's maximum means the tensor is not ternary: *not_ternary (a device word the caller
 * zeroes first) becomes nonzero, where the reference returns null and its loader quantizes
 * to int4 instead. K % 64 == 0. */
int ti_quant_tern_bf16(ti_ctx* ctx, const uint16_t* w_bf16, uint32_t* pack, uint16_t* scales,
                       int N, int K, uint32_t* not_ternary);
/* gemvTern2 / gemvTern_only (models/qwen3.js:449-503, 548-556): y (+)= W x over quantQ8's
 * int8 activation (xq, xs) and its per-16 sums xsum; each 32-group is an exact int32 sum
 * (sum c x - sum x) scaled by the weight and activation scales. */
int ti_gemv_tern2(ti_ctx* ctx, const uint32_t* xq, const float* xs, const int32_t* xsum,
                  const uint32_t* pack, const uint16_t* scales, float* y, int N, int K, int acc);
/* gateupTern2 (models/qwen3.js:747-810, 862-870): swi = silu(gate x) * (up x). */
int ti_gateup_silu_tern2(ti_ctx* ctx, const uint32_t* xq, const float* xs, const int32_t* xsum,
                         const uint32_t* gpack, const uint16_t* gscales, const uint32_t* upack,
                         const uint16_t* uscales, float* swi, int I, int H);

/* ---- activations ----------------------------------------------------------- */
/* quantQ8 (models/qwen3.js:414-420): per-32 int8 + per-16 sums. */
int ti_quant_act_q8(ti_ctx* ctx, const float* x, uint32_t* xq, float* xs, int32_t* xsum, int K);
/* QUANTQ8T (models/qwen3.js:1210-1231): T rows, per (token, group). */
int ti_quant_act_q8_t(ti_ctx* ctx, const float* x, uint32_t* xq, float* xs, int T, int K);
/* rmsnormQ (models/qwen3.js:569-621): fused RMSNorm + int8 quant. */
int ti_rmsnorm_q8(ti_ctx* ctx, const float* x, const uint16_t* w, uint32_t* xq, float* xs,
                  int32_t* xsum, int H, float eps);
/* rmsnorm (models/qwen3.js:60-88) + QUANTQ8T (:1210-1231) of T rows, the int8 input of the
 * T-token projections: xq[T][H/4], xs[T][H/32]. H = 256 * {1, 2, 4, 8, 16}. */
int ti_rmsnorm_q8_t(ti_ctx* ctx, const float* x, const uint16_t* w, uint32_t* xq, float* xs, int T, int H, float eps);
/* rmsnorm (models/qwen3.js:60-88), y[T,H]. */
int ti_rmsnorm(ti_ctx* ctx, const float* x, const uint16_t* w, float* y, int T, int H, float eps);

/* ---- GEMV (batch 1) --------------------------------------------------------- */
/* gemvDP4_only (models/qwen3.js:422-427): y (+)= W·x over the int8 activation. */
int ti_gemv_q4_q8(ti_ctx* ctx, const uint32_t* xq, const float* xs, const uint32_t* pack,
                  const uint16_t* scales, float* y, int N, int K, int acc);
/* gemvQ (models/qwen3.js:314-321): f32 activation, used for N >= 16384 (lm_head). */
int ti_gemv_q4_f32(ti_ctx* ctx, const float* x, const uint32_t* pack, const uint16_t* scales,
                   float* y, int N, int K, int acc);
/* gateUpSiluDP4_only (models/qwen3.js:861-877): swi = silu(gate·x)*(up·x). */
int ti_gateup_silu_q4(ti_ctx* ctx, const uint32_t* xq, const float* xs,
                      const uint32_t* gpack, const uint16_t* gsc,
                      const uint32_t* upack, const uint16_t* usc, float* swi, int I, int H);
/* linearQ router (models/qwen3.js:1588-1608): T==1 and N<16384 -> int8 quant +
 * gemvDP4; T==1 and N>=16384 -> gemvQ; T>1 -> per-token quant + int8 MFMA GEMM. */
int ti_linear_q4(ti_ctx* ctx, const float* x, const uint32_t* pack, const uint16_t* scales,
                 float* y, int T, int N, int K, int acc);
/* Integer per-(row, group) dots of gemvDP4 (debug/parity: exact int32). */
int ti_group_dots_q4_q8(ti_ctx* ctx, const uint32_t* xq, const uint32_t* pack, int32_t* dots,
                        int N, int K);

/* ---- fused decode-step launches ---------------------------------------------------
 * Each replaces a run of the reference's launchers with one kernel; the int8 codes
 * they produce internally are the ones the separate launchers produce, bit for bit. */
/* rmsnormQ (models/qwen3.js:614-621) + the projGemv calls that share its output
 * (q, k, v: models/qwen3.js:3981-3984): ys[i][0..Ns[i]) = W_i . rmsnormQ(x), for nmat
 * in 1..3 matrices of K columns. norm_w == NULL quantizes x as is (quantQ8).
 * xq_out/xs_out (both or neither) receive the int8 activation. K <= 16384. */
int ti_rmsnorm_gemv_q4(ti_ctx* ctx, const float* x, const uint16_t* norm_w, float eps, int K, int nmat,
                       const uint32_t* const* packs, const uint16_t* const* scales, float* const* ys,
                       const int* Ns, uint32_t* xq_out, float* xs_out);
/* rmsnormQ + gateUpSiluDP4_only (models/qwen3.js:4023-4024): swi = silu(gate.x)*(up.x).
 * swi (may be NULL when swi_q is given) receives the f32 values; swi_q/swi_s (both or
 * neither; I % 32 == 0) receive them quantized per 32 as linearQ's quantQ8 would
 * (models/qwen3.js:4033), ready for the down projection's gemvDP4. */
int ti_rmsnorm_gateup_silu_q4(ti_ctx* ctx, const float* x, const uint16_t* norm_w, float eps,
                              const uint32_t* gpack, const uint16_t* gsc, const uint32_t* upack,
                              const uint16_t* usc, float* swi, int I, int H, uint32_t* swi_q, float* swi_s);
/* final rmsnorm + lm_head gemvQ + argmaxKernel (models/qwen3.js:4037-4055):
 * logits (may be NULL) = W . rmsnorm(x), tok_hist[out_pos] = argmax with argmaxKernel's
 * tie order (below). K <= 8192. */
int ti_rmsnorm_lm_head_argmax(ti_ctx* ctx, const float* x, const uint16_t* norm_w, float eps,
                              const uint32_t* pack, const uint16_t* scales, float* logits, int N, int K,
                              uint32_t* tok_hist, int out_pos);
/* argmaxKernel (models/qwen3.js:2681-2690): tok_hist[out_pos] = argmax(logits[0..N)).
 * Equal maxima resolve as the reference's trees resolve them: N < 16384 by its one
 * 256-thread workgroup, larger N by its 64 x 256 two-stage pair (index 16394 beats 300).
 * Only logits above -3e38 are candidates; with none the token is 0. */
int ti_argmax(ti_ctx* ctx, const float* logits, int N, uint32_t* tok_hist, int out_pos);
/* gumbelNoise(logits, N, temp) (models/qwen3.js:2722-2740): logits[i] += temp * g_i with
 * g_i = -log(-log(u_i)), u_i = ((pcg(i ^ seed * 2654435761) >> 8) + 0.5) / 2^24, in
 * place; ti_argmax of the result samples softmax(logits / temp). `seed` is the already
 * advanced seed of this step (the reference advances _rngSeed before each call). */
int ti_gumbel_noise(ti_ctx* ctx, float* logits, int N, uint32_t seed, float temp);
/* embedGather (models/qwen3.js:1663-1676): y[t] = f32(emb[ids[id_off+t]]), t < T. */
int ti_embed(ti_ctx* ctx, const int32_t* ids, const uint16_t* emb, float* y, int T, int H, int id_off, int vocab);

/* ---- attention over the int8 KV cache ------------------------------------------ */
/* attnPrepQ8 (models/qwen3.js:2297-2308): per-head RMSNorm(q,k) + split-half RoPE at
 * `pos`, q -> qr, k and v snorm-quantized into the cache row `pos` (kq/ks/vq/vs are the
 * layer's cache base pointers). Bit-exact KV codes. */
int ti_attn_prep_q8(ti_ctx* ctx, const float* q, const float* k, const float* v,
                    const uint16_t* qn_w, const uint16_t* kn_w, float* qr,
                    uint32_t* kq, float* ks, uint32_t* vq, float* vs,
                    int nHq, int nKv, int hd, int pos, float theta, float eps);
/* attnDecodeStreamQ8 (models/qwen3.js:2165-2173): split-KV decode attention over
 * S cached positions plus the log-sum-exp combine; out[nHq*hd]. nsplit = 0 picks the
 * split count; otherwise it is the reference's nsplitOverride (splits of ceil(S/nsplit),
 * trailing ones may be empty). */
int ti_attn_decode_q8(ti_ctx* ctx, const float* qr, const uint32_t* kq, const float* ks,
                      const uint32_t* vq, const float* vs, float* out,
                      int S, int nHq, int nKv, int hd, int nsplit);
/* ti_attn_decode_q8 without a context, for callers that cannot allocate device memory
 * (code under graph capture, tight serving loops, harnesses that forbid hipMalloc). It has
 * no counterpart in the reference. It allocates nothing: the split partials live in a
 * file-scope device array of the library (2.03 MiB, held by every device the call runs on
 * until the process ends), so nHq * splits <= 4096 (splits as ti_attn_decode_q8 picks
 * them for nsplit = 0; at most 512); larger calls fail with TI_ERR_INVALID. `stream` is a
 * hipStream_t (NULL: the null stream); the call is ordered on it and does not block. The
 * array used is the copy on the stream's device (the current device for NULL), whatever
 * device is current; the first call on a device looks its address up once. All
 * calls on one device share the array, so calls whose execution overlaps on one device
 * (two streams, two threads) race; calls ordered on one stream do not. */
int ti_attn_decode_q8_noalloc(void* stream, const float* qr, const uint32_t* kq, const float* ks,
                              const uint32_t* vq, const float* vs, float* out,
                              int S, int nHq, int nKv, int hd, int nsplit);
/* attnPrepQ8 + attnDecodeStreamQ8 + combine as one launch (models/qwen3.js:4001-4002) for
 * one token at `pos` (< cap, the cache capacity in positions): q/k/v are the token's
 * projections [nHq*hd], [nKv*hd], [nKv*hd]; k and v are written into cache row pos;
 * out[nHq*hd] is the attention over positions 0..pos; out_q/out_s (both or neither)
 * receive it quantized per 32 (quantQ8, for o_proj's linearQ). max_splits workgroups
 * per KV head (0 = the default for pos + 1 positions: 16 up to 2048, 32 up to 14336,
 * then 64; at most 64).
 * Covers hd 64/128 with nHq/nKv <= 2. */
int ti_attn_step_q8(ti_ctx* ctx, const float* q, const float* k, const float* v,
                    const uint16_t* qn_w, const uint16_t* kn_w, uint32_t* kq, float* ks,
                    uint32_t* vq, float* vs, float* out, int nHq, int nKv, int hd, int pos, int cap,
                    float theta, float eps, int max_splits, uint32_t* out_q, float* out_s);
/* ropeQK (models/qwen3.js:1700-1760): out[t,h,:] = RoPE(RMSNorm(x[t,h,:]) * w) at
 * pos0+t for T tokens; w == NULL skips the norm. x and out must not alias. */
int ti_rope_qk(ti_ctx* ctx, const float* x, const uint16_t* w, float* out,
               int T, int nH, int hd, int pos0, float theta, float eps);
/* kvQuantWrite (models/qwen3.js:2211-2216): snorm int8 write of T rows of k (roped) and
 * v at positions pos..pos+T-1. */
int ti_kv_write_q8(ti_ctx* ctx, const float* kr, const float* v, uint32_t* kq, float* ks,
                   uint32_t* vq, float* vs, int T, int nKv, int hd, int pos);

/* ---- ternary Q2_0_g64 ------------------------------------------------------------ */
/* gemv_tern (native/crates/n2-kernels/src/tern.rs:56-71; cpu/kernel/src/lib.rs:438-441):
 * out[n] = sum_b s[n,b]*dot_b - sum_b s[n,b]*xsum[b], in units of 1/scale (the caller
 * multiplies by 1/scale, as the reference's callers do). K % 64 == 0. */
int ti_tern_gemv(ti_ctx* ctx, float* out, const uint8_t* codes, const float* scales,
                 const int8_t* act, const int32_t* xsum, int N, int K);
/* gemv_tern over 1..3 matrices that share the activation (q/k/v, gate/up) in one launch:
 * outs[i][0..Ns[i]) as ti_tern_gemv for each, bit for bit. K % 1024 == 0, K <= 8192. */
int ti_tern_gemv_multi(ti_ctx* ctx, const int8_t* act, const int32_t* xsum, int K, int nmat,
                       const uint8_t* const* codes, const float* const* scales, float* const* outs,
                       const int* Ns);
/* gemm_tern_b4 (cpu/kernel/src/lib.rs:331-367): B activation rows act[B*K], xsum[B*K/64];
 * row b of the output starts at out + b*out_stride. */
int ti_tern_gemm(ti_ctx* ctx, float* out, long out_stride, const uint8_t* codes, const float* scales,
                 const int8_t* act, const int32_t* xsum, int N, int K, int B);
/* quantize_act_into (tern.rs:206-222, mode 0) or WASM quantize (lib.rs:570-606,
 * mode 1): per-tensor int8 activation + per-64 sums; the scale (127/amax for mode 0,
 * amax/127 for mode 1) is written to the device float scale_out. */
int ti_quant_act_tern(ti_ctx* ctx, const float* x, int8_t* act, int32_t* xsum, float* scale_out,
                      int K, int mode);
/* Exact int32 per-(row, block) code dots of gemv_tern (debug/parity). */
int ti_tern_block_dots(ti_ctx* ctx, const uint8_t* codes, const int8_t* act, int32_t* dots, int N, int K);

/* ---- the .cpu.bin weight container (native/docs/FORMAT.md) ----------------------------
 * Reader of the native ternary engine's container (native/crates/n2-core/src/binfmt.rs:
 * 104-257, written by native/tools/pack_bin.py): [u32 le header_len][UTF-8 JSON header]
 * [blob], header {"G": 64, "tensors": {name: {...}}} with blob-relative offsets. Host
 * only (no GPU needed). Open and parse fail with TI_ERR_INVALID and the reference's
 * message for each rule it enforces: a header overrunning the file, a header that is not
 * UTF-8 or JSON, G != 64, no `tensors` object, a tensor without `kind` or of an unknown
 * kind, K % G != 0, codesLen != N*K/4, scalesLen != N*(K/G)*4, a byte range overrunning
 * the blob; and, when a tensor is viewed, f32 ranges that are not whole f32s at 4-byte-
 * aligned offsets. The blob lives in a 16-byte-aligned host allocation owned by the handle. */
typedef struct ti_cpubin ti_cpubin;
#define TI_CPUBIN_TERN      1   /* Q2_0_g64 codes u8[N*K/4] + f32 scales [N*K/64] */
#define TI_CPUBIN_EMBED_F16 2   /* f16 bit patterns, shape[] */
#define TI_CPUBIN_F32       3   /* f32, shape[] */
typedef struct {
    int kind;
    long long N, K;             /* tern */
    int ndim;                   /* embed_f16 / f32 */
    long long shape[4];
    const void* data;           /* codes (tern) or the values, in the container's blob */
    size_t data_bytes;
    const void* scales;         /* tern only */
    size_t scale_bytes;
} ti_cpubin_tensor_info;
/* Container::open (binfmt.rs:104-134): the header, then the blob streamed into its own
 * aligned allocation. */
int ti_cpubin_open(const char* path, ti_cpubin** out);
/* Container::from_bytes (binfmt.rs:136-157): a whole file held in memory (copied). */
int ti_cpubin_parse(const void* data, size_t bytes, ti_cpubin** out);
int ti_cpubin_close(ti_cpubin* c);
int ti_cpubin_summary(const ti_cpubin* c, int* group_size, int* n_tensors, size_t* blob_bytes);
/* the i-th tensor name, in name order (the reference's BTreeMap order) */
int ti_cpubin_name(const ti_cpubin* c, int i, const char** name);
/* ternary / view_f32 / the embedding table (binfmt.rs:260-320): a tensor's kind, shape and
 * host views into the blob (valid until ti_cpubin_close). */
int ti_cpubin_tensor(const ti_cpubin* c, const char* name, ti_cpubin_tensor_info* info);
/* embed_row (binfmt.rs:321-342): row `row` of an embed_f16 tensor decoded to f32. */
int ti_cpubin_embed_row(const ti_cpubin* c, const char* name, long long row, float* dst, int dim);

/* ---- the Bonsai-1.7B ternary decoder ----------------------------------------------------
 * The native engine's Model (native/crates/n2-core/src/model.rs:349-501, ops.rs) on the GPU:
 * ternary projections and lm_head in the .cpu.bin layout (Q2_0_g64 codes + f32 scales),
 * f32 norms, f16 embeddings, an f32 KV cache of max_ctx positions, a token history and a
 * device-side position. Per token: rmsnorm, per-tensor int8 quantize_act, ternary GEMVs
 * scaled by 1/scale, qk-norm, split-half RoPE, GQA attention, SwiGLU, residuals, final
 * norm, lm_head, argmax (ops::argmax, the lowest index on ties). head_dim 128 with two
 * query heads per KV head; hidden, intermediate and n_heads * head_dim multiples of 1024,
 * at most 8192. */
typedef struct ti_bonsai ti_bonsai;
typedef struct {
    int layers, hidden, intermediate, n_heads, n_kv_heads, head_dim, vocab;
    float rope_theta, rms_eps;
    int max_ctx;      /* KV capacity in positions, <= 40960 */
} ti_bonsai_config;
int ti_bonsai_create(ti_ctx* ctx, const ti_bonsai_config* cfg, ti_bonsai** out);
int ti_bonsai_destroy(ti_ctx* ctx, ti_bonsai* m);
/* Model::load + check_shapes (model.rs:256-322): every tensor the forward needs, of the kind
 * and size the config implies, uploaded from an open container (ti_cpubin_open). */
int ti_bonsai_load(ti_ctx* ctx, ti_bonsai* m, const ti_cpubin* bin);
/* device buffers of a tensor by its container name: ternary tensors return codes + scales,
 * norms f32, the embedding f16 */
int ti_bonsai_tensor(ti_bonsai* m, const char* name, void** data, size_t* data_bytes, void** scales,
                     size_t* scale_bytes);
int ti_bonsai_kv(ti_bonsai* m, int layer, float** kc, float** vc);   /* f32 [max_ctx][n_kv*head_dim] */
int ti_bonsai_logits(ti_bonsai* m, float** logits);                   /* f32 [vocab], last decode */
/* Model::forward per prompt token at positions pos.. (logits for the last one only, as n2's
 * prefill): history[pos..pos+T) = ids, argmax of the last logits -> history[pos+T], device
 * position = pos+T. ids == NULL takes the tokens already in the history. */
int ti_bonsai_forward(ti_ctx* ctx, ti_bonsai* m, const int32_t* ids, int T, int pos);
/* one token at the device position P: embeds history[P], writes KV row P, argmax ->
 * history[P+1], P += 1. Reads nothing from the host (capturable, replayable). */
int ti_bonsai_decode(ti_ctx* ctx, ti_bonsai* m);
int ti_bonsai_set_pos(ti_ctx* ctx, ti_bonsai* m, int pos);
int ti_bonsai_write_tokens(ti_ctx* ctx, ti_bonsai* m, int from, int count, const int32_t* ids);
int ti_bonsai_read_tokens(ti_ctx* ctx, ti_bonsai* m, int from, int count, int32_t* ids);
/* Parity trace (debug; no reference counterpart). With buf set, every later step also copies
 * per layer, in 32-bit words: x_in[H], xn[H], its int8 codes [H/4] and scale [1], q/k/v as
 * the GEMVs leave them (units of 1/scale) [nq][nkv][nkv], attn[nq], its codes [nq/4] and
 * scale [1], x_mid[H], xn2[H], codes [H/4], scale [1], gate[I], up[I] (units of 1/scale),
 * swi[I], codes [I/4], scale [1], down[H] (units of 1/scale); after the last layer x_final[H],
 * xn_final[H], codes [H/4], scale [1]. NULL switches it off. */
int ti_bonsai_trace(ti_bonsai* m, void* buf, size_t bytes);

/* ---- int3 MoE experts (LFM2.5) ----------------------------------------------------
 * int3 group of 32 weights: three u32 bitplanes (bit i of plane b = bit b of q3+4 for
 * element i) and one f16 scale; the rows of all experts are stacked expert-major
 * (row = e*N + n), p3 u32[nE*N*K/32*3], s3 f16[nE*N*K/32]. */
/* _requant43 (models/lfm25.js:833-856): int4 codes -> int3 bitplanes, s3 =
 * f32ToF16(s4*m/4) by the engine converter (engine/webgpu-engine.js:217-236); bit-exact
 * with the JavaScript f64 arithmetic. rows*K/32 groups; pack4 16-byte aligned. */
int ti_requant43(ti_ctx* ctx, const uint32_t* pack4, const uint16_t* sc4, int rows, int K,
                 uint32_t* p3, uint16_t* s3);
/* router / ROUTER_WGSL (models/lfm25.js:111-146): s = sigmoid(logit), top-k of s + bias
 * (strict '>', lowest index wins a tie), wt = s/(sum + 1e-6). bias may be NULL (zero).
 * logits f32[T*nE] -> idx i32[T*topk], wt f32[T*topk]; nE <= 256, topk <= 64. */
int ti_router(ti_ctx* ctx, const float* logits, const float* bias, int T, int nE, int topk,
              int32_t* idx, float* wt);
/* idxGemv3 (models/lfm25.js:1924-1980): y[k*N+n] = sum_g s3 * sum_32 q3*x over expert
 * idx[k]'s rows, x row k/xdiv of stride in_stride (f32); a pair whose id is outside
 * [0, nE) writes nothing. K % 32 == 0, K <= 4096. */
int ti_moe_gemv_q3(ti_ctx* ctx, const float* x, const uint32_t* p3, const uint16_t* s3,
                   const int32_t* idx, float* y, int pairs, int N, int K, int in_stride,
                   int xdiv, int nE);
/* moeGemm3 (models/lfm25.js:1503-1647): src f32[src_rows*K] is quantized per 32-group to
 * int8 (quantAct8, :1487-1494) into the context's scratch, then pair p (expert ridx[p],
 * activation row p/src_div) gives y[p*N+n] = sum_g int32 dot * s_x * s_w. Pairs are
 * grouped by expert inside the kernel; y stays in pair order. src_rows*K <= 2^24. */
int ti_moe_gemm_q3(ti_ctx* ctx, const float* src, int src_rows, const uint32_t* p3,
                   const uint16_t* s3, const int32_t* ridx, float* y, int P, int N, int K,
                   int src_div, int nE);
/* The MoE block of one decode token (models/lfm25.js:2145-2166 at T = 1, after the router
 * logits) in two launches: [router + w1/w3 + swiglu] and [w2 + combine]:
 * x[H] += sum_k wt[k] * w2_{idx[k]} (silu(w1 normed) * (w3 normed)). idx/wt[topk] receive
 * the routing, act[topk*I] the expert activations. nE <= 256, topk in {1, 2, 4, 8},
 * H and I multiples of 32, <= 4096. */
int ti_moe_decode_q3(ti_ctx* ctx, float* x, const float* normed, const float* logits, const float* bias,
                     const uint32_t* w1p, const uint16_t* w1s, const uint32_t* w3p, const uint16_t* w3s,
                     const uint32_t* w2p, const uint16_t* w2s, int32_t* idx, float* wt, float* act,
                     int H, int I, int nE, int topk);
/* The MoE block of T > 1 tokens (models/lfm25.js:2145-2158, the prefill branch after the
 * router logits: router, moeGemm3 w1 and w3, swiglu, moeGemm3 w2, moeCombine) in five
 * launches instead of nine: the router shares a launch with normed's quantizer, normed is
 * quantized once for w1 and w3, both run in one launch,
 * and the SwiGLU is formed inside the quantizer of w2's input. The same arithmetic as that
 * chain of ti_router, ti_moe_gemm_q3, ti_swiglu, ti_moe_gemm_q3, ti_moe_combine: idx/wt[T*topk]
 * the routing, gate/up/act[T*topk*I] and out[T*topk*H] its intermediates, x[T*H] += the
 * combined experts. nE <= 256, H and I multiples of 32 <= 4096, T*H and T*topk*I <= 2^24;
 * normed, gate, up and act 16-byte aligned. */
int ti_moe_prefill_q3(ti_ctx* ctx, float* x, const float* normed, const float* logits, const float* bias,
                      const uint32_t* w1p, const uint16_t* w1s, const uint32_t* w3p, const uint16_t* w3s,
                      const uint32_t* w2p, const uint16_t* w2s, int32_t* idx, float* wt, float* gate, float* up,
                      float* act, float* out, int T, int H, int I, int nE, int topk);
/* swiglu (models/lfm25.js:1831-1847): y[i] = g[i] / (1 + e^-g[i]) * u[i]. */
int ti_swiglu(ti_ctx* ctx, const float* g, const float* u, float* y, long n);
/* moeCombine / MOECOMBINE_WGSL (models/lfm25.js:1982-2000): x[t*H+h] += sum_k
 * wt[t*K+k] * o[(t*K+k)*H+h]. */
int ti_moe_combine(ti_ctx* ctx, float* x, const float* o, const float* wt, int H, int K, int T);

/* ---- Qwen3 decoder ---------------------------------------------------------------
 * The model-level forward of models/qwen3.js (forward :3938-4069, loadModel layout
 * :3470-3531) as a native object: int4 projections and lm_head, f16 norms and
 * embeddings, the int8 KV cache, the token history and a device-side position. */
typedef struct ti_qwen3 ti_qwen3;
typedef struct {
    int layers, hidden, intermediate, n_heads, n_kv_heads, head_dim, vocab;
    float rope_theta, rms_eps;
    int max_ctx;      /* KV capacity in positions */
    int max_tokens;   /* largest T accepted by ti_qwen3_forward; <= 256 and max_tokens *
                         n_heads <= 4096 (the T-query attention's rows) */
} ti_qwen3_config;
int ti_qwen3_create(ti_ctx* ctx, const ti_qwen3_config* cfg, ti_qwen3** out);
int ti_qwen3_destroy(ti_ctx* ctx, ti_qwen3* m);
/* Device buffers of a checkpoint tensor by its Hugging Face name (e.g.
 * "model.layers.3.self_attn.q_proj.weight"): int4 tensors return pack + scales
 * (fill them with ti_quant_int4_bf16), f16 tensors return data only. */
int ti_qwen3_tensor(ti_qwen3* m, const char* name, void** data, size_t* data_bytes,
                    void** scales, size_t* scale_bytes);
int ti_qwen3_kv(ti_qwen3* m, int layer, uint32_t** kq, float** ks, uint32_t** vq, float** vs);
/* The layout of those buffers. Scales: [max_ctx][n_kv_heads][head_dim/32] f32, as the
 * reference's. Codes: [max_ctx][slots][head_dim] int8, where *slots >= n_kv_heads; the
 * decoder keeps one spare head slot per position (with 4 or more KV heads), so that a
 * head's slice does not sit at the same offset of every row (no reference counterpart:
 * the reference's cache is its own buffer). Head h of position p is slot h. */
int ti_qwen3_kv_layout(const ti_qwen3* m, int* slots);
/* kvQuantWrite (models/qwen3.js:2180-2216) into the decoder's own cache of `layer`: rows
 * [pos, pos+T) from the roped K rows kr and the V rows v ([T][n_kv_heads*head_dim] f32,
 * 16-byte aligned). */
int ti_qwen3_kv_write(ti_ctx* ctx, ti_qwen3* m, int layer, const float* kr, const float* v, int T, int pos);
int ti_qwen3_logits(ti_qwen3* m, float** logits);
/* forward(ids, pos) at T >= 1 (models/qwen3.js:3938): history[pos..pos+T) = ids, KV
 * written, argmax of the last logits to history[pos+T], device position = pos+T.
 * ids == NULL takes the tokens already in the history (ti_qwen3_write_tokens), which
 * makes the call capturable into a graph. */
int ti_qwen3_forward(ti_ctx* ctx, ti_qwen3* m, const int32_t* ids, int T, int pos);
/* forward(null, pos, {chain: true}) (models/qwen3.js:3951-3959, 4055): one step at the
 * device position P: embeds history[P], writes KV row P, argmax -> history[P+1], P += 1.
 * Reads nothing from the host, so it can be captured once and replayed per token. */
int ti_qwen3_decode(ti_ctx* ctx, ti_qwen3* m);
int ti_qwen3_set_pos(ti_ctx* ctx, ti_qwen3* m, int pos);
/* The reference picks the decode attention's split count from the context on every
 * dispatch (_decNsplit, models/qwen3.js:2354). A captured step fixes it when it is
 * captured, from the position last set on the host (ti_qwen3_set_pos, or the end of a
 * ti_qwen3_forward): *splits receives the count a step captured at pos uses (16 up to
 * 4096 positions, then about one per 512 positions, between 24 and 64). A caller that
 * replays a captured step captures it again when this value changes for its position;
 * a step replayed past its capture's tier stays correct. */
int ti_qwen3_decode_splits(const ti_qwen3* m, int pos, int* splits);
/* forward(..., {temp}) (models/qwen3.js:4052, 4538-4567): the temperature of the following
 * decode steps and forwards, read on the device (so one captured step serves any
 * temperature); <= 0 is greedy (the default). With temp > 0 each step's lm_head adds
 * temp * g to every logit (ti_gumbel_noise's g) before its argmax, with the seed
 * s = 1664525 s + 1013904223 advanced once per sampled step, as the reference's
 * _rngSeed (:2733-2737); the logits buffer keeps the logits without the noise.
 * Stream-ordered, capturable. */
int ti_qwen3_sampling(ti_ctx* ctx, ti_qwen3* m, float temperature);
/* The seed stream's state: the last seed used (a new decoder holds 0x9E3779B9, the
 * reference's initial _rngSeed). ti_qwen3_seed is stream-ordered; get waits. */
int ti_qwen3_seed(ti_ctx* ctx, ti_qwen3* m, uint32_t state);
int ti_qwen3_get_seed(ti_ctx* ctx, ti_qwen3* m, uint32_t* state);
/* Parity trace (debug; no reference counterpart: it exposes the intermediate values the
 * reference's forward keeps in its own buffers, models/qwen3.js:3959-4049). With buf set,
 * every later ti_qwen3_decode / ti_qwen3_forward also copies into buf, per layer l, 13
 * fields of cfg.max_tokens rows each, in this order (32-bit words per row; nq = n_heads *
 * head_dim, nkv = n_kv_heads * head_dim, H = hidden, I = intermediate):
 *   x_in f32[H]      residual entering the layer
 *   xn_q u32[H/4]    rmsnormQ codes of x_in (input of q/k/v), xn_s f32[H/32] their scales
 *   q f32[nq], k f32[nkv], v f32[nkv]   the projections (before the q/k norms and RoPE)
 *   attn f32[nq]     attention output; a_q u32[nq/4], a_s f32[nq/32] its quantQ8 codes
 *   x_mid f32[H]     residual after o_proj
 *   swi f32[I]       silu(gate)*up; s_q u32[I/4], s_s f32[I/32] its quantQ8 codes
 * then, after the last layer, x_final f32[max_tokens][H]. A call fills rows [0, T). Fields
 * a path does not materialise are left as they were: xn_* for 2 <= T <= 4 (the
 * projections normalise in their prologue), attn and swi for fused T >= 2 (codes only).
 * bytes must cover 4 * (layers * sum of the fields' words * max_tokens + max_tokens * H).
 * buf == NULL switches tracing off (the default; the traced step launches extra copies). */
int ti_qwen3_trace(ti_qwen3* m, void* buf, size_t bytes);
int ti_qwen3_write_tokens(ti_ctx* ctx, ti_qwen3* m, int from, int count, const int32_t* ids);
int ti_qwen3_read_tokens(ti_ctx* ctx, ti_qwen3* m, int from, int count, int32_t* ids);
/* The same read queued behind the steps already issued (decodeLoop's readU32Range,
 * models/qwen3.js:4423), without waiting: see ti_buf_read_async. */
int ti_qwen3_read_tokens_async(ti_ctx* ctx, ti_qwen3* m, int from, int count, int32_t* ids);
/* T-query causal attention over the int8 KV cache (models/qwen3.js:2534-2577): query t
 * (positions pos0+t) attends keys [0, pos0+t]; qr/out are [T][nHq][hd]. */
int ti_attn_causal_q8(ti_ctx* ctx, const float* qr, const uint32_t* kq, const float* ks,
                      const uint32_t* vq, const float* vs, float* out,
                      int T, int pos0, int nHq, int nKv, int hd);

#ifdef __cplusplus
}
#endif
#endif
