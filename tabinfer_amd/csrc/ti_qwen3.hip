// ti_qwen3.hip — native Qwen3 decoder over the decode-path kernels.
//
// Replaces the reference's forward() (models/qwen3.js:3938-4069) and its
// GPU-resident token chaining (_tokHist, models/qwen3.js:3890, 4055): the model
// owns its weights (int4 projections + lm_head, f16 norms and embeddings), the
// int8 KV cache, a token history and a device-side position counter. A decode
// step reads its position on the device, so one captured HIP graph decodes
// token after token with no host round trip: embed(tok[pos]) -> 28 layers ->
// final norm -> lm_head -> argmax writes tok[pos+1] and advances pos.
#include "ti_internal.h"
#include <string.h>
#include <stdio.h>
#include <string>
#include <vector>

int ti_gemv_q4_q8_launch(ti_ctx*, const uint32_t*, const float*, const uint32_t*, const uint16_t*, float*, int, int, int);
int ti_gemv_q4_f32_launch(ti_ctx*, const float*, const uint32_t*, const uint16_t*, float*, int, int, int);
int ti_gateup_launch(ti_ctx*, const uint32_t*, const float*, const uint32_t*, const uint16_t*, const uint32_t*,
                     const uint16_t*, float*, int, int);
int ti_quant_act_q8_async(ti_ctx*, const float*, uint32_t*, float*, int32_t*, int);
int ti_attn_prep_launch(ti_ctx*, const float*, const float*, const float*, const uint16_t*, const uint16_t*, float*,
                        uint32_t*, float*, uint32_t*, float*, int, int, int, int, float, float, const int*);
int ti_attn_decode_launch(ti_ctx*, const float*, const uint32_t*, const float*, const uint32_t*, const float*, float*,
                          int, int, int, int, int, int, const int*, int, int);
int ti_kv_write_launch(ti_ctx*, const float*, const float*, uint32_t*, float*, uint32_t*, float*, int, int, int, int, int);
int ti_attn_decode_splits(int S);
int ti_attn_fused_launch(ti_ctx*, const float*, const float*, const float*, const uint16_t*, const uint16_t*, uint32_t*,
                         float*, uint32_t*, float*, float*, int, int, int, const int*, int, int, float, float, int,
                         const float*, uint32_t*, float*, int);
void ti_rope_row(float* cs, int pos, int hd, float theta);
int ti_fused_qkv_launch(ti_ctx*, const float*, const uint16_t*, float, int, int, const uint32_t* const*,
                        const uint16_t* const*, float* const*, const int*, uint32_t*, float*);
int ti_fused_linear_launch(ti_ctx*, const float*, const uint32_t*, const uint16_t*, float*, int, int, int);
int ti_fused_gateup_launch(ti_ctx*, const float*, const uint16_t*, float, const uint32_t*, const uint16_t*,
                           const uint32_t*, const uint16_t*, float*, int, int, uint32_t*, float*);
int ti_fused_lmhead_launch(ti_ctx*, const float*, const uint16_t*, float, const uint32_t*, const uint16_t*, float*, int,
                           int, uint32_t*, int*, int, int, const float*, float*, int, uint32_t*);
int ti_fused_kmax(int lm);
int ti_attn_qkv_launch(ti_ctx*, const float*, const uint16_t*, float, int, const uint32_t* const*, const uint16_t* const*,
                       float* const*, int, uint32_t*, float*, const uint16_t*, const uint16_t*, uint32_t*, float*,
                       uint32_t*, float*, float*, int, int, int, const int*, int, float, float, int, const float*,
                       uint32_t*, float*, int);

// ---------------------------------------------------------------------------
// glue kernels
// ---------------------------------------------------------------------------
// embed gather (models/qwen3.js:1621-1633): y[t,h] = f32(emb[ids[off+t]*H + h]);
// ids out of range are clamped to the vocabulary (a garbage id never reads out of bounds)
__global__ void k_embed(const uint32_t* __restrict__ ids, const uint16_t* __restrict__ emb, float* __restrict__ y, int T,
                        int H, int off, const int* __restrict__ dpos, int vocab) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * H) return;
    if (dpos) off = *dpos;
    int t = (int)(i / H), h = (int)(i % H);
    uint32_t id = ids[off + t];
    id = id < (uint32_t)vocab ? id : (uint32_t)(vocab - 1);
    y[i] = ti_h2f(emb[(size_t)id * H + h]);
}

// two-stage argmax (models/qwen3.js:2624-2690): 256 workgroups fold interleaved slices,
// one workgroup folds their partials; ties resolve by the reference's rank (ti_amx_take)
constexpr int AMX_THREADS = 256;
constexpr int AMX_PARTS = 256;

__device__ __forceinline__ void amx_fold_lds(float* sv, int* si, int n, int N) {
    for (int s = n / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            float v = sv[threadIdx.x];
            int i = si[threadIdx.x];
            ti_amx_take(v, i, sv[threadIdx.x + s], si[threadIdx.x + s], N);
            sv[threadIdx.x] = v;
            si[threadIdx.x] = i;
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(AMX_THREADS) void k_argmax_p1(const float* __restrict__ logits, int N, float* __restrict__ pv,
                                                           uint32_t* __restrict__ pi) {
    __shared__ float sv[AMX_THREADS];
    __shared__ int si[AMX_THREADS];
    float bv = -3.0e38f;
    int bi = 0;
    for (int i = blockIdx.x * AMX_THREADS + threadIdx.x; i < N; i += AMX_PARTS * AMX_THREADS) ti_amx_take(bv, bi, logits[i], i, N);
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    amx_fold_lds(sv, si, AMX_THREADS, N);
    if (threadIdx.x == 0) { pv[blockIdx.x] = sv[0]; pi[blockIdx.x] = (uint32_t)si[0]; }
}

// writes the token to hist[out_pos] (device position: hist[*dpos + 1], then *dpos += 1)
__global__ __launch_bounds__(AMX_PARTS) void k_argmax_p2(const float* __restrict__ pv, const uint32_t* __restrict__ pi, int N,
                                                         uint32_t* __restrict__ hist, int out_pos, int* __restrict__ dpos,
                                                         int advance) {
    __shared__ float sv[AMX_PARTS];
    __shared__ int si[AMX_PARTS];
    sv[threadIdx.x] = pv[threadIdx.x];
    si[threadIdx.x] = (int)pi[threadIdx.x];
    __syncthreads();
    amx_fold_lds(sv, si, AMX_PARTS, N);
    if (threadIdx.x == 0) {
        int p = dpos ? *dpos + 1 : out_pos;
        hist[p] = (uint32_t)ti_amx_result(sv[0], si[0]);
        if (dpos && advance) *dpos = p;
    }
}

// device position := pos, and its rotary row into rope_cur (hd threads)
__global__ void k_set_pos(int* __restrict__ dpos, int pos, const float* __restrict__ rope, float* __restrict__ rope_cur,
                          int hd, int cap) {
    if (threadIdx.x == 0) *dpos = pos;
    if (pos < cap && (int)threadIdx.x < hd) rope_cur[threadIdx.x] = rope[(size_t)pos * hd + threadIdx.x];
}

// swi = silu(g) * u (models/qwen3.js swiglu; silu(g) = g / (1 + e^-g))
__global__ void k_swiglu(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ y, long n) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { float a = g[i]; y[i] = a / (1.0f + expf(-a)) * u[i]; }
}

__global__ void k_copy_f32(const float* __restrict__ s, float* __restrict__ d, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = s[i];
}

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
namespace {
struct Lin {
    uint32_t* pack = nullptr;
    uint16_t* sc = nullptr;
    int N = 0, K = 0;
};
struct Layer {
    Lin q, k, v, o, gate, up, down;
    uint16_t *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    uint32_t *kq = nullptr, *vq = nullptr;
    float *ks = nullptr, *vs = nullptr;
};
}  // namespace

struct ti_qwen3 {
    ti_qwen3_config cfg;
    std::vector<Layer> L;
    uint16_t* embed = nullptr;
    uint16_t* final_norm = nullptr;
    Lin lm;
    float *x, *normed, *q, *k, *v, *qr, *kr, *attn, *gate, *up, *swi, *last, *logits;
    uint32_t* xq;
    float* xs;
    int32_t* xsum;
    float* psum;          // [16][256] RMSNorm partial sums of x (the T-token forward)
    uint32_t* hist;
    int* dpos;
    uint32_t* samp;       // sampling words: temperature, seed state (TI_SAMP_*)
    float* rope;          // [max_ctx][head_dim] cos/sin rows of the rotary embedding
    float* rope_cur;      // the row of the device position (kept in step with dpos)
    float* amx_v;
    uint32_t* amx_i;
    uint32_t* trace = nullptr;   // caller's trace buffer (ti_qwen3_trace), or null
    int pos_hint = 0;            // the position last set from the host (set_pos, or a forward's end)
    int kvs = 0;                 // K/V code slots per cached position (ti_qwen3_kv_layout)
    std::vector<void*> allocs;
};

// The decoder's K/V code rows carry one spare head slot per position when there are 4 or
// more KV heads: a head's 128-byte slice then moves to the next slot of the row from one
// position to the next, instead of sitting at the same offset of every (power-of-two)
// row. Measured on the decode attention: at a 1 KB row the workgroups of the heads whose
// slices lie at offsets 384 and 896 stream their keys ~10% slower than the others (the
// slowness moves with the offset when the cache base is shifted), and a layer waits for
// its slowest head; with the spare slot every head sees every offset. The scale rows
// (128 B per position for 8 heads) are left dense.
static int kv_slots(const ti_qwen3_config& C) { return C.n_kv_heads >= 4 ? C.n_kv_heads + 1 : C.n_kv_heads; }

// ---- the parity trace (ti_qwen3_trace) -------------------------------------------------
// Per layer, fields of max_tokens rows each, in this order (32-bit words per row):
enum TraceField { TR_X_IN, TR_XN_Q, TR_XN_S, TR_Q, TR_K, TR_V, TR_ATTN, TR_A_Q, TR_A_S, TR_X_MID, TR_SWI, TR_S_Q, TR_S_S,
                  TR_NFIELDS };
static size_t trace_row_words(const ti_qwen3_config& C, int f) {
    const size_t H = C.hidden, I = C.intermediate, nq = (size_t)C.n_heads * C.head_dim, nkv = (size_t)C.n_kv_heads * C.head_dim;
    switch (f) {
        case TR_X_IN: case TR_X_MID: return H;
        case TR_XN_Q: return H / 4;
        case TR_XN_S: return H / 32;
        case TR_Q: case TR_ATTN: return nq;
        case TR_K: case TR_V: return nkv;
        case TR_A_Q: return nq / 4;
        case TR_A_S: return nq / 32;
        case TR_SWI: return I;
        case TR_S_Q: return I / 4;
        default: return I / 32;   // TR_S_S
    }
}
static size_t trace_layer_words(const ti_qwen3_config& C) {
    size_t w = 0;
    for (int f = 0; f < TR_NFIELDS; f++) w += trace_row_words(C, f) * C.max_tokens;
    return w;
}
// the slot of (layer, field); layer == layers is the final residual (TR_X_IN only)
static uint32_t* trace_slot(ti_qwen3* m, int layer, int f) {
    size_t off = (size_t)layer * trace_layer_words(m->cfg);
    for (int g = 0; g < f; g++) off += trace_row_words(m->cfg, g) * m->cfg.max_tokens;
    return m->trace + off;
}

__global__ void k_copy_u32(const uint32_t* __restrict__ s, uint32_t* __restrict__ d, long n) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) d[i] = s[i];
}

// copy `rows` rows of field f from src into the trace (nothing when no trace is set)
static int trace_put(ti_ctx* c, ti_qwen3* m, int layer, int f, const void* src, int rows) {
    if (!m->trace) return TI_OK;
    const long n = (long)trace_row_words(m->cfg, f) * rows;
    const long blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
    k_copy_u32<<<(unsigned)blocks, 256, 0, c->stream>>>(static_cast<const uint32_t*>(src), trace_slot(m, layer, f), n);
    TI_LAUNCHED("k_copy_u32 (trace)");
    return TI_OK;
}

static int mk(ti_qwen3* m, void** p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 4);
    if (e != hipSuccess) return ti_hip_fail(e, "ti_qwen3_create hipMalloc");
    m->allocs.push_back(*p);
    return TI_OK;
}

static void release(ti_qwen3* m) {
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
}

extern "C" int ti_qwen3_create(ti_ctx* c, const ti_qwen3_config* cfg, ti_qwen3** out) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(cfg && out, "ti_qwen3_create: null argument");
    *out = nullptr;
    const ti_qwen3_config& C = *cfg;
    TI_REQUIRE(C.layers > 0 && C.hidden > 0 && C.intermediate > 0 && C.n_heads > 0 && C.n_kv_heads > 0 &&
               C.n_heads % C.n_kv_heads == 0 && C.vocab > 0 && C.max_ctx > 0 && C.max_tokens > 0,
               "ti_qwen3_create: bad config");
    TI_REQUIRE(C.hidden % 32 == 0 && C.intermediate % 32 == 0 && C.head_dim % 32 == 0 && C.head_dim <= 128,
               "ti_qwen3_create: hidden/intermediate/head_dim must be multiples of 32 (head_dim <= 128)");
    TI_REQUIRE(C.max_tokens <= TI_ACT_TMAX && C.max_tokens * C.n_heads <= TI_ATTN_ROWS_MAX,
               "ti_qwen3_create: max_tokens too large");
    TI_REQUIRE((C.max_ctx + 127) / 128 <= TI_ATTN_SPLITS_MAX, "ti_qwen3_create: max_ctx > %d", TI_ATTN_SPLITS_MAX * 128);
    TI_REQUIRE(C.n_heads / C.n_kv_heads <= 2 && (C.head_dim == 64 || C.head_dim == 128),
               "ti_qwen3_create: the decode step covers head_dim 64/128 with at most 2 query heads per KV head");
    {
        int kmax = C.hidden > C.intermediate ? C.hidden : C.intermediate;
        kmax = kmax > C.n_heads * C.head_dim ? kmax : C.n_heads * C.head_dim;
        TI_REQUIRE(kmax <= ti_fused_kmax(0) && C.hidden <= ti_fused_kmax(1),
                   "ti_qwen3_create: hidden <= %d and projection inputs <= %d required", ti_fused_kmax(1), ti_fused_kmax(0));
    }
    TI_REQUIRE(!c->capturing, "ti_qwen3_create: not during graph capture");
    TI_HIP(hipSetDevice(c->device));
    ti_qwen3* m = new ti_qwen3();
    m->cfg = C;
    const int H = C.hidden, I = C.intermediate, hd = C.head_dim;
    const int nq = C.n_heads * hd, nkv = C.n_kv_heads * hd, T = C.max_tokens;
    auto lin = [&](Lin& l, int N, int K) -> int {
        l.N = N;
        l.K = K;
        int rc = mk(m, (void**)&l.pack, (size_t)N * K / 2);
        if (!rc) rc = mk(m, (void**)&l.sc, (size_t)N * K / 16);
        return rc;
    };
    int rc = 0;
    m->L.resize(C.layers);
    m->kvs = kv_slots(C);
    const size_t kvw = (size_t)C.max_ctx * nkv;   // int8 elements per layer per K or V (scales: kvw / 32)
    const size_t kvc = (size_t)C.max_ctx * m->kvs * hd;   // code bytes per layer per K or V (padded rows)
    for (int l = 0; l < C.layers && !rc; l++) {
        Layer& y = m->L[l];
        rc = lin(y.q, nq, H); if (!rc) rc = lin(y.k, nkv, H); if (!rc) rc = lin(y.v, nkv, H);
        if (!rc) rc = lin(y.o, H, nq); if (!rc) rc = lin(y.gate, I, H); if (!rc) rc = lin(y.up, I, H);
        if (!rc) rc = lin(y.down, H, I);
        if (!rc) rc = mk(m, (void**)&y.in_norm, H * 2);
        if (!rc) rc = mk(m, (void**)&y.post_norm, H * 2);
        if (!rc) rc = mk(m, (void**)&y.q_norm, hd * 2);
        if (!rc) rc = mk(m, (void**)&y.k_norm, hd * 2);
        if (!rc) rc = mk(m, (void**)&y.kq, kvc);
        if (!rc) rc = mk(m, (void**)&y.vq, kvc);
        if (!rc) rc = mk(m, (void**)&y.ks, kvw / 32 * 4);
        if (!rc) rc = mk(m, (void**)&y.vs, kvw / 32 * 4);
    }
    if (!rc) rc = mk(m, (void**)&m->embed, (size_t)C.vocab * H * 2);
    if (!rc) rc = mk(m, (void**)&m->final_norm, H * 2);
    if (!rc) rc = lin(m->lm, C.vocab, H);
    struct { float** p; size_t n; } fb[] = {{&m->x, (size_t)T * H}, {&m->normed, (size_t)T * H}, {&m->q, (size_t)T * nq},
                                            {&m->k, (size_t)T * nkv}, {&m->v, (size_t)T * nkv}, {&m->qr, (size_t)T * nq},
                                            {&m->kr, (size_t)T * nkv}, {&m->attn, (size_t)T * nq}, {&m->gate, (size_t)T * I},
                                            {&m->up, (size_t)T * I}, {&m->swi, (size_t)T * I}, {&m->last, (size_t)H},
                                            {&m->logits, (size_t)C.vocab}, {&m->amx_v, (size_t)AMX_PARTS}};
    for (auto& f : fb) if (!rc) rc = mk(m, (void**)f.p, f.n * 4);
    const size_t kmax = (size_t)(H > I ? (H > nq ? H : nq) : (I > nq ? I : nq));   // widest GEMV input
    if (!rc) rc = mk(m, (void**)&m->xq, (size_t)T * kmax);                          // [T][kmax] int8 codes
    if (!rc) rc = mk(m, (void**)&m->xs, (size_t)T * kmax / 32 * 4);
    if (!rc) rc = mk(m, (void**)&m->xsum, kmax / 16 * 4);
    if (!rc) rc = mk(m, (void**)&m->psum, 16 * 256 * 4);
    if (!rc) rc = mk(m, (void**)&m->hist, (size_t)(C.max_ctx + 1) * 4);
    if (!rc) rc = mk(m, (void**)&m->dpos, 4);
    if (!rc) rc = mk(m, (void**)&m->samp, 2 * 4);
    if (!rc) {
        const uint32_t s0[2] = {0u, TI_SEED_INIT};   // greedy; the reference's first seed state
        hipError_t e = hipMemcpy(m->samp, s0, sizeof(s0), hipMemcpyHostToDevice);
        if (e != hipSuccess) rc = ti_hip_fail(e, "ti_qwen3_create sampling words");
    }
    if (!rc) rc = mk(m, (void**)&m->rope, (size_t)C.max_ctx * hd * 4);
    if (!rc) rc = mk(m, (void**)&m->rope_cur, (size_t)hd * 4);
    if (!rc) {
        std::vector<float> tab((size_t)C.max_ctx * hd);
        for (int p = 0; p < C.max_ctx; p++) ti_rope_row(tab.data() + (size_t)p * hd, p, hd, C.rope_theta);
        hipError_t e = hipMemcpy(m->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(m->rope_cur, tab.data(), (size_t)hd * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) rc = ti_hip_fail(e, "ti_qwen3_create rope table");
    }
    if (!rc) rc = mk(m, (void**)&m->amx_i, (size_t)AMX_PARTS * 4);
    if (!rc) {
        hipError_t e = hipMemset(m->hist, 0, (size_t)(C.max_ctx + 1) * 4);
        if (e == hipSuccess) e = hipMemset(m->dpos, 0, 4);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) rc = ti_hip_fail(e, "ti_qwen3_create clear");
    }
    if (rc) { release(m); return rc; }
    *out = m;
    return TI_OK;
}

extern "C" int ti_qwen3_destroy(ti_ctx* c, ti_qwen3* m) {
    TI_CHECK_CTX(c);
    if (!m) return TI_OK;
    TI_REQUIRE(!c->capturing, "ti_qwen3_destroy: not during graph capture");
    TI_HIP(hipStreamSynchronize(c->stream));
    release(m);
    return TI_OK;
}

// Tensor names follow the Hugging Face checkpoint (models/qwen3.js:3470, 3945-4049).
extern "C" int ti_qwen3_tensor(ti_qwen3* m, const char* name, void** data, size_t* data_bytes, void** scales,
                               size_t* scale_bytes) {
    TI_REQUIRE(m && name && data && data_bytes, "ti_qwen3_tensor: null argument");
    const ti_qwen3_config& C = m->cfg;
    *data = nullptr;
    *data_bytes = 0;
    if (scales) *scales = nullptr;
    if (scale_bytes) *scale_bytes = 0;
    auto f16 = [&](uint16_t* p, size_t n) { *data = p; *data_bytes = n * 2; return TI_OK; };
    auto lin = [&](Lin& l) {
        *data = l.pack;
        *data_bytes = (size_t)l.N * l.K / 2;
        if (scales) *scales = l.sc;
        if (scale_bytes) *scale_bytes = (size_t)l.N * l.K / 16;
        return TI_OK;
    };
    std::string s(name);
    if (s == "model.embed_tokens.weight") return f16(m->embed, (size_t)C.vocab * C.hidden);
    if (s == "model.norm.weight") return f16(m->final_norm, C.hidden);
    if (s == "lm_head.weight") return lin(m->lm);
    int l = -1;
    char rest[128] = {0};
    if (sscanf(name, "model.layers.%d.%127s", &l, rest) == 2 && l >= 0 && l < C.layers) {
        Layer& y = m->L[l];
        std::string r(rest);
        if (r == "input_layernorm.weight") return f16(y.in_norm, C.hidden);
        if (r == "post_attention_layernorm.weight") return f16(y.post_norm, C.hidden);
        if (r == "self_attn.q_norm.weight") return f16(y.q_norm, C.head_dim);
        if (r == "self_attn.k_norm.weight") return f16(y.k_norm, C.head_dim);
        if (r == "self_attn.q_proj.weight") return lin(y.q);
        if (r == "self_attn.k_proj.weight") return lin(y.k);
        if (r == "self_attn.v_proj.weight") return lin(y.v);
        if (r == "self_attn.o_proj.weight") return lin(y.o);
        if (r == "mlp.gate_proj.weight") return lin(y.gate);
        if (r == "mlp.up_proj.weight") return lin(y.up);
        if (r == "mlp.down_proj.weight") return lin(y.down);
    }
    return ti_fail(TI_ERR_INVALID, "ti_qwen3_tensor: unknown tensor '%s'", name);
}

extern "C" int ti_qwen3_kv(ti_qwen3* m, int layer, uint32_t** kq, float** ks, uint32_t** vq, float** vs) {
    TI_REQUIRE(m && layer >= 0 && layer < m->cfg.layers && kq && ks && vq && vs, "ti_qwen3_kv: bad argument");
    *kq = m->L[layer].kq;
    *ks = m->L[layer].ks;
    *vq = m->L[layer].vq;
    *vs = m->L[layer].vs;
    return TI_OK;
}

extern "C" int ti_qwen3_kv_layout(const ti_qwen3* m, int* slots) {
    TI_REQUIRE(m && slots, "ti_qwen3_kv_layout: null argument");
    *slots = m->kvs;
    return TI_OK;
}

extern "C" int ti_qwen3_kv_write(ti_ctx* c, ti_qwen3* m, int layer, const float* kr, const float* v, int T, int pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && layer >= 0 && layer < m->cfg.layers && kr && v, "ti_qwen3_kv_write: bad argument");
    TI_REQUIRE(T > 0 && pos >= 0 && pos + T <= m->cfg.max_ctx, "ti_qwen3_kv_write: rows [%d, %d) outside the cache (%d)", pos,
               pos + T, m->cfg.max_ctx);
    TI_REQUIRE(((uintptr_t)kr & 15u) == 0 && ((uintptr_t)v & 15u) == 0, "ti_qwen3_kv_write: kr/v must be 16-byte aligned");
    const Layer& y = m->L[layer];
    return ti_kv_write_launch(c, kr, v, y.kq, y.ks, y.vq, y.vs, T, m->cfg.n_kv_heads, m->cfg.head_dim, pos, m->kvs);
}

extern "C" int ti_qwen3_logits(ti_qwen3* m, float** logits) {
    TI_REQUIRE(m && logits, "ti_qwen3_logits: null argument");
    *logits = m->logits;
    return TI_OK;
}

extern "C" int ti_qwen3_trace(ti_qwen3* m, void* buf, size_t bytes) {
    TI_REQUIRE(m, "ti_qwen3_trace: null model");
    if (!buf) { m->trace = nullptr; return TI_OK; }
    const size_t need = (trace_layer_words(m->cfg) * m->cfg.layers + (size_t)m->cfg.hidden * m->cfg.max_tokens) * 4;
    TI_REQUIRE(bytes >= need, "ti_qwen3_trace: the trace needs %zu bytes (got %zu)", need, bytes);
    TI_REQUIRE(((uintptr_t)buf & 15) == 0, "ti_qwen3_trace: buffer must be 16-byte aligned");
    m->trace = static_cast<uint32_t*>(buf);
    return TI_OK;
}

extern "C" int ti_qwen3_set_pos(ti_ctx* c, ti_qwen3* m, int pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && pos >= 0 && pos < m->cfg.max_ctx, "ti_qwen3_set_pos: pos %d out of [0, %d)", pos, m ? m->cfg.max_ctx : 0);
    k_set_pos<<<1, 256, 0, c->stream>>>(m->dpos, pos, m->rope, m->rope_cur, m->cfg.head_dim, m->cfg.max_ctx);
    TI_LAUNCHED("k_set_pos");
    m->pos_hint = pos;
    return TI_OK;
}

// The decode step's attention splits per KV head for a step at pos: the reference picks its
// split count from the context on every dispatch (_decNsplit, models/qwen3.js:2354); a
// captured step fixes it when it is captured, from the position last set on the host.
static int decode_splits(const ti_qwen3* m, int pos) {
    const int S = pos + 1 < m->cfg.max_ctx ? pos + 1 : m->cfg.max_ctx;
    return ti_attn_decode_splits(S);
}

extern "C" int ti_qwen3_decode_splits(const ti_qwen3* m, int pos, int* splits) {
    TI_REQUIRE(m && splits, "ti_qwen3_decode_splits: null argument");
    TI_REQUIRE(pos >= 0 && pos < m->cfg.max_ctx, "ti_qwen3_decode_splits: pos %d out of [0, %d)", pos, m->cfg.max_ctx);
    *splits = decode_splits(m, pos);
    return TI_OK;
}

__global__ void k_set_word(uint32_t* __restrict__ dst, uint32_t v) {
    if (threadIdx.x == 0) *dst = v;
}

// forward(..., {temp}) (models/qwen3.js:4052): the temperature of the following steps and
// forwards (<= 0: greedy), read on the device, so a captured decode step samples at
// whatever temperature was last set. Stream-ordered; may be captured.
extern "C" int ti_qwen3_sampling(ti_ctx* c, ti_qwen3* m, float temperature) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m, "ti_qwen3_sampling: null model");
    TI_REQUIRE(temperature == temperature, "ti_qwen3_sampling: temperature is NaN");
    const float t = temperature > 0.0f ? temperature : 0.0f;
    k_set_word<<<1, 64, 0, c->stream>>>(m->samp + TI_SAMP_TEMP, __builtin_bit_cast(uint32_t, t));
    TI_LAUNCHED("k_set_word");
    return TI_OK;
}

// The seed stream's state (_rngSeed, models/qwen3.js:2733): each sampled step first
// advances it (s = 1664525 s + 1013904223) and samples with the result. A new decoder
// starts at 0x9E3779B9, as the reference's module does.
extern "C" int ti_qwen3_seed(ti_ctx* c, ti_qwen3* m, uint32_t state) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m, "ti_qwen3_seed: null model");
    k_set_word<<<1, 64, 0, c->stream>>>(m->samp + TI_SAMP_STATE, state);
    TI_LAUNCHED("k_set_word");
    return TI_OK;
}

extern "C" int ti_qwen3_get_seed(ti_ctx* c, ti_qwen3* m, uint32_t* state) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && state, "ti_qwen3_get_seed: null argument");
    return ti_buf_read(c, m->samp, TI_SAMP_STATE * 4, state, 4);
}

extern "C" int ti_qwen3_write_tokens(ti_ctx* c, ti_qwen3* m, int from, int count, const int32_t* ids) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && ids && from >= 0 && count >= 0 && from + count <= m->cfg.max_ctx + 1, "ti_qwen3_write_tokens: bad range");
    return ti_buf_write(c, m->hist, (size_t)from * 4, ids, (size_t)count * 4);
}

extern "C" int ti_qwen3_read_tokens(ti_ctx* c, ti_qwen3* m, int from, int count, int32_t* ids) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && ids && from >= 0 && count >= 0 && from + count <= m->cfg.max_ctx + 1, "ti_qwen3_read_tokens: bad range");
    return ti_buf_read(c, m->hist, (size_t)from * 4, ids, (size_t)count * 4);
}

// readU32Range(_tokHist, from, count) as submitted in decodeLoop (models/qwen3.js:4423): the
// copy is queued behind the steps already issued and does not wait
extern "C" int ti_qwen3_read_tokens_async(ti_ctx* c, ti_qwen3* m, int from, int count, int32_t* ids) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && ids && from >= 0 && count >= 0 && from + count <= m->cfg.max_ctx + 1,
               "ti_qwen3_read_tokens_async: bad range");
    return ti_buf_read_async(c, m->hist, (size_t)from * 4, ids, (size_t)count * 4);
}

// argmaxKernel (models/qwen3.js:2681-2690): tok_hist[out_pos] = argmax(logits[0..N)),
// ties resolved as the reference's one-stage (N < 16384) or two-stage trees resolve them.
extern "C" int ti_argmax(ti_ctx* c, const float* logits, int N, uint32_t* tok_hist, int out_pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(logits && tok_hist, "ti_argmax: null buffer");
    TI_REQUIRE(N > 0 && out_pos >= 0, "ti_argmax: need N > 0 and out_pos >= 0 (N=%d out_pos=%d)", N, out_pos);
    TI_REQUIRE(AMX_PARTS <= TI_AMAX_PARTS, "ti_argmax: partial buffer too small");
    k_argmax_p1<<<AMX_PARTS, AMX_THREADS, 0, c->stream>>>(logits, N, c->amax_v, c->amax_i);
    TI_LAUNCHED("k_argmax_p1");
    k_argmax_p2<<<1, AMX_PARTS, 0, c->stream>>>(c->amax_v, c->amax_i, N, tok_hist, out_pos, nullptr, 0);
    TI_LAUNCHED("k_argmax_p2");
    return TI_OK;
}

// gumbelNoise (models/qwen3.js:2722-2740): logits[i] += temp * (-log(-log(u_i))), u_i from
// the PCG hash of i and `seed` (the caller advances the seed stream, as the reference's
// host does before each sampled step); an argmax of the result is the sample.
__global__ void k_gumbel(float* __restrict__ logits, int N, uint32_t seed, float temp) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const float g = temp * ti_gumbel((uint32_t)i, seed);
    logits[i] = logits[i] + g;
}

extern "C" int ti_gumbel_noise(ti_ctx* c, float* logits, int N, uint32_t seed, float temp) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(logits && N > 0, "ti_gumbel_noise: need logits and N > 0 (N=%d)", N);
    TI_REQUIRE(temp == temp, "ti_gumbel_noise: temperature is NaN");
    k_gumbel<<<(unsigned)((N + 255) / 256), 256, 0, c->stream>>>(logits, N, seed, temp);
    TI_LAUNCHED("k_gumbel");
    return TI_OK;
}

// embedGather (models/qwen3.js:1663-1676): y[t, :] = f32(emb[ids[id_off + t], :]) for
// t < T; ids at or past `vocab` read the last row (no out-of-bounds read).
extern "C" int ti_embed(ti_ctx* c, const int32_t* ids, const uint16_t* emb, float* y, int T, int H, int id_off,
                        int vocab) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(ids && emb && y, "ti_embed: null buffer");
    TI_REQUIRE(T > 0 && H > 0 && id_off >= 0 && vocab > 0, "ti_embed: bad shape (T=%d H=%d off=%d vocab=%d)", T, H, id_off, vocab);
    k_embed<<<(unsigned)(((long)T * H + 255) / 256), 256, 0, c->stream>>>(reinterpret_cast<const uint32_t*>(ids), emb, y,
                                                                           T, H, id_off, nullptr, vocab);
    TI_LAUNCHED("k_embed");
    return TI_OK;
}

// One decode step at the device position (forward(null, pos, {chain: true}),
// models/qwen3.js:3951-4055) in 2 + 4 x layers launches:
//   embed(tok[pos])
//   per layer: [rmsnormQ + q/k/v GEMV + attnPrep + split-KV attention + combine +
//               quantQ8 of the output] (the q/k/v rows handed between the attention's own
//               workgroups, k_attn.hip; as two launches where that kernel does not apply)
//              [o_proj GEMV + residual]
//              [rmsnormQ + gate/up + SiLU + quantQ8 of swi]
//              [down_proj GEMV + residual]
//   [final rmsnorm + lm_head + argmax -> tok[pos+1], pos += 1]
extern "C" int ti_qwen3_decode(ti_ctx* c, ti_qwen3* m) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m, "ti_qwen3_decode: null model");
    const ti_qwen3_config& C = m->cfg;
    const int H = C.hidden, I = C.intermediate, hd = C.head_dim, nHq = C.n_heads, nKv = C.n_kv_heads;
    const int nq = nHq * hd, nkv = nKv * hd;
    int rc;
#define RC(x) do { rc = (x); if (rc) return rc; } while (0)
    k_embed<<<(H + 255) / 256, 256, 0, c->stream>>>(m->hist, m->embed, m->x, 1, H, 0, m->dpos, C.vocab);
    TI_LAUNCHED("k_embed");
    const bool tr = m->trace != nullptr;
    for (int l = 0; l < C.layers; l++) {
        Layer& y = m->L[l];
        const uint32_t* packs[3] = {y.q.pack, y.k.pack, y.v.pack};
        const uint16_t* scs[3] = {y.q.sc, y.k.sc, y.v.sc};
        float* ys[3] = {m->q, m->k, m->v};
        RC(trace_put(c, m, l, TR_X_IN, m->x, 1));
        RC(ti_attn_qkv_launch(c, m->x, y.in_norm, C.rms_eps, H, packs, scs, ys, tr ? 1 : 0,
                              tr ? trace_slot(m, l, TR_XN_Q) : nullptr,
                              tr ? reinterpret_cast<float*>(trace_slot(m, l, TR_XN_S)) : nullptr, y.q_norm, y.k_norm,
                              y.kq, y.ks, y.vq, y.vs, m->attn, nHq, nKv, hd, m->dpos, C.max_ctx, C.rope_theta,
                              C.rms_eps, decode_splits(m, m->pos_hint), m->rope_cur, m->xq, m->xs, m->kvs));
        RC(trace_put(c, m, l, TR_Q, m->q, 1));
        RC(trace_put(c, m, l, TR_K, m->k, 1));
        RC(trace_put(c, m, l, TR_V, m->v, 1));
        RC(trace_put(c, m, l, TR_ATTN, m->attn, 1));
        RC(trace_put(c, m, l, TR_A_Q, m->xq, 1));
        RC(trace_put(c, m, l, TR_A_S, m->xs, 1));
        RC(ti_gemv_q4_q8_launch(c, m->xq, m->xs, y.o.pack, y.o.sc, m->x, H, nq, 1));
        RC(trace_put(c, m, l, TR_X_MID, m->x, 1));
        RC(ti_fused_gateup_launch(c, m->x, y.post_norm, C.rms_eps, y.gate.pack, y.gate.sc, y.up.pack, y.up.sc,
                                  tr ? reinterpret_cast<float*>(trace_slot(m, l, TR_SWI)) : nullptr, I, H, m->xq, m->xs));
        RC(trace_put(c, m, l, TR_S_Q, m->xq, 1));
        RC(trace_put(c, m, l, TR_S_S, m->xs, 1));
        RC(ti_gemv_q4_q8_launch(c, m->xq, m->xs, y.down.pack, y.down.sc, m->x, H, I, 1));
    }
    RC(trace_put(c, m, C.layers, TR_X_IN, m->x, 1));
    RC(ti_fused_lmhead_launch(c, m->x, m->final_norm, C.rms_eps, m->lm.pack, m->lm.sc, m->logits, C.vocab, H, m->hist,
                              m->dpos, 0, C.max_ctx, m->rope, m->rope_cur, hd, m->samp));
    return TI_OK;
}

// forward(ids, pos) for T >= 1 host tokens (prefill, or the T-token batch): writes
// the ids into the token history at [pos, pos+T), runs the T-token forward, puts
// the argmax of the last token's logits at hist[pos+T] and sets the device
// position to pos+T, so the next chained step embeds hist[pos+T].
extern "C" int ti_qwen3_forward(ti_ctx* c, ti_qwen3* m, const int32_t* ids, int T, int pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m, "ti_qwen3_forward: null model");
    const ti_qwen3_config& C = m->cfg;
    TI_REQUIRE(T > 0 && T <= C.max_tokens && pos >= 0 && pos + T <= C.max_ctx,
               "ti_qwen3_forward: T=%d pos=%d outside max_tokens=%d / max_ctx=%d", T, pos, C.max_tokens, C.max_ctx);
    const int H = C.hidden, I = C.intermediate, hd = C.head_dim, nHq = C.n_heads, nKv = C.n_kv_heads;
    const int nq = nHq * hd, nkv = nKv * hd;
    int rc;
    if (ids) RC(ti_buf_write(c, m->hist, (size_t)pos * 4, ids, (size_t)T * 4));   // else already in the history
    k_embed<<<(unsigned)(((long)T * H + 255) / 256), 256, 0, c->stream>>>(m->hist, m->embed, m->x, T, H, pos, nullptr, C.vocab);
    TI_LAUNCHED("k_embed");
    // 2..16 tokens: per layer [rmsnorm + quantQ8T + q/k/v] [attention] [split merge +
    // quantQ8T] [o_proj + residual] [rmsnorm + quantQ8T + gate/up + SiLU + quantQ8T]
    // [down + residual], the projections on the matrix cores (k_tgemm.hip, k_tattn.hip).
    // Up to 4 tokens the residual projections also write the RMSNorm partial sums of the
    // new x (m->psum), from which the next projection normalises and quantises x in its
    // prologue (two launches fewer per layer); past 4 tokens that prologue (every
    // workgroup quantises all T x H elements) costs more than the launch it saves, and a
    // per-token norm kernel writes the codes into the context's activation scratch
    // first (1.7B geometry at 8k: T = 2 1.22 against 1.29 ms, T = 4 1.26 against 1.32,
    // T = 8 1.39 against 1.36, T = 16 3.13 against 2.94; with the pairwise-group MFMA,
    // T = 8 1.37 against 1.32 at 8k and 1.60 against 1.55 at 32k; both paths give the same
    // bits).
    // The attention and SwiGLU codes live in the model's scratch.
    const bool fused = ti_tnorm_ok(H) && ti_tgemm_gateup_ok(T, H) && ti_tgemm_ok(T, nq) && ti_tgemm_ok(T, I) &&
                       nq % 16 == 0 && nkv % 16 == 0 && I % 32 == 0;
    const bool fused_attn = ti_tattn_ok(T, nHq, nKv, hd);
    const bool norm_in = fused && T <= 4 && ti_tgemm_norm_ok(T, H);
    if (norm_in) RC(ti_tsumsq_launch(c, m->x, m->psum, T, H));
    float* const pout = norm_in ? m->psum : nullptr;
    const TgIn codes_in = {c->act_q, c->act_s, nullptr, nullptr, 0.0f, nullptr};
    const TgIn attn_in = {m->xq, m->xs, nullptr, nullptr, 0.0f, nullptr};
    for (int l = 0; l < C.layers; l++) {
        Layer& y = m->L[l];
        RC(trace_put(c, m, l, TR_X_IN, m->x, T));
        if (fused) {
            const uint32_t* packs[3] = {y.q.pack, y.k.pack, y.v.pack};
            const uint16_t* scs[3] = {y.q.sc, y.k.sc, y.v.sc};
            float* ys[3] = {m->q, m->k, m->v};
            const int Ns[3] = {nq, nkv, nkv};
            const TgIn in_norm = {nullptr, nullptr, m->x, y.in_norm, C.rms_eps, m->psum};
            if (!norm_in) {
                RC(ti_tnorm_q8_launch(c, m->x, y.in_norm, C.rms_eps, c->act_q, c->act_s, T, H));
                RC(trace_put(c, m, l, TR_XN_Q, c->act_q, T));
                RC(trace_put(c, m, l, TR_XN_S, c->act_s, T));
            }
            RC(ti_tgemm_launch(c, norm_in ? in_norm : codes_in, 3, packs, scs, ys, Ns, T, H, 0, nullptr));
        } else {
            RC(ti_rmsnorm(c, m->x, y.in_norm, m->normed, T, H, C.rms_eps));
            RC(ti_linear_q4(c, m->normed, y.q.pack, y.q.sc, m->q, T, nq, H, 0));
            RC(ti_linear_q4(c, m->normed, y.k.pack, y.k.sc, m->k, T, nkv, H, 0));
            RC(ti_linear_q4(c, m->normed, y.v.pack, y.v.sc, m->v, T, nkv, H, 0));
        }
        if (fused && fused_attn) {
            RC(ti_tattn_launch(c, m->q, m->k, m->v, y.q_norm, y.k_norm, m->rope, y.kq, y.ks, y.vq, y.vs, pos, T, nHq, nKv,
                               hd, C.rms_eps, m->xq, m->xs, m->kvs));
        } else {
            RC(ti_rope_qk(c, m->q, y.q_norm, m->qr, T, nHq, hd, pos, C.rope_theta, C.rms_eps));
            RC(ti_rope_qk(c, m->k, y.k_norm, m->kr, T, nKv, hd, pos, C.rope_theta, C.rms_eps));
            RC(ti_kv_write_launch(c, m->kr, m->v, y.kq, y.ks, y.vq, y.vs, T, nKv, hd, pos, m->kvs));
            RC(ti_attn_decode_launch(c, m->qr, y.kq, y.ks, y.vq, y.vs, m->attn, pos + 1, T, nHq, nKv, hd, 0, nullptr, 0,
                                     m->kvs));
        }
        RC(trace_put(c, m, l, TR_Q, m->q, T));
        RC(trace_put(c, m, l, TR_K, m->k, T));
        RC(trace_put(c, m, l, TR_V, m->v, T));
        if (fused) {
            if (!fused_attn) {
                RC(trace_put(c, m, l, TR_ATTN, m->attn, T));
                RC(ti_quant_act_q8_async(c, m->attn, m->xq, m->xs, nullptr, T * (nq / 32)));
            }
            RC(trace_put(c, m, l, TR_A_Q, m->xq, T));
            RC(trace_put(c, m, l, TR_A_S, m->xs, T));
            RC(ti_tgemm_launch(c, attn_in, 1, &y.o.pack, &y.o.sc, &m->x, &H, T, nq, 1, pout));
            RC(trace_put(c, m, l, TR_X_MID, m->x, T));
            const TgIn post_norm = {nullptr, nullptr, m->x, y.post_norm, C.rms_eps, m->psum};
            if (!norm_in) RC(ti_tnorm_q8_launch(c, m->x, y.post_norm, C.rms_eps, c->act_q, c->act_s, T, H));
            RC(ti_tgemm_gateup_launch(c, norm_in ? post_norm : codes_in, y.gate.pack, y.gate.sc, y.up.pack, y.up.sc, I, H,
                                      T, m->xq, m->xs));
            RC(trace_put(c, m, l, TR_S_Q, m->xq, T));
            RC(trace_put(c, m, l, TR_S_S, m->xs, T));
            RC(ti_tgemm_launch(c, attn_in, 1, &y.down.pack, &y.down.sc, &m->x, &H, T, I, 1, pout));
            continue;
        }
        RC(trace_put(c, m, l, TR_ATTN, m->attn, T));
        RC(ti_linear_q4(c, m->attn, y.o.pack, y.o.sc, m->x, T, H, nq, 1));
        RC(trace_put(c, m, l, TR_X_MID, m->x, T));
        RC(ti_rmsnorm(c, m->x, y.post_norm, m->normed, T, H, C.rms_eps));
        RC(ti_linear_q4(c, m->normed, y.gate.pack, y.gate.sc, m->gate, T, I, H, 0));
        RC(ti_linear_q4(c, m->normed, y.up.pack, y.up.sc, m->up, T, I, H, 0));
        k_swiglu<<<(unsigned)(((long)T * I + 255) / 256), 256, 0, c->stream>>>(m->gate, m->up, m->swi, (long)T * I);
        TI_LAUNCHED("k_swiglu");
        RC(trace_put(c, m, l, TR_SWI, m->swi, T));
        RC(ti_linear_q4(c, m->swi, y.down.pack, y.down.sc, m->x, T, H, I, 1));
    }
    RC(trace_put(c, m, C.layers, TR_X_IN, m->x, T));
    k_copy_f32<<<(H + 255) / 256, 256, 0, c->stream>>>(m->x + (size_t)(T - 1) * H, m->last, H);
    TI_LAUNCHED("k_copy_f32");
    RC(ti_fused_lmhead_launch(c, m->last, m->final_norm, C.rms_eps, m->lm.pack, m->lm.sc, m->logits, C.vocab, H, m->hist,
                              nullptr, pos + T, C.max_ctx, nullptr, nullptr, 0, m->samp));
    k_set_pos<<<1, 256, 0, c->stream>>>(m->dpos, pos + T, m->rope, m->rope_cur, hd, C.max_ctx);
    TI_LAUNCHED("k_set_pos");
    m->pos_hint = pos + T < C.max_ctx ? pos + T : C.max_ctx - 1;
    return TI_OK;
#undef RC
}
