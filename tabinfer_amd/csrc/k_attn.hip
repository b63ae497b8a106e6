// k_attn.hip — int8-KV attention of the decode path:
//  A7 fused QK-RMSNorm + RoPE + int8 KV write   attnPrepQ8     models/qwen3.js:2228-2308
//     RMSNorm + RoPE for T tokens               ropeQK         models/qwen3.js:1700-1760
//     int8 KV write for T tokens                kvQuantWrite   models/qwen3.js:2180-2216
//  A8 split-KV decode attention (partials)      attnDecStreamQ8 models/qwen3.js:2077-2173
//  A9 log-sum-exp combine                        ATTN_DEC_COMBINE models/qwen3.js:2048-2068
//
// KV layout is the reference's: per layer, position-major, then head, then dim;
// int8 codes packed 4 per u32 (snorm: code/127 * group max), one f32 scale per
// 32 dims.
#include "ti_internal.h"

// ---------------------------------------------------------------------------
// snorm int8 (pack4x8snorm): code = floor(0.5 + 127*clamp(x/mx, -1, 1)),
// evaluated exactly (double) on the f32 quotient; mx = max(1e-12, max|x|).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t snorm_code(float x, float mx) {
    float e = x / mx;
    e = e > 1.0f ? 1.0f : (e < -1.0f ? -1.0f : e);
    return (uint32_t)((int)floor(0.5 + 127.0 * (double)e) & 0xff);
}

// Quantize 32 values held by one thread into 8 words + a scale.
__device__ __forceinline__ void snorm_group(const float* v, uint32_t* q, float* s) {
    float mx = 1e-12f;
#pragma unroll
    for (int j = 0; j < 32; j++) mx = fmaxf(mx, fabsf(v[j]));
    *s = mx;
#pragma unroll
    for (int w = 0; w < 8; w++)
        q[w] = snorm_code(v[4 * w], mx) | (snorm_code(v[4 * w + 1], mx) << 8) |
               (snorm_code(v[4 * w + 2], mx) << 16) | (snorm_code(v[4 * w + 3], mx) << 24);
}

// RMSNorm over one head row (thread j holds element j; 128 threads, tree from 64)
// then split-half RoPE at `pos`. The angle pos*theta^(-2i/hd) and its sin/cos are
// evaluated in f64 and rounded to f32 (the reference's f32 builtins are only
// specified on [-pi, pi], and positions reach 32768 rad).
__device__ float rope_norm(float x, int j, int hd, const uint16_t* __restrict__ w, int pos, float theta, float eps,
                           bool norm, float* red, float* rk) {
    if (norm) {
        red[j] = j < hd ? x * x : 0.0f;
        __syncthreads();
        for (int st = 64; st > 0; st >>= 1) {
            if (j < st) red[j] = red[j] + red[j + st];
            __syncthreads();
        }
        float m = red[0] / (float)hd;
        m = m + eps;
        float inv = 1.0f / sqrtf(m);
        if (j < hd) { float a = x * inv; rk[j] = a * ti_h2f(w[j]); }
    } else {
        if (j < hd) rk[j] = x;
    }
    __syncthreads();
    float out = 0.0f;
    if (j < hd) {
        int half = hd / 2;
        int fi = j < half ? j : j - half;
        double ang = (double)pos * pow((double)theta, -2.0 * (double)fi / (double)hd);
        float c = (float)cos(ang), s = (float)sin(ang);
        float partner = j < half ? rk[j + half] : rk[j - half];
        float rot = j < half ? -partner : partner;
        float a = rk[j] * c, b = rot * s;
        out = a + b;
    }
    __syncthreads();
    return out;
}

// A7: workgroup roles [0,nHq) q-head rope+norm -> qr ; [nHq, nHq+nKv) k-head
// rope+norm+quantize into the cache ; [nHq+nKv, nHq+2nKv) v-head quantize.
__global__ __launch_bounds__(128) void k_attn_prep_q8(const float* __restrict__ q, const float* __restrict__ k,
                                                      const float* __restrict__ v, const uint16_t* __restrict__ qw,
                                                      const uint16_t* __restrict__ kw, float* __restrict__ qr,
                                                      uint32_t* __restrict__ kq, float* __restrict__ ks,
                                                      uint32_t* __restrict__ vq, float* __restrict__ vs,
                                                      int nHq, int nKv, int hd, int pos, float theta, float eps,
                                                      const int* __restrict__ dpos) {
    __shared__ float red[128];
    __shared__ float rk[128];
    __shared__ float row[128];
    if (dpos) pos = *dpos;
    const int j = threadIdx.x;
    const int role = blockIdx.x;
    const bool isQ = role < nHq;
    const bool isK = !isQ && role < nHq + nKv;
    const int head = isQ ? role : (isK ? role - nHq : role - nHq - nKv);
    const float* src = isQ ? q : (isK ? k : v);
    float x = j < hd ? src[head * hd + j] : 0.0f;
    if (isQ || isK) x = rope_norm(x, j, hd, isQ ? qw : kw, pos, theta, eps, true, red, rk);
    if (isQ) {
        if (j < hd) qr[head * hd + j] = x;
        return;
    }
    if (j < hd) row[j] = x;
    __syncthreads();
    if (j < hd / 32) {
        float vals[32];
#pragma unroll
        for (int i = 0; i < 32; i++) vals[i] = row[j * 32 + i];
        size_t wbase = ((size_t)pos * nKv + head) * (hd / 4) + j * 8;
        size_t gbase = ((size_t)pos * nKv + head) * (hd / 32) + j;
        snorm_group(vals, (isK ? kq : vq) + wbase, (isK ? ks : vs) + gbase);
    }
}

// ropeQK for T tokens (prefill): out[t, h, :] = rope(norm(x[t, h, :])) at pos0+t.
__global__ __launch_bounds__(128) void k_rope_qk(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                 float* __restrict__ out, int nH, int hd, int pos0, float theta,
                                                 float eps, int norm) {
    __shared__ float red[128];
    __shared__ float rk[128];
    const int j = threadIdx.x;
    const int t = blockIdx.x / nH, h = blockIdx.x % nH;
    size_t base = ((size_t)t * nH + h) * hd;
    float xv = j < hd ? x[base + j] : 0.0f;
    float o = rope_norm(xv, j, hd, w, pos0 + t, theta, eps, norm != 0, red, rk);
    if (j < hd) out[base + j] = o;
}

// kvQuantWrite: thread = one 32-group; threads [0,nG) quantize K rows, [nG,2nG) V rows.
__global__ void k_kv_write_q8(const float* __restrict__ kr, const float* __restrict__ vv, uint32_t* __restrict__ kq,
                              float* __restrict__ ks, uint32_t* __restrict__ vq, float* __restrict__ vs, long nG,
                              long dst_g0) {
    long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= 2 * nG) return;
    const bool isV = idx >= nG;
    const long g = isV ? idx - nG : idx;
    const float4* src = reinterpret_cast<const float4*>((isV ? vv : kr) + g * 32);
    float vals[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float4 t = src[i];
        vals[4 * i] = t.x; vals[4 * i + 1] = t.y; vals[4 * i + 2] = t.z; vals[4 * i + 3] = t.w;
    }
    snorm_group(vals, (isV ? vq : kq) + (dst_g0 + g) * 8, (isV ? vs : ks) + dst_g0 + g);
}

// ---------------------------------------------------------------------------
// A8: split-KV decode attention. Workgroup (256 threads) = (kv head hk, split).
// All G = nHq/nKv query heads of the group are served from one read of K/V.
// Token rows are read 16 bytes per lane, LPT = hd/16 lanes per row, so one pass
// covers 256/LPT tokens; a split is walked in tiles of TILE tokens: scores for
// the tile -> tile max -> exp -> P*V, with the running (m, l, acc) rescaled per
// tile (online softmax). Output: unnormalised o, and (m, l) per (q head, split).
// ---------------------------------------------------------------------------
namespace {
constexpr int ATT_THREADS = 256;
constexpr int ATT_TILE = 256;

__device__ __forceinline__ float i8f(uint32_t w, int b) { return (float)(int)(int8_t)((w >> (8 * b)) & 0xffu); }

template <int HD, int G>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_split_q8(const float* __restrict__ qr, const uint4* __restrict__ kq,
                                                               const float* __restrict__ ks, const uint4* __restrict__ vq,
                                                               const float* __restrict__ vs, float* __restrict__ po,
                                                               float* __restrict__ pml, int S, int nKv, int nsplit,
                                                               int per, int ns_stride, const int* __restrict__ dpos) {
    constexpr int LPT = HD / 16;              // lanes per token row
    constexpr int TPP = ATT_THREADS / LPT;    // tokens per pass
    constexpr int PASSES = ATT_TILE / TPP;
    __shared__ float sc[G][ATT_TILE];
    __shared__ float redm[G][ATT_THREADS / 64];
    __shared__ float reds[G][ATT_THREADS / 64];
    __shared__ float pvred[TPP][G * HD + 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const int hk = blockIdx.x % nKv;
    const int split = blockIdx.x / nKv;
    // query t of a T-token call attends keys [0, S+t); with a device position
    // the context is *dpos + 1 and splits past it have nothing to do
    const int qt = blockIdx.y;
    if (dpos) {
        S = *dpos + 1;
        nsplit = (S + per - 1) / per;
        if (split >= nsplit) return;
    }
    S += qt;
    qr += (size_t)qt * (nKv * G) * HD;
    po += (size_t)qt * (nKv * G) * ns_stride * HD;
    pml += (size_t)qt * (nKv * G) * ns_stride * 2;
    const int tp = tid / LPT, sl = tid % LPT;       // token slot in a pass, 16-dim slice
    const int c0 = split * per;
    const int c1 = min(S, c0 + per);
    const int row_words4 = nKv * HD / 16;           // uint4 per cached position
    const int row_groups = nKv * HD / 32;
    const float qk_scale = 1.0f / (127.0f * sqrtf((float)HD));

    float qv[G][16];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int i = 0; i < 16; i++) qv[h][i] = qr[(size_t)(hk * G + h) * HD + sl * 16 + i];

    float m_run[G], l_run[G], acc[G][16];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m_run[h] = -3.0e38f;
        l_run[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) acc[h][i] = 0.0f;
    }

    for (int t0 = c0; t0 < c1; t0 += ATT_TILE) {
        const int n = min(ATT_TILE, c1 - t0);
        // ---- scores: all K loads of the tile issued first
        uint4 kw[PASSES];
        float ksc[PASSES];
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            int t = t0 + p * TPP + tp;
            t = t < c1 ? t : c1 - 1;
            kw[p] = ti_ld_nt(kq + (size_t)t * row_words4 + hk * LPT + sl);
            ksc[p] = ks[(size_t)t * row_groups + hk * (HD / 32) + sl / 2];
        }
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const uint32_t ww[4] = {kw[p].x, kw[p].y, kw[p].z, kw[p].w};
            float part[G];
#pragma unroll
            for (int h = 0; h < G; h++) {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; i++) d = fmaf(qv[h][i], i8f(ww[i >> 2], i & 3), d);
                part[h] = d * ksc[p];
            }
#pragma unroll
            for (int o = LPT / 2; o > 0; o >>= 1)
#pragma unroll
                for (int h = 0; h < G; h++) part[h] += __shfl_xor(part[h], o, 64);
            const int j = p * TPP + tp;
            if (sl == 0 && j < ATT_TILE)
#pragma unroll
                for (int h = 0; h < G; h++) sc[h][j] = j < n ? part[h] * qk_scale : -3.0e38f;
        }
        __syncthreads();
        // ---- tile max and exp
        float mt[G];
#pragma unroll
        for (int h = 0; h < G; h++) {
            float v = -3.0e38f;
            for (int j = tid; j < ATT_TILE; j += ATT_THREADS) v = fmaxf(v, sc[h][j]);
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
            if (lane == 0) redm[h][wv] = v;
        }
        __syncthreads();
        float corr[G];
#pragma unroll
        for (int h = 0; h < G; h++) {
            float v = redm[h][0];
#pragma unroll
            for (int w = 1; w < ATT_THREADS / 64; w++) v = fmaxf(v, redm[h][w]);
            mt[h] = fmaxf(m_run[h], v);
            corr[h] = expf(m_run[h] - mt[h]);
            float s = 0.0f;
            for (int j = tid; j < ATT_TILE; j += ATT_THREADS) {
                float pe = j < n ? expf(sc[h][j] - mt[h]) : 0.0f;
                sc[h][j] = pe;
                s += pe;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
            if (lane == 0) reds[h][wv] = s;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < G; h++) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < ATT_THREADS / 64; w++) s += reds[h][w];
            l_run[h] = l_run[h] * corr[h] + s;
            m_run[h] = mt[h];
#pragma unroll
            for (int i = 0; i < 16; i++) acc[h][i] *= corr[h];
        }
        // ---- P * V
        uint4 vw[PASSES];
        float vsc[PASSES];
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            int t = t0 + p * TPP + tp;
            t = t < c1 ? t : c1 - 1;
            vw[p] = ti_ld_nt(vq + (size_t)t * row_words4 + hk * LPT + sl);
            vsc[p] = vs[(size_t)t * row_groups + hk * (HD / 32) + sl / 2];
        }
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const int j = p * TPP + tp;          // p_j is 0 past the tile's last token
            const uint32_t ww[4] = {vw[p].x, vw[p].y, vw[p].z, vw[p].w};
#pragma unroll
            for (int h = 0; h < G; h++) {
                float pw = sc[h][j] * vsc[p] * (1.0f / 127.0f);
#pragma unroll
                for (int i = 0; i < 16; i++) acc[h][i] = fmaf(pw, i8f(ww[i >> 2], i & 3), acc[h][i]);
            }
        }
        __syncthreads();   // sc is rewritten by the next tile
    }
    // ---- reduce the TPP token slots and write the partials
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int i = 0; i < 16; i++) pvred[tp][h * HD + sl * 16 + i] = acc[h][i];
    __syncthreads();
    for (int o = tid; o < G * HD; o += ATT_THREADS) {
        float s = 0.0f;
        for (int r = 0; r < TPP; r++) s += pvred[r][o];
        const int h = o / HD, d = o % HD;
        po[((size_t)(hk * G + h) * ns_stride + split) * HD + d] = s;
    }
    if (tid < G) {
        pml[((size_t)(hk * G + tid) * ns_stride + split) * 2] = m_run[tid];
        pml[((size_t)(hk * G + tid) * ns_stride + split) * 2 + 1] = l_run[tid];
    }
}

// A9: O = sum_i o_i e^(m_i-M) / sum_i l_i e^(m_i-M); an empty split carries
// (m = -3e38, l = 0, o = 0) and contributes nothing.
__global__ void k_attn_combine(const float* __restrict__ po, const float* __restrict__ pml, float* __restrict__ out,
                               int nsplit, int hd, int ns_stride, int per, const int* __restrict__ dpos) {
    const int d = threadIdx.x;
    const int qt = blockIdx.y;
    const int hq = blockIdx.x + qt * gridDim.x;        // row of [T][nHq]
    if (dpos) nsplit = (*dpos + 1 + per - 1) / per;
    const float* ml = pml + (size_t)hq * ns_stride * 2;
    float M = -3.0e38f;
    for (int i = 0; i < nsplit; i++) M = fmaxf(M, ml[2 * i]);
    float L = 0.0f, o = 0.0f;
    for (int i = 0; i < nsplit; i++) {
        float e = expf(ml[2 * i] - M);
        L += ml[2 * i + 1] * e;
        if (d < hd) o += po[((size_t)hq * ns_stride + i) * hd + d] * e;
    }
    if (d < hd) out[(size_t)hq * hd + d] = o / L;
}
}  // namespace

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// default split count on MI355X: ~128 keys per split, at least ~512 workgroups
// per layer when the context allows it, at most TI_ATTN_SPLITS_MAX
static int auto_nsplit(int S, int nKv) {
    int ns = (S + 127) / 128;
    int want = (512 + nKv - 1) / nKv;
    if (ns < want) ns = min(want, (S + 31) / 32);
    if (ns < 1) ns = 1;
    if (ns > TI_ATTN_SPLITS_MAX) ns = TI_ATTN_SPLITS_MAX;
    return ns;
}

// T queries (T >= 1) at contexts S, S+1, ..., S+T-1 (causal); with dpos != NULL the
// context is read on the device (S = *dpos + 1, T must be 1) and the grid covers
// `cap` positions in splits of `per` keys.
int ti_attn_decode_launch(ti_ctx* c, const float* qr, const uint32_t* kq, const float* ks, const uint32_t* vq,
                          const float* vs, float* out, int S, int T, int nHq, int nKv, int hd, int nsplit,
                          const int* dpos, int cap) {
    int per, ns_stride;
    if (dpos) {
        per = 128;
        nsplit = (cap + per - 1) / per;
        ns_stride = nsplit;
    } else {
        int Smax = S + T - 1;
        if (nsplit <= 0) nsplit = auto_nsplit(Smax, nKv);
        per = (Smax + nsplit - 1) / nsplit;
        ns_stride = nsplit;
    }
    if (nsplit > TI_ATTN_SPLITS_MAX) return ti_fail(TI_ERR_INVALID, "ti_attn_decode_q8: %d splits > %d", nsplit, TI_ATTN_SPLITS_MAX);
    if ((long)T * nHq > TI_ATTN_ROWS_MAX) return ti_fail(TI_ERR_INVALID, "ti_attn_decode_q8: T*nHq = %d > %d", T * nHq, TI_ATTN_ROWS_MAX);
    int G = nHq / nKv;
    dim3 grid(nKv * nsplit, T);
    const uint4* k4 = reinterpret_cast<const uint4*>(kq);
    const uint4* v4 = reinterpret_cast<const uint4*>(vq);
#define ATT(HD_, G_) \
    if (hd == HD_ && G == G_) { k_attn_split_q8<HD_, G_><<<grid, ATT_THREADS, 0, c->stream>>>(qr, k4, ks, v4, vs, c->attn_po, c->attn_ml, S, nKv, nsplit, per, ns_stride, dpos); }
    ATT(128, 1) else ATT(128, 2) else ATT(128, 4) else ATT(64, 1) else ATT(64, 2) else ATT(32, 2)
    else return ti_fail(TI_ERR_INVALID, "ti_attn_decode_q8: unsupported hd=%d / group=%d", hd, G);
#undef ATT
    TI_LAUNCHED("k_attn_split_q8");
    k_attn_combine<<<dim3(nHq, T), hd < 64 ? 64 : hd, 0, c->stream>>>(c->attn_po, c->attn_ml, out, nsplit, hd, ns_stride, per, dpos);
    TI_LAUNCHED("k_attn_combine");
    return TI_OK;
}

extern "C" int ti_attn_decode_q8(ti_ctx* c, const float* qr, const uint32_t* kq, const float* ks, const uint32_t* vq,
                                 const float* vs, float* out, int S, int nHq, int nKv, int hd, int nsplit) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(qr && kq && ks && vq && vs && out, "ti_attn_decode_q8: null buffer");
    TI_REQUIRE(S > 0 && nKv > 0 && nHq % nKv == 0 && nHq <= TI_ATTN_HEADS_MAX, "ti_attn_decode_q8: bad heads/context (S=%d nHq=%d nKv=%d)", S, nHq, nKv);
    TI_REQUIRE(hd % 32 == 0 && hd <= TI_ATTN_HD_MAX, "ti_attn_decode_q8: hd must be a multiple of 32 and <= %d", TI_ATTN_HD_MAX);
    TI_REQUIRE(al16(kq) && al16(vq), "ti_attn_decode_q8: kq/vq must be 16-byte aligned");
    return ti_attn_decode_launch(c, qr, kq, ks, vq, vs, out, S, 1, nHq, nKv, hd, nsplit, nullptr, 0);
}

extern "C" int ti_attn_causal_q8(ti_ctx* c, const float* qr, const uint32_t* kq, const float* ks, const uint32_t* vq,
                                 const float* vs, float* out, int T, int pos0, int nHq, int nKv, int hd) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(qr && kq && ks && vq && vs && out, "ti_attn_causal_q8: null buffer");
    TI_REQUIRE(T > 0 && pos0 >= 0 && nKv > 0 && nHq % nKv == 0, "ti_attn_causal_q8: bad shape (T=%d pos0=%d)", T, pos0);
    TI_REQUIRE(hd % 32 == 0 && hd <= TI_ATTN_HD_MAX, "ti_attn_causal_q8: bad hd=%d", hd);
    TI_REQUIRE(al16(kq) && al16(vq), "ti_attn_causal_q8: kq/vq must be 16-byte aligned");
    return ti_attn_decode_launch(c, qr, kq, ks, vq, vs, out, pos0 + 1, T, nHq, nKv, hd, 0, nullptr, 0);
}

int ti_attn_prep_launch(ti_ctx* c, const float* q, const float* k, const float* v, const uint16_t* qw,
                        const uint16_t* kw, float* qr, uint32_t* kq, float* ks, uint32_t* vq, float* vs,
                        int nHq, int nKv, int hd, int pos, float theta, float eps, const int* dpos) {
    k_attn_prep_q8<<<nHq + 2 * nKv, 128, 0, c->stream>>>(q, k, v, qw, kw, qr, kq, ks, vq, vs, nHq, nKv, hd, pos, theta,
                                                         eps, dpos);
    TI_LAUNCHED("k_attn_prep_q8");
    return TI_OK;
}

extern "C" int ti_attn_prep_q8(ti_ctx* c, const float* q, const float* k, const float* v, const uint16_t* qw,
                               const uint16_t* kw, float* qr, uint32_t* kq, float* ks, uint32_t* vq, float* vs,
                               int nHq, int nKv, int hd, int pos, float theta, float eps) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(q && k && v && qw && kw && qr && kq && ks && vq && vs, "ti_attn_prep_q8: null buffer");
    TI_REQUIRE(nHq > 0 && nKv > 0 && pos >= 0, "ti_attn_prep_q8: bad heads/pos");
    TI_REQUIRE(hd % 32 == 0 && hd <= 128, "ti_attn_prep_q8: hd must be a multiple of 32 and <= 128 (hd=%d)", hd);
    return ti_attn_prep_launch(c, q, k, v, qw, kw, qr, kq, ks, vq, vs, nHq, nKv, hd, pos, theta, eps, nullptr);
}

extern "C" int ti_rope_qk(ti_ctx* c, const float* x, const uint16_t* w, float* out, int T, int nH, int hd, int pos0,
                          float theta, float eps) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && out && (w || eps < 0), "ti_rope_qk: null buffer");
    TI_REQUIRE(T > 0 && nH > 0 && hd % 2 == 0 && hd <= 128 && pos0 >= 0, "ti_rope_qk: bad shape");
    TI_REQUIRE(x != out, "ti_rope_qk: in-place call (x == out) is not allowed");
    k_rope_qk<<<T * nH, 128, 0, c->stream>>>(x, w, out, nH, hd, pos0, theta, eps, w != nullptr);
    TI_LAUNCHED("k_rope_qk");
    return TI_OK;
}

extern "C" int ti_kv_write_q8(ti_ctx* c, const float* kr, const float* v, uint32_t* kq, float* ks, uint32_t* vq,
                              float* vs, int T, int nKv, int hd, int pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(kr && v && kq && ks && vq && vs, "ti_kv_write_q8: null buffer");
    TI_REQUIRE(T > 0 && nKv > 0 && hd % 32 == 0 && pos >= 0, "ti_kv_write_q8: bad shape");
    TI_REQUIRE(al16(kr) && al16(v), "ti_kv_write_q8: kr/v must be 16-byte aligned");
    long nG = (long)T * nKv * hd / 32;
    long g0 = (long)pos * nKv * hd / 32;
    k_kv_write_q8<<<(unsigned)((2 * nG + 63) / 64), 64, 0, c->stream>>>(kr, v, kq, ks, vq, vs, nG, g0);
    TI_LAUNCHED("k_kv_write_q8");
    return TI_OK;
}

// ---------------------------------------------------------------------------
// Fused decode attention: one launch per layer at T = 1 does attnPrepQ8
// (models/qwen3.js:2228-2308), attnDecodeStreamQ8 (:2077-2164) and the combine
// (:2048-2068). Workgroup (256 threads) = (KV head hk, split):
//  1. RMSNorm + RoPE of the G = nHq/nKv query heads of hk into LDS (each
//     workgroup recomputes them: 2 x 128 values);
//  2. the split that holds position pos normalises/ropes k and quantizes k, v
//     into the cache row pos (snorm int8, as attnPrepQ8) and uses that row from
//     LDS, so no workgroup waits for another one's write;
//  3. online softmax over the split in tiles of ATTF_TILE keys; K and V of a tile
//     are loaded together and the next tile is prefetched during the current one;
//  4. partials (unnormalised o, m, l) go to scratch; the last workgroup of hk to
//     finish (device-scope counter, release/acquire fences) merges them by
//     log-sum-exp and writes the head outputs, then resets the counter.
// The split count adapts to the context on the device: at least min_per keys
// per split, at most max_splits splits.
// ---------------------------------------------------------------------------
namespace {
constexpr int ATTF_TILE = 128;
constexpr int ATTF_MAXS = 64;

struct AttnFArgs {
    const float* q;
    const float* k;
    const float* v;
    const uint16_t* qw;
    const uint16_t* kw;
    uint32_t* kq;
    float* ks;
    uint32_t* vq;
    float* vs;
    float* out;
    float* po;
    float* pml;
    uint32_t* counter;     // [nKv]
    const int* dpos;       // device position, or null: use pos
    int pos;
    int nKv, max_splits, min_per, cap;
    float theta, eps;
};

template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_fused_q8(AttnFArgs a) {
    static_assert(G >= 1 && G <= 2 && HD <= 128 && HD % 32 == 0, "fused attention: G <= 2, HD <= 128");
    constexpr int LPT = HD / 16;               // lanes per token row (16 bytes each)
    constexpr int TPP = 256 / LPT;             // tokens per pass
    constexpr int PASSES = ATTF_TILE / TPP;
    constexpr int NG = HD / 32;                // scale groups per head row
    __shared__ float red[256];
    __shared__ float rk[256];
    __shared__ float s_q[G][HD];
    __shared__ float s_row[2][128];
    __shared__ __align__(16) uint32_t s_kw[HD / 4];
    __shared__ __align__(16) uint32_t s_vw[HD / 4];
    __shared__ float s_ksc[NG], s_vsc[NG];
    __shared__ float sc[G][ATTF_TILE];
    __shared__ float redm[G][4];
    __shared__ float reds[G][4];
    __shared__ float pvred[TPP][G * HD + 1];
    __shared__ float s_ml[G][ATTF_MAXS][2];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const int hk = blockIdx.x % a.nKv;
    const int split = blockIdx.x / a.nKv;
    const int pos = a.dpos ? *a.dpos : a.pos;
    if (pos < 0 || pos >= a.cap) return;       // outside the cache: nothing is read or written
    const int S = pos + 1;
    int ns0 = (S + a.min_per - 1) / a.min_per;
    ns0 = ns0 < a.max_splits ? ns0 : a.max_splits;
    const int per = (S + ns0 - 1) / ns0;
    const int nsplit = (S + per - 1) / per;
    if (split >= nsplit) return;
    const int c0 = split * per;
    const int c1 = min(S, c0 + per);
    const bool has_pos = c1 == S;

    // 1. query heads
    const int h = tid >> 7, j = tid & 127;
    {
        float x = (h < G && j < HD) ? a.q[(size_t)(hk * G + h) * HD + j] : 0.0f;
        float r = rope_norm(x, j, HD, a.qw, pos, a.theta, a.eps, true, red + h * 128, rk + h * 128);
        if (h < G && j < HD) s_q[h][j] = r;
    }
    // 2. this token's K/V row
    if (has_pos) {
        float x = (h == 0 && j < HD) ? a.k[(size_t)hk * HD + j] : 0.0f;
        float r = rope_norm(x, j, HD, a.kw, pos, a.theta, a.eps, true, red + h * 128, rk + h * 128);
        if (j < HD) s_row[h][j] = h == 0 ? r : a.v[(size_t)hk * HD + j];
        __syncthreads();
        if (tid < 2 * NG) {
            const int which = tid / NG, g = tid % NG;
            float vals[32];
#pragma unroll
            for (int i = 0; i < 32; i++) vals[i] = s_row[which][g * 32 + i];
            uint32_t wds[8];
            float scl;
            snorm_group(vals, wds, &scl);
            uint32_t* dq = (which ? a.vq : a.kq) + ((size_t)pos * a.nKv + hk) * (HD / 4) + g * 8;
            float* ds = (which ? a.vs : a.ks) + ((size_t)pos * a.nKv + hk) * NG + g;
            uint32_t* lw = which ? s_vw : s_kw;
#pragma unroll
            for (int w = 0; w < 8; w++) { dq[w] = wds[w]; lw[g * 8 + w] = wds[w]; }
            *ds = scl;
            (which ? s_vsc : s_ksc)[g] = scl;
        }
    }
    __syncthreads();

    const int tp = tid / LPT, sl = tid % LPT;
    const int row_words4 = a.nKv * HD / 16;
    const int row_groups = a.nKv * NG;
    const float qk_scale = 1.0f / (127.0f * sqrtf((float)HD));
    const uint4* kq4 = reinterpret_cast<const uint4*>(a.kq);
    const uint4* vq4 = reinterpret_cast<const uint4*>(a.vq);
    float qv[G][16];
#pragma unroll
    for (int hh = 0; hh < G; hh++)
#pragma unroll
        for (int i = 0; i < 16; i++) qv[hh][i] = s_q[hh][sl * 16 + i];
    float m_run[G], l_run[G], acc[G][16];
#pragma unroll
    for (int hh = 0; hh < G; hh++) {
        m_run[hh] = -3.0e38f;
        l_run[hh] = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) acc[hh][i] = 0.0f;
    }

    uint4 kw[2][PASSES], vw[2][PASSES];
    float ksc[2][PASSES], vsc[2][PASSES];
    auto load = [&](int buf, int t0) {
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            int t = t0 + p * TPP + tp;
            t = t < c1 ? t : c1 - 1;
            kw[buf][p] = ti_ld_nt(kq4 + (size_t)t * row_words4 + hk * LPT + sl);
            vw[buf][p] = ti_ld_nt(vq4 + (size_t)t * row_words4 + hk * LPT + sl);
            ksc[buf][p] = a.ks[(size_t)t * row_groups + hk * NG + sl / 2];
            vsc[buf][p] = a.vs[(size_t)t * row_groups + hk * NG + sl / 2];
        }
    };
    auto process = [&](int buf, int t0) {
        const int n = min(ATTF_TILE, c1 - t0);
        if (has_pos) {   // the row at pos (and the clamped reads past it) come from LDS
#pragma unroll
            for (int p = 0; p < PASSES; p++) {
                if (min(t0 + p * TPP + tp, c1 - 1) == pos) {
                    kw[buf][p] = reinterpret_cast<const uint4*>(s_kw)[sl];
                    vw[buf][p] = reinterpret_cast<const uint4*>(s_vw)[sl];
                    ksc[buf][p] = s_ksc[sl / 2];
                    vsc[buf][p] = s_vsc[sl / 2];
                }
            }
        }
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const uint32_t ww[4] = {kw[buf][p].x, kw[buf][p].y, kw[buf][p].z, kw[buf][p].w};
            float part[G];
#pragma unroll
            for (int hh = 0; hh < G; hh++) {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; i++) d = fmaf(qv[hh][i], i8f(ww[i >> 2], i & 3), d);
                part[hh] = d * ksc[buf][p];
            }
#pragma unroll
            for (int o = LPT / 2; o > 0; o >>= 1)
#pragma unroll
                for (int hh = 0; hh < G; hh++) part[hh] += __shfl_xor(part[hh], o, 64);
            const int jj = p * TPP + tp;
            if (sl == 0)
#pragma unroll
                for (int hh = 0; hh < G; hh++) sc[hh][jj] = jj < n ? part[hh] * qk_scale : -3.0e38f;
        }
        __syncthreads();
        float mt[G], corr[G];
#pragma unroll
        for (int hh = 0; hh < G; hh++) {
            float v = -3.0e38f;
            for (int q = tid; q < ATTF_TILE; q += 256) v = fmaxf(v, sc[hh][q]);
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
            if (lane == 0) redm[hh][wv] = v;
        }
        __syncthreads();
#pragma unroll
        for (int hh = 0; hh < G; hh++) {
            float v = fmaxf(fmaxf(redm[hh][0], redm[hh][1]), fmaxf(redm[hh][2], redm[hh][3]));
            mt[hh] = fmaxf(m_run[hh], v);
            corr[hh] = expf(m_run[hh] - mt[hh]);
            float s = 0.0f;
            for (int q = tid; q < ATTF_TILE; q += 256) {
                float pe = q < n ? expf(sc[hh][q] - mt[hh]) : 0.0f;
                sc[hh][q] = pe;
                s += pe;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
            if (lane == 0) reds[hh][wv] = s;
        }
        __syncthreads();
#pragma unroll
        for (int hh = 0; hh < G; hh++) {
            float s = (reds[hh][0] + reds[hh][1]) + (reds[hh][2] + reds[hh][3]);
            l_run[hh] = l_run[hh] * corr[hh] + s;
            m_run[hh] = mt[hh];
#pragma unroll
            for (int i = 0; i < 16; i++) acc[hh][i] *= corr[hh];
        }
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const int jj = p * TPP + tp;
            const uint32_t ww[4] = {vw[buf][p].x, vw[buf][p].y, vw[buf][p].z, vw[buf][p].w};
#pragma unroll
            for (int hh = 0; hh < G; hh++) {
                float pw = sc[hh][jj] * vsc[buf][p] * (1.0f / 127.0f);
#pragma unroll
                for (int i = 0; i < 16; i++) acc[hh][i] = fmaf(pw, i8f(ww[i >> 2], i & 3), acc[hh][i]);
            }
        }
        __syncthreads();   // sc is rewritten by the next tile
    };
    int t0 = c0;
    load(0, t0);
    for (;;) {
        int nt = t0 + ATTF_TILE;
        if (nt < c1) load(1, nt);
        process(0, t0);
        if (nt >= c1) break;
        t0 = nt;
        nt = t0 + ATTF_TILE;
        if (nt < c1) load(0, nt);
        process(1, t0);
        if (nt >= c1) break;
        t0 = nt;
    }

    // 4. partials of this split, then the last workgroup of hk merges them
#pragma unroll
    for (int hh = 0; hh < G; hh++)
#pragma unroll
        for (int i = 0; i < 16; i++) pvred[tp][hh * HD + sl * 16 + i] = acc[hh][i];
    __syncthreads();
    const size_t ms = (size_t)a.max_splits;
    for (int o = tid; o < G * HD; o += 256) {
        float s = 0.0f;
        for (int r = 0; r < TPP; r++) s += pvred[r][o];
        const int hh = o / HD, d = o % HD;
        a.po[((size_t)(hk * G + hh) * ms + split) * HD + d] = s;
    }
    if (tid < G) {
        a.pml[((size_t)(hk * G + tid) * ms + split) * 2] = m_run[tid];
        a.pml[((size_t)(hk * G + tid) * ms + split) * 2 + 1] = l_run[tid];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = __hip_atomic_fetch_add(a.counter + hk, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (unsigned)(nsplit - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int e = tid; e < G * nsplit * 2; e += 256) {
        const int hh = e / (nsplit * 2), r = e % (nsplit * 2);
        s_ml[hh][r >> 1][r & 1] = a.pml[((size_t)(hk * G + hh) * ms + (r >> 1)) * 2 + (r & 1)];
    }
    __syncthreads();
    if (tid < G * HD) {
        const int hh = tid / HD, d = tid % HD;
        float M = -3.0e38f;
        for (int i = 0; i < nsplit; i++) M = fmaxf(M, s_ml[hh][i][0]);
        float L = 0.0f, o = 0.0f;
        const float* pp = a.po + (size_t)(hk * G + hh) * ms * HD + d;
#pragma unroll 16
        for (int i = 0; i < nsplit; i++) {
            float e = expf(s_ml[hh][i][0] - M);
            L += s_ml[hh][i][1] * e;
            o += pp[(size_t)i * HD] * e;
        }
        a.out[(size_t)(hk * G + hh) * HD + d] = o / L;
    }
    if (tid == 0) __hip_atomic_store(a.counter + hk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
}  // namespace

// Fused decode attention; returns TI_ERR_INVALID for head shapes it does not cover
// (the caller then issues prep + split + combine).
int ti_attn_fused_launch(ti_ctx* c, const float* q, const float* k, const float* v, const uint16_t* qw,
                         const uint16_t* kw, uint32_t* kq, float* ks, uint32_t* vq, float* vs, float* out, int nHq,
                         int nKv, int hd, const int* dpos, int pos, int cap, float theta, float eps, int max_splits) {
    const int G = nHq / nKv;
    if (nKv > TI_SYNC_WORDS - TI_SYNC_ATTN) return ti_fail(TI_ERR_INVALID, "fused attention: too many KV heads");
    if (max_splits <= 0 || max_splits > ATTF_MAXS) max_splits = ATTF_MAXS;
    AttnFArgs a = {q, k, v, qw, kw, kq, ks, vq, vs, out, c->attn_po, c->attn_ml, c->sync + TI_SYNC_ATTN, dpos, pos,
                   nKv, max_splits, 128, cap, theta, eps};
    dim3 grid(nKv * max_splits);
#define AF(HD_, G_) \
    if (hd == HD_ && G == G_) { k_attn_fused_q8<HD_, G_><<<grid, 256, 0, c->stream>>>(a); TI_LAUNCHED("k_attn_fused_q8"); return TI_OK; }
    AF(128, 2) AF(128, 1) AF(64, 2) AF(64, 1)
#undef AF
    return ti_fail(TI_ERR_INVALID, "fused attention: no kernel for hd=%d group=%d", hd, G);
}

extern "C" int ti_attn_step_q8(ti_ctx* c, const float* q, const float* k, const float* v, const uint16_t* qn_w,
                               const uint16_t* kn_w, uint32_t* kq, float* ks, uint32_t* vq, float* vs, float* out,
                               int nHq, int nKv, int hd, int pos, int cap, float theta, float eps, int max_splits) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(q && k && v && qn_w && kn_w && kq && ks && vq && vs && out, "ti_attn_step_q8: null buffer");
    TI_REQUIRE(nKv > 0 && nHq % nKv == 0 && nHq <= TI_ATTN_HEADS_MAX, "ti_attn_step_q8: bad heads (nHq=%d nKv=%d)", nHq, nKv);
    TI_REQUIRE(pos >= 0 && pos < cap, "ti_attn_step_q8: pos %d outside the cache [0, %d)", pos, cap);
    TI_REQUIRE(al16(kq) && al16(vq), "ti_attn_step_q8: kq/vq must be 16-byte aligned");
    TI_REQUIRE(max_splits >= 0 && max_splits <= ATTF_MAXS, "ti_attn_step_q8: max_splits in [0, %d]", ATTF_MAXS);
    return ti_attn_fused_launch(c, q, k, v, qn_w, kn_w, kq, ks, vq, vs, out, nHq, nKv, hd, nullptr, pos, cap, theta, eps,
                                max_splits);
}
