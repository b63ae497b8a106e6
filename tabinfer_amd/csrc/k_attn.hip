// k_attn.hip — int8-KV attention of the decode path:
//  fused QK-RMSNorm + RoPE + int8 KV write   attnPrepQ8     models/qwen3.js:2228-2308
//     RMSNorm + RoPE for T tokens               ropeQK         models/qwen3.js:1700-1760
//     int8 KV write for T tokens                kvQuantWrite   models/qwen3.js:2180-2216
//  split-KV decode attention (partials)      attnDecStreamQ8 models/qwen3.js:2077-2173
//  log-sum-exp combine                        ATTN_DEC_COMBINE models/qwen3.js:2048-2068
//
// KV layout is the reference's: per layer, position-major, then head, then dim;
// int8 codes packed 4 per u32 (snorm: code/127 * group max), one f32 scale per
// 32 dims.
#include "ti_dev.h"
#include <math.h>
#include <mutex>

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

// rope_norm with the rotation's cos/sin given: cs[i] = cos(pos*theta^(-2i/hd)),
// cs[hd/2 + i] = sin(...), i < hd/2, evaluated in f64 and rounded to f32 on the host
// (the same values rope_norm computes on the device), so the hot kernels call no
// f64 library routine.
__device__ float rope_norm_tab(float x, int j, int hd, const uint16_t* __restrict__ w, const float* cs, float eps,
                               float* red, float* rk) {
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
    __syncthreads();
    float out = 0.0f;
    if (j < hd) {
        const int half = hd / 2;
        const int fi = j < half ? j : j - half;
        const float c = cs[fi], sn = cs[half + fi];
        float partner = j < half ? rk[j + half] : rk[j - half];
        float rot = j < half ? -partner : partner;
        float a = rk[j] * c, b = rot * sn;
        out = a + b;
    }
    __syncthreads();
    return out;
}

// workgroup roles [0,nHq) q-head rope+norm -> qr ; [nHq, nHq+nKv) k-head
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
// Group gg (flat over positions x heads x groups, rowg groups per position) has its scale
// at gg and its codes at group slot (gg / rowg) * crowg + gg % rowg (crowg >= rowg: the
// code rows may carry spare slots).
__global__ void k_kv_write_q8(const float* __restrict__ kr, const float* __restrict__ vv, uint32_t* __restrict__ kq,
                              float* __restrict__ ks, uint32_t* __restrict__ vq, float* __restrict__ vs, long nG,
                              long dst_g0, int rowg, int crowg) {
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
    const long gg = dst_g0 + g;
    const long cg = (gg / rowg) * crowg + gg % rowg;
    snorm_group(vals, (isV ? vq : kq) + cg * 8, (isV ? vs : ks) + gg);
}

// ---------------------------------------------------------------------------
// split-KV decode attention. Workgroup (256 threads) = (kv head hk, split).
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
                                                               int per, int ns_stride, const int* __restrict__ dpos,
                                                               int kvs) {
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
    const int row_words4 = kvs * HD / 16;           // uint4 per cached position (codes: kvs slots)
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
                for (int h = 0; h < G; h++) part[h] += ti_xor(part[h], o);
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
            for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, ti_xor(v, o));
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
            for (int o = 32; o > 0; o >>= 1) s += ti_xor(s, o);
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

// ---------------------------------------------------------------------------
// T > 1 queries (a prefill chunk or a T-token batch, models/qwen3.js:2534-2577): one
// pass over a split's keys serves every query row of the KV head, instead of one pass
// per query. Workgroup (256 threads) = (split, KV head, group of 16 query rows; row
// ri = (t, h) with t = query, h = head of the group). Key tiles of 64:
//  - S = Q K^T on the matrix cores: v_mfma_f32_16x16x32_f16, one MFMA per 32-dim scale
//    group and per 16 keys (wave w: keys 16w..16w+15). K codes are exact in f16; q is
//    split into f16 hi + lo (q = hi + lo to ~2^-22), two MFMAs per group, so the
//    scores keep f32 accuracy. Each group's partial is scaled by its key's K scale.
//  - causal mask (key < S0 + t), online softmax per row (tile maxima and sums through
//    LDS, the running (m, l) in LDS);
//  - P V with f32 FMAs from the V tile staged in LDS: wave w owns the 32 dims of scale
//    group w, each lane one dim and 8 rows.
// Partials (o, m, l) go to the split-KV scratch in k_attn_split_q8's layout; the same
// k_attn_combine merges them.
// ---------------------------------------------------------------------------
typedef _Float16 am_half8 __attribute__((ext_vector_type(8)));
typedef float am_f4 __attribute__((ext_vector_type(4)));
constexpr int AM_ROWS = 16, AM_KT = 64;

struct AttnMArgs {
    const float* qr;
    const uint8_t* kq;
    const float* ks;
    const uint4* vq;
    const float* vs;
    float* po;
    float* pml;
    int S0, T, nHq, nKv, G, nsplit, per, ns_stride;
    int kvs;   // K/V code slots per cached position
};

__global__ __launch_bounds__(256) void k_attn_multi_q8(AttnMArgs a) {
    constexpr int HD = 128, NG = HD / 32;
    __shared__ __align__(16) int8_t s_v[AM_KT][HD];
    __shared__ float s_vs[AM_KT][NG];
    __shared__ __align__(16) float s_p[AM_KT][AM_ROWS];
    __shared__ float s_mx[2][4][AM_ROWS], s_sm[2][4][AM_ROWS];
    __shared__ float s_m[AM_ROWS], s_l[AM_ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x % a.nsplit, hk = blockIdx.x / a.nsplit;
    const int rg = blockIdx.y;
    const int nrows = a.G * a.T;
    const int Smax = a.S0 + a.T - 1;
    const int c0 = split * a.per;
    const int c1 = min(Smax, c0 + a.per);
    const int row_bytes = a.kvs * HD, row_words4 = a.kvs * HD / 16, row_groups = a.nKv * NG;
    const float qk_scale = 1.0f / (127.0f * sqrtf((float)HD));
    if (tid < AM_ROWS) {
        s_m[tid] = -3.0e38f;
        s_l[tid] = 0.0f;
    }
    // A operands: query row (lane % 16), dims 32g + 8 (lane / 16) .. +8, as f16 hi + lo
    const int ak = lane >> 4;
    am_half8 qh[NG], ql[NG];
    {
        const int gr = rg * AM_ROWS + (lane & 15);
        const bool ok = gr < nrows;
        const int t = ok ? gr / a.G : 0, h = ok ? gr % a.G : 0;
        const float* q = a.qr + ((size_t)t * a.nHq + hk * a.G + h) * HD;
#pragma unroll
        for (int g = 0; g < NG; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float v = ok ? q[32 * g + 8 * ak + e] : 0.0f;
                const _Float16 hi = (_Float16)v;
                qh[g][e] = hi;
                ql[g][e] = (_Float16)(v - (float)hi);
            }
    }
    // this lane's score rows (4 (lane / 16) + i) and their causal limits
    int lim[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int gr = rg * AM_ROWS + 4 * ak + i;
        lim[i] = gr < nrows ? min(c1, a.S0 + gr / a.G) : 0;     // keys [c0, lim) are visible
    }
    // this lane's P V rows (8 (lane / 32) + i) and dim
    const int pr0 = 8 * (lane >> 5), d = 32 * wave + (lane & 31);
    float acc[8] = {};
    int it = 0;
    for (int t0 = c0; t0 < c1; t0 += AM_KT, it ^= 1) {
        // V tile and its scales into LDS (coalesced)
        for (int i = tid; i < AM_KT * HD / 16; i += 256) {
            const int j = i / (HD / 16), c = i % (HD / 16);
            int key = t0 + j;
            key = key < c1 ? key : c1 - 1;
            *reinterpret_cast<uint4*>(&s_v[j][c * 16]) = ti_ld_nt(a.vq + (size_t)key * row_words4 + hk * (HD / 16) + c);
        }
        {
            const int j = tid / NG, g = tid % NG;
            int key = t0 + j;
            key = key < c1 ? key : c1 - 1;
            s_vs[j][g] = a.vs[(size_t)key * row_groups + hk * NG + g];
        }
        // K operands of this wave's 16 keys: key (lane % 16), dims 32g + 8 (lane / 16) .. +8
        const int kk = t0 + 16 * wave + (lane & 15);
        const int kc = kk < c1 ? kk : c1 - 1;
        am_half8 kb[NG];
        float ksc[NG];
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const uint2 w = *reinterpret_cast<const uint2*>(a.kq + (size_t)kc * row_bytes + hk * HD + 32 * g + 8 * ak);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                kb[g][e] = (_Float16)(int)(int8_t)((w.x >> (8 * e)) & 0xffu);
                kb[g][4 + e] = (_Float16)(int)(int8_t)((w.y >> (8 * e)) & 0xffu);
            }
            ksc[g] = a.ks[(size_t)kc * row_groups + hk * NG + g];
        }
        am_f4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const am_f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            am_f4 dg = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[g], kb[g], z, 0, 0, 0);
            dg = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[g], kb[g], dg, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) sc[i] = fmaf(dg[i], ksc[g], sc[i]);
        }
        // mask, scale, tile maxima of this wave's 16 keys per row
        float s[4], mx[4];
        bool ok[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            ok[i] = kk < lim[i];
            s[i] = ok[i] ? sc[i] * qk_scale : -3.0e38f;
            mx[i] = s[i];
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) mx[i] = fmaxf(mx[i], ti_xor(mx[i], o));
        }
        if ((lane & 15) == 0)
#pragma unroll
            for (int i = 0; i < 4; i++) s_mx[it][wave][4 * ak + i] = mx[i];
        __syncthreads();                                   // (1) tile maxima, V tile
        float ps[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 4 * ak + i;
            float mt = s_mx[it][0][r];
#pragma unroll
            for (int w = 1; w < 4; w++) mt = fmaxf(mt, s_mx[it][w][r]);
            const float mnew = fmaxf(s_m[r], mt);
            const float p = ok[i] ? expf(s[i] - mnew) : 0.0f;
            s_p[16 * wave + (lane & 15)][r] = p;
            ps[i] = p;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) ps[i] += ti_xor(ps[i], o);
        }
        if ((lane & 15) == 0)
#pragma unroll
            for (int i = 0; i < 4; i++) s_sm[it][wave][4 * ak + i] = ps[i];
        __syncthreads();                                   // (2) p
        // P V for this lane's 8 rows and dim d (scale group = wave)
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int r = pr0 + i;
            float mt = s_mx[it][0][r];
#pragma unroll
            for (int w = 1; w < 4; w++) mt = fmaxf(mt, s_mx[it][w][r]);
            const float mo = s_m[r], mnew = fmaxf(mo, mt);
            acc[i] *= mo == mnew ? 1.0f : expf(mo - mnew);
        }
        // every key of the tile (p is 0 past the split's end; the clamped V rows are finite)
#pragma unroll 16
        for (int j = 0; j < AM_KT; j++) {
            const float cv = (float)s_v[j][d] * s_vs[j][wave];
            const float4 pa = *reinterpret_cast<const float4*>(&s_p[j][pr0]);
            const float4 pb = *reinterpret_cast<const float4*>(&s_p[j][pr0 + 4]);
            acc[0] = fmaf(pa.x, cv, acc[0]); acc[1] = fmaf(pa.y, cv, acc[1]);
            acc[2] = fmaf(pa.z, cv, acc[2]); acc[3] = fmaf(pa.w, cv, acc[3]);
            acc[4] = fmaf(pb.x, cv, acc[4]); acc[5] = fmaf(pb.y, cv, acc[5]);
            acc[6] = fmaf(pb.z, cv, acc[6]); acc[7] = fmaf(pb.w, cv, acc[7]);
        }
        __syncthreads();                                   // (3) s_v, s_p, s_m read
        if (tid < AM_ROWS) {
            const int r = tid;
            float mt = s_mx[it][0][r], sum = 0.0f;
#pragma unroll
            for (int w = 1; w < 4; w++) mt = fmaxf(mt, s_mx[it][w][r]);
#pragma unroll
            for (int w = 0; w < 4; w++) sum += s_sm[it][w][r];
            const float mo = s_m[r], mnew = fmaxf(mo, mt);
            s_l[r] = s_l[r] * (mo == mnew ? 1.0f : expf(mo - mnew)) + sum;
            s_m[r] = mnew;
        }
    }
    __syncthreads();
    // partials, in k_attn_split_q8's layout: row (t, hq) -> [t][hq][split]
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int gr = rg * AM_ROWS + pr0 + i;
        if (gr < nrows) {
            const int t = gr / a.G, hq = hk * a.G + gr % a.G;
            a.po[(((size_t)t * a.nHq + hq) * a.ns_stride + split) * HD + d] = acc[i] * (1.0f / 127.0f);
        }
    }
    if (tid < AM_ROWS) {
        const int gr = rg * AM_ROWS + tid;
        if (gr < nrows) {
            const int t = gr / a.G, hq = hk * a.G + gr % a.G;
            float* ml = a.pml + (((size_t)t * a.nHq + hq) * a.ns_stride + split) * 2;
            ml[0] = s_m[tid];
            ml[1] = s_l[tid];
        }
    }
}

// O = sum_i o_i e^(m_i-M) / sum_i l_i e^(m_i-M); an empty split carries
// (m = -3e38, l = 0, o = 0) and contributes nothing.
__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ po, const float* __restrict__ pml,
                                                      float* __restrict__ out, int nsplit, int hd, int ns_stride, int per,
                                                      const int* __restrict__ dpos) {
    // one workgroup per output row: the splits' (m, l) into LDS and their weights
    // e_i = exp(m_i - M) computed once; then 2 threads per dim sum o_i e_i over
    // alternate chunks of 16 splits (16 loads in flight), and the halves meet in LDS
    __shared__ float s_e[TI_ATTN_SPLITS_MAX];
    __shared__ float s_red[2][TI_ATTN_HD_MAX];
    __shared__ float s_w[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qt = blockIdx.y;
    const int hq = blockIdx.x + qt * gridDim.x;        // row of [T][nHq]
    if (dpos) nsplit = (*dpos + 1 + per - 1) / per;
    const float* ml = pml + (size_t)hq * ns_stride * 2;
    float M = -3.0e38f;
    for (int i = tid; i < nsplit; i += 256) M = fmaxf(M, ml[2 * i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, ti_xor(M, o));
    if (lane == 0) s_w[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(s_w[0], s_w[1]), fmaxf(s_w[2], s_w[3]));
    float L = 0.0f;
    for (int i = tid; i < nsplit; i += 256) {
        const float e = expf(ml[2 * i] - M);
        s_e[i] = e;
        L += ml[2 * i + 1] * e;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) L += ti_xor(L, o);
    __syncthreads();                       // s_w (maxima) read by everyone before reuse
    if (lane == 0) s_w[wave] = L;
    __syncthreads();
    L = (s_w[0] + s_w[1]) + (s_w[2] + s_w[3]);
    const int d = tid % TI_ATTN_HD_MAX, q4 = tid / TI_ATTN_HD_MAX;    // 2 x 128 threads
    float o = 0.0f;
    if (d < hd) {
        const float* pp = po + (size_t)hq * ns_stride * hd + d;
        for (int i0 = q4 * 16; i0 < nsplit; i0 += 32) {
            float v[16];
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = i0 + k < nsplit ? pp[(size_t)(i0 + k) * hd] : 0.0f;
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (i0 + k < nsplit) o += v[k] * s_e[i0 + k];
        }
    }
    s_red[q4][d] = o;
    __syncthreads();
    if (q4 == 0 && d < hd) out[(size_t)hq * hd + d] = (s_red[0][d] + s_red[1][d]) / L;
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

// The per-split kernel and the log-sum-exp combine on stream `st`, the partials in
// po[T*nHq*ns_stride*hd] and ml[T*nHq*ns_stride*2] (every slot below nsplit is written
// before it is read, so nothing in them needs clearing).
static int split_combine(hipStream_t st, float* po, float* ml, const float* qr, const uint32_t* kq, const float* ks,
                         const uint32_t* vq, const float* vs, float* out, int S, int T, int nHq, int nKv, int hd,
                         int nsplit, int per, int ns_stride, const int* dpos, int kvs) {
    const int G = nHq / nKv;
    dim3 grid(nKv * nsplit, T);
    const uint4* k4 = reinterpret_cast<const uint4*>(kq);
    const uint4* v4 = reinterpret_cast<const uint4*>(vq);
#define ATT(HD_, G_) \
    if (hd == HD_ && G == G_) { k_attn_split_q8<HD_, G_><<<grid, ATT_THREADS, 0, st>>>(qr, k4, ks, v4, vs, po, ml, S, nKv, nsplit, per, ns_stride, dpos, kvs); }
    ATT(128, 1) else ATT(128, 2) else ATT(128, 4) else ATT(64, 1) else ATT(64, 2) else ATT(32, 2)
    else return ti_fail(TI_ERR_INVALID, "ti_attn_decode_q8: unsupported hd=%d / group=%d", hd, G);
#undef ATT
    TI_LAUNCHED("k_attn_split_q8");
    k_attn_combine<<<dim3(nHq, T), 256, 0, st>>>(po, ml, out, nsplit, hd, ns_stride, per, dpos);
    TI_LAUNCHED("k_attn_combine");
    return TI_OK;
}

// T queries (T >= 1) at contexts S, S+1, ..., S+T-1 (causal); with dpos != NULL the
// context is read on the device (S = *dpos + 1, T must be 1) and the grid covers
// `cap` positions in splits of `per` keys.
int ti_attn_decode_launch(ti_ctx* c, const float* qr, const uint32_t* kq, const float* ks, const uint32_t* vq,
                          const float* vs, float* out, int S, int T, int nHq, int nKv, int hd, int nsplit,
                          const int* dpos, int cap, int kvs) {
    if (kvs < nKv) return ti_fail(TI_ERR_INVALID, "attention: %d code slots per position < %d KV heads", kvs, nKv);
    int per, ns_stride;
    if (dpos) {
        per = 128;
        nsplit = (cap + per - 1) / per;
        ns_stride = nsplit;
    } else {
        int Smax = S + T - 1;
        if (nsplit <= 0) {
            nsplit = auto_nsplit(Smax, nKv);
            const long fit = TI_ATTN_ROWSPLITS / ((long)T * nHq > 0 ? (long)T * nHq : 1);
            if (nsplit > fit) nsplit = fit > 0 ? (int)fit : 1;   // many query rows: fewer, longer splits
        }
        per = (Smax + nsplit - 1) / nsplit;
        ns_stride = nsplit;
    }
    if (nsplit > TI_ATTN_SPLITS_MAX) return ti_fail(TI_ERR_INVALID, "ti_attn_decode_q8: %d splits > %d", nsplit, TI_ATTN_SPLITS_MAX);
    if ((long)T * nHq > TI_ATTN_ROWS_MAX) return ti_fail(TI_ERR_INVALID, "ti_attn_decode_q8: T*nHq = %d > %d", T * nHq, TI_ATTN_ROWS_MAX);
    if ((long)T * nHq * nsplit > TI_ATTN_ROWSPLITS)
        return ti_fail(TI_ERR_INVALID, "ti_attn_decode_q8: T*nHq*nsplit = %ld > %d", (long)T * nHq * nsplit, TI_ATTN_ROWSPLITS);
    int G = nHq / nKv;
    if (!dpos && T > 1 && hd == 128) {   // one pass over the keys for all T queries
        const int Smax = S + T - 1;
        const int want = (1024 + nKv - 1) / nKv;
        int per2 = (Smax + want - 1) / want;
        per2 = ((per2 + AM_KT - 1) / AM_KT) * AM_KT;
        if (per2 < AM_KT) per2 = AM_KT;
        int ns2 = (Smax + per2 - 1) / per2;
        while (ns2 > TI_ATTN_SPLITS_MAX || (long)ns2 * T * nHq > TI_ATTN_ROWSPLITS) {
            per2 += AM_KT;
            ns2 = (Smax + per2 - 1) / per2;
        }
        AttnMArgs m = {qr, reinterpret_cast<const uint8_t*>(kq), ks, reinterpret_cast<const uint4*>(vq), vs,
                       c->attn_po, c->attn_ml, S, T, nHq, nKv, G, ns2, per2, ns2, kvs};
        dim3 g2(nKv * ns2, (G * T + AM_ROWS - 1) / AM_ROWS);
        k_attn_multi_q8<<<g2, 256, 0, c->stream>>>(m);
        TI_LAUNCHED("k_attn_multi_q8");
        k_attn_combine<<<dim3(nHq, T), 256, 0, c->stream>>>(c->attn_po, c->attn_ml, out, ns2, hd, ns2, per2, nullptr);
        TI_LAUNCHED("k_attn_combine");
        return TI_OK;
    }
    return split_combine(c->stream, c->attn_po, c->attn_ml, qr, kq, ks, vq, vs, out, S, T, nHq, nKv, hd, nsplit, per,
                         ns_stride, dpos, kvs);
}

extern "C" int ti_attn_decode_q8(ti_ctx* c, const float* qr, const uint32_t* kq, const float* ks, const uint32_t* vq,
                                 const float* vs, float* out, int S, int nHq, int nKv, int hd, int nsplit) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(qr && kq && ks && vq && vs && out, "ti_attn_decode_q8: null buffer");
    TI_REQUIRE(S > 0 && nKv > 0 && nHq % nKv == 0 && nHq <= TI_ATTN_HEADS_MAX, "ti_attn_decode_q8: bad heads/context (S=%d nHq=%d nKv=%d)", S, nHq, nKv);
    TI_REQUIRE(hd % 32 == 0 && hd <= TI_ATTN_HD_MAX, "ti_attn_decode_q8: hd must be a multiple of 32 and <= %d", TI_ATTN_HD_MAX);
    TI_REQUIRE(al16(kq) && al16(vq), "ti_attn_decode_q8: kq/vq must be 16-byte aligned");
    return ti_attn_decode_launch(c, qr, kq, ks, vq, vs, out, S, 1, nHq, nKv, hd, nsplit, nullptr, 0, nKv);
}

// ---- the same call without a context (nothing allocated) ---------------------------------
// Callers that cannot allocate device memory (code under graph capture, serving loops,
// harnesses that forbid hipMalloc) get the split partials from this file-scope array.
// Every device the call runs on holds its own copy until the process ends. In host code
// the array's name is not a device address: its address on each device is looked up once
// (hipGetSymbolAddress, with that device current) and only that address is used.
constexpr int NOALLOC_ROWSPLITS = 4096;   // query heads x splits of one call, at most
constexpr int NOALLOC_DEVICES = 64;
static __device__ __align__(256) float scratch[NOALLOC_ROWSPLITS * (TI_ATTN_HD_MAX + 2)];

static std::mutex g_scratch_mu;
static float* g_scratch_addr[NOALLOC_DEVICES];

// the array's address on device dev (looked up with dev current, the caller's device restored)
static int scratch_address(int dev, float** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        int cur = -1;
        TI_HIP(hipGetDevice(&cur));
        if (cur != dev) TI_HIP(hipSetDevice(dev));
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) TI_HIP(hipSetDevice(cur));
        if (e != hipSuccess) return ti_hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return ti_fail(TI_ERR_HIP, "ti_attn_decode_q8_noalloc: no device address for the scratch array");
        g_scratch_addr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_addr[dev];
    return TI_OK;
}

extern "C" int ti_attn_decode_q8_noalloc(void* stream, const float* qr, const uint32_t* kq, const float* ks,
                                         const uint32_t* vq, const float* vs, float* out, int S, int nHq, int nKv,
                                         int hd, int nsplit) {
    TI_REQUIRE(qr && kq && ks && vq && vs && out, "ti_attn_decode_q8_noalloc: null buffer");
    TI_REQUIRE(S > 0 && nKv > 0 && nHq % nKv == 0 && nHq <= TI_ATTN_HEADS_MAX,
               "ti_attn_decode_q8_noalloc: bad heads/context (S=%d nHq=%d nKv=%d)", S, nHq, nKv);
    TI_REQUIRE(hd % 32 == 0 && hd <= TI_ATTN_HD_MAX, "ti_attn_decode_q8_noalloc: hd must be a multiple of 32 and <= %d",
               TI_ATTN_HD_MAX);
    TI_REQUIRE(al16(kq) && al16(vq), "ti_attn_decode_q8_noalloc: kq/vq must be 16-byte aligned");
    if (nsplit <= 0) nsplit = auto_nsplit(S, nKv);
    TI_REQUIRE(nsplit <= TI_ATTN_SPLITS_MAX && (long)nHq * nsplit <= NOALLOC_ROWSPLITS,
               "ti_attn_decode_q8_noalloc: %d heads x %d splits exceed the scratch array (%d head-splits, %d splits at most)",
               nHq, nsplit, NOALLOC_ROWSPLITS, TI_ATTN_SPLITS_MAX);
    // the kernels run on the stream's device, so the scratch address is that device's
    // (the null stream: the current device's)
    int dev = -1;
    if (stream) TI_HIP(hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev));
    else TI_HIP(hipGetDevice(&dev));
    TI_REQUIRE(dev >= 0 && dev < NOALLOC_DEVICES, "ti_attn_decode_q8_noalloc: device %d out of range", dev);
    float* base = nullptr;
    const int rc = scratch_address(dev, &base);
    if (rc) return rc;
    const int per = (S + nsplit - 1) / nsplit;
    return split_combine(static_cast<hipStream_t>(stream), base, base + (size_t)NOALLOC_ROWSPLITS * TI_ATTN_HD_MAX, qr, kq,
                         ks, vq, vs, out, S, 1, nHq, nKv, hd, nsplit, per, nsplit, nullptr, nKv);
}

extern "C" int ti_attn_causal_q8(ti_ctx* c, const float* qr, const uint32_t* kq, const float* ks, const uint32_t* vq,
                                 const float* vs, float* out, int T, int pos0, int nHq, int nKv, int hd) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(qr && kq && ks && vq && vs && out, "ti_attn_causal_q8: null buffer");
    TI_REQUIRE(T > 0 && pos0 >= 0 && nKv > 0 && nHq % nKv == 0, "ti_attn_causal_q8: bad shape (T=%d pos0=%d)", T, pos0);
    TI_REQUIRE(hd % 32 == 0 && hd <= TI_ATTN_HD_MAX, "ti_attn_causal_q8: bad hd=%d", hd);
    TI_REQUIRE(al16(kq) && al16(vq), "ti_attn_causal_q8: kq/vq must be 16-byte aligned");
    return ti_attn_decode_launch(c, qr, kq, ks, vq, vs, out, pos0 + 1, T, nHq, nKv, hd, 0, nullptr, 0, nKv);
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

// the write into a cache whose code rows hold kvs >= nKv slots per position
int ti_kv_write_launch(ti_ctx* c, const float* kr, const float* v, uint32_t* kq, float* ks, uint32_t* vq, float* vs,
                       int T, int nKv, int hd, int pos, int kvs) {
    TI_REQUIRE(kvs >= nKv, "kv write: %d code slots per position < %d KV heads", kvs, nKv);
    const long nG = (long)T * nKv * hd / 32;
    const long g0 = (long)pos * nKv * hd / 32;
    k_kv_write_q8<<<(unsigned)((2 * nG + 63) / 64), 64, 0, c->stream>>>(kr, v, kq, ks, vq, vs, nG, g0, nKv * hd / 32,
                                                                        kvs * hd / 32);
    TI_LAUNCHED("k_kv_write_q8");
    return TI_OK;
}

extern "C" int ti_kv_write_q8(ti_ctx* c, const float* kr, const float* v, uint32_t* kq, float* ks, uint32_t* vq,
                              float* vs, int T, int nKv, int hd, int pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(kr && v && kq && ks && vq && vs, "ti_kv_write_q8: null buffer");
    TI_REQUIRE(T > 0 && nKv > 0 && hd % 32 == 0 && pos >= 0, "ti_kv_write_q8: bad shape");
    TI_REQUIRE(al16(kr) && al16(v), "ti_kv_write_q8: kr/v must be 16-byte aligned");
    return ti_kv_write_launch(c, kr, v, kq, ks, vq, vs, T, nKv, hd, pos, nKv);
}

// ---------------------------------------------------------------------------
// Fused decode attention: one launch per layer at T = 1 does attnPrepQ8
// (models/qwen3.js:2228-2308), attnDecodeStreamQ8 (:2077-2164) and the combine
// (:2048-2068). Workgroup (256 threads) = (KV head hk, split w of NS):
//  - the keys are cut into tiles of ATTF_TILE positions and workgroup w takes
//    tiles w, w+NS, w+2NS, ... : the first tile's address does not depend on the
//    context length, so its K/V loads are issued together with the loads of the
//    device position, the rope row and the q/k/v projections — the kernel pays one
//    memory round trip before it computes, not three;
//  - RMSNorm + RoPE of the G = nHq/nKv query heads of hk into LDS (every
//    workgroup; 2 x 128 values);
//  - the workgroup holding the last tile normalises/ropes k and quantizes k, v
//    into cache row pos (snorm int8, as attnPrepQ8) and takes that row from LDS;
//  - online softmax over its tiles, K and V of a tile loaded together, the next
//    tile prefetched during the current one;
//  - partials (unnormalised o, m, l) are published with device-scope stores; the
//    last workgroup of hk to arrive merges the NS partials by log-sum-exp, writes
//    the head outputs and resets the counter.
// ---------------------------------------------------------------------------
namespace {
constexpr int ATTF_MAXS = 64;
// default workgroups per KV head, by cache capacity (the split count is fixed when a
// decode step is captured, the context length is not): measured on MI355X, 32 is best
// for contexts up to ~16k, 64 beyond (more waves streaming the keys)
constexpr int ATTF_SPLITS_SHORT = 32, ATTF_SPLITS_LONG = 64, ATTF_LONG_CAP = 16384;
// rounds of the q/k/v hand-off's poll (each a device-scope round trip of ~1 us plus a
// short sleep) before a wave gives up and computes its rows itself
constexpr int ATTF_QKV_POLLS = 1 << 15;

// the activation prologue's inputs (act_regs_load / act_regs_quant read these fields)
struct AttnNormIn {
    const float* x;
    const uint16_t* nw;
    int K;
    float eps;
    uint32_t* xq_out;
    float* xs_out;
};

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
    uint32_t* counter;     // KV head hk's at counter[hk * TI_SYNC_ATTN_STRIDE]
    // the position and its rotary row come from device memory (dev = 1: the decode
    // step's device position) or from these arguments; both pointers are always
    // valid so the kernel loads them unconditionally (no branch, no flat access)
    const int* dpos;
    const float* rope_cur;
    int dev;
    int pos;
    int nKv, ns, cap;
    int kvs;               // K/V code slots per cached position (>= nKv; the scale rows stay nKv wide)
    float eps;
    uint32_t* oq;          // optional: the output quantized per 32 (quantQ8, for o_proj's linearQ)
    float* os;
    float rope_row[TI_ATTN_HD_MAX];
    // The q/k/v projection of the same launch (k_attn_fused_pv with QL > 0): rmsnormQ of
    // the residual stream (nin), the int4 q, k and v matrices (packs and f16 scales, rows of
    // nin.K / 32 groups), the tagged words that carry the rows between the workgroups, and
    // optional plain copies of q, k and v (nullptr: none)
    AttnNormIn nin;
    const uint4* wpk[3];
    const uint16_t* wsc[3];
    uint64_t* pub;
    float* qkv_copy[3];
    int qkv_polls;         // poll rounds before a wave computes its rows itself
};

// RMSNorm over one head row held by 128 threads (j = element, 0 past hd) in the
// reference's reduction order — slot j and j+64, then a 32..1 tree — with the last
// levels as a wave butterfly (a pair's float sum is the same in either order), then
// split-half RoPE with the given cos/sin row. red/rk: this head's 128-float slices.
__device__ __forceinline__ float head_norm_rope(float x, int j, int hd, float wj, const float* cs, float eps, float* red,
                                               float* rk, float* tot) {
    const float sq = j < hd ? x * x : 0.0f;
    red[j] = sq;
    __syncthreads();
    float v = 0.0f;
    if (j < 64) {
        v = red[j] + red[j + 64];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v = v + ti_xor(v, o);
        if (j == 0) *tot = v;
    }
    __syncthreads();
    float m = *tot / (float)hd;
    m = m + eps;
    const float inv = 1.0f / sqrtf(m);
    if (j < hd) { float t = x * inv; rk[j] = t * wj; }
    __syncthreads();
    float out = 0.0f;
    if (j < hd) {
        const int half = hd / 2;
        const int fi = j < half ? j : j - half;
        const float c = cs[fi], sn = cs[half + fi];
        const float partner = j < half ? rk[j + half] : rk[j - half];
        const float rot = j < half ? -partner : partner;
        const float p0 = rk[j] * c, p1 = rot * sn;
        out = p0 + p1;
    }
    return out;
}

// signed int8 code k of a packed word as (code + 128): one v_cvt_f32_ubyte
__device__ __forceinline__ float ub(uint32_t wflip, int k) { return (float)((wflip >> (8 * k)) & 0xffu); }

// The end of a fused attention workgroup, shared by the decode kernels: merge the 4
// waves' slots (s_red: unnormalised outputs with the +128 code offset already removed,
// s_wml: per-wave (m, l)) into this split's partial and publish it; the last split of
// KV head hk to arrive merges the NS partials by log-sum-exp, writes the head outputs
// (and their quantQ8 codes) and resets the counter. s_part: 1024 floats of LDS that the
// last arriver may use once the publish has read s_red.
template <int HD, int G, int TPW>
__device__ __forceinline__ void attn_merge_tail(const AttnFArgs& a, int hk, int w, int NS, int ntiles, bool valid,
                                                float (&s_red)[4][TPW][G * HD], float (&s_wml)[4][G][2],
                                                float (&s_ml)[G][ATTF_MAXS][2], float (&s_e)[G][ATTF_MAXS], float* s_L,
                                                int* s_last_p, float* s_part, uint32_t epoch = 0) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int NW = NS * 4;
    int& s_last = *s_last_p;
    uint32_t* counter = a.counter + (size_t)hk * TI_SYNC_ATTN_STRIDE;
    __syncthreads();
    // merge the 4 waves x TPW slots into this split's partial and publish it
    const size_t ms = (size_t)NS;
    if (tid < G * HD) {
        const int hh = tid / HD, d = tid % HD;
        float M = s_wml[0][hh][0];
#pragma unroll
        for (int q = 1; q < 4; q++) M = fmaxf(M, s_wml[q][hh][0]);
        float O = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float sq = 0.0f;
#pragma unroll
            for (int t = 0; t < TPW; t++) sq += s_red[q][t][tid];
            O += sq * expf(s_wml[q][hh][0] - M);
        }
        ti_pub_store(a.po + ((size_t)(hk * G + hh) * ms + w) * HD + d, O);
    }
    if (tid < G) {
        float M = s_wml[0][tid][0];
#pragma unroll
        for (int q = 1; q < 4; q++) M = fmaxf(M, s_wml[q][tid][0]);
        float L = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; q++) L += s_wml[q][tid][1] * expf(s_wml[q][tid][0] - M);
        ti_pub_store(a.pml + ((size_t)(hk * G + tid) * ms + w) * 2, M);
        ti_pub_store(a.pml + ((size_t)(hk * G + tid) * ms + w) * 2 + 1, L);
    }
    ti_stores_done();
    __syncthreads();
    if (tid == 0) s_last = ti_arrive(counter) == (unsigned)(NS - 1);
    __syncthreads();
    if (!s_last) return;
    // the last split of hk: log-sum-exp over the splits that saw a tile
    const int nused = ntiles < NW ? (ntiles > 0 ? (ntiles + 3) / 4 : 1) : NS;   // >= 1: no index -1
    // Loads in the order they are needed (vmcnt counts in order): every used split's
    // (m, l) first, one word a thread, then the outputs as 16-byte agent-scope loads —
    // thread (sg, dg) takes 4 consecutive dims 4 dg of splits sg, sg + SG, ... (an index
    // past nused repeats the last split and gets weight 0). The splits' weights are formed
    // while the outputs are still arriving.
    constexpr int GHD = G * HD, D4 = GHD / 4, SG = 256 / D4, MAXL = ATTF_MAXS / SG;
    static_assert(SG * GHD == 1024 && SG * MAXL == ATTF_MAXS, "merge layout");
    const int nml = G * nused * 2;
    float mlv = 0.0f;
    if (tid < nml) {
        const int hh = tid / (nused * 2), r = tid % (nused * 2);
        mlv = ti_pub_load(a.pml + ((size_t)(hk * G + hh) * ms + (r >> 1)) * 2 + (r & 1));
    }
    TI_ISSUE_FENCE();
    const int dg = tid % D4, sg = tid / D4;
    const int oh = (4 * dg) / HD, od = (4 * dg) % HD;
    const __amdgpu_buffer_rsrc_t rpo = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(a.po + (size_t)hk * G * ms * HD), (short)0, (int)(G * ms * HD * 4), 0x00020000);
    float4 ov[MAXL];
#pragma unroll
    for (int j = 0; j < MAXL; j++) {
        const int i = sg + SG * j < nused ? sg + SG * j : nused - 1;
        ov[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rpo, (uint32_t)(((size_t)oh * ms + i) * HD + od) * 4u, 0, TI_CPOL_SC1));
    }
    TI_ISSUE_FENCE();
    if (tid < nml) {
        const int hh = tid / (nused * 2), r = tid % (nused * 2);
        s_ml[hh][r >> 1][r & 1] = mlv;
    }
    __syncthreads();
    if (wave < G) {
        const bool in = lane < nused;
        const float m = in ? s_ml[wave][lane][0] : -3.0e38f;
        float M = m;
#pragma unroll
        for (int o2 = 32; o2 > 0; o2 >>= 1) M = fmaxf(M, ti_xor(M, o2));
        const float e = in ? expf(m - M) : 0.0f;
        float L = in ? s_ml[wave][lane][1] * e : 0.0f;
#pragma unroll
        for (int o2 = 32; o2 > 0; o2 >>= 1) L += ti_xor(L, o2);
        s_e[wave][lane] = e;
        if (lane == 0) s_L[wave] = L;
    }
    __syncthreads();
    {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int j = 0; j < MAXL; j++) {
            const float e = s_e[oh][sg + SG * j];   // 0 past nused
            acc.x = fmaf(ov[j].x, e, acc.x);
            acc.y = fmaf(ov[j].y, e, acc.y);
            acc.z = fmaf(ov[j].z, e, acc.z);
            acc.w = fmaf(ov[j].w, e, acc.w);
        }
        *reinterpret_cast<float4*>(s_part + sg * GHD + 4 * dg) = acc;
    }
    __syncthreads();
    if (valid && tid < GHD) {
        const int hh = tid / HD, d = tid % HD;
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < SG; q++) o += s_part[q * GHD + tid];
        const float L = s_L[hh];
        const float res = o / L;
        const size_t e = (size_t)(hk * G + hh) * HD + d;
        a.out[e] = res;
        if (a.oq) {   // quantQ8 of 32 consecutive outputs = 32 consecutive lanes (q8_group's arithmetic)
            float mx = fabsf(res);
#pragma unroll
            for (int o2 = 16; o2 > 0; o2 >>= 1) mx = fmaxf(mx, ti_xor(mx, o2));
            const float scale = mx / 127.0f;
            const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
            const float pq = res * inv;
            int qi = (int)rintf(pq);
            qi = qi < -127 ? -127 : (qi > 127 ? 127 : qi);
            const uint32_t b = (uint32_t)(qi & 0xff);
            const uint32_t word = ti_quad_or(b << (8 * (lane & 3)));
            if ((lane & 3) == 0) a.oq[e / 4] = word;
            if ((lane & 31) == 0) a.os[e / 32] = scale;
        }
    }
    if (tid == 0) {
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // the q/k/v hand-off of this launch is over (every split of hk has arrived here):
        // the next launch's words carry the next epoch
        if (epoch) __hip_atomic_store(counter + TI_SYNC_ATTN_EPOCH, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int HD, int G>
__global__ __launch_bounds__(256, 2) void k_attn_fused_q8(AttnFArgs a) {
    static_assert(G >= 1 && G <= 2 && (HD == 64 || HD == 128), "fused attention: G <= 2, HD 64 or 128");
    constexpr int LPT = HD / 16;               // lanes per token row (16 bytes each)
    constexpr int TPW = 64 / LPT;              // tokens per wave pass
    constexpr int PASSES = 4;
    constexpr int WT = PASSES * TPW;           // tokens per wave tile
    constexpr int NG = HD / 32;                // scale groups per head row
    __shared__ float red[256];
    __shared__ float rk[256];
    __shared__ float tot[2];
    __shared__ float s_q[G][HD];
    __shared__ __align__(16) uint32_t s_kw[HD / 4];
    __shared__ __align__(16) uint32_t s_vw[HD / 4];
    __shared__ float s_ksc[NG], s_vsc[NG];
    __shared__ __align__(16) float s_red[4][TPW][G * HD];
    __shared__ float s_wml[4][G][2];
    __shared__ float s_ml[G][ATTF_MAXS][2];
    __shared__ float s_e[G][ATTF_MAXS];
    __shared__ float s_L[G];
    __shared__ float rope_cs[HD];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    // split-major across the XCDs (workgroup i runs on XCD i % 8): the NS/8 splits of an
    // XCD are the same for every KV head, so one position's scale line (all heads' groups,
    // 128 B) is fetched into one XCD's L2 and shared by the 8 head workgroups, not into 8
    const int w = blockIdx.x % a.ns;
    const int hk = blockIdx.x / a.ns;
    const int NS = a.ns;
    const int NW = NS * 4;                     // waves per KV head
    const int gw = w * 4 + wave;               // this wave's index among them
    const int h = tid >> 7, j = tid & 127;
    const int tp = lane / LPT, sl = lane % LPT;
    const int row_words4 = a.kvs * HD / 16;
    const int row_groups = a.nKv * NG;
    const float qk_scale = 1.0f / (127.0f * sqrtf((float)HD));
    const uint4* kq4 = reinterpret_cast<const uint4*>(a.kq);
    const uint4* vq4 = reinterpret_cast<const uint4*>(a.vq);

    // ---- every load that does not depend on the position, in one batch
    const int pos_dev = *a.dpos;
    const float cs_dev = a.rope_cur[j < HD ? j : 0];
    const float cs_arg = a.rope_row[j < HD ? j : 0];
    const float qx = a.q[(size_t)(hk * G + (h < G ? h : 0)) * HD + (j < HD ? j : 0)];
    const float kx = a.k[(size_t)hk * HD + (j < HD ? j : 0)];
    const float vx = a.v[(size_t)hk * HD + (j < HD ? j : 0)];
    // the norm weights too: a load issued after the tiles' would wait for them (vmcnt is in order)
    const float qwj = ti_h2f(a.qw[j < HD ? j : 0]);
    const float kwj = ti_h2f(a.kw[j < HD ? j : 0]);
    uint4 kw[2][PASSES], vw[2][PASSES];
    float ksc[2][PASSES], vsc[2][PASSES];
    int lim = a.cap;                           // clamp bound until the context is known
    auto load = [&](int buf, int t0) {
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            int t = t0 + p * TPW + tp;
            t = t < lim ? t : lim - 1;
            kw[buf][p] = ti_ld_nt(kq4 + (size_t)t * row_words4 + hk * LPT + sl);
            vw[buf][p] = ti_ld_nt(vq4 + (size_t)t * row_words4 + hk * LPT + sl);
            ksc[buf][p] = a.ks[(size_t)t * row_groups + hk * NG + sl / 2];
            vsc[buf][p] = a.vs[(size_t)t * row_groups + hk * NG + sl / 2];
        }
    };
    load(0, gw * WT);
    TI_ISSUE_FENCE();

    const int pos = a.dev ? pos_dev : a.pos;
    const float csj = a.dev ? cs_dev : cs_arg;
    const bool valid = pos >= 0 && pos < a.cap;          // outside the cache: nothing is written
    const int S = valid ? pos + 1 : 0;
    const int ntiles = (S + WT - 1) / WT;                 // wave tiles of the context
    const int last_gw = ntiles > 0 ? (ntiles - 1) % NW : -1;
    const bool has_pos = valid && (last_gw >> 2) == w;    // this workgroup writes/uses cache row pos
    lim = S > 0 ? S : 1;

    if (tid < HD) rope_cs[tid] = csj;
    {   // query heads (the first barrier inside publishes rope_cs)
        const float x = (h < G && j < HD) ? qx : 0.0f;
        const float r = head_norm_rope(x, j, HD, qwj, rope_cs, a.eps, red + h * 128, rk + h * 128, tot + h);
        if (h < G && j < HD) s_q[h][j] = r;
    }
    if (has_pos) {   // this token's K (normed, roped) and V rows, snorm int8, into the cache and LDS
        const float x = (h == 0 && j < HD) ? kx : 0.0f;
        const float r = head_norm_rope(x, j, HD, kwj, rope_cs, a.eps, red + h * 128, rk + h * 128, tot + h);
        // one element per lane, a 32-group = 32 lanes of one wave: group max by shuffles,
        // the code of each element (snorm_code), 4 codes packed by the group's lanes
        const float val = h == 0 ? r : vx;
        float mx = j < HD ? fabsf(val) : 0.0f;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, ti_xor(mx, o));
        mx = fmaxf(mx, 1e-12f);
        const uint32_t code = snorm_code(val, mx);
        const uint32_t word = ti_quad_or(code << (8 * (lane & 3)));
        if (j < HD) {
            const size_t rowq = ((size_t)pos * a.kvs + hk) * (HD / 4), rows = ((size_t)pos * a.nKv + hk) * NG;
            if ((j & 3) == 0) {
                (h ? a.vq : a.kq)[rowq + j / 4] = word;
                (h ? s_vw : s_kw)[j / 4] = word;
            }
            if ((j & 31) == 0) {
                (h ? a.vs : a.ks)[rows + j / 32] = mx;
                (h ? s_vsc : s_ksc)[j / 32] = mx;
            }
        }
    }
    __syncthreads();

    float qv[G][16], qsum[G];
#pragma unroll
    for (int hh = 0; hh < G; hh++) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) { qv[hh][i] = s_q[hh][sl * 16 + i]; s += qv[hh][i]; }
        qsum[hh] = 128.0f * s;
    }
    float m_run[G], l_run[G], acc[G][16], pws[G];
#pragma unroll
    for (int hh = 0; hh < G; hh++) {
        m_run[hh] = -3.0e38f;
        l_run[hh] = 0.0f;
        pws[hh] = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) acc[hh][i] = 0.0f;
    }

    // one wave tile, no barriers: scores -> wave max -> exp -> P*V. Codes enter as
    // (code + 128) (v_cvt_f32_ubyte); the offset is removed once per dot (q) and once
    // at the end (p), where it is exact bookkeeping, not an approximation.
    auto process = [&](int buf, int t0) {
        if (has_pos && t0 + WT >= S) {   // the tile holding pos: that row (and clamped reads past it) from LDS
#pragma unroll
            for (int p = 0; p < PASSES; p++) {
                if (t0 + p * TPW + tp >= pos) {
                    kw[buf][p] = reinterpret_cast<const uint4*>(s_kw)[sl];
                    vw[buf][p] = reinterpret_cast<const uint4*>(s_vw)[sl];
                    ksc[buf][p] = s_ksc[sl / 2];
                    vsc[buf][p] = s_vsc[sl / 2];
                }
            }
        }
        float sc[PASSES][G];
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const uint32_t ww[4] = {kw[buf][p].x ^ 0x80808080u, kw[buf][p].y ^ 0x80808080u,
                                    kw[buf][p].z ^ 0x80808080u, kw[buf][p].w ^ 0x80808080u};
#pragma unroll
            for (int hh = 0; hh < G; hh++) {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; i++) d = fmaf(qv[hh][i], ub(ww[i >> 2], i & 3), d);
                sc[p][hh] = (d - qsum[hh]) * ksc[buf][p];
            }
#pragma unroll
            for (int o = LPT / 2; o > 0; o >>= 1)
#pragma unroll
                for (int hh = 0; hh < G; hh++) sc[p][hh] += ti_xor(sc[p][hh], o);
            const bool live = t0 + p * TPW + tp < S;
#pragma unroll
            for (int hh = 0; hh < G; hh++) sc[p][hh] = live ? sc[p][hh] * qk_scale : -3.0e38f;
        }
        float corr[G];
#pragma unroll
        for (int hh = 0; hh < G; hh++) {
            float mx = sc[0][hh];
#pragma unroll
            for (int p = 1; p < PASSES; p++) mx = fmaxf(mx, sc[p][hh]);
#pragma unroll
            for (int o = LPT; o < 64; o <<= 1) mx = fmaxf(mx, ti_xor(mx, o));
            const float mn = fmaxf(m_run[hh], mx);
            corr[hh] = expf(m_run[hh] - mn);
            m_run[hh] = mn;
        }
        float ps[G];
#pragma unroll
        for (int hh = 0; hh < G; hh++) {
            ps[hh] = 0.0f;
            pws[hh] *= corr[hh];
#pragma unroll
            for (int i = 0; i < 16; i++) acc[hh][i] *= corr[hh];
        }
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const bool live = t0 + p * TPW + tp < S;
            const uint32_t ww[4] = {vw[buf][p].x ^ 0x80808080u, vw[buf][p].y ^ 0x80808080u,
                                    vw[buf][p].z ^ 0x80808080u, vw[buf][p].w ^ 0x80808080u};
#pragma unroll
            for (int hh = 0; hh < G; hh++) {
                const float e = live ? expf(sc[p][hh] - m_run[hh]) : 0.0f;
                ps[hh] += e;
                // rows past the context may hold anything (even a NaN scale): weight exactly 0
                const float pw = live ? e * vsc[buf][p] * (1.0f / 127.0f) : 0.0f;
                pws[hh] += pw;
#pragma unroll
                for (int i = 0; i < 16; i++) acc[hh][i] = fmaf(pw, ub(ww[i >> 2], i & 3), acc[hh][i]);
            }
        }
#pragma unroll
        for (int hh = 0; hh < G; hh++) {
#pragma unroll
            for (int o = LPT; o < 64; o <<= 1) ps[hh] += ti_xor(ps[hh], o);
            l_run[hh] = l_run[hh] * corr[hh] + ps[hh];
        }
    };
    const int step = NW * WT;
    int t0 = gw * WT;
    while (t0 < S) {
        int nt = t0 + step;
        if (nt < S) load(1, nt);
        process(0, t0);
        if (nt >= S) break;
        t0 = nt;
        nt = t0 + step;
        if (nt < S) load(0, nt);
        process(1, t0);
        t0 = nt;
    }

    // wave state -> LDS, one row per token slot with the +128 offset removed (a shuffle
    // tree over the slots costs more than the 32 LDS reads of the merge below)
#pragma unroll
    for (int hh = 0; hh < G; hh++) {
        float4* dst = reinterpret_cast<float4*>(&s_red[wave][tp][hh * HD + sl * 16]);
        const float off = 128.0f * pws[hh];
#pragma unroll
        for (int i = 0; i < 4; i++)
            dst[i] = make_float4(acc[hh][4 * i] - off, acc[hh][4 * i + 1] - off, acc[hh][4 * i + 2] - off,
                                 acc[hh][4 * i + 3] - off);
        if (lane == 0) {
            s_wml[wave][hh][0] = m_run[hh];
            s_wml[wave][hh][1] = l_run[hh];
        }
    }
    attn_merge_tail<HD, G, TPW>(a, hk, w, NS, ntiles, valid, s_red, s_wml, s_ml, s_e, s_L, &s_last, &s_red[0][0][0]);
}

// head_dim 128 decode attention with both products on the matrix cores.
//
// A wave tile is 32 keys. Its K and V codes and its scale rows reach LDS by buffer loads
// written straight to LDS; the tile's buffer resources start at the tile and end at the
// last valid key, so no lane clamps its index (keys past the end read as zero, and are
// masked anyway). In LDS a key row's 16-byte slices are XOR-permuted by (key >> 1) & 7,
// which leaves both operand reads below free of bank conflicts.
//  - Q K^T: q (normed and roped, f32) split per head into three int8 limbs,
//    q = S0*c0 + S1*c1 + S2*c2 with S0 = max|q|/127, S1 = S0/254, S2 = S1/254 (each limb's
//    residual is within half its step, so |c| <= 127 and the representation error is
//    below max|q| * 6.2e-8, the size of f32 rounding). Per 32-dim scale group two
//    v_mfma_i32_16x16x32_i8 accumulate into one result: the first holds the limbs in A
//    rows 0..7 (row 4 h + limb) against keys 0..15, the second in rows 8..15 against
//    keys 16..31. So lane l ends with the three limb dots of head (l >> 4) & 1 and key
//    16 (l >> 5) + (l & 15): one score per lane, in base-2 units (log2 e and
//    1/(127 sqrt(hd)) ride on the limb scales).
//  - softmax per head over its 32 lanes, p = 2^(s - m) against the running maximum.
//  - P V: P'_g = p * vs(key, g), the V scale of the key's 32-dim group g, as f16 hi + lo
//    (~2^-22 relative), parked in LDS per (head, group, key). A (16 x 32) row
//    m = 8 (g >> 1) + 4 h + 2 (g & 1) + (hi: 0, lo: 1); B = the V codes of 8 keys per
//    lane group for 16 dims, transposed by ds_read_b64_tr_b8 and converted to f16
//    exactly; one v_mfma_f32_16x16x32_f16 per 16 dims. Lane group q holds rows
//    4q .. 4q+3 = head q & 1, groups 2 (q >> 1) + {0, 1}: the head's outputs at dims
//    64 (q >> 1) .. +63 are the sums of its hi and lo rows there (the other rows of those
//    columns pair P' of another group with these dims and are never read).
//  The head of a lane's scores and of its P V rows is the same ((l >> 4) & 1), so the
//  rescale by the moved maximum needs no exchange.
constexpr int PV_WT = 32;                  // keys per wave tile
constexpr int PV_TB = PV_WT * 128;         // bytes of one tile's K (or V) codes
constexpr int PV_PH = 640;                 // bytes between the two heads' P' rows (conflict-free stores)

typedef int pv_v4i __attribute__((ext_vector_type(4)));
typedef int pv_v2i __attribute__((ext_vector_type(2)));
typedef float pv_f4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* pv_lds_t;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pv_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes > 0 ? bytes : 0, 0x00020000);
}

// The LDS reads of a tile's P V step, issued as one block that ends with its own wait:
// the P' words other lanes of the wave wrote just before (a wave's LDS instructions
// execute in order; the block is a compiler memory barrier, so the writes stay above it)
// and the 8 transposing reads of the V tile (ds_read_b64_tr_b8). Written by hand because
// the compiler puts a wait for every direct-to-LDS load in flight before such reads (it
// cannot tell that those loads fill the other tile buffer), which would hold each tile's
// P V products until the next tile had arrived. This tile's loads were waited for at the
// top of its iteration.
__device__ __forceinline__ void pv_read_pv(const uint8_t* pa, const uint8_t* vt, const uint32_t (&voff8)[8], uint4& wa,
                                           uint4& wb, pv_v2i (&vb)[8]) {
    typedef __attribute__((address_space(3))) const uint8_t* lds_p;
    const uint32_t pw = (uint32_t)reinterpret_cast<uintptr_t>((lds_p)pa);
    uint32_t ad[8];
#pragma unroll
    for (int D = 0; D < 8; D++) ad[D] = (uint32_t)reinterpret_cast<uintptr_t>((lds_p)(vt + voff8[D]));
    __builtin_amdgcn_wave_barrier();
    asm volatile(
        "ds_read_b128 %0, %10\n\t"
        "ds_read_b128 %1, %10 offset:16\n\t"
        "ds_read_b64_tr_b8 %2, %11\n\t"
        "ds_read_b64_tr_b8 %3, %12\n\t"
        "ds_read_b64_tr_b8 %4, %13\n\t"
        "ds_read_b64_tr_b8 %5, %14\n\t"
        "ds_read_b64_tr_b8 %6, %15\n\t"
        "ds_read_b64_tr_b8 %7, %16\n\t"
        "ds_read_b64_tr_b8 %8, %17\n\t"
        "ds_read_b64_tr_b8 %9, %18\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(wa), "=&v"(wb), "=&v"(vb[0]), "=&v"(vb[1]), "=&v"(vb[2]), "=&v"(vb[3]), "=&v"(vb[4]), "=&v"(vb[5]),
          "=&v"(vb[6]), "=&v"(vb[7])
        : "v"(pw), "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]), "v"(ad[7])
        : "memory");
}

// max / sum over the 16 lanes of a row (DPP), every lane receiving the result
__device__ __forceinline__ float pv_row_max(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
    return v;
}
__device__ __forceinline__ float pv_row_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    return v;
}

template <int G, int QL = 0, int QR = 2>
__global__ __launch_bounds__(256, 2) void k_attn_fused_pv(AttnFArgs a) {
    static_assert(G == 1 || G == 2, "MFMA decode attention: G <= 2");
    constexpr int HD = 128, NG = HD / 32;
    __shared__ float s_qmax[2];
    __shared__ __align__(16) int8_t s_ql[G][3][HD];
    __shared__ __align__(16) uint32_t s_kw[HD / 4];
    __shared__ __align__(16) uint32_t s_vw[HD / 4];
    __shared__ __align__(16) float s_ksc[NG];
    __shared__ __align__(16) float s_vsc[NG];
    __shared__ __align__(16) uint8_t s_k[4][2][PV_TB];            // [wave][buffer] K tiles
    __shared__ __align__(16) uint8_t s_v[4][2][PV_TB];            // V tiles
    __shared__ __align__(16) float s_sc[4][2][2][PV_WT][NG];      // [wave][buffer][K, V][key][group] scales
    __shared__ __align__(16) uint8_t s_pa[4][2 * PV_PH];          // P' words [head][group][key]: hi | lo << 16
    __shared__ float s_wml[4][G][2];
    __shared__ float s_L[G];
    __shared__ int s_last;
    // after the tile loop: the waves' outputs over the K tiles, the split merge's (m, l)
    // and weights over the V tiles
    float (&s_red)[4][1][G * HD] = *reinterpret_cast<float (*)[4][1][G * HD]>(&s_k[0][0][0]);
    float (&s_ml)[G][ATTF_MAXS][2] = *reinterpret_cast<float (*)[G][ATTF_MAXS][2]>(&s_v[0][0][0]);
    float (&s_e)[G][ATTF_MAXS] = *reinterpret_cast<float (*)[G][ATTF_MAXS]>(&s_v[1][0][0]);
    static_assert(4 * G * HD * 4 <= (int)sizeof(s_k) && G * ATTF_MAXS * 8 <= 2 * PV_TB, "merge areas fit the tiles");

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int w = blockIdx.x % a.ns;           // split-major across the XCDs (see k_attn_fused_q8)
    const int hk = blockIdx.x / a.ns;
    const int NS = a.ns;
    const int NW = NS * 4;
    const int gw = w * 4 + wave;
    const int r16 = lane & 15, kq = lane >> 4;    // MFMA lanes: row / column, K quarter
    const int sh = kq & 1;                        // head of this lane's scores and P V rows
    const int key_t = 16 * (lane >> 5) + r16;     // key (in the tile) of this lane's score
    const uint32_t rowb = (uint32_t)a.kvs * HD;   // cache bytes per position (codes)
    const uint32_t rows16 = (uint32_t)a.nKv * 16; // bytes per position (the 4 group scales)
    const float l2s = 1.4426950408889634f / (127.0f * sqrtf((float)HD));

    // tile lanes: pass p carries key 8p + lane/8; LDS slot lane%8 of it holds slice
    // (lane%8) ^ ((key >> 1) & 7). Scale rows in LDS as [K, V][key][group]: the first
    // tile's by lane (lane < 32 the K row of key lane, else the V row of key lane - 32),
    // the others' as dwords (lane: key 16j + lane/4, group lane%4).
    uint32_t toff[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int key = 8 * p + (lane >> 3);
        toff[p] = (uint32_t)key * rowb + 16u * (uint32_t)((lane & 7) ^ ((key >> 1) & 7));
    }
    const uint32_t soff = (uint32_t)(lane & 31) * rows16;
    const uint32_t soff4[2] = {(uint32_t)(lane >> 2) * rows16 + 4u * (uint32_t)(lane & 3),
                               (uint32_t)(16 + (lane >> 2)) * rows16 + 4u * (uint32_t)(lane & 3)};
    const uint8_t* kq_b = reinterpret_cast<const uint8_t*>(a.kq);
    const uint8_t* vq_b = reinterpret_cast<const uint8_t*>(a.vq);
    const uint8_t* ks_b = reinterpret_cast<const uint8_t*>(a.ks);
    const uint8_t* vs_b = reinterpret_cast<const uint8_t*>(a.vs);
    // the resources of the tile at t0 when positions below lim are valid
    auto tile_rs = [&](int t0, int lim, __amdgpu_buffer_rsrc_t& rk, __amdgpu_buffer_rsrc_t& rv,
                       __amdgpu_buffer_rsrc_t& rks, __amdgpu_buffer_rsrc_t& rvs) {
        const int n = lim - t0;
        const size_t crow0 = (size_t)t0 * a.kvs + hk, srow0 = (size_t)t0 * a.nKv + hk;
        const int cb = n > 0 ? (int)((uint32_t)(n - 1) * rowb + HD) : 0;
        const int sb = n > 0 ? (int)((uint32_t)(n - 1) * rows16 + 16) : 0;
        rk = pv_rsrc(kq_b + crow0 * HD, cb);
        rv = pv_rsrc(vq_b + crow0 * HD, cb);
        rks = pv_rsrc(ks_b + srow0 * 16, sb);
        rvs = pv_rsrc(vs_b + srow0 * 16, sb);
    };

    // ---- every load that does not depend on the position, in one batch. Wave 0 (and 1
    // when G = 2) holds query head `wave`, wave 2 the new K row, wave 3 the new V row;
    // lane L holds elements L and L + 64, so RMSNorm, RoPE and the limb split of q run in
    // registers
    const uint16_t* nwrow = wave < 2 ? a.qw : a.kw;
    // The device position is read with a vector load issued behind the first tile's, and
    // the value is held opaque (an empty asm that rewrites the register) until it is
    // needed: as a scalar load at the top it held every vector load of the prologue for
    // its own round trip (the compiler waits for all scalar loads before the first vector
    // one), and a use the compiler is free to hoist (a readfirstlane right after the load)
    // makes the wave wait for every load issued before it, the first tile's included,
    // before the prologue's arithmetic. Without a device position the load reads a word
    // that is always there, unused.
    uint32_t pos_raw = 0;
    auto pos_load = [&]() {
        pos_raw = ti_pub_load(a.dev ? reinterpret_cast<const uint32_t*>(a.dpos) : a.counter);
    };
    auto pos_now = [&]() {
        asm volatile("" : "+v"(pos_raw));
        return a.dev ? (int)pos_raw : a.pos;
    };
    // the first tile through registers, bounded by the capacity until the context is known
    // (a load straight to LDS in flight would make the prologue's waits full ones)
    uint4 kf[4], vf[4], sf;
    auto first_tile = [&](int wt_gw, uint4 (&tk)[4], uint4 (&tv)[4], uint4& ts) {
        __amdgpu_buffer_rsrc_t rk, rv, rks, rvs;
        tile_rs(wt_gw * PV_WT, a.cap, rk, rv, rks, rvs);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            tk[p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, toff[p], 0, 2));
            tv[p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, toff[p], 0, 2));
        }
        const uint4 sk = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rks, soff, 0, 2));
        const uint4 sv = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rvs, soff, 0, 2));
        ts = lane < 32 ? sk : sv;
    };
    float x0, x1;
    uint32_t epoch = 0;
    if constexpr (QL == 0) {
        const float* xrow = wave < 2 ? a.q + (size_t)(hk * G + (wave < G ? wave : 0)) * HD
                                     : (wave == 2 ? a.k : a.v) + (size_t)hk * HD;
        x0 = xrow[lane];
        x1 = xrow[lane + 64];
    }
    const float w0 = ti_h2f(nwrow[lane]), w1 = ti_h2f(nwrow[lane + 64]);
    const float c_dev = a.rope_cur[lane], s_dev = a.rope_cur[lane + 64];
    const float c_arg = a.rope_row[lane], s_arg = a.rope_row[lane + 64];
    if constexpr (QL == 0) {
        first_tile(gw, kf, vf, sf);
        pos_load();
        TI_ISSUE_FENCE();
    } else {
        // ---- q, k and v of this KV head, computed by its NS workgroups together.
        // rmsnormQ of x in every workgroup (the q/k/v GEMV's prologue: the same codes),
        // then each wave takes units of RS rows of the head's (G + 2) * HD rows (q heads
        // hk*G.., the k head, the v head), units gw, gw + 4 NS, ...: QL lanes per row, one
        // 32-group a lane, the exact int32 group dots scaled and summed as the stand-alone
        // GEMV does (k_fgemv), so the rows are the same bits. Each row goes out as a 64-bit
        // word, its value beside the launch's epoch; the wave that needs a row (its q head,
        // the k or the v row) polls those words until all carry the epoch. No counter: a
        // word is complete when it lands. The epoch of KV head hk sits beside its merge
        // counter; the merge's last arriver (every split of hk has passed its poll by then)
        // advances it for the next launch. A poll that does not complete in
        // ATTF_QKV_POLLS rounds (workgroups of the head not resident) gives up, and the
        // wave computes its 128 rows itself, with the same arithmetic.
        constexpr int RPP = 64 / QL, R = QR, RS = RPP * R, NU = (G + 2) * HD / RS, SPAN = QL / R, EPT = QL / 8;
        static_assert(HD % RS == 0, "a unit of rows never straddles two heads");
        const int sub = lane / QL, li = lane % QL;
        uint32_t* s_xq = reinterpret_cast<uint32_t*>(&s_v[0][1][0]);      // free until the tile loop
        float* s_xs = reinterpret_cast<float*>(&s_v[0][1][2048]);
        float* s_nred = reinterpret_cast<float*>(&s_v[1][1][0]);
        uint32_t* ctr = a.counter + (size_t)hk * TI_SYNC_ATTN_STRIDE;
        epoch = ti_pub_load(ctr + TI_SYNC_ATTN_EPOCH) + 1u;
        uint64_t* pub = a.pub + (size_t)hk * (G + 2) * HD;
        ActRegs<EPT, true> ar;
        act_regs_load<MODE_NORM>(a.nin, ar);
        // a unit's rows: local rows u*RS + sub + r*RPP (r < R); its matrix and first row
        // are wave-uniform (selects of argument pointers stay scalar)
        auto unit_rows = [&](int u, const uint4*& P, const uint16_t*& SC, int& grow0) {
            const int lr0 = u * RS, seg = lr0 / HD;
            P = seg < G ? a.wpk[0] : (seg == G ? a.wpk[1] : a.wpk[2]);
            SC = seg < G ? a.wsc[0] : (seg == G ? a.wsc[1] : a.wsc[2]);
            grow0 = (seg < G ? (hk * G + seg) * HD : hk * HD) + lr0 - seg * HD;
        };
        uint4 wq[R];
        uint16_t sq[R];
        const int gwv = w * 4 + wave, wstep = 4 * NS;
        auto unit_load = [&](int j) {
            int u = gwv + j * wstep;
            u = u < NU ? u : NU - 1;                      // past the head's units: a repeat, unused
            const uint4* P;
            const uint16_t* SC;
            int grow0;
            unit_rows(u, P, SC, grow0);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const size_t gi = (size_t)(grow0 + sub + r * RPP) * QL + li;
                wq[r] = ti_ld_nt(P + gi);
                sq[r] = __builtin_nontemporal_load(SC + gi);
            }
        };
        unit_load(0);
        first_tile(gw, kf, vf, sf);
        pos_load();
        TI_ISSUE_FENCE();
        act_regs_quant<MODE_NORM>(a.nin, ar, s_xq, s_xs, s_nred);
        ActQ8 act;
        load_act_q8(s_xq, s_xs, li, act);
        // the unit's R rows, summed over the QL lanes of each: lane li holds row li / SPAN
        // (the same butterfly tree for every R, so the same bits as the stand-alone GEMV)
        auto unit_dot = [&](const uint4 (&wu)[R], const uint16_t (&su)[R]) {
            float ga[R];
#pragma unroll
            for (int r = 0; r < R; r++) ga[r] = fmaf((float)group_dot_q8(wu[r], act), ti_h2f(su[r]) * act.s, 0.0f);
            return transpose_reduce<QL, R>(ga, li);
        };
        const int rounds = (NU + wstep - 1) / wstep;
        for (int j = 0; j < rounds; j++) {
            if (j > 0) unit_load(j);
            const int u = gwv + j * wstep;
            const float tot = unit_dot(wq, sq);
            if (u < NU && li % SPAN == 0) {
                const int lr = u * RS + sub + (li / SPAN) * RPP;
                ti_pub_store(pub + lr, ((uint64_t)epoch << 32) | __builtin_bit_cast(uint32_t, tot));
                const int seg = lr / HD;                  // plain copy: row of q, k or v
                float* cp = seg < G ? a.qkv_copy[0] : (seg == G ? a.qkv_copy[1] : a.qkv_copy[2]);
                if (cp) cp[(seg < G ? (hk * G + seg) * HD : hk * HD) + lr - seg * HD] = tot;
            }
        }
        // this wave's row: q head (wave < G), k (wave 2) or v (wave 3); local rows cb..cb+127
        // (the k and v rows only in the split that holds the position: no other reads them)
        const int cb = (wave < 2 ? (wave < G ? wave : 0) : (wave == 2 ? G : G + 1)) * HD;
        const int pos_e = pos_now();
        const int ntiles_e = pos_e >= 0 && pos_e < a.cap ? (pos_e + PV_WT) / PV_WT : 0;
        const bool need = wave < 2 || (ntiles_e > 0 && ((ntiles_e - 1) % NW) >> 2 == w);
        uint64_t e0 = 0, e1 = 0;
        bool got = !need;
        for (int it = 0; need && it < a.qkv_polls; it++) {
            e0 = ti_pub_load(pub + cb + lane);
            e1 = ti_pub_load(pub + cb + lane + 64);
            got = __all((uint32_t)(e0 >> 32) == epoch && (uint32_t)(e1 >> 32) == epoch);
            if (got) break;
            __builtin_amdgcn_s_sleep(2);
        }
        if (got) {
            x0 = __builtin_bit_cast(float, (uint32_t)e0);
            x1 = __builtin_bit_cast(float, (uint32_t)e1);
        } else {   // the wave's 128 rows here (LDS of its second K tile, unused until the loop)
            float* fb = reinterpret_cast<float*>(&s_k[wave][1][0]);
            for (int u = cb / RS; u < (cb + HD) / RS; u++) {
                const uint4* P;
                const uint16_t* SC;
                int grow0;
                unit_rows(u, P, SC, grow0);
                uint4 wu[R];
                uint16_t su[R];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const size_t gi = (size_t)(grow0 + sub + r * RPP) * QL + li;
                    wu[r] = ti_ld_nt(P + gi);
                    su[r] = __builtin_nontemporal_load(SC + gi);
                }
                const float tot = unit_dot(wu, su);
                if (li % SPAN == 0) fb[u * RS + sub + (li / SPAN) * RPP - cb] = tot;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            x0 = fb[lane];
            x1 = fb[lane + 64];
        }
    }

    const int pos = pos_now();
    const bool valid = pos >= 0 && pos < a.cap;
    const int S = valid ? pos + 1 : 0;
    const int ntiles = (S + PV_WT - 1) / PV_WT;
    const int last_gw = ntiles > 0 ? (ntiles - 1) % NW : -1;
    const bool has_pos = valid && (last_gw >> 2) == w;

    const float cr = a.dev ? c_dev : c_arg, sr = a.dev ? s_dev : s_arg;
    float o0 = x0, o1 = x1;
    if (wave < 3) {   // RMSNorm in attnPrepQ8's order, split-half RoPE
        float v = x0 * x0 + x1 * x1;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v = v + ti_xor(v, o);
        float m = v / (float)HD;
        m = m + a.eps;
        const float inv = 1.0f / sqrtf(m);
        const float t0n = x0 * inv, t1n = x1 * inv;
        const float r0 = t0n * w0, r1 = t1n * w1;
        const float p00 = r0 * cr, p01 = (-r1) * sr;
        const float p10 = r1 * cr, p11 = r0 * sr;
        o0 = p00 + p01;
        o1 = p10 + p11;
    }
    if (has_pos && wave >= 2) {   // this token's K (normed, roped) and V rows, snorm int8, into LDS
        // (into the cache after the tile loop)
        const bool isv = wave == 3;
        const float mx0 = fmaxf(ti_max32_nonneg(fabsf(o0)), 1e-12f);
        const float mx1 = fmaxf(ti_max32_nonneg(fabsf(o1)), 1e-12f);
        const uint32_t wd0 = ti_quad_or(snorm_code(o0, mx0) << (8 * (lane & 3)));
        const uint32_t wd1 = ti_quad_or(snorm_code(o1, mx1) << (8 * (lane & 3)));
        uint32_t* lq = isv ? s_vw : s_kw;
        float* lsc = isv ? s_vsc : s_ksc;
        if ((lane & 3) == 0) {
            lq[lane / 4] = wd0;
            lq[16 + lane / 4] = wd1;
        }
        if ((lane & 31) == 0) {
            lsc[lane / 32] = mx0;
            lsc[2 + lane / 32] = mx1;
        }
    }
    if (wave < G) {   // q limbs: q = S0*c0 + S1*c1 + S2*c2, codes into LDS
        float qm = fmaxf(fabsf(o0), fabsf(o1));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) qm = fmaxf(qm, ti_xor(qm, o));
        const float S0 = qm / 127.0f, S1 = S0 / 254.0f, S2 = S1 / 254.0f;
        const float i0 = S0 > 0.0f ? 1.0f / S0 : 0.0f, i1 = S1 > 0.0f ? 1.0f / S1 : 0.0f, i2 = S2 > 0.0f ? 1.0f / S2 : 0.0f;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const float v = e ? o1 : o0;
            const float c0 = fminf(fmaxf(rintf(v * i0), -127.0f), 127.0f);
            const float r1 = fmaf(-S0, c0, v);
            const float c1 = fminf(fmaxf(rintf(r1 * i1), -127.0f), 127.0f);
            const float r2 = fmaf(-S1, c1, r1);
            const float c2 = fminf(fmaxf(rintf(r2 * i2), -127.0f), 127.0f);
            s_ql[wave][0][lane + 64 * e] = (int8_t)c0;
            s_ql[wave][1][lane + 64 * e] = (int8_t)c1;
            s_ql[wave][2][lane + 64 * e] = (int8_t)c2;
        }
        if (lane == 0) s_qmax[wave] = qm;
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {   // the first tile into buffer 0, in the order the direct loads use
        *reinterpret_cast<uint4*>(&s_k[wave][0][p * 1024 + 16 * lane]) = kf[p];
        *reinterpret_cast<uint4*>(&s_v[wave][0][p * 1024 + 16 * lane]) = vf[p];
    }
    *reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(&s_sc[wave][0][0][0][0]) + 16 * lane) = sf;
    __syncthreads();

    // ---- score operands: A0 rows 0..7 / A1 rows 8..15 = (head, limb), limb 3 zero; this
    // lane's K quarter of each group is dims 32g + 8kq .. +7
    long qa0[NG], qa1[NG];
    {
        const int m = r16 & 7, ah = G == 2 ? m >> 2 : 0, al = m & 3;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const long v = *reinterpret_cast<const long*>(&s_ql[ah][al < 3 ? al : 0][g * 32 + 8 * kq]);
            const long vv = al < 3 ? v : 0;
            qa0[g] = r16 < 8 ? vv : 0;
            qa1[g] = r16 < 8 ? 0 : vv;
        }
    }
    float L0, L1, L2;
    {
        const float qm = s_qmax[G == 2 ? sh : 0];
        const float S0 = qm / 127.0f, S1 = S0 / 254.0f, S2 = S1 / 254.0f;
        L0 = S0 * l2s;
        L1 = S1 * l2s;
        L2 = S2 * l2s;
    }
    // operand offsets in a tile: K of block b (keys 16b..16b+15) and group g for this lane's
    // key r16 and quarter kq; V (transposing read) of 16-dim block D: lanes 2r, 2r+1 of lane
    // group kq address key 8kq + r, 8-byte half r16 & 1
    uint32_t koff[2][NG], voff8[8];
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const int key = 16 * b + r16;
            koff[b][g] = (uint32_t)(key * 128 + 16 * ((2 * g + (kq >> 1)) ^ ((key >> 1) & 7)) + 8 * (kq & 1));
        }
    {
        const int key = 8 * kq + (r16 >> 1);
#pragma unroll
        for (int D = 0; D < 8; D++) voff8[D] = (uint32_t)(key * 128 + 16 * (D ^ ((key >> 1) & 7)) + 8 * (r16 & 1));
    }
    // P' words: this lane's (head sh, key key_t) at [sh][g][key_t]; the A row of this lane
    // (m = r16: g = 2 (m >> 3) + ((m >> 1) & 1), head (m >> 2) & 1, hi/lo m & 1) over keys 8kq..8kq+7
    const uint32_t pa_w = (uint32_t)(sh * PV_PH + 4 * key_t);
    const uint32_t pa_r = (uint32_t)(((r16 >> 2) & 1) * PV_PH + (2 * (r16 >> 3) + ((r16 >> 1) & 1)) * 128 + 32 * kq);
    const uint32_t psel = (r16 & 1) ? 0x07060302u : 0x05040100u;   // the lo or hi halves of two words
    const bool pa_zero = G == 1 && sh == 1;                           // rows of a head that is not there

    float m_run = -3.0e38f, l_lane = 0.0f;
    pv_f4 O[8];
#pragma unroll
    for (int D = 0; D < 8; D++) O[D] = pv_f4{0.0f, 0.0f, 0.0f, 0.0f};

    auto process = [&](int b, int t0) {
        const uint8_t* kt = &s_k[wave][b][0];
        const uint8_t* vt = &s_v[wave][b][0];
        uint8_t* pa = &s_pa[wave][0];
        const float4 kg = *reinterpret_cast<const float4*>(&s_sc[wave][b][0][key_t][0]);
        const float4 vg = *reinterpret_cast<const float4*>(&s_sc[wave][b][1][key_t][0]);
        const float kgs[NG] = {kg.x, kg.y, kg.z, kg.w};
        const float vgs[NG] = {vg.x, vg.y, vg.z, vg.w};
        float d = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const long k0 = *reinterpret_cast<const long*>(kt + koff[0][g]);
            const long k1 = *reinterpret_cast<const long*>(kt + koff[1][g]);
            pv_v4i c = {0, 0, 0, 0};
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa0[g], k0, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa1[g], k1, c, 0, 0, 0);
            const float lq = fmaf(L2, (float)c[2], fmaf(L1, (float)c[1], L0 * (float)c[0]));
            d = fmaf(kgs[g], lq, d);
        }
        const bool live = t0 + key_t < S;
        const float s2 = live ? d : -3.0e38f;
        // the head's 32 lanes: r16 + 16 {sh, sh + 2}
        float mt = pv_row_max(s2);
        mt = fmaxf(mt, ti_xor(mt, 32));
        const float mn = fmaxf(m_run, mt);
        const float corr = __builtin_amdgcn_exp2f(m_run - mn);
        m_run = mn;
        const float p = live ? __builtin_amdgcn_exp2f(s2 - mn) : 0.0f;
        l_lane = fmaf(l_lane, corr, p);
        if (__any(corr != 1.0f)) {   // a head's maximum moved: rescale its rows
#pragma unroll
            for (int D = 0; D < 8; D++) O[D] *= corr;
        }
        // P'_g as f16 hi | lo << 16 (keys past the context: exactly 0, whatever their scale holds)
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const float pv = (live && !pa_zero) ? p * vgs[g] : 0.0f;
            const _Float16 hi = (_Float16)pv;
            const _Float16 lo = (_Float16)(pv - (float)hi);
            *reinterpret_cast<uint32_t*>(pa + pa_w + 128 * g) =
                (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
        }
        // the other lanes' P' words, then the V tile (8 keys of one dimension per lane)
        uint4 wa, wb;
        pv_v2i vb[8];
        pv_read_pv(pa + pa_r, vt, voff8, wa, wb, vb);
        const uint4 ap = make_uint4(__builtin_amdgcn_perm(wa.y, wa.x, psel), __builtin_amdgcn_perm(wa.w, wa.z, psel),
                                    __builtin_amdgcn_perm(wb.y, wb.x, psel), __builtin_amdgcn_perm(wb.w, wb.z, psel));
        const ti_h8 A = __builtin_bit_cast(ti_h8, ap);
#pragma unroll
        for (int D = 0; D < 8; D++)
            O[D] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, ti_i8x8_h8((uint32_t)vb[D].x, (uint32_t)vb[D].y), O[D], 0, 0, 0);
    };
    // the tile holding pos: that key's rows from the prologue's LDS copy (this launch writes
    // them to the cache)
    auto own_row = [&](int b, int t0) {
        const int i = pos - t0, swz = (i >> 1) & 7;
        if (lane < 8) {
            *reinterpret_cast<uint4*>(&s_k[wave][b][i * 128 + 16 * (lane ^ swz)]) = reinterpret_cast<const uint4*>(s_kw)[lane];
        } else if (lane < 16) {
            *reinterpret_cast<uint4*>(&s_v[wave][b][i * 128 + 16 * ((lane - 8) ^ swz)]) = reinterpret_cast<const uint4*>(s_vw)[lane - 8];
        } else if (lane == 16) {
            *reinterpret_cast<float4*>(&s_sc[wave][b][0][i][0]) = *reinterpret_cast<const float4*>(s_ksc);
        } else if (lane == 17) {
            *reinterpret_cast<float4*>(&s_sc[wave][b][1][i][0]) = *reinterpret_cast<const float4*>(s_vsc);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    auto load_tile = [&](int b, int t0) {
        __amdgpu_buffer_rsrc_t rk, rv, rks, rvs;
        tile_rs(t0, S, rk, rv, rks, rvs);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (pv_lds_t)&s_k[wave][b][p * 1024], 16, toff[p], 0, 0, 2);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (pv_lds_t)&s_v[wave][b][p * 1024], 16, toff[p], 0, 0, 2);
        }
        // scale rows as dwords (one resource per instruction: a lane-dependent choice of
        // resource would become a loop over the distinct values)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rks, (pv_lds_t)&s_sc[wave][b][0][16 * j][0], 4, soff4[j], 0, 0, 2);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rvs, (pv_lds_t)&s_sc[wave][b][1][16 * j][0], 4, soff4[j], 0, 0, 2);
        }
    };

    // every memory operation in flight at the top of an iteration belongs to the tile about
    // to be processed: wait for all of them, then start the next tile's loads into the
    // other buffer and compute (measured: a second tile in flight per wave, through
    // registers, is slower)
    const int step = NW * PV_WT;
    int t0 = gw * PV_WT;
    while (t0 < S) {
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        TI_ISSUE_FENCE();
        if (has_pos && pos >= t0 && pos < t0 + PV_WT) own_row(0, t0);
        int nt = t0 + step;
        if (nt < S) load_tile(1, nt);
        process(0, t0);
        if (nt >= S) break;
        t0 = nt;
        __builtin_amdgcn_s_waitcnt(0x0F70);
        TI_ISSUE_FENCE();
        if (has_pos && pos >= t0 && pos < t0 + PV_WT) own_row(1, t0);
        nt = t0 + step;
        if (nt < S) load_tile(0, nt);
        process(1, t0);
        t0 = nt;
    }
    if (has_pos && wave >= 2) {   // the new K / V row into the cache, from LDS
        const bool isv = wave == 3;
        const size_t rowq = ((size_t)pos * a.kvs + hk) * (HD / 4), rows = ((size_t)pos * a.nKv + hk) * NG;
        if (lane < HD / 4) (isv ? a.vq : a.kq)[rowq + lane] = (isv ? s_vw : s_kw)[lane];
        if (lane < NG) (isv ? a.vs : a.ks)[rows + lane] = (isv ? s_vsc : s_ksc)[lane];
    }
    __syncthreads();   // the tiles become s_red: no wave still reads them

    // wave state -> LDS: lane group q holds head q & 1 at dims 16 D + r16, D = 4 (q >> 1) + j,
    // as its rows 2 (j >> 1) (hi) and 2 (j >> 1) + 1 (lo); then (m, l) of each head in
    // natural-log units
    {
        float l32 = pv_row_sum(l_lane);
        l32 += ti_xor(l32, 32);
        const bool upper = kq >= 2;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i0 = 2 * (j >> 1);
            const float hi = upper ? O[4 + j][i0] : O[j][i0];
            const float lo = upper ? O[4 + j][i0 + 1] : O[j][i0 + 1];
            const int D = 4 * (kq >> 1) + j;
            if (sh < G) s_red[wave][0][sh * HD + 16 * D + r16] = (hi + lo) * (1.0f / 127.0f);
        }
        if (sh < G && r16 == 0 && kq < 2) {
            s_wml[wave][sh][0] = m_run * 0.6931471805599453f;
            s_wml[wave][sh][1] = l32;
        }
    }
    attn_merge_tail<HD, G, 1>(a, hk, w, NS, ntiles, valid, s_red, s_wml, s_ml, s_e, s_L, &s_last,
                              reinterpret_cast<float*>(&s_k[2][0][0]), epoch);
}
}  // namespace

// Fused decode attention; returns TI_ERR_INVALID for head shapes it does not cover
// (the caller then issues prep + split + combine).
// rope rows: cs[i] = cos(pos * theta^(-2i/hd)), cs[hd/2 + i] = sin(...), in f64 then f32
void ti_rope_row(float* cs, int pos, int hd, float theta) {
    for (int i = 0; i < hd / 2; i++) {
        double ang = (double)pos * pow((double)theta, -2.0 * (double)i / (double)hd);
        cs[i] = (float)cos(ang);
        cs[hd / 2 + i] = (float)sin(ang);
    }
}

// Splits per KV head of the fused decode attention over S positions when the caller leaves
// the count open: about 512 keys per split (four 32-key tiles per wave), at least 24 once
// the context passes 4096 (fewer workgroups leave CUs without a stream) and 16 below,
// at most 64. Measured on the Qwen3-1.7B step (8 KV heads, head_dim 128): within ~3% of
// the best count at every context from 1k to 32k, and up to 10% faster than 64 splits.
int ti_attn_decode_splits(int S) {
    // the grid is 8 x NS workgroups: 32 and 64 splits fill the 256 CUs once or twice over;
    // counts in between leave some CUs two workgroups and the rest one, and the step waits
    // for the CUs that stream twice (a sweep of the 1.7B step, 4k-32k, over 16-64 splits:
    // 32 best up to ~12k, 64 from ~16k; 1159 / 1003 tok/s at 16k for 32 / 33 splits)
    if (S <= 2048) return 16;
    return S <= 14336 ? 32 : 64;
}

int ti_attn_fused_launch(ti_ctx* c, const float* q, const float* k, const float* v, const uint16_t* qw,
                         const uint16_t* kw, uint32_t* kq, float* ks, uint32_t* vq, float* vs, float* out, int nHq,
                         int nKv, int hd, const int* dpos, int pos, int cap, float theta, float eps, int max_splits,
                         const float* rope_cur, uint32_t* oq, float* os, int kvs) {
    const int G = nHq / nKv;
    if (kvs < nKv) return ti_fail(TI_ERR_INVALID, "fused attention: %d code slots per position < %d KV heads", kvs, nKv);
    if (nKv > TI_ATTN_COUNTERS) return ti_fail(TI_ERR_INVALID, "fused attention: more than %d KV heads", TI_ATTN_COUNTERS);
    if (hd > TI_ATTN_HD_MAX) return ti_fail(TI_ERR_INVALID, "fused attention: hd=%d > %d", hd, TI_ATTN_HD_MAX);
    if (dpos && !rope_cur) return ti_fail(TI_ERR_INVALID, "fused attention: a device position needs its rope row");
    if (max_splits <= 0 || max_splits > ATTF_MAXS)   // a host position gives the context; a device one only the cache
        max_splits = dpos ? (cap > ATTF_LONG_CAP ? ATTF_SPLITS_LONG : ATTF_SPLITS_SHORT) : ti_attn_decode_splits(pos + 1);
    // no more splits than the cache has wave tiles for their 4 waves
    const int wt = 4 * (64 / (hd / 16));
    const int cap_splits = (cap + 4 * wt - 1) / (4 * wt);
    if (max_splits > cap_splits) max_splits = cap_splits;
    // without a device position, dpos/rope_cur point at a valid dummy (the spare sync words)
    const int* dp = dpos ? dpos : reinterpret_cast<const int*>(c->sync + TI_SYNC_DUMMY);
    const float* rc = rope_cur ? rope_cur : reinterpret_cast<const float*>(c->sync + TI_SYNC_DUMMY);
    AttnFArgs a = {q, k, v, qw, kw, kq, ks, vq, vs, out, c->attn_po, c->attn_ml, c->sync + TI_SYNC_ATTN, dp, rc,
                   dpos ? 1 : 0, pos, nKv, max_splits, cap, kvs, eps, oq, os, {}};
    if (!dpos) ti_rope_row(a.rope_row, pos, hd, theta);
    dim3 grid(nKv * max_splits);
#define AF(HD_, G_) \
    if (hd == HD_ && G == G_) { k_attn_fused_q8<HD_, G_><<<grid, 256, 0, c->stream>>>(a); TI_LAUNCHED("k_attn_fused_q8"); return TI_OK; }
    // head_dim 128 (the Qwen3 heads): Q K^T on the matrix cores
    if (hd == 128 && G == 2) { k_attn_fused_pv<2><<<grid, 256, 0, c->stream>>>(a); TI_LAUNCHED("k_attn_fused_pv"); return TI_OK; }
    if (hd == 128 && G == 1) { k_attn_fused_pv<1><<<grid, 256, 0, c->stream>>>(a); TI_LAUNCHED("k_attn_fused_pv"); return TI_OK; }
    AF(64, 2) AF(64, 1)
#undef AF
    return ti_fail(TI_ERR_INVALID, "fused attention: no kernel for hd=%d group=%d", hd, G);
}

int ti_fused_qkv_launch(ti_ctx*, const float*, const uint16_t*, float, int, int, const uint32_t* const*,
                        const uint16_t* const*, float* const*, const int*, uint32_t*, float*);

// The decode step's q/k/v projection and its attention as one launch (k_attn_fused_pv with
// QL > 0): rmsnormQ(x) -> q, k, v rows (int4 GEMV) -> attnPrep + split-KV attention +
// combine + quantQ8 of the output. Taken for head_dim 128, two query heads per KV head and
// H = 1024 or 2048 (QL = H / 32 lanes per row) when the whole grid can be resident at once
// (its workgroups wait for each other's rows); otherwise the q/k/v GEMV and the attention
// run as two launches, with the same results. ys: q, k and v row buffers ([nHq*hd],
// [nKv*hd] x 2), written by the two-launch path always and by the fused kernel when
// copy_rows is set; xq_out / xs_out: the normed x's int8 codes (or null).
bool ti_attn_qkv_ok(int nHq, int nKv, int hd, int H) {
    return hd == 128 && nKv > 0 && nHq == 2 * nKv && (H == 1024 || H == 2048) && nKv <= TI_ATTN_COUNTERS &&
           nKv * (nHq / nKv + 2) * hd <= TI_QKV_PUB_WORDS;
}

int ti_attn_qkv_launch(ti_ctx* c, const float* x, const uint16_t* in_norm, float in_eps, int H,
                       const uint32_t* const* packs, const uint16_t* const* scs, float* const* ys, int copy_rows,
                       uint32_t* xq_out, float* xs_out, const uint16_t* qw, const uint16_t* kw, uint32_t* kq,
                       float* ks, uint32_t* vq, float* vs, float* out, int nHq, int nKv, int hd, const int* dpos,
                       int cap, float theta, float eps, int max_splits, const float* rope_cur, uint32_t* oq,
                       float* os, int kvs) {
    auto two_launches = [&]() {
        const int Ns[3] = {nHq * hd, nKv * hd, nKv * hd};
        int rc = ti_fused_qkv_launch(c, x, in_norm, in_eps, H, 3, packs, scs, ys, Ns, xq_out, xs_out);
        if (!rc) rc = ti_attn_fused_launch(c, ys[0], ys[1], ys[2], qw, kw, kq, ks, vq, vs, out, nHq, nKv, hd, dpos, 0,
                                           cap, theta, eps, max_splits, rope_cur, oq, os, kvs);
        return rc;
    };
    if (c->qkv_separate || !ti_attn_qkv_ok(nHq, nKv, hd, H) || !dpos || !rope_cur || kvs < nKv) return two_launches();
    int NS = max_splits;
    if (NS <= 0 || NS > ATTF_MAXS) NS = cap > ATTF_LONG_CAP ? ATTF_SPLITS_LONG : ATTF_SPLITS_SHORT;
    const int wt = 4 * (64 / (hd / 16));
    const int cap_splits = (cap + 4 * wt - 1) / (4 * wt);   // as ti_attn_fused_launch clamps it
    if (NS > cap_splits) NS = cap_splits;
    // rows per unit: 4, or 8 where 4-row units would not fit in one round (at most 4 NS units,
    // one per wave of the head's workgroups), so that every unit is done in the first round
    // whenever NS >= 16 (and no row waits for a second); 2-row units at 64 splits, where they
    // also fit, measured 1% slower at 32k than 4-row ones (a wave's poll waits on more of
    // them). R rows per lane group, 64 / QL lane groups a wave
    const int QL = H / 32, G = 2;
    int RS = 4;
    while (RS < 8 && (G + 2) * hd / RS > 4 * NS) RS *= 2;
    const int QR = RS * QL / 64;
    const void* fn = nullptr;
#define QV(QL_, QR_) if (QL == QL_ && QR == QR_) fn = reinterpret_cast<const void*>(k_attn_fused_pv<2, QL_, QR_>);
    QV(32, 2) QV(32, 4) QV(64, 4) QV(64, 8)
#undef QV
    int per_cu = 0;
    if (fn) TI_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, 0));
    const long grid = (long)nKv * NS;
    if (!fn || grid > (long)per_cu * c->cus) return two_launches();
    AttnFArgs a = {nullptr, nullptr, nullptr, qw, kw, kq, ks, vq, vs, out, c->attn_po, c->attn_ml, c->sync + TI_SYNC_ATTN,
                   dpos, rope_cur, 1, 0, nKv, NS, cap, kvs, eps, oq, os, {}};
    a.nin = {x, in_norm, H, in_eps, xq_out, xs_out};
    for (int i = 0; i < 3; i++) {
        a.wpk[i] = reinterpret_cast<const uint4*>(packs[i]);
        a.wsc[i] = scs[i];
        a.qkv_copy[i] = copy_rows ? ys[i] : nullptr;
    }
    a.pub = c->qkv_pub;
    a.qkv_polls = c->qkv_polls >= 0 ? c->qkv_polls : ATTF_QKV_POLLS;
#define QV(QL_, QR_)                                                                      \
    if (QL == QL_ && QR == QR_) {                                                         \
        k_attn_fused_pv<2, QL_, QR_><<<dim3((unsigned)grid), 256, 0, c->stream>>>(a);       \
        TI_LAUNCHED("k_attn_fused_pv (q/k/v)");                                           \
        return TI_OK;                                                                     \
    }
    QV(32, 2) QV(32, 4) QV(64, 4) QV(64, 8)
#undef QV
    return two_launches();
}

extern "C" int ti_attn_step_q8(ti_ctx* c, const float* q, const float* k, const float* v, const uint16_t* qn_w,
                               const uint16_t* kn_w, uint32_t* kq, float* ks, uint32_t* vq, float* vs, float* out,
                               int nHq, int nKv, int hd, int pos, int cap, float theta, float eps, int max_splits,
                               uint32_t* out_q, float* out_s) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(q && k && v && qn_w && kn_w && kq && ks && vq && vs && out, "ti_attn_step_q8: null buffer");
    TI_REQUIRE(nKv > 0 && nHq % nKv == 0 && nHq <= TI_ATTN_HEADS_MAX, "ti_attn_step_q8: bad heads (nHq=%d nKv=%d)", nHq, nKv);
    TI_REQUIRE(pos >= 0 && pos < cap, "ti_attn_step_q8: pos %d outside the cache [0, %d)", pos, cap);
    TI_REQUIRE(al16(kq) && al16(vq), "ti_attn_step_q8: kq/vq must be 16-byte aligned");
    TI_REQUIRE(max_splits >= 0 && max_splits <= ATTF_MAXS, "ti_attn_step_q8: max_splits in [0, %d]", ATTF_MAXS);
    TI_REQUIRE((out_q == nullptr) == (out_s == nullptr), "ti_attn_step_q8: out_q and out_s go together");
    return ti_attn_fused_launch(c, q, k, v, qn_w, kn_w, kq, ks, vq, vs, out, nHq, nKv, hd, nullptr, pos, cap, theta, eps,
                                max_splits, nullptr, out_q, out_s, nKv);
}
