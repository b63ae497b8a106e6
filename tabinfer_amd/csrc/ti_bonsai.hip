// ti_bonsai.hip — the Bonsai-1.7B ternary decoder on the GPU: the native engine's forward
// (native/crates/n2-core/src/model.rs:349-501 with ops.rs) around the ternary GEMV.
//
// Per token, as model.rs computes it: embed (f16 row) -> per layer: rmsnorm, per-tensor
// int8 quantize (n2 quantize_act), q/k/v ternary GEMVs scaled by 1/scale, per-head
// qk-norm, split-half RoPE (theta 1e6), the post-RoPE key and the value appended to an
// f32 KV cache, GQA attention (softmax over 1/sqrt(hd)-scaled scores), quantize, o_proj,
// residual, rmsnorm, quantize, gate/up, SwiGLU, quantize, down, residual -> final rmsnorm,
// quantize, ternary lm_head scaled by 1/scale -> logits, argmax (ops::argmax: the lowest
// index on ties). The ternary GEMVs are the library's bit-exact kernels (k_tern.hip); the
// int8 codes are exact functions of their f32 inputs; every 1/scale product and residual
// add uses the reference's f32 operations in its order. The reductions (norm sums, the
// attention) run as trees, not the reference's sequential sums.
//
// The position lives on the device (the decode step is one graph, replayed per token):
// the step embeds hist[P], writes KV row P, and (with logits) puts the argmax in hist[P+1]
// and advances P.
#include "ti_internal.h"
#include <math.h>
#include <string.h>
#include <stdio.h>
#include <string>
#include <vector>

namespace {

constexpr int BN_THREADS = 1024;
constexpr int BN_AMAX_PARTS = 256;

// total of one float per thread over a 1024-thread workgroup (a tree; every thread gets it)
__device__ __forceinline__ float wg_sum_1024(float v, float* red) {
    v = ti_wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; w++) s += red[w];
    return s;
}

__device__ __forceinline__ float wg_max_1024(float v, float* red) {
    v = ti_wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < 16; w++) m = fmaxf(m, red[w]);
    return m;
}

// n2 quantize_act of v[n] held EPT per thread (tern.rs:206-222): scale = 127/amax (1 if
// amax = 0), a = clamp(round-half-away(v * scale), -127, 127), xsum per 64.
template <int EPT>
__device__ __forceinline__ void quant_n2(const float (&v)[EPT], int n, int8_t* __restrict__ act,
                                         int32_t* __restrict__ xsum, float* __restrict__ scale_out, float* red) {
    const int t = threadIdx.x;
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < EPT; i++)
        if (t + BN_THREADS * i < n) m = fmaxf(m, fabsf(v[i]));
    const float amax = wg_max_1024(m, red);
    const float scale = amax > 0.0f ? 127.0f / amax : 1.0f;
    if (t == 0) *scale_out = scale;
    // element e = t + 1024 i: its 64-block is e / 64, one wave's lanes cover one block
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = t + BN_THREADS * i;
        int q = 0;
        if (e < n) {
            float r = roundf(v[i] * scale);
            r = fminf(fmaxf(r, -127.0f), 127.0f);
            q = (int)r;
            act[e] = (int8_t)q;
        }
        const int sum = ti_wave_sum_i(q);
        if ((t & 63) == 0 && e < n) xsum[e / 64] = sum;
    }
}

// ---- embed: x = f32(emb[hist[P]]) ---------------------------------------------------------
__global__ void k_bn_embed(const uint32_t* __restrict__ hist, const int* __restrict__ dpos, const uint16_t* __restrict__ emb,
                           float* __restrict__ x, int H, int vocab, int cap) {
    const int P = *dpos;
    if (P >= cap) return;                              // past the cache: the step writes nothing
    uint32_t id = hist[P];
    id = id < (uint32_t)vocab ? id : (uint32_t)(vocab - 1);
    for (int i = threadIdx.x; i < H; i += blockDim.x) x[i] = ti_h2f(emb[(size_t)id * H + i]);
}

// ---- residual add + rmsnorm + quantize (one workgroup) --------------------------------------
// with add: x[i] = x[i] + add[i] * (1 / add_scale) (model.rs linear's scaling, then the
// residual add); then xn = x * (1 / sqrt(mean(x^2) + eps)) * w (ops.rs:14-22) and the n2
// quantizer of xn.
template <int EPT>
__global__ __launch_bounds__(BN_THREADS) void k_bn_norm_quant(float* __restrict__ x, const float* __restrict__ add,
                                                             const float* __restrict__ add_scale, const float* __restrict__ w,
                                                             float eps, int H, float* __restrict__ xn_out,
                                                             int8_t* __restrict__ act, int32_t* __restrict__ xsum,
                                                             float* __restrict__ scale_out) {
    __shared__ float red[16];
    const int t = threadIdx.x;
    float v[EPT], a[EPT], wv[EPT];
    // every load first (clamped indices), so they are in flight together
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = min(t + BN_THREADS * i, H - 1);
        v[i] = x[e];
        a[i] = add ? add[e] : 0.0f;
        wv[i] = w[e];
    }
    const float inv_add = add ? 1.0f / *add_scale : 0.0f;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = t + BN_THREADS * i;
        if (e < H) {
            float xe = v[i];
            if (add) {
                const float d = a[i] * inv_add;
                xe = xe + d;
                x[e] = xe;
            }
            v[i] = xe;
            ss = ss + xe * xe;
        } else {
            v[i] = 0.0f;
        }
    }
    const float mean = wg_sum_1024(ss, red) / (float)H;
    const float inv = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = t + BN_THREADS * i;
        if (e < H) {
            v[i] = v[i] * inv * wv[i];
            if (xn_out) xn_out[e] = v[i];
        }
    }
    quant_n2<EPT>(v, H, act, xsum, scale_out, red);
}

// ---- SwiGLU of the scaled gate/up + quantize (ops.rs:110-117) ---------------------------------
template <int EPT>
__global__ __launch_bounds__(BN_THREADS) void k_bn_swiglu_quant(const float* __restrict__ graw, const float* __restrict__ uraw,
                                                               const float* __restrict__ gu_scale, int n,
                                                               float* __restrict__ swi_out, int8_t* __restrict__ act,
                                                               int32_t* __restrict__ xsum, float* __restrict__ scale_out) {
    __shared__ float red[16];
    float g[EPT], u[EPT], v[EPT];
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = min((int)threadIdx.x + BN_THREADS * i, n - 1);
        g[i] = graw[e];
        u[i] = uraw[e];
    }
    const float inv = 1.0f / *gu_scale;
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = threadIdx.x + BN_THREADS * i;
        v[i] = 0.0f;
        if (e < n) {
            const float gg = g[i] * inv;
            const float uu = u[i] * inv;
            v[i] = (gg / (1.0f + expf(-gg))) * uu;
            if (swi_out) swi_out[e] = v[i];
        }
    }
    quant_n2<EPT>(v, n, act, xsum, scale_out, red);
}

// ---- GQA attention over the f32 cache (model.rs:421-447) ------------------------------------
// keys per attention workgroup for a cache of cap positions: 64, or more for longer caches, so
// that the grid (8 KV heads x splits) stays within one round of resident workgroups (three
// 4-wave workgroups per CU) up to 12288 positions, and the split count within 160
constexpr int BN_MAX_CTX = 256 * 160;
__host__ __device__ inline int bn_chunk(int cap) {
    return cap <= 64 * 96 ? 64 : (cap <= 128 * 96 ? 128 : 256);
}

// workgroup (KV head hk, split of CH keys), the G = 2 query heads of hk (hd 128):
//  prologue (model.rs:399-418): q of both heads scaled by 1/scale, per-head RMSNorm (the sum
//          of squares as a 64..1 tree), the q_norm weight and split-half RoPE at position P
//          (the rotary row kept beside the device position), into LDS (every workgroup), with
//          the first 64 keys' K and V rows already in flight; the workgroup whose split holds
//          P also forms K (scaled, k_norm, RoPE) and V (scaled) of hk at P, stores them into
//          the cache for later tokens and uses them from LDS for its own key P (no other
//          workgroup reads row P);
//  scores: 4 lanes per key, 32 dims each (8 float4 loads a lane, in flight together), a quad
//          sum, 64 keys per pass;
//  max / exp / sum over the split's keys;
//  P V: lane (key group kg = t / 32, dims 4 (t % 32) ..) over keys kg, kg + 8, .. (one float4
//       of V serves both heads), then the 8 key-group partials summed in order;
//  partials (o, m, l) per (query head, split).
// RMSNorm of one head row held one element per thread (the 128 threads with act, element
// i, LDS slots from `base`): the sum of squares as a 64..1 tree in red, then split-half RoPE
// with the rotary row's cos c and sin s of element i's pair. Every thread of the workgroup
// calls it (it holds barriers); only those with act write.
__device__ __forceinline__ float bn_head_norm_rope(float a, int i, float nw, float c, float s, float eps, float* red,
                                                   float* y, int base, bool act) {
    constexpr int HD = 128, half = HD / 2;
    if (act) red[base + i] = a * a;
    __syncthreads();
    for (int st = 64; st > 0; st >>= 1) {
        if (act && i < st) red[base + i] = red[base + i] + red[base + i + st];
        __syncthreads();
    }
    const float mean = red[base] / (float)HD;
    const float rinv = 1.0f / sqrtf(mean + eps);
    if (act) y[base + i] = a * rinv * nw;
    __syncthreads();
    const int j = i < half ? i : i - half;
    const float x0 = y[base + j], x1 = y[base + half + j];
    return i < half ? x0 * c - x1 * s : x1 * c + x0 * s;
}

template <int CH>
__global__ __launch_bounds__(256) void k_bn_attn(const float* __restrict__ qraw, const float* __restrict__ kraw,
                                                 const float* __restrict__ vraw, const float* __restrict__ act_scale,
                                                 const float* __restrict__ qn, const float* __restrict__ kn,
                                                 const float* __restrict__ rope_cur, float eps, float* __restrict__ kc,
                                                 float* __restrict__ vc, const int* __restrict__ dpos, int nKv,
                                                 float* __restrict__ po, float* __restrict__ pml, int ns_stride, int cap) {
    constexpr int G = 2, HD = 128, half = HD / 2;
    __shared__ float sc[G][CH];
    __shared__ float4 so[8][G][HD / 4];
    __shared__ float red[G][4];
    __shared__ __align__(16) float s_q[G][HD];
    __shared__ __align__(16) float s_kp[HD];           // K and V of row P (the own split)
    __shared__ __align__(16) float s_vp[HD];
    __shared__ float s_red[G * HD], s_y[G * HD];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hk = blockIdx.x % nKv, split = blockIdx.x / nKv;
    const int c0 = split * CH;
    const size_t kvd = (size_t)nKv * HD;
    const float scale = 1.0f / sqrtf((float)HD);
    const int qd = t & 3;
    const int pg = t >> 7, pi = t & 127;
    const int kg = t >> 5, d4 = t & 31;
    // ---- the prologue's loads: the device position first (a vector load: as a scalar one it
    // would hold every vector load behind the kernel arguments' wait), then raw q (thread t:
    // head t / 128, dim t % 128), the activation scale, the norm weights, the rotary row of
    // the device position (kept beside it by the kernels that move it) and the new token's
    // raw K (threads 0..127) or V (128..255) row of hk, none of which depends on the
    // position, so all of them arrive in one round trip; then a split past the context
    // leaves, and the others request the first 64 keys' V rows (as the P V pass reads them)
    // and, for one-pass splits, K rows (4 lanes a key, 32 dims each) before the norm.
    const uint32_t praw = ti_pub_load(reinterpret_cast<const uint32_t*>(dpos));
    float qr = qraw[(size_t)(hk * G + pg) * HD + pi];
    float asc = ti_pub_load(act_scale);                 // a vector load: no scalar wait before the others
    float qnw = qn[pi], knw = kn[pi];
    const int jr = pi < half ? pi : pi - half;
    float rc = rope_cur[jr], rs = rope_cur[half + jr];
    float kvr = (pg == 0 ? kraw : vraw)[(size_t)hk * HD + pi];
    uint32_t pv = praw;
    // every load above is issued, and has landed, before the exit test (the compiler would
    // otherwise sink them past it, behind the position's round trip)
    asm volatile("" : "+v"(pv), "+v"(qr), "+v"(asc), "+v"(qnw), "+v"(knw), "+v"(rc), "+v"(rs), "+v"(kvr));
    const int P = (int)pv;
    const int S = min(P + 1, cap);
    if (c0 >= S) return;                               // the merge reads splits below ceil(S / CH) only
    const int n = min(CH, S - c0);
    const bool own = P < cap && P < c0 + CH;           // this split holds row P: it writes K, V there
    // the first pass's K rows are prefetched only when the split is one pass (CH = 64): with
    // more, the prefetched rows and the second pass's together cost a wave per SIMD
    constexpr bool KPRE = CH == 64;
    float4 kpre[8], vpre[8];
    if (KPRE) {
        const int j = t >> 2;
        const float4* kr = reinterpret_cast<const float4*>(kc + (size_t)(c0 + (j < n ? j : n - 1)) * kvd +
                                                           (size_t)hk * HD + qd * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) kpre[i] = kr[i];
    }
    const float4* vb = reinterpret_cast<const float4*>(vc + (size_t)c0 * kvd + (size_t)hk * HD) + d4;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int j = kg + 8 * i;
        vpre[i] = vb[(size_t)(j < n ? j : n - 1) * (kvd / 4)];
    }
    TI_ISSUE_FENCE();
    const float inv = 1.0f / asc;
    s_q[pg][pi] = bn_head_norm_rope(qr * inv, pi, qnw, rc, rs, eps, s_red, s_y, pg * HD, true);
    if (own) {   // K (threads 0..127) and V (128..255) of hk at P (model.rs:405-418): into the cache
        // for later tokens, and through LDS for this split's own key P (its cache row may not
        // have landed before the loads above, which were issued before it was formed)
        const size_t row = (size_t)P * kvd + (size_t)hk * HD + pi;
        __syncthreads();   // every thread has read the q tree's slots
        const float kr = bn_head_norm_rope(kvr * inv, pi, knw, rc, rs, eps, s_red, s_y, 0, pg == 0);
        if (pg == 0) {
            kc[row] = kr;
            s_kp[pi] = kr;
        } else {
            const float vv = kvr * inv;
            vc[row] = vv;
            s_vp[pi] = vv;
        }
    }
    __syncthreads();
    float4 q[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int i = 0; i < 8; i++) q[g][i] = reinterpret_cast<const float4*>(&s_q[g][qd * 32])[i];
    const int jp = own ? P - c0 : -1;                  // the split's key P, if it holds it
    for (int k0 = 0; k0 < n; k0 += 64) {
        const int j = k0 + (t >> 2);
        const int key = c0 + (j < n ? j : n - 1);
        float4 kv[8];
        if (KPRE && k0 == 0) {
#pragma unroll
            for (int i = 0; i < 8; i++) kv[i] = kpre[i];
        } else {
            const float4* kr = reinterpret_cast<const float4*>(kc + (size_t)key * kvd + (size_t)hk * HD + qd * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) kv[i] = kr[i];
        }
        if (j == jp)
#pragma unroll
            for (int i = 0; i < 8; i++) kv[i] = reinterpret_cast<const float4*>(&s_kp[qd * 32])[i];
        float part[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                s = s + kv[i].x * q[g][i].x;
                s = s + kv[i].y * q[g][i].y;
                s = s + kv[i].z * q[g][i].z;
                s = s + kv[i].w * q[g][i].w;
            }
            part[g] = s;
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            part[g] += ti_xor(part[g], 1);
            part[g] += ti_xor(part[g], 2);
        }
        if (qd == 0 && j < n)
#pragma unroll
            for (int g = 0; g < G; g++) sc[g][j] = part[g] * scale;
    }
    __syncthreads();
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float v = -INFINITY;
        for (int j = t; j < n; j += 256) v = fmaxf(v, sc[g][j]);
        v = ti_wave_max(v);
        if (lane == 0) red[g][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) m[g] = fmaxf(fmaxf(red[g][0], red[g][1]), fmaxf(red[g][2], red[g][3]));
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) {
        float s = 0.0f;
        for (int j = t; j < n; j += 256) {
            const float p = expf(sc[g][j] - m[g]);
            sc[g][j] = p;
            s += p;
        }
        s = ti_wave_sum(s);
        if (lane == 0) red[g][wave] = s;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) l[g] = (red[g][0] + red[g][1]) + (red[g][2] + red[g][3]);
    float4 o[G];
#pragma unroll
    for (int g = 0; g < G; g++) o[g] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 vp = reinterpret_cast<const float4*>(s_vp)[d4];   // used only by the own split
#pragma unroll
    for (int i = 0; i < 8; i++) {                      // keys kg + 8i < 64: the prefetched rows
        const int j = kg + 8 * i;
        if (j < n) {
            const float4 vv = j == jp ? vp : vpre[i];
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float p = sc[g][j];
                o[g].x = fmaf(p, vv.x, o[g].x);
                o[g].y = fmaf(p, vv.y, o[g].y);
                o[g].z = fmaf(p, vv.z, o[g].z);
                o[g].w = fmaf(p, vv.w, o[g].w);
            }
        }
    }
#pragma unroll 4
    for (int j = kg + 64; j < n; j += 8) {
        const float4 vl = vb[(size_t)j * (kvd / 4)];    // always loaded: the select below stays a
        const bool mine = j == jp;                         // value select, and the loads pipeline
        const float4 vv = make_float4(mine ? vp.x : vl.x, mine ? vp.y : vl.y, mine ? vp.z : vl.z, mine ? vp.w : vl.w);
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float p = sc[g][j];
            o[g].x = fmaf(p, vv.x, o[g].x);
            o[g].y = fmaf(p, vv.y, o[g].y);
            o[g].z = fmaf(p, vv.z, o[g].z);
            o[g].w = fmaf(p, vv.w, o[g].w);
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) so[kg][g][d4] = o[g];
    __syncthreads();
    {
        const int g = t >> 7, d = t & 127;
        const float* sof = reinterpret_cast<const float*>(so);
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) acc += sof[(k * G + g) * HD + d];
        const size_t slot = (size_t)(hk * G + g) * ns_stride + split;
        po[slot * HD + d] = acc;
        if (d == 0) {
            pml[slot * 2] = g == 0 ? m[0] : m[1];
            pml[slot * 2 + 1] = g == 0 ? l[0] : l[1];
        }
    }
}

// out[h][d] = sum_i o_i e^(m_i - M) / sum_i l_i e^(m_i - M) over the splits that hold keys,
// then the n2 quantizer of the whole output. One workgroup per KV head (its G = 2 query
// heads), 1024 threads: thread (quarter q, head g, dim d) loads its quarter of the splits'
// partials (every load in flight at once, before the split weights are known: one memory
// round trip), waves 0 and 1 find their head's M, the weights e^(m_i - M) and L, and each
// (g, d) adds its four quarter sums in order. The last of the nKv workgroups to finish
// quantizes the whole output (the per-tensor scale needs every element); the head outputs
// reach it through device-scope stores and loads, and it resets the counter.
constexpr int BN_MERGE_SPLITS = 160;   // split slots per head: bn_chunk keeps a cache of BN_MAX_CTX within them
constexpr int BN_MQ = BN_MERGE_SPLITS / 4;   // splits per quarter, at most

template <int EPT>
__global__ __launch_bounds__(BN_THREADS) void k_bn_merge_quant(const float* __restrict__ po, const float* __restrict__ pml,
                                                              const int* __restrict__ dpos, int ns_stride, int nq,
                                                              int chunk, float* __restrict__ out, int8_t* __restrict__ act,
                                                              int32_t* __restrict__ xsum, float* __restrict__ scale_out,
                                                              uint32_t* __restrict__ counter, int cap) {
    constexpr int HD = 128, G = 2;
    __shared__ float red[16];
    __shared__ float s_w[G][BN_MERGE_SPLITS];
    __shared__ float s_l[G];
    __shared__ float s_part[4][G][HD];
    __shared__ int s_last;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int q = t >> 8, g = (t >> 7) & 1, d = t & 127;
    const int hk = blockIdx.x;
    const int ns = (min(*dpos + 1, cap) + chunk - 1) / chunk;
    // this thread's partials: splits q, q + 4, .. of query head 2 hk + g
    const float* ob = po + (size_t)(hk * G + g) * ns_stride * HD + d;
    float ov[BN_MQ];
#pragma unroll
    for (int i = 0; i < BN_MQ; i++) {
        const int k = q + 4 * i;
        ov[i] = k < ns ? ob[(size_t)k * HD] : 0.0f;
    }
    if (wave < G) {
        const float* ml = pml + (size_t)(hk * G + wave) * ns_stride * 2;
        float mk[BN_MERGE_SPLITS / 64 + 1], lk[BN_MERGE_SPLITS / 64 + 1];
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i * 64 < BN_MERGE_SPLITS; i++) {
            const int k = lane + 64 * i;
            mk[i] = k < ns ? ml[2 * k] : -INFINITY;
            lk[i] = k < ns ? ml[2 * k + 1] : 0.0f;
            M = fmaxf(M, mk[i]);
        }
        M = ti_wave_max(M);
        float L = 0.0f;
#pragma unroll
        for (int i = 0; i * 64 < BN_MERGE_SPLITS; i++) {
            const int k = lane + 64 * i;
            if (k < ns) {
                const float e2 = expf(mk[i] - M);
                s_w[wave][k] = e2;
                L += lk[i] * e2;
            }
        }
        L = ti_wave_sum(L);
        if (lane == 0) s_l[wave] = L;
    }
    __syncthreads();
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < BN_MQ; i++) {
        const int k = q + 4 * i;
        if (k < ns) o = fmaf(ov[i], s_w[g][k], o);
    }
    s_part[q][g][d] = o;
    __syncthreads();
    if (q == 0) {
        const float v = ((s_part[0][g][d] + s_part[1][g][d]) + (s_part[2][g][d] + s_part[3][g][d])) / s_l[g];
        ti_pub_store(out + (size_t)(hk * G + g) * HD + d, v);
    }
    if (!act) return;                                  // the next launch quantizes out
    ti_stores_done();
    __syncthreads();
    if (t == 0) s_last = ti_arrive(counter) == gridDim.x - 1;
    __syncthreads();
    if (!s_last) return;
    float v[EPT];
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = t + BN_THREADS * i;
        v[i] = e < nq ? ti_pub_load(out + e) : 0.0f;
    }
    quant_n2<EPT>(v, nq, act, xsum, scale_out, red);
    if (t == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- logits = raw * (1 / scale), argmax (ops::argmax: larger wins, the lower index on ties,
// only values above -inf) in two stages; the second writes hist[P + 1] and advances P.
__device__ __forceinline__ void n2_take(float& v, int& i, float v2, int i2) {
    if (v2 > v || (v2 == v && v2 > -INFINITY && i2 < i)) {
        v = v2;
        i = i2;
    }
}

__global__ __launch_bounds__(256) void k_bn_logits(const float* __restrict__ raw, const float* __restrict__ scale, int N,
                                                   float* __restrict__ logits, float* __restrict__ pv, int* __restrict__ pi) {
    __shared__ float sv[256];
    __shared__ int si[256];
    const float inv = 1.0f / *scale;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < N; i += gridDim.x * 256) {
        const float v = raw[i] * inv;
        logits[i] = v;
        n2_take(bv, bi, v, i);
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            float v = sv[threadIdx.x];
            int i = si[threadIdx.x];
            n2_take(v, i, sv[threadIdx.x + s], si[threadIdx.x + s]);
            sv[threadIdx.x] = v;
            si[threadIdx.x] = i;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = sv[0];
        pi[blockIdx.x] = si[0];
    }
}

__global__ __launch_bounds__(BN_AMAX_PARTS) void k_bn_argmax(const float* __restrict__ pv, const int* __restrict__ pi, int parts,
                                                            uint32_t* __restrict__ hist, int* __restrict__ dpos, int cap,
                                                            const float* __restrict__ rope, float* __restrict__ rope_cur,
                                                            int hd) {
    __shared__ float sv[BN_AMAX_PARTS];
    __shared__ int si[BN_AMAX_PARTS];
    const int t = threadIdx.x;
    const int P = *dpos;   // every thread, before thread 0 advances it (barriers below)
    sv[t] = t < parts ? pv[t] : -INFINITY;
    si[t] = t < parts ? pi[t] : 0x7fffffff;
    __syncthreads();
    for (int s = BN_AMAX_PARTS / 2; s > 0; s >>= 1) {
        if (t < s) {
            float v = sv[t];
            int i = si[t];
            n2_take(v, i, sv[t + s], si[t + s]);
            sv[t] = v;
            si[t] = i;
        }
        __syncthreads();
    }
    if (t == 0) {
        if (P + 1 <= cap) hist[P + 1] = (uint32_t)(sv[0] > -INFINITY ? si[0] : 0);
        *dpos = P + 1;
    }
    for (int i = t; i < hd; i += BN_AMAX_PARTS)
        if (P + 1 < cap) rope_cur[i] = rope[(size_t)(P + 1) * hd + i];
}

// device position + 1 and its rotary row (one workgroup, hd threads or more)
__global__ void k_bn_advance(int* __restrict__ dpos, const float* __restrict__ rope, float* __restrict__ rope_cur, int hd,
                             int cap) {
    const int P = *dpos;
    __syncthreads();   // every thread has read it
    if (threadIdx.x == 0) *dpos = P + 1;
    if ((int)threadIdx.x < hd && P + 1 < cap) rope_cur[threadIdx.x] = rope[(size_t)(P + 1) * hd + threadIdx.x];
}
// device position := pos, and its rotary row
__global__ void k_bn_set_pos(int* __restrict__ dpos, int pos, const float* __restrict__ rope, float* __restrict__ rope_cur,
                             int hd, int cap) {
    if (threadIdx.x == 0) *dpos = pos;
    if ((int)threadIdx.x < hd && pos < cap) rope_cur[threadIdx.x] = rope[(size_t)pos * hd + threadIdx.x];
}

__global__ void k_bn_copy_u32(const uint32_t* __restrict__ s, uint32_t* __restrict__ d, long n) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) d[i] = s[i];
}

struct TLin {
    uint8_t* codes = nullptr;
    float* scales = nullptr;
    int N = 0, K = 0;
};
struct BLayer {
    TLin q, k, v, o, gate, up, down;
    float *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    float *kc = nullptr, *vc = nullptr;
};

}  // namespace

struct ti_bonsai {
    ti_bonsai_config cfg;
    std::vector<BLayer> L;
    uint16_t* embed = nullptr;
    float* final_norm = nullptr;
    TLin lm;
    float *x, *x2, *xn, *qraw, *kraw, *vraw, *attn, *oraw, *graw, *uraw, *swi, *draw, *lraw, *logits;
    int8_t* act;
    int32_t* xsum;
    float* scales;        // [4]: a (input norm), b (attention), c (post norm), d (swi)
    float *po, *pml;      // attention split partials
    float* amax_v;
    int* amax_i;
    uint32_t* hist;
    int* dpos;
    float* rope;          // [max_ctx][head_dim]: cos then sin of each position (ops.rs rope_table)
    float* rope_cur;      // the row of the device position, kept in step with dpos
    uint32_t* trace = nullptr;
    std::vector<void*> allocs;
};

// ---- the parity trace (ti_bonsai_trace) -----------------------------------------------------
namespace {
enum BField { B_X_IN, B_XN, B_A_ACT, B_A_SCALE, B_Q, B_K, B_V, B_ATTN, B_B_ACT, B_B_SCALE, B_X_MID, B_XN2, B_C_ACT,
              B_C_SCALE, B_G, B_U, B_SWI, B_D_ACT, B_D_SCALE, B_D, B_NFIELDS };
size_t bfield_words(const ti_bonsai_config& C, int f) {
    const size_t H = C.hidden, I = C.intermediate, nq = (size_t)C.n_heads * C.head_dim, nkv = (size_t)C.n_kv_heads * C.head_dim;
    switch (f) {
        case B_X_IN: case B_XN: case B_X_MID: case B_XN2: case B_D: return H;
        case B_A_ACT: case B_C_ACT: return H / 4;
        case B_Q: case B_ATTN: return nq;
        case B_B_ACT: return nq / 4;
        case B_K: case B_V: return nkv;
        case B_G: case B_U: case B_SWI: return I;
        case B_D_ACT: return I / 4;
        default: return 1;    // the scales
    }
}
size_t blayer_words(const ti_bonsai_config& C) {
    size_t w = 0;
    for (int f = 0; f < B_NFIELDS; f++) w += bfield_words(C, f);
    return w;
}
}  // namespace

static uint32_t* bslot(ti_bonsai* m, int layer, int f) {
    size_t off = (size_t)layer * blayer_words(m->cfg);
    for (int g = 0; g < f; g++) off += bfield_words(m->cfg, g);
    return m->trace + off;
}

static int bput(ti_ctx* c, ti_bonsai* m, int layer, int f, const void* src) {
    if (!m->trace) return TI_OK;
    const long n = (long)bfield_words(m->cfg, f);
    k_bn_copy_u32<<<(unsigned)((n + 255) / 256 < 256 ? (n + 255) / 256 : 256), 256, 0, c->stream>>>(
        static_cast<const uint32_t*>(src), bslot(m, layer, f), n);
    TI_LAUNCHED("k_bn_copy_u32 (trace)");
    return TI_OK;
}

static int bmk(ti_bonsai* m, void** p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 4);
    if (e != hipSuccess) return ti_hip_fail(e, "ti_bonsai_create hipMalloc");
    m->allocs.push_back(*p);
    return TI_OK;
}

static void brelease(ti_bonsai* m) {
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
}

extern "C" int ti_bonsai_create(ti_ctx* c, const ti_bonsai_config* cfg, ti_bonsai** out) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(cfg && out, "ti_bonsai_create: null argument");
    *out = nullptr;
    const ti_bonsai_config& C = *cfg;
    TI_REQUIRE(C.layers > 0 && C.hidden > 0 && C.intermediate > 0 && C.n_heads > 0 && C.n_kv_heads > 0 && C.vocab > 0 &&
               C.max_ctx > 0 && C.n_heads % C.n_kv_heads == 0, "ti_bonsai_create: bad config");
    TI_REQUIRE(C.hidden % 1024 == 0 && C.hidden <= 8192 && C.intermediate % 1024 == 0 && C.intermediate <= 8192,
               "ti_bonsai_create: hidden and intermediate must be multiples of 1024, at most 8192");
    TI_REQUIRE(C.head_dim == 128 && C.n_heads / C.n_kv_heads == 2 && (C.n_heads * C.head_dim) % 1024 == 0 &&
               C.n_heads * C.head_dim <= 8192, "ti_bonsai_create: the decoder covers head_dim 128 with 2 query heads per KV head");
    TI_REQUIRE(C.max_ctx <= BN_MAX_CTX, "ti_bonsai_create: max_ctx %d is above the decoder's %d positions", C.max_ctx,
               BN_MAX_CTX);
    TI_REQUIRE(!c->capturing, "ti_bonsai_create: not during graph capture");
    TI_HIP(hipSetDevice(c->device));
    ti_bonsai* m = new ti_bonsai();
    m->cfg = C;
    const int H = C.hidden, I = C.intermediate, hd = C.head_dim;
    const int nq = C.n_heads * hd, nkv = C.n_kv_heads * hd;
    int rc = 0;
    auto lin = [&](TLin& l, int N, int K) {
        l.N = N;
        l.K = K;
        int r = bmk(m, (void**)&l.codes, (size_t)N * K / 4);
        if (!r) r = bmk(m, (void**)&l.scales, (size_t)N * (K / 64) * 4);
        return r;
    };
    m->L.resize(C.layers);
    const size_t kvf = (size_t)C.max_ctx * nkv * 4;
    for (int l = 0; l < C.layers && !rc; l++) {
        BLayer& y = m->L[l];
        rc = lin(y.q, nq, H); if (!rc) rc = lin(y.k, nkv, H); if (!rc) rc = lin(y.v, nkv, H);
        if (!rc) rc = lin(y.o, H, nq); if (!rc) rc = lin(y.gate, I, H); if (!rc) rc = lin(y.up, I, H);
        if (!rc) rc = lin(y.down, H, I);
        if (!rc) rc = bmk(m, (void**)&y.in_norm, H * 4);
        if (!rc) rc = bmk(m, (void**)&y.post_norm, H * 4);
        if (!rc) rc = bmk(m, (void**)&y.q_norm, hd * 4);
        if (!rc) rc = bmk(m, (void**)&y.k_norm, hd * 4);
        if (!rc) rc = bmk(m, (void**)&y.kc, kvf);
        if (!rc) rc = bmk(m, (void**)&y.vc, kvf);
    }
    if (!rc) rc = bmk(m, (void**)&m->embed, (size_t)C.vocab * H * 2);
    if (!rc) rc = bmk(m, (void**)&m->final_norm, H * 4);
    if (!rc) rc = lin(m->lm, C.vocab, H);
    const int widest = I > H ? (I > nq ? I : nq) : (H > nq ? H : nq);
    const int nsplit = (C.max_ctx + bn_chunk(C.max_ctx) - 1) / bn_chunk(C.max_ctx);
    struct { float** p; size_t n; } fb[] = {{&m->x, (size_t)H}, {&m->x2, (size_t)H}, {&m->xn, (size_t)H}, {&m->qraw, (size_t)nq},
                                            {&m->kraw, (size_t)nkv}, {&m->vraw, (size_t)nkv},
                                            {&m->attn, (size_t)nq}, {&m->oraw, (size_t)H}, {&m->graw, (size_t)I},
                                            {&m->uraw, (size_t)I}, {&m->swi, (size_t)I}, {&m->draw, (size_t)H},
                                            {&m->lraw, (size_t)C.vocab}, {&m->logits, (size_t)C.vocab}, {&m->scales, 4},
                                            {&m->po, (size_t)C.n_heads * nsplit * hd}, {&m->pml, (size_t)C.n_heads * nsplit * 2},
                                            {&m->amax_v, BN_AMAX_PARTS}};
    for (auto& f : fb) if (!rc) rc = bmk(m, (void**)f.p, f.n * 4);
    if (!rc) rc = bmk(m, (void**)&m->act, (size_t)widest);
    if (!rc) rc = bmk(m, (void**)&m->xsum, (size_t)widest / 64 * 4);
    if (!rc) rc = bmk(m, (void**)&m->amax_i, BN_AMAX_PARTS * 4);
    if (!rc) rc = bmk(m, (void**)&m->hist, (size_t)(C.max_ctx + 1) * 4);
    if (!rc) rc = bmk(m, (void**)&m->dpos, 4);
    if (!rc) rc = bmk(m, (void**)&m->rope, (size_t)C.max_ctx * hd * 4);
    if (!rc) rc = bmk(m, (void**)&m->rope_cur, (size_t)hd * 4);
    if (!rc) {
        // ops.rs:79-90 in f32 with the platform's powf / cosf / sinf, the functions Rust's
        // f32::powf and sin_cos call on Linux
        std::vector<float> tab((size_t)C.max_ctx * hd);
        const int half = hd / 2;
        for (int p = 0; p < C.max_ctx; p++)
            for (int i = 0; i < half; i++) {
                const float e = -((float)(2 * i)) / (float)hd;
                const float ang = (float)p * powf(C.rope_theta, e);
                tab[(size_t)p * hd + i] = cosf(ang);
                tab[(size_t)p * hd + half + i] = sinf(ang);
            }
        hipError_t e = hipMemcpy(m->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(m->rope_cur, tab.data(), (size_t)hd * 4, hipMemcpyHostToDevice);   // position 0
        if (e == hipSuccess) e = hipMemset(m->hist, 0, (size_t)(C.max_ctx + 1) * 4);
        if (e == hipSuccess) e = hipMemset(m->dpos, 0, 4);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) rc = ti_hip_fail(e, "ti_bonsai_create set-up");
    }
    if (rc) { brelease(m); return rc; }
    *out = m;
    return TI_OK;
}

extern "C" int ti_bonsai_destroy(ti_ctx* c, ti_bonsai* m) {
    TI_CHECK_CTX(c);
    if (!m) return TI_OK;
    TI_REQUIRE(!c->capturing, "ti_bonsai_destroy: not during graph capture");
    TI_HIP(hipStreamSynchronize(c->stream));
    brelease(m);
    return TI_OK;
}

// Tensor names and kinds are the container's (native/tools/pack_bin.py; model.rs:275-304):
// ternary projections and lm_head return codes + scales, norms f32, the embedding f16.
extern "C" int ti_bonsai_tensor(ti_bonsai* m, const char* name, void** data, size_t* data_bytes, void** scales,
                                size_t* scale_bytes) {
    TI_REQUIRE(m && name && data && data_bytes, "ti_bonsai_tensor: null argument");
    const ti_bonsai_config& C = m->cfg;
    *data = nullptr;
    *data_bytes = 0;
    if (scales) *scales = nullptr;
    if (scale_bytes) *scale_bytes = 0;
    auto vec = [&](void* p, size_t bytes) { *data = p; *data_bytes = bytes; return TI_OK; };
    auto lin = [&](TLin& l) {
        *data = l.codes;
        *data_bytes = (size_t)l.N * l.K / 4;
        if (scales) *scales = l.scales;
        if (scale_bytes) *scale_bytes = (size_t)l.N * (l.K / 64) * 4;
        return TI_OK;
    };
    std::string s(name);
    if (s == "model.embed_tokens.weight") return vec(m->embed, (size_t)C.vocab * C.hidden * 2);
    if (s == "model.norm.weight") return vec(m->final_norm, (size_t)C.hidden * 4);
    if (s == "lm_head.weight") return lin(m->lm);
    int l = -1;
    char rest[128] = {0};
    if (sscanf(name, "model.layers.%d.%127s", &l, rest) == 2 && l >= 0 && l < C.layers) {
        BLayer& y = m->L[l];
        std::string r(rest);
        if (r == "input_layernorm.weight") return vec(y.in_norm, (size_t)C.hidden * 4);
        if (r == "post_attention_layernorm.weight") return vec(y.post_norm, (size_t)C.hidden * 4);
        if (r == "self_attn.q_norm.weight") return vec(y.q_norm, (size_t)C.head_dim * 4);
        if (r == "self_attn.k_norm.weight") return vec(y.k_norm, (size_t)C.head_dim * 4);
        if (r == "self_attn.q_proj.weight") return lin(y.q);
        if (r == "self_attn.k_proj.weight") return lin(y.k);
        if (r == "self_attn.v_proj.weight") return lin(y.v);
        if (r == "self_attn.o_proj.weight") return lin(y.o);
        if (r == "mlp.gate_proj.weight") return lin(y.gate);
        if (r == "mlp.up_proj.weight") return lin(y.up);
        if (r == "mlp.down_proj.weight") return lin(y.down);
    }
    return ti_fail(TI_ERR_INVALID, "ti_bonsai_tensor: unknown tensor '%s'", name);
}

// [N, K] of a ternary tensor by its name, as check_shapes (model.rs:288-309) derives them
// from the config: q [nq, H], k/v [nkv, H], o [H, nq], gate/up [I, H], down [H, I],
// lm_head [vocab, H]
static void tern_shape(const ti_bonsai_config& C, const std::string& n, long long& N, long long& K) {
    const long long H = C.hidden, I = C.intermediate, nq = (long long)C.n_heads * C.head_dim,
                    nkv = (long long)C.n_kv_heads * C.head_dim;
    auto ends = [&](const char* suf) {
        const size_t ls = strlen(suf);
        return n.size() >= ls && n.compare(n.size() - ls, ls, suf) == 0;
    };
    N = K = 0;
    if (ends("q_proj.weight")) { N = nq; K = H; }
    else if (ends("k_proj.weight") || ends("v_proj.weight")) { N = nkv; K = H; }
    else if (ends("o_proj.weight")) { N = H; K = nq; }
    else if (ends("gate_proj.weight") || ends("up_proj.weight")) { N = I; K = H; }
    else if (ends("down_proj.weight")) { N = H; K = I; }
    else if (n == "lm_head.weight") { N = C.vocab; K = H; }
}

// Model::load + check_shapes (model.rs:256-322): every tensor the forward needs, of the
// kind and shape the config implies (each ternary tensor's N and K compared with the
// config's, in every layer), uploaded from the container.
extern "C" int ti_bonsai_load(ti_ctx* c, ti_bonsai* m, const ti_cpubin* bin) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && bin, "ti_bonsai_load: null argument");
    TI_REQUIRE(!c->capturing, "ti_bonsai_load: not during graph capture");
    const ti_bonsai_config& C = m->cfg;
    std::vector<std::string> names = {"model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"};
    const char* per[] = {"input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_norm.weight",
                         "self_attn.k_norm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
                         "self_attn.v_proj.weight", "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
                         "mlp.down_proj.weight"};
    for (int l = 0; l < C.layers; l++)
        for (const char* p : per) names.push_back("model.layers." + std::to_string(l) + "." + p);
    for (auto& n : names) {
        ti_cpubin_tensor_info t;
        if (ti_cpubin_tensor(bin, n.c_str(), &t)) return ti_fail(TI_ERR_INVALID, "missing tensor `%s`", n.c_str());
        void *d = nullptr, *s = nullptr;
        size_t db = 0, sb = 0;
        int rc = ti_bonsai_tensor(m, n.c_str(), &d, &db, &s, &sb);
        if (rc) return rc;
        const int want = s ? TI_CPUBIN_TERN : (n == "model.embed_tokens.weight" ? TI_CPUBIN_EMBED_F16 : TI_CPUBIN_F32);
        const char* wk = want == TI_CPUBIN_TERN ? "tern" : want == TI_CPUBIN_F32 ? "f32" : "embed_f16";
        if (t.kind != want) return ti_fail(TI_ERR_INVALID, "%s: expected `%s`", n.c_str(), wk);
        if (want == TI_CPUBIN_TERN) {
            // the [N, K] the config implies, compared dimension by dimension: a transposed
            // projection has the byte counts of the right one
            long long en = 0, ek = 0;
            tern_shape(C, n, en, ek);
            if (t.N != en || t.K != ek)
                return ti_fail(TI_ERR_INVALID, "%s: container says [%lld, %lld], config implies [%lld, %lld]", n.c_str(), t.N,
                               t.K, en, ek);
            if ((size_t)t.N * t.K / 4 != db || t.scale_bytes != sb)
                return ti_fail(TI_ERR_INVALID, "%s: container holds %zu code and %zu scale bytes, the config implies %zu and %zu",
                               n.c_str(), t.data_bytes, t.scale_bytes, db, sb);
        }
        if (t.data_bytes != db)
            return ti_fail(TI_ERR_INVALID, "%s: container holds %zu bytes, the config implies %zu", n.c_str(), t.data_bytes, db);
        TI_HIP(hipMemcpyAsync(d, t.data, db, hipMemcpyHostToDevice, c->stream));
        if (s) TI_HIP(hipMemcpyAsync(s, t.scales, sb, hipMemcpyHostToDevice, c->stream));
    }
    TI_HIP(hipStreamSynchronize(c->stream));
    return TI_OK;
}

extern "C" int ti_bonsai_kv(ti_bonsai* m, int layer, float** kc, float** vc) {
    TI_REQUIRE(m && kc && vc && layer >= 0 && layer < m->cfg.layers, "ti_bonsai_kv: bad argument");
    *kc = m->L[layer].kc;
    *vc = m->L[layer].vc;
    return TI_OK;
}

extern "C" int ti_bonsai_logits(ti_bonsai* m, float** logits) {
    TI_REQUIRE(m && logits, "ti_bonsai_logits: null argument");
    *logits = m->logits;
    return TI_OK;
}

extern "C" int ti_bonsai_set_pos(ti_ctx* c, ti_bonsai* m, int pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && pos >= 0 && pos < m->cfg.max_ctx, "ti_bonsai_set_pos: pos %d out of [0, %d)", pos, m ? m->cfg.max_ctx : 0);
    k_bn_set_pos<<<1, 256, 0, c->stream>>>(m->dpos, pos, m->rope, m->rope_cur, m->cfg.head_dim, m->cfg.max_ctx);
    TI_LAUNCHED("k_bn_set_pos");
    return TI_OK;
}

extern "C" int ti_bonsai_write_tokens(ti_ctx* c, ti_bonsai* m, int from, int count, const int32_t* ids) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && ids && from >= 0 && count >= 0 && from + count <= m->cfg.max_ctx + 1, "ti_bonsai_write_tokens: bad range");
    return ti_buf_write(c, m->hist, (size_t)from * 4, ids, (size_t)count * 4);
}

extern "C" int ti_bonsai_read_tokens(ti_ctx* c, ti_bonsai* m, int from, int count, int32_t* ids) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m && ids && from >= 0 && count >= 0 && from + count <= m->cfg.max_ctx + 1, "ti_bonsai_read_tokens: bad range");
    return ti_buf_read(c, m->hist, (size_t)from * 4, ids, (size_t)count * 4);
}

extern "C" int ti_bonsai_trace(ti_bonsai* m, void* buf, size_t bytes) {
    TI_REQUIRE(m, "ti_bonsai_trace: null model");
    if (!buf) { m->trace = nullptr; return TI_OK; }
    const size_t need = (blayer_words(m->cfg) * m->cfg.layers + 2 * (size_t)m->cfg.hidden + m->cfg.hidden / 4 + 1) * 4;
    TI_REQUIRE(bytes >= need, "ti_bonsai_trace: the trace needs %zu bytes (got %zu)", need, bytes);
    TI_REQUIRE(((uintptr_t)buf & 15) == 0, "ti_bonsai_trace: buffer must be 16-byte aligned");
    m->trace = static_cast<uint32_t*>(buf);
    return TI_OK;
}

static int bn_norm_quant(ti_ctx* c, float* x, const float* add, const float* add_scale, const float* w, float eps, int H,
                         float* xn, int8_t* act, int32_t* xsum, float* scale) {
    const int ept = (H + BN_THREADS - 1) / BN_THREADS;
#define NQ(E) if (ept <= E) { k_bn_norm_quant<E><<<1, BN_THREADS, 0, c->stream>>>(x, add, add_scale, w, eps, H, xn, act, xsum, scale); }
    NQ(2) else NQ(4) else NQ(8) else return ti_fail(TI_ERR_INVALID, "bonsai: hidden %d too wide", H);
#undef NQ
    TI_LAUNCHED("k_bn_norm_quant");
    return TI_OK;
}

// One token at the device position P (model.rs:349-501): with logits, the argmax goes to
// hist[P + 1]; P advances either way.
static int bonsai_step(ti_ctx* c, ti_bonsai* m, bool want_logits) {
    const ti_bonsai_config& C = m->cfg;
    const int H = C.hidden, I = C.intermediate, hd = C.head_dim, nHq = C.n_heads, nKv = C.n_kv_heads;
    const int nq = nHq * hd, nkv = nKv * hd;
    const int nsplit = (C.max_ctx + bn_chunk(C.max_ctx) - 1) / bn_chunk(C.max_ctx);
    float* sa = m->scales;
    float* sb = m->scales + 1;
    float* scl = m->scales + 2;
    float* sd = m->scales + 3;
    // the residual add + norm + quantizer before q/k/v and gate/up run in those projections'
    // prologues (ti_tern_gemv_multi_norm) where the hidden width allows
    const bool fuse = ti_tern_norm_ok(H);
    int rc;
#define RC(x) do { rc = (x); if (rc) return rc; } while (0)
    k_bn_embed<<<1, 256, 0, c->stream>>>(m->hist, m->dpos, m->embed, m->x, H, C.vocab, C.max_ctx);
    TI_LAUNCHED("k_bn_embed");
    for (int l = 0; l < C.layers; l++) {
        BLayer& y = m->L[l];
        const bool first = l == 0;
        // the previous layer's down projection is added in this norm's prologue
        if (m->trace && !first) RC(bput(c, m, l - 1, B_D, m->draw));
        const uint8_t* cq[3] = {y.q.codes, y.k.codes, y.v.codes};
        const float* sq[3] = {y.q.scales, y.k.scales, y.v.scales};
        float* oq[3] = {m->qraw, m->kraw, m->vraw};
        const int nqkv[3] = {nq, nkv, nkv};
        // with the norm in the projections' prologue the residual moves x -> x2 here and
        // back x2 -> x in the post-attention norm (a launch's workgroups still read its input)
        float* xmid = fuse ? m->x2 : m->x;
        if (fuse) {
            const ti_tern_norm nin = {m->x, first ? nullptr : m->draw, sd, y.in_norm, C.rms_eps,
                                      m->x2, m->xn, m->act, m->xsum, sa};
            RC(ti_tern_gemv_multi_norm(c, &nin, H, 3, cq, sq, oq, nqkv));
        } else {
            RC(bn_norm_quant(c, m->x, first ? nullptr : m->draw, sd, y.in_norm, C.rms_eps, H, m->xn, m->act, m->xsum, sa));
        }
        if (m->trace) {
            // x_in of this layer: x before the add is the previous x_out; trace the sum
            RC(bput(c, m, l, B_X_IN, xmid));
            RC(bput(c, m, l, B_XN, m->xn));
            RC(bput(c, m, l, B_A_ACT, m->act));
            RC(bput(c, m, l, B_A_SCALE, sa));
        }
        if (!fuse) RC(ti_tern_gemv_multi(c, m->act, m->xsum, H, 3, cq, sq, oq, nqkv));
        if (m->trace) {
            RC(bput(c, m, l, B_Q, m->qraw));
            RC(bput(c, m, l, B_K, m->kraw));
            RC(bput(c, m, l, B_V, m->vraw));
        }
        const int chunk = bn_chunk(C.max_ctx);
#define BA(CH_) k_bn_attn<CH_><<<nKv * nsplit, 256, 0, c->stream>>>(m->qraw, m->kraw, m->vraw, sa, y.q_norm, y.k_norm, m->rope_cur, \
                                                                    C.rms_eps, y.kc, y.vc, m->dpos, nKv, m->po, m->pml, nsplit, C.max_ctx)
        if (chunk == 64) BA(64);
        else if (chunk == 128) BA(128);
        else BA(256);
#undef BA
        TI_LAUNCHED("k_bn_attn");
        const int eq = (nq + BN_THREADS - 1) / BN_THREADS;
        // with the quantizer in the o projection's prologue the merge only merges
        const bool fuse_o = ti_tern_norm_ok(nq);
        int8_t* mact = fuse_o ? nullptr : m->act;
#define MQ(E) if (eq <= E) { k_bn_merge_quant<E><<<nKv, BN_THREADS, 0, c->stream>>>(m->po, m->pml, m->dpos, nsplit, nq, chunk, m->attn, mact, m->xsum, sb, c->sync + TI_SYNC_BONSAI, C.max_ctx); }
        MQ(2) else MQ(4) else MQ(8) else return ti_fail(TI_ERR_INVALID, "bonsai: q width %d", nq);
#undef MQ
        TI_LAUNCHED("k_bn_merge_quant");
        if (fuse_o) {
            const ti_tern_norm nqo = {m->attn, nullptr, nullptr, nullptr, 0.0f, nullptr, nullptr, m->act, m->xsum, sb};
            float* oo[1] = {m->oraw};
            const uint8_t* co[1] = {y.o.codes};
            const float* so[1] = {y.o.scales};
            const int no[1] = {H};
            RC(ti_tern_gemv_multi_norm(c, &nqo, nq, 1, co, so, oo, no));
        }
        if (m->trace) {
            RC(bput(c, m, l, B_ATTN, m->attn));
            RC(bput(c, m, l, B_B_ACT, m->act));
            RC(bput(c, m, l, B_B_SCALE, sb));
        }
        if (!fuse_o) RC(ti_tern_gemv(c, m->oraw, y.o.codes, y.o.scales, m->act, m->xsum, H, nq));
        const uint8_t* cg[2] = {y.gate.codes, y.up.codes};
        const float* sg[2] = {y.gate.scales, y.up.scales};
        float* og[2] = {m->graw, m->uraw};
        const int ngu[2] = {I, I};
        if (fuse) {
            const ti_tern_norm npost = {xmid, m->oraw, sb, y.post_norm, C.rms_eps, m->x, m->xn, m->act, m->xsum, scl};
            RC(ti_tern_gemv_multi_norm(c, &npost, H, 2, cg, sg, og, ngu));
        } else {
            RC(bn_norm_quant(c, m->x, m->oraw, sb, y.post_norm, C.rms_eps, H, m->xn, m->act, m->xsum, scl));
        }
        if (m->trace) {
            RC(bput(c, m, l, B_X_MID, m->x));
            RC(bput(c, m, l, B_XN2, m->xn));
            RC(bput(c, m, l, B_C_ACT, m->act));
            RC(bput(c, m, l, B_C_SCALE, scl));
        }
        if (!fuse) RC(ti_tern_gemv_multi(c, m->act, m->xsum, H, 2, cg, sg, og, ngu));
        const bool fuse_swi = ti_tern_swiglu_ok(I);
        if (fuse_swi) {
            // the SwiGLU and its quantizer run in the down projection's prologue
            const ti_tern_swiglu swd = {m->graw, m->uraw, scl, m->swi, m->act, m->xsum, sd};
            RC(ti_tern_gemv_swiglu(c, &swd, m->draw, y.down.codes, y.down.scales, H, I));
        } else {
            const int ei = (I + BN_THREADS - 1) / BN_THREADS;
#define SQ(E) if (ei <= E) { k_bn_swiglu_quant<E><<<1, BN_THREADS, 0, c->stream>>>(m->graw, m->uraw, scl, I, m->swi, m->act, m->xsum, sd); }
            SQ(2) else SQ(4) else SQ(8) else return ti_fail(TI_ERR_INVALID, "bonsai: intermediate %d", I);
#undef SQ
            TI_LAUNCHED("k_bn_swiglu_quant");
        }
        if (m->trace) {
            RC(bput(c, m, l, B_G, m->graw));
            RC(bput(c, m, l, B_U, m->uraw));
            RC(bput(c, m, l, B_SWI, m->swi));
            RC(bput(c, m, l, B_D_ACT, m->act));
            RC(bput(c, m, l, B_D_SCALE, sd));
        }
        if (!fuse_swi) RC(ti_tern_gemv(c, m->draw, y.down.codes, y.down.scales, m->act, m->xsum, H, I));
    }
    if (m->trace) RC(bput(c, m, C.layers - 1, B_D, m->draw));
    if (!want_logits) {
        // a prompt token: its KV rows are written; the residual restarts at the next
        // token's embedding, so nothing past the last layer is computed (model.rs:486-490)
        k_bn_advance<<<1, 256, 0, c->stream>>>(m->dpos, m->rope, m->rope_cur, hd, C.max_ctx);
        TI_LAUNCHED("k_bn_advance");
        return TI_OK;
    }
    RC(bn_norm_quant(c, m->x, m->draw, sd, m->final_norm, C.rms_eps, H, m->xn, m->act, m->xsum, sa));
    if (m->trace) {
        uint32_t* fin = bslot(m, C.layers, 0);
        // x_final, xn_final, its codes and scale after the last layer
        k_bn_copy_u32<<<8, 256, 0, c->stream>>>(reinterpret_cast<const uint32_t*>(m->x), fin, H);
        k_bn_copy_u32<<<8, 256, 0, c->stream>>>(reinterpret_cast<const uint32_t*>(m->xn), fin + H, H);
        k_bn_copy_u32<<<8, 256, 0, c->stream>>>(reinterpret_cast<const uint32_t*>(m->act), fin + 2 * H, H / 4);
        k_bn_copy_u32<<<1, 64, 0, c->stream>>>(reinterpret_cast<const uint32_t*>(sa), fin + 2 * H + H / 4, 1);
        TI_LAUNCHED("k_bn_copy_u32 (trace)");
    }
    RC(ti_tern_gemv(c, m->lraw, m->lm.codes, m->lm.scales, m->act, m->xsum, C.vocab, H));
    k_bn_logits<<<BN_AMAX_PARTS, 256, 0, c->stream>>>(m->lraw, sa, C.vocab, m->logits, m->amax_v, m->amax_i);
    TI_LAUNCHED("k_bn_logits");
    k_bn_argmax<<<1, BN_AMAX_PARTS, 0, c->stream>>>(m->amax_v, m->amax_i, BN_AMAX_PARTS, m->hist, m->dpos, C.max_ctx, m->rope,
                                                    m->rope_cur, hd);
    TI_LAUNCHED("k_bn_argmax");
    return TI_OK;
#undef RC
}

// Model::forward at the device position (model.rs:349-501), logits and greedy token:
// graph-capturable (reads nothing from the host).
extern "C" int ti_bonsai_decode(ti_ctx* c, ti_bonsai* m) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m, "ti_bonsai_decode: null model");
    return bonsai_step(c, m, true);
}

// Prompt tokens ids[0..T) at positions pos.. (Model::forward per token, logits only for the
// last, as n2-cli's prefill calls it): the argmax of the last token's logits goes to
// hist[pos + T] and the device position becomes pos + T.
extern "C" int ti_bonsai_forward(ti_ctx* c, ti_bonsai* m, const int32_t* ids, int T, int pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(m, "ti_bonsai_forward: null model");
    TI_REQUIRE(T > 0 && pos >= 0 && pos + T <= m->cfg.max_ctx, "ti_bonsai_forward: T=%d pos=%d outside max_ctx=%d", T, pos,
               m->cfg.max_ctx);
    int rc;
    if (ids && (rc = ti_buf_write(c, m->hist, (size_t)pos * 4, ids, (size_t)T * 4))) return rc;
    if ((rc = ti_bonsai_set_pos(c, m, pos))) return rc;
    for (int t = 0; t < T; t++)
        if ((rc = bonsai_step(c, m, t == T - 1))) return rc;
    return TI_OK;
}
