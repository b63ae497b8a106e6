// k_moe.hip — the int3 MoE expert path of LFM2.5 (models/lfm25.js):
//  int4 -> int3 cascade requant into bitplanes    _requant43        lfm25.js:833-856
//  sigmoid + bias top-k router                     ROUTER_WGSL       lfm25.js:111-146
//  pair-indexed int3 GEMV, f32 activation (T = 1) idxGemv3          lfm25.js:1924-1980
//      expert-grouped int3 x int8 GEMM (T > 1)        moeSort+moeGemm3  lfm25.js:1503-1647
//      weighted combine into the residual              MOECOMBINE_WGSL   lfm25.js:1982-2000
//
// int3 group (32 weights): three u32 bitplanes, bit i of plane b = bit b of (q3 + 4) for
// element i, then one f16 scale; rows of all experts stacked expert-major (row = e*N + n).
// The kernels turn a group's three planes into eight words of (q3 + 4) bytes, word c
// holding elements c, c+8, c+16, c+24 (q3_cols), and dot them with v_dot4_i32_i8 against
// activation words packed in the same order; the +4 offset is removed once per group from
// the activation sum. The int32 group dot is the same integer in any element order.
#include "ti_dev.h"

namespace {

// ---- requant -----------------------------------------------------------------------------
// engine/webgpu-engine.js:217-236 f32 -> f16 (rounding by +0x1000 and OR-ing the carry
// into the exponent field, as that routine does)
__device__ __forceinline__ uint16_t f32_to_f16_eng(float v) {
    const uint32_t x = __float_as_uint(v);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x007fffffu;
    const int exp = (int)((x >> 23) & 0xffu);
    if (exp == 255) return (uint16_t)(sign | (mant ? 0x7e00u : 0x7c00u));
    const int e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant = (mant | 0x00800000u) >> (1 - e);
        return (uint16_t)(sign | ((mant + 0x00001000u) >> 13));
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | ((mant + 0x00001000u) >> 13));
}

// JS Math.round: ties toward +infinity
__device__ __forceinline__ double js_round(double x) {
    const double f = floor(x);
    return (x - f >= 0.5) ? f + 1.0 : f;
}

// one thread per (row, group); JS number (f64) arithmetic as _requant43 does it
__global__ __launch_bounds__(256) void k_requant43(const uint32_t* __restrict__ pack4, const uint16_t* __restrict__ sc4,
                                                   uint32_t* __restrict__ p3, uint16_t* __restrict__ s3, long ngroups) {
    const long gi = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= ngroups) return;
    const uint4 w4 = reinterpret_cast<const uint4*>(pack4)[gi];
    const uint32_t words[4] = {w4.x, w4.y, w4.z, w4.w};
    int q4[32];
    int m = 0;
#pragma unroll
    for (int wI = 0; wI < 4; wI++)
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int q = (int)((words[wI] >> (4 * i)) & 15u) - 8;
            q4[wI * 8 + i] = q;
            const int a = q < 0 ? -q : q;
            m = a > m ? a : m;
        }
    if (m == 0) {
        s3[gi] = f32_to_f16_eng(0.0f);
        p3[gi * 3] = 0u;
        p3[gi * 3 + 1] = 0u;
        p3[gi * 3 + 2] = 0xFFFFFFFFu;
        return;
    }
    const double ratio = 4.0 / (double)m;
    const double s3d = (double)ti_h2f(sc4[gi]) * (double)m / 4.0;
    s3[gi] = f32_to_f16_eng((float)s3d);
    uint32_t b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        double q = js_round((double)q4[i] * ratio);
        q = q > 3.0 ? 3.0 : (q < -4.0 ? -4.0 : q);
        const uint32_t st = (uint32_t)((int)q + 4);
        b0 |= (st & 1u) << i;
        b1 |= ((st >> 1) & 1u) << i;
        b2 |= ((st >> 2) & 1u) << i;
    }
    p3[gi * 3] = b0;
    p3[gi * 3 + 1] = b1;
    p3[gi * 3 + 2] = b2;
}

// ---- router ------------------------------------------------------------------------------
// one wave per token: s = sigmoid(logit) in f32, top-k of s + bias by strict '>' (the
// lowest index wins a tie), weights s / (sum + 1e-6)
constexpr int ROUTER_EMAX = 256;
__device__ __forceinline__ void router_token(int t, const float* __restrict__ logits, const float* __restrict__ bias,
                                             int nE, int topk, int32_t* __restrict__ idx, float* __restrict__ wt) {
    __shared__ float sc[ROUTER_EMAX], sel[ROUTER_EMAX];
    __shared__ int chosen[ROUTER_EMAX];
    const int lane = threadIdx.x;
    for (int e = lane; e < nE; e += 64) {
        const float l = logits[(size_t)t * nE + e];
        const float s = 1.0f / (1.0f + expf(-l));
        sc[e] = s;
        sel[e] = s + (bias ? bias[e] : 0.0f);
    }
    __syncthreads();
    float sum = 0.0f;
    for (int k = 0; k < topk; k++) {
        float bv = -1.0e30f;
        int bi = 0x7fffffff;
        for (int e = lane; e < nE; e += 64) {
            const float v = sel[e];
            if (v > bv) { bv = v; bi = e; }          // per lane: ascending e, strict '>'
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = ti_xor(bv, o);
            const int oi = ti_xor_i(bi, o);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (bi == 0x7fffffff) bi = 0;                   // nothing above -1e30: index 0, as a scan would
        if (lane == 0) {
            chosen[k] = bi;
            sel[bi] = -2.0e30f;
        }
        __syncthreads();
        const int b = chosen[k];
        sum = sum + sc[b];
    }
    if (lane < topk) {
        const int b = chosen[lane];
        idx[(size_t)t * topk + lane] = b;
        wt[(size_t)t * topk + lane] = sc[b] / (sum + 1e-6f);
    }
}

__global__ __launch_bounds__(64) void k_router(const float* __restrict__ logits, const float* __restrict__ bias, int nE,
                                               int topk, int32_t* __restrict__ idx, float* __restrict__ wt) {
    router_token(blockIdx.x, logits, bias, nE, topk, idx, wt);
}

// the router (workgroups 0 .. T-1, one per token) and, in the same launch, quantAct8 of
// the normed rows (the remaining workgroups, a 32-group per thread, words in
// k_moe_gemm_q3's element order): the two do not depend on each other
__global__ __launch_bounds__(64) void k_router_quant(const float* __restrict__ logits, const float* __restrict__ bias,
                                                     int nE, int topk, int32_t* __restrict__ idx, float* __restrict__ wt,
                                                     int T, const float* __restrict__ x, uint32_t* __restrict__ xq,
                                                     float* __restrict__ xs, int ng) {
    if ((int)blockIdx.x < T) {
        router_token(blockIdx.x, logits, bias, nE, topk, idx, wt);
        return;
    }
    const int gi = ((int)blockIdx.x - T) * 64 + threadIdx.x;
    if (gi >= ng) return;
    float v[32];
    load32(x + (size_t)gi * 32, v);
    q8_group<true>(v, xq + (size_t)gi * 8, xs + gi, nullptr);
}

// ---- decode: pair-indexed GEMV with the f32 activation ----------------------------
// A group's (q3 + 4) codes as bytes, q[c] byte i = element 8i + c. Elements 4t + r
// (r = 0..3, t = 0..7) take plane bit positions 4t + r; gathering plane b's bits of one r
// beside each other gives X_r with element 4t + r's code in nibble t (bits 4t + r + b for
// r < 2, shifted down by 2 for r >= 2 so nothing leaves the word), then q[4h + r] is
// nibbles h, h+2, h+4, h+6 of X_r, one per byte. 36 VALU operations per 32 codes.
__device__ __forceinline__ void q3_cols(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t (&q)[8]) {
    constexpr uint32_t M = 0x11111111u, B = 0x07070707u;
    const uint32_t x0 = (b0 & M) | ((b1 & M) << 1) | ((b2 & M) << 2);
    const uint32_t x1 = (b0 & (M << 1)) | ((b1 & (M << 1)) << 1) | ((b2 & (M << 1)) << 2);
    const uint32_t x2 = ((b0 & (M << 2)) >> 2) | ((b1 & (M << 2)) >> 1) | (b2 & (M << 2));
    const uint32_t x3 = ((b0 & (M << 3)) >> 2) | ((b1 & (M << 3)) >> 1) | (b2 & (M << 3));
    q[0] = x0 & B;
    q[4] = (x0 >> 4) & B;
    q[1] = (x1 >> 1) & B;
    q[5] = (x1 >> 5) & B;
    q[2] = x2 & B;
    q[6] = (x2 >> 4) & B;
    q[3] = (x3 >> 1) & B;
    q[7] = (x3 >> 5) & B;
}

// f32 activation group as exact fixed point (as k_gemv_q4_f32): x_j = X_j * 2^(ex-22),
// X = l2*65536 + l1*256 + l0 with signed int8 limbs, words in q3_cols's element order
struct Limbs {
    int l[3][8];        // limb, word c = elements c, c+8, c+16, c+24
    int sum[3];         // sum of each limb over the 32 elements
    float S;            // 2^(ex-22)
};
__device__ __forceinline__ void make_limbs(const float* v, Limbs& L) {
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) mx = fmaxf(mx, fabsf(v[j]));
    int ex = 0;
    if (mx > 0.0f) (void)frexpf(mx, &ex);
    L.S = ldexpf(1.0f, ex - 22);
    int b[3][32];
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const int X = mx > 0.0f ? (int)rintf(ldexpf(v[j], 22 - ex)) : 0;
        const int l0 = ((X & 0xff) ^ 0x80) - 0x80;
        const int X1 = (X - l0) >> 8;
        const int l1 = ((X1 & 0xff) ^ 0x80) - 0x80;
        b[0][j] = l0;
        b[1][j] = l1;
        b[2][j] = (X1 - l1) >> 8;
    }
#pragma unroll
    for (int q = 0; q < 3; q++) {
        int s = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            L.l[q][w] = (int)((uint32_t)(b[q][w] & 0xff) | ((uint32_t)(b[q][w + 8] & 0xff) << 8) |
                              ((uint32_t)(b[q][w + 16] & 0xff) << 16) | ((uint32_t)(b[q][w + 24] & 0xff) << 24));
            s += b[q][w] + b[q][w + 8] + b[q][w + 16] + b[q][w + 24];
        }
        L.sum[q] = s;
    }
}

// sum_i (q3_i) * x_i over one group, q3 = stored - 4
__device__ __forceinline__ float group_dot_q3_limbs(uint32_t b0, uint32_t b1, uint32_t b2, const Limbs& L) {
    int d[3] = {0, 0, 0};
    uint32_t q[8];
    q3_cols(b0, b1, b2, q);
#pragma unroll
    for (int w = 0; w < 8; w++)
#pragma unroll
        for (int k = 0; k < 3; k++) d[k] = __builtin_amdgcn_sdot4((int)q[w], L.l[k][w], d[k], false);
    const int t = (d[2] - 4 * L.sum[2]) * 256 + (d[1] - 4 * L.sum[1]);   // |t| < 2^24
    return fmaf((float)t, 256.0f, (float)(d[0] - 4 * L.sum[0])) * L.S;
}

// grid (row blocks of 16, pairs); each wave takes 4 rows, lane l the groups l and l + 64;
// the pair's activation groups become limbs once per wave. A pair whose expert id is out
// of range writes nothing.
constexpr int MOE_R = 4;           // rows per wave
template <int GL>
__global__ __launch_bounds__(256) void k_moe_gemv_q3(const float* __restrict__ x, const uint32_t* __restrict__ p3,
                                                     const uint16_t* __restrict__ s3, const int32_t* __restrict__ idx,
                                                     float* __restrict__ y, int N, int K, int in_stride, int xdiv,
                                                     int nE) {
    const int k = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gpr = K / 32;
    const int e = idx[k];
    if (e < 0 || e >= nE) return;
    const float* xr = x + (size_t)(k / xdiv) * in_stride;
    const int row0 = (blockIdx.x * 4 + wave) * MOE_R;
    uint32_t pl[GL][MOE_R][3];
    uint16_t sv[GL][MOE_R];
    float v[GL][32];
#pragma unroll
    for (int h = 0; h < GL; h++) {
        const int g = lane + 64 * h;
        const int gc = g < gpr ? g : gpr - 1;
        const float4* src = reinterpret_cast<const float4*>(xr + (size_t)gc * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 t = src[i];
            v[h][4 * i] = t.x; v[h][4 * i + 1] = t.y; v[h][4 * i + 2] = t.z; v[h][4 * i + 3] = t.w;
        }
#pragma unroll
        for (int r = 0; r < MOE_R; r++) {
            const int n = min(row0 + r, N - 1);
            const size_t gi = ((size_t)e * N + n) * gpr + gc;
            pl[h][r][0] = __builtin_nontemporal_load(p3 + gi * 3);
            pl[h][r][1] = __builtin_nontemporal_load(p3 + gi * 3 + 1);
            pl[h][r][2] = __builtin_nontemporal_load(p3 + gi * 3 + 2);
            sv[h][r] = s3[gi];
        }
    }
    float accv[MOE_R] = {};
#pragma unroll
    for (int h = 0; h < GL; h++) {
        Limbs L;
        make_limbs(v[h], L);
        const bool live = lane + 64 * h < gpr;
#pragma unroll
        for (int r = 0; r < MOE_R; r++) {
            const float d = group_dot_q3_limbs(pl[h][r][0], pl[h][r][1], pl[h][r][2], L);
            accv[r] = live ? fmaf(d, ti_h2f(sv[h][r]), accv[r]) : accv[r];
        }
    }
    const float tot = transpose_reduce<64, MOE_R>(accv, lane);
    const int n = row0 + lane / (64 / MOE_R);
    if ((lane % (64 / MOE_R)) == 0 && n < N) y[(size_t)k * N + n] = tot;
}

// ---- T > 1: rows of one expert against all pairs routed to it ----------------------
// grid (row blocks of 16, experts). The workgroup scans the routing ids 256 at a time and
// lists its expert's pairs in pair order (ballot compaction in LDS). Each wave turns its 4
// rows' bitplanes into (q + 4) bytes (q3_cols), kept in registers; the listed pairs then
// read their int8 activation groups (L2-resident, words in the same element order) and
// scales, four pairs' loads in flight at once:
//   dot = sum (q + 4) a - 4 sum a   (exact int32),   y[pair, n] = sum_g dot * s_x * s_w.
// spec (most experts are routed to, as at 16 tokens x top-4 over 32 experts): the weight
// loads are issued before the scan, so their round trip overlaps it; otherwise they wait
// for the first hit and the workgroups of experts nobody chose read only the ids.
constexpr int MOE_PB = 4;          // pairs whose activation loads are in flight together
template <int GL>
// grid.z = 2 runs a second matrix (p3b, s3b -> yb) of the same shape on the same activation.
__global__ __launch_bounds__(256) void k_moe_gemm_q3(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                     const uint32_t* __restrict__ p3a, const uint16_t* __restrict__ s3a,
                                                     const int32_t* __restrict__ ridx, float* __restrict__ ya, int P, int N,
                                                     int K, int src_div, int spec, const uint32_t* __restrict__ p3b,
                                                     const uint16_t* __restrict__ s3b, float* __restrict__ yb) {
    const uint32_t* __restrict__ p3 = blockIdx.z ? p3b : p3a;
    const uint16_t* __restrict__ s3 = blockIdx.z ? s3b : s3a;
    float* __restrict__ y = blockIdx.z ? yb : ya;
    __shared__ int s_list[256];
    __shared__ int s_wcnt[4];
    const int e = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gpr = K / 32;
    const int row0 = blockIdx.x * 16 + wave * MOE_R;
    uint32_t pb[MOE_R][GL][3];
    uint16_t sr[MOE_R][GL];
    auto wload = [&]() {
#pragma unroll
        for (int r = 0; r < MOE_R; r++) {
            const int n = min(row0 + r, N - 1);
#pragma unroll
            for (int h = 0; h < GL; h++) {
                const int g = lane + 64 * h;
                const int gc = g < gpr ? g : gpr - 1;
                const size_t gi = ((size_t)e * N + n) * gpr + gc;
#pragma unroll
                for (int b = 0; b < 3; b++) pb[r][h][b] = __builtin_nontemporal_load(p3 + gi * 3 + b);
                sr[r][h] = s3[gi];
            }
        }
    };
    // the first chunk's routing ids are loaded before the weights, so that the scan waits
    // for them alone; at GL = 1 the first pairs' activation loads are then issued before the
    // codes are expanded, and their round trip overlaps the weights' (at GL = 2 the codes
    // and four pairs' activations together would not fit in the registers)
    constexpr bool ACT_FIRST = GL == 1;
    const int rid0 = tid < P ? ridx[tid] : -1;
    if (spec) wload();
    uint32_t qb[MOE_R][GL][8];
    float sw[MOE_R][GL];
    bool have = false;
    for (int c0 = 0; c0 < P; c0 += 256) {
        const int p = c0 + tid;
        const bool hit = p < P && (c0 == 0 ? rid0 : ridx[p]) == e;
        const uint64_t m = __ballot(hit);
        __syncthreads();                                    // the previous chunk's list is consumed
        if (lane == 0) s_wcnt[wave] = __popcll(m);
        __syncthreads();
        int base = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) base += w < wave ? s_wcnt[w] : 0;
        const int tot = (s_wcnt[0] + s_wcnt[1]) + (s_wcnt[2] + s_wcnt[3]);
        if (hit) s_list[base + __popcll(m & ((1ull << lane) - 1ull))] = p;
        __syncthreads();
        if (tot == 0) continue;
        if (!have && !spec) wload();
        auto expand = [&]() {
#pragma unroll
            for (int r = 0; r < MOE_R; r++)
#pragma unroll
                for (int h = 0; h < GL; h++) {
                    const int g = lane + 64 * h;
                    sw[r][h] = g < gpr ? ti_h2f(sr[r][h]) : 0.0f;
                    q3_cols(pb[r][h][0], pb[r][h][1], pb[r][h][2], qb[r][h]);
                }
        };
        if (!ACT_FIRST && !have) {
            have = true;
            expand();
        }
        for (int i0 = 0; i0 < tot; i0 += MOE_PB) {
            uint4 u0[MOE_PB][GL], u1[MOE_PB][GL];
            float as[MOE_PB][GL];
            int pairs[MOE_PB];
#pragma unroll
            for (int q = 0; q < MOE_PB; q++) {   // every pair's loads first (past tot: the last pair again)
                pairs[q] = s_list[min(i0 + q, tot - 1)];
                const int src = pairs[q] / src_div;
#pragma unroll
                for (int h = 0; h < GL; h++) {
                    const int g = lane + 64 * h;
                    const int gc = g < gpr ? g : gpr - 1;
                    const uint4* a4 = reinterpret_cast<const uint4*>(xq + (size_t)src * (K / 4) + gc * 8);
                    u0[q][h] = a4[0];
                    u1[q][h] = a4[1];
                    as[q][h] = xs[(size_t)src * gpr + gc];
                }
            }
            if (ACT_FIRST && !have) {                       // workgroup-uniform
                have = true;
                expand();
            }
#pragma unroll
            for (int q = 0; q < MOE_PB; q++) {
                if (i0 + q >= tot) break;                   // workgroup-uniform
                float accv[MOE_R] = {};
#pragma unroll
                for (int h = 0; h < GL; h++) {
                    const int a[8] = {(int)u0[q][h].x, (int)u0[q][h].y, (int)u0[q][h].z, (int)u0[q][h].w,
                                      (int)u1[q][h].x, (int)u1[q][h].y, (int)u1[q][h].z, (int)u1[q][h].w};
                    int asum = 0;
#pragma unroll
                    for (int w = 0; w < 8; w++) asum = __builtin_amdgcn_sdot4(a[w], 0x01010101, asum, false);
#pragma unroll
                    for (int r = 0; r < MOE_R; r++) {
                        int d = 0;
#pragma unroll
                        for (int w = 0; w < 8; w++) d = __builtin_amdgcn_sdot4((int)qb[r][h][w], a[w], d, false);
                        accv[r] = fmaf((float)(d - 4 * asum), as[q][h] * sw[r][h], accv[r]);
                    }
                }
                const float tot_r = transpose_reduce<64, MOE_R>(accv, lane);
                const int n = row0 + lane / (64 / MOE_R);
                if ((lane % (64 / MOE_R)) == 0 && n < N) y[(size_t)pairs[q] * N + n] = tot_r;
            }
        }
    }
}

// ---- one decode token, fused: [router + w1/w3 + swiglu] and [w2 + combine] ----------------
// The router's top-k for one token, computed by one wave (every wave that needs it gets
// the same answer, so no barrier): experts e = lane + 64 i, sigmoid and selection as
// k_router (strict '>', lowest index on ties, weights s / (sum + 1e-6)).
constexpr int RT_EPL = 4;     // experts per lane (nE <= 256)
constexpr int RT_KMAX = 8;    // top-k held in registers
__device__ __forceinline__ void wave_route(const float* __restrict__ logits, const float* __restrict__ bias, int nE,
                                           int topk, int lane, int* ek, float* wk) {
    float sc[RT_EPL], sel[RT_EPL];
#pragma unroll
    for (int i = 0; i < RT_EPL; i++) {
        const int e = lane + 64 * i;
        const int ec = e < nE ? e : 0;
        const float l = logits[ec];
        const float sg = 1.0f / (1.0f + expf(-l));
        sc[i] = sg;
        sel[i] = e < nE ? sg + (bias ? bias[ec] : 0.0f) : -3.0e38f;
    }
    float sum = 0.0f;
    float chosen_s[RT_KMAX];
#pragma unroll
    for (int k = 0; k < RT_KMAX; k++) {
        if (k < topk) {
            float bv = -1.0e30f;
            int bi = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < RT_EPL; i++)
                if (sel[i] > bv) { bv = sel[i]; bi = lane + 64 * i; }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = ti_xor(bv, o);
                const int oi = ti_xor_i(bi, o);
                if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
            }
            if (bi == 0x7fffffff) bi = 0;
            const int owner = bi & 63, slot = bi >> 6;
            float mine = sc[0];
#pragma unroll
            for (int i = 1; i < RT_EPL; i++) mine = slot == i ? sc[i] : mine;
            const float s_b = __shfl(mine, owner, 64);
#pragma unroll
            for (int i = 0; i < RT_EPL; i++)
                if (lane == owner && slot == i) sel[i] = -2.0e30f;
            ek[k] = bi;
            chosen_s[k] = s_b;
            sum = sum + s_b;
        }
    }
#pragma unroll
    for (int k = 0; k < RT_KMAX; k++)
        if (k < topk) wk[k] = chosen_s[k] / (sum + 1e-6f);
}

// a group's Limbs as 28 words (l[3][8], then sum[3] and the scale's bits), for LDS
struct LimbsPacked {
    int4 w[7];          // l[3][8] as 6 int4, then sum[3] and the scale's bits
};
__device__ __forceinline__ void unpack_limbs(const LimbsPacked& d, Limbs& L) {
#pragma unroll
    for (int q = 0; q < 3; q++) {
        const int4 a = d.w[2 * q], b = d.w[2 * q + 1];
        L.l[q][0] = a.x; L.l[q][1] = a.y; L.l[q][2] = a.z; L.l[q][3] = a.w;
        L.l[q][4] = b.x; L.l[q][5] = b.y; L.l[q][6] = b.z; L.l[q][7] = b.w;
    }
    const int4 t = d.w[6];
    L.sum[0] = t.x; L.sum[1] = t.y; L.sum[2] = t.z; L.S = __int_as_float(t.w);
}

// make_limbs of one 32-element group shared by TPG adjacent lanes, each converting the
// 32/TPG elements of words part*CPW .. part*CPW + CPW-1 (part = the lane's index among
// them): the group's max through a butterfly over the TPG lanes, then the same
// per-element conversion, words and sums as make_limbs (so the same bits). Every lane of
// the TPG must take part.
template <int TPG>
__device__ __forceinline__ void coop_limbs(const float* grp, int part, LimbsPacked& d) {
    constexpr int EPT = 32 / TPG, CPW = 8 / TPG;
    float v[EPT];   // v[4j + i] = element part*CPW + j + 8i
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < CPW; j++) v[4 * j + i] = grp[part * CPW + j + 8 * i];
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < EPT; i++) mx = fmaxf(mx, fabsf(v[i]));
#pragma unroll
    for (int o = 1; o < TPG; o <<= 1) mx = fmaxf(mx, ti_xor(mx, o));
    int ex = 0;
    if (mx > 0.0f) (void)frexpf(mx, &ex);
    int* out = reinterpret_cast<int*>(&d);
    int sum[3] = {0, 0, 0};
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        uint32_t word[3] = {0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int X = mx > 0.0f ? (int)rintf(ldexpf(v[4 * j + e], 22 - ex)) : 0;
            const int l0 = ((X & 0xff) ^ 0x80) - 0x80;
            const int X1 = (X - l0) >> 8;
            const int l1 = ((X1 & 0xff) ^ 0x80) - 0x80;
            const int l2 = (X1 - l1) >> 8;
            word[0] |= (uint32_t)(l0 & 0xff) << (8 * e);
            word[1] |= (uint32_t)(l1 & 0xff) << (8 * e);
            word[2] |= (uint32_t)(l2 & 0xff) << (8 * e);
            sum[0] += l0;
            sum[1] += l1;
            sum[2] += l2;
        }
#pragma unroll
        for (int q = 0; q < 3; q++) out[8 * q + part * CPW + j] = (int)word[q];
    }
#pragma unroll
    for (int o = 1; o < TPG; o <<= 1)
#pragma unroll
        for (int q = 0; q < 3; q++) sum[q] += ti_xor(sum[q], o);
    if (part == 0) {
        out[24] = sum[0];
        out[25] = sum[1];
        out[26] = sum[2];
        out[27] = __float_as_int(ldexpf(1.0f, ex - 22));
    }
}

// grid (row blocks of 4R, topk): workgroup (., k) runs the router, takes expert e of
// slot k, and computes act[k*I + n] = silu(w1_e x)_n * (w3_e x)_n for its 4R rows
// (R per wave) with the exact fixed-point dot of k_moe_gemv_q3. Workgroup (0, k) stores
// slot k's expert id and weight.
template <int GL, int R>
__global__ __launch_bounds__(256) void k_moe_gateup_dec(const float* __restrict__ x, const float* __restrict__ logits,
                                                        const float* __restrict__ bias, int nE, int topk,
                                                        const uint32_t* __restrict__ p1, const uint16_t* __restrict__ s1,
                                                        const uint32_t* __restrict__ p3, const uint16_t* __restrict__ s3,
                                                        float* __restrict__ act, int32_t* __restrict__ idx,
                                                        float* __restrict__ wt, int I, int H) {
    const int k = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gpr = H / 32;
    // x once per workgroup, coalesced, into LDS (group g padded to 36 floats: conflict-free
    // 16-byte reads of a lane's group); the loads do not wait for the router
    __shared__ __align__(16) float s_x[GL * 64 * 36];
    for (int i = threadIdx.x; i < H / 4; i += 256) {
        const float4 t = reinterpret_cast<const float4*>(x)[i];
        *reinterpret_cast<float4*>(&s_x[(i / 8) * 36 + (i % 8) * 4]) = t;
    }
    int ek[RT_KMAX];
    float wk[RT_KMAX];
    wave_route(logits, bias, nE, topk, lane, ek, wk);
    int e = ek[0];
    float w = wk[0];
#pragma unroll
    for (int i = 1; i < RT_KMAX; i++) {
        e = k == i ? ek[i] : e;
        w = k == i ? wk[i] : w;
    }
    if (blockIdx.x == 0 && wave == 0 && lane == 0) {
        idx[k] = e;
        wt[k] = w;
    }
    const int row0 = (blockIdx.x * 4 + wave) * R;
    __shared__ LimbsPacked s_lb[GL * 64];
    uint32_t pg[GL][R][3], pu[GL][R][3];
    uint16_t sg[GL][R], su[GL][R];
#pragma unroll
    for (int h = 0; h < GL; h++) {
        const int g = lane + 64 * h;
        const int gc = g < gpr ? g : gpr - 1;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int n = min(row0 + r, I - 1);
            const size_t gi = ((size_t)e * I + n) * gpr + gc;
#pragma unroll
            for (int b = 0; b < 3; b++) {
                pg[h][r][b] = __builtin_nontemporal_load(p1 + gi * 3 + b);
                pu[h][r][b] = __builtin_nontemporal_load(p3 + gi * 3 + b);
            }
            sg[h][r] = s1[gi];
            su[h][r] = s3[gi];
        }
    }
    __syncthreads();
    {   // every group's limbs once per workgroup: 4 / GL threads a group (the waves would
        // otherwise each convert the same 64 GL groups)
        constexpr int TPG = 4 / GL;
        const int grp = threadIdx.x / TPG;
        if (grp < gpr) coop_limbs<TPG>(&s_x[grp * 36], threadIdx.x % TPG, s_lb[grp]);   // uniform per TPG lanes
    }
    __syncthreads();
    float accv[2 * R] = {};
#pragma unroll
    for (int h = 0; h < GL; h++) {
        const int g = lane + 64 * h;
        const int gc = g < gpr ? g : gpr - 1;
        Limbs L;
        unpack_limbs(s_lb[gc], L);
        const bool live = lane + 64 * h < gpr;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float dg = group_dot_q3_limbs(pg[h][r][0], pg[h][r][1], pg[h][r][2], L);
            const float du = group_dot_q3_limbs(pu[h][r][0], pu[h][r][1], pu[h][r][2], L);
            accv[r] = live ? fmaf(dg, ti_h2f(sg[h][r]), accv[r]) : accv[r];
            accv[R + r] = live ? fmaf(du, ti_h2f(su[h][r]), accv[R + r]) : accv[R + r];
        }
    }
    // slot s (gate rows 0..R-1, up rows R..2R-1) ends in lanes s*SPAN .. s*SPAN+SPAN-1
    constexpr int SPAN = 64 / (2 * R);
    const float tot = transpose_reduce<64, 2 * R>(accv, lane);
    const float up = __shfl(tot, lane + SPAN * R, 64);
    const int r = lane / SPAN;
    const int n = row0 + r;
    if (lane % SPAN == 0 && r < R && n < I) act[(size_t)k * I + n] = tot / (1.0f + expf(-tot)) * up;
}

// grid (row blocks of 16): rows n of w2 for every slot k (expert idx[k], activation row
// act[k*I ..]), then x[n] += sum_k wt[k] * out_k[n] in slot order (moeCombine's order).
template <int GL, int P>
__global__ __launch_bounds__(256) void k_moe_down_dec(const float* __restrict__ act, const uint32_t* __restrict__ p2,
                                                      const uint16_t* __restrict__ s2, const int32_t* __restrict__ idx,
                                                      const float* __restrict__ wt, float* __restrict__ x, int H, int I,
                                                      int nE) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gpr = I / 32;
    const int row0 = (blockIdx.x * 4 + wave) * MOE_R;
    int ek[P];
#pragma unroll
    for (int k = 0; k < P; k++) {
        const int e = idx[k];
        ek[k] = e < 0 ? 0 : (e >= nE ? nE - 1 : e);   // ids come from the router: always in range
    }
    float accv[MOE_R * P] = {};
#pragma unroll
    for (int h = 0; h < GL; h++) {
        const int g = lane + 64 * h;
        const int gc = g < gpr ? g : gpr - 1;
        const bool live = g < gpr;
        uint32_t pl[P][MOE_R][3];
        uint16_t sv[P][MOE_R];
#pragma unroll
        for (int k = 0; k < P; k++)
#pragma unroll
            for (int r = 0; r < MOE_R; r++) {
                const int n = min(row0 + r, H - 1);
                const size_t gi = ((size_t)ek[k] * H + n) * gpr + gc;
#pragma unroll
                for (int b = 0; b < 3; b++) pl[k][r][b] = __builtin_nontemporal_load(p2 + gi * 3 + b);
                sv[k][r] = s2[gi];
            }
#pragma unroll
        for (int k = 0; k < P; k++) {
            float vv[32];
            const float4* src = reinterpret_cast<const float4*>(act + (size_t)k * I + (size_t)gc * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 t = src[i];
                vv[4 * i] = t.x; vv[4 * i + 1] = t.y; vv[4 * i + 2] = t.z; vv[4 * i + 3] = t.w;
            }
            Limbs L;
            make_limbs(vv, L);
#pragma unroll
            for (int r = 0; r < MOE_R; r++) {
                const float d = group_dot_q3_limbs(pl[k][r][0], pl[k][r][1], pl[k][r][2], L);
                accv[r * P + k] = live ? fmaf(d, ti_h2f(sv[k][r]), accv[r * P + k]) : accv[r * P + k];
            }
        }
    }
    constexpr int SLOTS = MOE_R * P, SPAN = 64 / SLOTS;
    const float tot = transpose_reduce<64, SLOTS>(accv, lane);
    // row r's P slots are in lanes (r*P + k) * SPAN
    const int r = lane / (P * SPAN);
    float o[P];
#pragma unroll
    for (int k = 0; k < P; k++) o[k] = __shfl(tot, (r * P + k) * SPAN, 64);
    const int n = row0 + r;
    if (lane % (P * SPAN) == 0 && n < H) {
        float sacc = 0.0f;
#pragma unroll
        for (int k = 0; k < P; k++) {
            const float pr = wt[k] * o[k];
            sacc = sacc + pr;
        }
        x[n] = x[n] + sacc;
    }
}

// the same with the slots' activation limbs computed once per workgroup (wave k: slot k,
// P <= 4) and shared through LDS; R rows per wave (I <= 2048)
template <int P, int R>
__global__ __launch_bounds__(256) void k_moe_down_dec_pl(const float* __restrict__ act, const uint32_t* __restrict__ p2,
                                                         const uint16_t* __restrict__ s2, const int32_t* __restrict__ idx,
                                                         const float* __restrict__ wt, float* __restrict__ x, int H, int I,
                                                         int nE) {
    static_assert(P >= 1 && P <= 4, "one wave per slot");
    __shared__ LimbsPacked s_l[P][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gpr = I / 32;
    const int g = lane, gc = g < gpr ? g : gpr - 1;
    const bool live = g < gpr;
    const int row0 = (blockIdx.x * 4 + wave) * R;
    int ek[P];
#pragma unroll
    for (int k = 0; k < P; k++) {
        const int e = idx[k];
        ek[k] = e < 0 ? 0 : (e >= nE ? nE - 1 : e);   // ids come from the router: always in range
    }
    uint32_t pl[P][R][3];
    uint16_t sv[P][R];
#pragma unroll
    for (int k = 0; k < P; k++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int n = min(row0 + r, H - 1);
            const size_t gi = ((size_t)ek[k] * H + n) * gpr + gc;
#pragma unroll
            for (int b = 0; b < 3; b++) pl[k][r][b] = __builtin_nontemporal_load(p2 + gi * 3 + b);
            sv[k][r] = s2[gi];
        }
    if (wave < P) {
        float vv[32];
        const float4* src = reinterpret_cast<const float4*>(act + (size_t)wave * I + (size_t)gc * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 t = src[i];
            vv[4 * i] = t.x; vv[4 * i + 1] = t.y; vv[4 * i + 2] = t.z; vv[4 * i + 3] = t.w;
        }
        Limbs L;
        make_limbs(vv, L);
        LimbsPacked& d = s_l[wave][lane];
#pragma unroll
        for (int q = 0; q < 3; q++) {
            d.w[2 * q] = make_int4(L.l[q][0], L.l[q][1], L.l[q][2], L.l[q][3]);
            d.w[2 * q + 1] = make_int4(L.l[q][4], L.l[q][5], L.l[q][6], L.l[q][7]);
        }
        d.w[6] = make_int4(L.sum[0], L.sum[1], L.sum[2], __float_as_int(L.S));
    }
    __syncthreads();
    float accv[R * P];
#pragma unroll
    for (int k = 0; k < P; k++) {
        Limbs L;
        unpack_limbs(s_l[k][lane], L);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float dd = group_dot_q3_limbs(pl[k][r][0], pl[k][r][1], pl[k][r][2], L);
            accv[r * P + k] = live ? dd * ti_h2f(sv[k][r]) : 0.0f;
        }
    }
    constexpr int SLOTS = R * P, SPAN = 64 / SLOTS;
    const float tot = transpose_reduce<64, SLOTS>(accv, lane);
    const int r = lane / (P * SPAN);
    float o[P];
#pragma unroll
    for (int k = 0; k < P; k++) o[k] = __shfl(tot, (r * P + k) * SPAN, 64);
    const int n = row0 + r;
    if (lane % (P * SPAN) == 0 && r < R && n < H) {
        float sacc = 0.0f;
#pragma unroll
        for (int k = 0; k < P; k++) {
            const float pr = wt[k] * o[k];
            sacc = sacc + pr;
        }
        x[n] = x[n] + sacc;
    }
}

// swiglu (lfm25.js:1831-1847): y = g / (1 + e^-g) * u
__global__ void k_swiglu_f32(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ y, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float a = g[i];
        y[i] = a / (1.0f + expf(-a)) * u[i];
    }
}

// ---- combine: x[t] += sum_k wt[t,k] * o[t*K + k] ------------------------------------------
__global__ void k_moe_combine(float* __restrict__ x, const float* __restrict__ o, const float* __restrict__ wt, int H,
                              int K, long TH) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= TH) return;
    const long t = i / H, h = i % H;
    float s = 0.0f;
    for (int k = 0; k < K; k++) {
        const float p = wt[t * K + k] * o[(t * K + k) * H + h];
        s = s + p;
    }
    x[i] = x[i] + s;
}

}  // namespace

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int ti_requant43(ti_ctx* c, const uint32_t* pack4, const uint16_t* sc4, int rows, int K, uint32_t* p3,
                            uint16_t* s3) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(pack4 && sc4 && p3 && s3, "ti_requant43: null buffer");
    TI_REQUIRE(rows > 0 && K > 0 && K % 32 == 0, "ti_requant43: need rows > 0 and K %% 32 == 0 (rows=%d K=%d)", rows, K);
    TI_REQUIRE(al16(pack4), "ti_requant43: pack4 must be 16-byte aligned");
    const long ng = (long)rows * (K / 32);
    k_requant43<<<(unsigned)((ng + 255) / 256), 256, 0, c->stream>>>(pack4, sc4, p3, s3, ng);
    TI_LAUNCHED("k_requant43");
    return TI_OK;
}

extern "C" int ti_router(ti_ctx* c, const float* logits, const float* bias, int T, int nE, int topk, int32_t* idx,
                         float* wt) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(logits && idx && wt, "ti_router: null buffer");
    TI_REQUIRE(T > 0 && nE > 0 && nE <= ROUTER_EMAX && topk > 0 && topk <= nE && topk <= 64,
               "ti_router: need T > 0, 0 < topk <= nE <= %d (T=%d nE=%d topk=%d)", ROUTER_EMAX, T, nE, topk);
    k_router<<<T, 64, 0, c->stream>>>(logits, bias, nE, topk, idx, wt);
    TI_LAUNCHED("k_router");
    return TI_OK;
}

extern "C" int ti_moe_gemv_q3(ti_ctx* c, const float* x, const uint32_t* p3, const uint16_t* s3, const int32_t* idx,
                              float* y, int pairs, int N, int K, int in_stride, int xdiv, int nE) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && p3 && s3 && idx && y, "ti_moe_gemv_q3: null buffer");
    TI_REQUIRE(pairs > 0 && pairs < 65536 && N > 0 && nE > 0, "ti_moe_gemv_q3: bad pairs/N/nE (pairs=%d N=%d nE=%d)",
               pairs, N, nE);
    TI_REQUIRE(K > 0 && K % 32 == 0 && K <= 4096, "ti_moe_gemv_q3: need K %% 32 == 0 and K <= 4096 (K=%d)", K);
    TI_REQUIRE(xdiv > 0 && in_stride >= K && in_stride % 4 == 0, "ti_moe_gemv_q3: bad in_stride/xdiv");
    TI_REQUIRE(al16(x), "ti_moe_gemv_q3: x must be 16-byte aligned");
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)pairs);
    if (K <= 2048) k_moe_gemv_q3<1><<<grid, 256, 0, c->stream>>>(x, p3, s3, idx, y, N, K, in_stride, xdiv, nE);
    else k_moe_gemv_q3<2><<<grid, 256, 0, c->stream>>>(x, p3, s3, idx, y, N, K, in_stride, xdiv, nE);
    TI_LAUNCHED("k_moe_gemv_q3");
    return TI_OK;
}

extern "C" int ti_moe_gemm_q3(ti_ctx* c, const float* src, int src_rows, const uint32_t* p3, const uint16_t* s3,
                              const int32_t* ridx, float* y, int P, int N, int K, int src_div, int nE) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(src && p3 && s3 && ridx && y, "ti_moe_gemm_q3: null buffer");
    TI_REQUIRE(P > 0 && N > 0 && nE > 0 && nE < 65536 && src_div > 0, "ti_moe_gemm_q3: bad P/N/nE/src_div");
    TI_REQUIRE(K > 0 && K % 32 == 0 && K <= 4096, "ti_moe_gemm_q3: need K %% 32 == 0 and K <= 4096 (K=%d)", K);
    TI_REQUIRE(src_rows > 0 && (P - 1) / src_div < src_rows, "ti_moe_gemm_q3: pair %d reads row %d of %d", P - 1,
               (P - 1) / src_div, src_rows);
    TI_REQUIRE((long)src_rows * K <= (long)TI_ACT_CAP * TI_ACT_TMAX, "ti_moe_gemm_q3: src_rows*K=%ld exceeds %ld",
               (long)src_rows * K, (long)TI_ACT_CAP * TI_ACT_TMAX);
    // quantAct8 (lfm25.js:1487-1494): per row, per 32-group int8 into the context's scratch,
    // words in the GEMM's element order (k_router_quant with no router workgroups)
    const int nq = src_rows * (K / 32);
    k_router_quant<<<(unsigned)((nq + 63) / 64), 64, 0, c->stream>>>(nullptr, nullptr, 0, 0, nullptr, nullptr, 0, src,
                                                                     c->act_q, c->act_s, nq);
    TI_LAUNCHED("k_router_quant (quantizer only)");
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)nE);
    const int spec = 2 * P >= nE;   // most experts are routed to: weights loaded before the scan
    if (K <= 2048) k_moe_gemm_q3<1><<<grid, 256, 0, c->stream>>>(c->act_q, c->act_s, p3, s3, ridx, y, P, N, K, src_div, spec, p3, s3, y);
    else k_moe_gemm_q3<2><<<grid, 256, 0, c->stream>>>(c->act_q, c->act_s, p3, s3, ridx, y, P, N, K, src_div, spec, p3, s3, y);
    TI_LAUNCHED("k_moe_gemm_q3");
    return TI_OK;
}

// quantAct8 of swiglu(g, u) (lfm25.js:1831-1847 then :1487-1494): group gi's 32 values
// a / (1 + e^-a) * u with k_swiglu_f32's operations, written to act as well, then q8_group
// (words in k_moe_gemm_q3's element order).
__global__ __launch_bounds__(64) void k_quant_swiglu_q8(const float* __restrict__ g, const float* __restrict__ u,
                                                        float* __restrict__ act, uint32_t* __restrict__ xq,
                                                        float* __restrict__ xs, int ng) {
    const int gi = blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= ng) return;
    float v[32], w[32];
    load32(g + (size_t)gi * 32, v);
    load32(u + (size_t)gi * 32, w);
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const float a = v[j];
        v[j] = a / (1.0f + expf(-a)) * w[j];
    }
    float4* ao = reinterpret_cast<float4*>(act + (size_t)gi * 32);
#pragma unroll
    for (int j = 0; j < 8; j++) ao[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    q8_group<true>(v, xq + (size_t)gi * 8, xs + gi, nullptr);
}

extern "C" int ti_moe_prefill_q3(ti_ctx* c, float* x, const float* normed, const float* logits, const float* bias,
                                 const uint32_t* w1p, const uint16_t* w1s, const uint32_t* w3p, const uint16_t* w3s,
                                 const uint32_t* w2p, const uint16_t* w2s, int32_t* idx, float* wt, float* gate,
                                 float* up, float* act, float* out, int T, int H, int I, int nE, int topk) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && normed && logits && w1p && w1s && w3p && w3s && w2p && w2s && idx && wt && gate && up && act && out,
               "ti_moe_prefill_q3: null buffer");
    TI_REQUIRE(T > 0 && nE > 0 && nE <= ROUTER_EMAX && nE < 65536 && topk > 0 && topk <= nE && topk <= 64,
               "ti_moe_prefill_q3: need T > 0, 0 < topk <= nE <= %d (T=%d nE=%d topk=%d)", ROUTER_EMAX, T, nE, topk);
    TI_REQUIRE(H > 0 && I > 0 && H % 32 == 0 && I % 32 == 0 && H <= 4096 && I <= 4096,
               "ti_moe_prefill_q3: H, I multiples of 32, <= 4096 (H=%d I=%d)", H, I);
    const long P = (long)T * topk;
    const long cap = (long)TI_ACT_CAP * TI_ACT_TMAX;
    TI_REQUIRE((long)T * H <= cap && P * I <= cap, "ti_moe_prefill_q3: T*H=%ld or P*I=%ld exceeds %ld", (long)T * H,
               P * I, cap);
    TI_REQUIRE(al16(normed) && al16(gate) && al16(up) && al16(act),
               "ti_moe_prefill_q3: normed, gate, up and act must be 16-byte aligned");
    const int nq = T * (H / 32);
    k_router_quant<<<(unsigned)(T + (nq + 63) / 64), 64, 0, c->stream>>>(logits, bias, nE, topk, idx, wt, T, normed,
                                                                          c->act_q, c->act_s, nq);
    TI_LAUNCHED("k_router_quant");
    const int spec = 2 * P >= nE;
    dim3 g13((unsigned)((I + 15) / 16), (unsigned)nE, 2);
    if (H <= 2048) k_moe_gemm_q3<1><<<g13, 256, 0, c->stream>>>(c->act_q, c->act_s, w1p, w1s, idx, gate, (int)P, I, H, topk, spec, w3p, w3s, up);
    else k_moe_gemm_q3<2><<<g13, 256, 0, c->stream>>>(c->act_q, c->act_s, w1p, w1s, idx, gate, (int)P, I, H, topk, spec, w3p, w3s, up);
    TI_LAUNCHED("k_moe_gemm_q3 (w1, w3)");
    const long ng = P * (I / 32);
    k_quant_swiglu_q8<<<(unsigned)((ng + 63) / 64), 64, 0, c->stream>>>(gate, up, act, c->act_q, c->act_s, (int)ng);
    TI_LAUNCHED("k_quant_swiglu_q8");
    dim3 g2((unsigned)((H + 15) / 16), (unsigned)nE, 1);
    if (I <= 2048) k_moe_gemm_q3<1><<<g2, 256, 0, c->stream>>>(c->act_q, c->act_s, w2p, w2s, idx, out, (int)P, H, I, 1, spec, w2p, w2s, out);
    else k_moe_gemm_q3<2><<<g2, 256, 0, c->stream>>>(c->act_q, c->act_s, w2p, w2s, idx, out, (int)P, H, I, 1, spec, w2p, w2s, out);
    TI_LAUNCHED("k_moe_gemm_q3 (w2)");
    const long th = (long)T * H;
    k_moe_combine<<<(unsigned)((th + 255) / 256), 256, 0, c->stream>>>(x, out, wt, H, topk, th);
    TI_LAUNCHED("k_moe_combine");
    return TI_OK;
}

extern "C" int ti_moe_decode_q3(ti_ctx* c, float* x, const float* normed, const float* logits, const float* bias,
                                const uint32_t* w1p, const uint16_t* w1s, const uint32_t* w3p, const uint16_t* w3s,
                                const uint32_t* w2p, const uint16_t* w2s, int32_t* idx, float* wt, float* act, int H, int I,
                                int nE, int topk) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && normed && logits && w1p && w1s && w3p && w3s && w2p && w2s && idx && wt && act,
               "ti_moe_decode_q3: null buffer");
    TI_REQUIRE(nE > 0 && nE <= RT_EPL * 64 && (topk == 1 || topk == 2 || topk == 4 || topk == 8) && topk <= nE,
               "ti_moe_decode_q3: need nE <= 256 and topk in {1, 2, 4, 8} (nE=%d topk=%d)", nE, topk);
    TI_REQUIRE(H > 0 && I > 0 && H % 32 == 0 && I % 32 == 0 && H <= 4096 && I <= 4096,
               "ti_moe_decode_q3: H, I multiples of 32, <= 4096 (H=%d I=%d)", H, I);
    TI_REQUIRE(al16(normed) && al16(act), "ti_moe_decode_q3: normed and act must be 16-byte aligned");
    // measured on MI355X (LFM2.5 shapes): 4 rows per wave for w1/w3, 2 for w2
    constexpr int K1R = 4, R2 = 2;
    dim3 g1((unsigned)((I + 4 * K1R - 1) / (4 * K1R)), (unsigned)topk);
    if (H <= 2048) k_moe_gateup_dec<1, K1R><<<g1, 256, 0, c->stream>>>(normed, logits, bias, nE, topk, w1p, w1s, w3p, w3s, act, idx, wt, I, H);
    else k_moe_gateup_dec<2, K1R><<<g1, 256, 0, c->stream>>>(normed, logits, bias, nE, topk, w1p, w1s, w3p, w3s, act, idx, wt, I, H);
    TI_LAUNCHED("k_moe_gateup_dec");
    if (I <= 2048 && topk <= 4) {
        const unsigned g4 = (unsigned)((H + 4 * R2 - 1) / (4 * R2));
        if (topk == 1) k_moe_down_dec_pl<1, R2><<<g4, 256, 0, c->stream>>>(act, w2p, w2s, idx, wt, x, H, I, nE);
        else if (topk == 2) k_moe_down_dec_pl<2, R2><<<g4, 256, 0, c->stream>>>(act, w2p, w2s, idx, wt, x, H, I, nE);
        else k_moe_down_dec_pl<4, R2><<<g4, 256, 0, c->stream>>>(act, w2p, w2s, idx, wt, x, H, I, nE);
        TI_LAUNCHED("k_moe_down_dec");
        return TI_OK;
    }
    const unsigned g2 = (unsigned)((H + 15) / 16);
#define DD(GL_, P_) \
    if ((I <= 2048) == (GL_ == 1) && topk == P_) { k_moe_down_dec<GL_, P_><<<g2, 256, 0, c->stream>>>(act, w2p, w2s, idx, wt, x, H, I, nE); TI_LAUNCHED("k_moe_down_dec"); return TI_OK; }
    DD(1, 1) DD(1, 2) DD(1, 4) DD(1, 8) DD(2, 1) DD(2, 2) DD(2, 4) DD(2, 8)
#undef DD
    return ti_fail(TI_ERR_INVALID, "ti_moe_decode_q3: no kernel for I=%d topk=%d", I, topk);
}

extern "C" int ti_swiglu(ti_ctx* c, const float* g, const float* u, float* y, long n) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(g && u && y && n > 0, "ti_swiglu: null buffer or n <= 0");
    TI_REQUIRE(n < (1L << 40), "ti_swiglu: n too large");
    k_swiglu_f32<<<(unsigned)((n + 255) / 256), 256, 0, c->stream>>>(g, u, y, n);
    TI_LAUNCHED("k_swiglu_f32");
    return TI_OK;
}

extern "C" int ti_moe_combine(ti_ctx* c, float* x, const float* o, const float* wt, int H, int K, int T) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && o && wt, "ti_moe_combine: null buffer");
    TI_REQUIRE(H > 0 && K > 0 && T > 0, "ti_moe_combine: bad shape");
    const long th = (long)T * H;
    k_moe_combine<<<(unsigned)((th + 255) / 256), 256, 0, c->stream>>>(x, o, wt, H, K, th);
    TI_LAUNCHED("k_moe_combine");
    return TI_OK;
}
