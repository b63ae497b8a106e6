// k_moe.hip — the int3 MoE expert path of LFM2.5 (models/lfm25.js):
//  int4 -> int3 cascade requant into bitplanes    _requant43        lfm25.js:833-856
//  sigmoid + bias top-k router                     ROUTER_WGSL       lfm25.js:111-146
//  pair-indexed int3 GEMV, f32 activation (T = 1) idxGemv3          lfm25.js:1924-1980
//      expert-grouped int3 x int8 GEMM (T > 1)        moeSort+moeGemm3  lfm25.js:1503-1647
//      weighted combine into the residual              MOECOMBINE_WGSL   lfm25.js:1982-2000
//
// int3 group (32 weights): three u32 bitplanes, bit i of plane b = bit b of (q3 + 4) for
// element i, then one f16 scale; rows of all experts stacked expert-major (row = e*N + n).
// The kernels turn 4 elements' plane bits into 4 bytes of (q3 + 4) with the bit-spread
// multiply ((b >> i) & 15) * 0x00204081 & 0x01010101 (bit k lands at bit 8k) and dot them
// with v_dot4_i32_i8; the +4 offset is removed once per group from the activation sum.
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
__global__ __launch_bounds__(64) void k_router(const float* __restrict__ logits, const float* __restrict__ bias, int nE,
                                               int topk, int32_t* __restrict__ idx, float* __restrict__ wt) {
    __shared__ float sc[ROUTER_EMAX], sel[ROUTER_EMAX];
    __shared__ int chosen[ROUTER_EMAX];
    const int t = blockIdx.x, lane = threadIdx.x;
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
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
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

// ---- decode: pair-indexed GEMV with the f32 activation ----------------------------
// 4 elements' (q3 + 4) as bytes from the three planes' bits i..i+3
__device__ __forceinline__ uint32_t q3_bytes(uint32_t b0, uint32_t b1, uint32_t b2, int i) {
    const uint32_t s0 = (((b0 >> i) & 15u) * 0x00204081u) & 0x01010101u;
    const uint32_t s1 = (((b1 >> i) & 15u) * 0x00204081u) & 0x01010101u;
    const uint32_t s2 = (((b2 >> i) & 15u) * 0x00204081u) & 0x01010101u;
    return s0 | (s1 << 1) | (s2 << 2);
}

// f32 activation group as exact fixed point (as k_gemv_q4_f32): x_j = X_j * 2^(ex-22),
// X = l2*65536 + l1*256 + l0 with signed int8 limbs, natural element order
struct Limbs {
    int l[3][8];        // limb, word of 4 elements
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
            L.l[q][w] = (int)((uint32_t)(b[q][4 * w] & 0xff) | ((uint32_t)(b[q][4 * w + 1] & 0xff) << 8) |
                              ((uint32_t)(b[q][4 * w + 2] & 0xff) << 16) | ((uint32_t)(b[q][4 * w + 3] & 0xff) << 24));
            s += b[q][4 * w] + b[q][4 * w + 1] + b[q][4 * w + 2] + b[q][4 * w + 3];
        }
        L.sum[q] = s;
    }
}

// sum_i (q3_i) * x_i over one group, q3 = stored - 4
__device__ __forceinline__ float group_dot_q3_limbs(uint32_t b0, uint32_t b1, uint32_t b2, const Limbs& L) {
    int d[3] = {0, 0, 0};
#pragma unroll
    for (int w = 0; w < 8; w++) {
        const int q = (int)q3_bytes(b0, b1, b2, 4 * w);
#pragma unroll
        for (int k = 0; k < 3; k++) d[k] = __builtin_amdgcn_sdot4(q, L.l[k][w], d[k], false);
    }
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
// lists its expert's pairs in pair order (ballot compaction in LDS). On the first hit each
// wave turns its 4 rows' bitplanes into (q + 4) bytes, kept in registers; every listed
// pair then reads its int8 activation group (L2-resident) and scale:
//   dot = sum (q + 4) a - 4 sum a   (exact int32),   y[pair, n] = sum_g dot * s_x * s_w.
// Workgroups of experts nobody chose read only the ids.
template <int GL>
__global__ __launch_bounds__(256) void k_moe_gemm_q3(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                     const uint32_t* __restrict__ p3, const uint16_t* __restrict__ s3,
                                                     const int32_t* __restrict__ ridx, float* __restrict__ y, int P, int N,
                                                     int K, int src_div) {
    __shared__ int s_list[256];
    __shared__ int s_wcnt[4];
    const int e = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gpr = K / 32;
    const int row0 = blockIdx.x * 16 + wave * MOE_R;
    uint32_t qb[MOE_R][GL][8];
    float sw[MOE_R][GL];
    bool have = false;
    for (int c0 = 0; c0 < P; c0 += 256) {
        const int p = c0 + tid;
        const bool hit = p < P && ridx[p] == e;
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
        if (!have) {
            have = true;
#pragma unroll
            for (int r = 0; r < MOE_R; r++) {
                const int n = min(row0 + r, N - 1);
#pragma unroll
                for (int h = 0; h < GL; h++) {
                    const int g = lane + 64 * h;
                    const int gc = g < gpr ? g : gpr - 1;
                    const size_t gi = ((size_t)e * N + n) * gpr + gc;
                    const uint32_t b0 = __builtin_nontemporal_load(p3 + gi * 3);
                    const uint32_t b1 = __builtin_nontemporal_load(p3 + gi * 3 + 1);
                    const uint32_t b2 = __builtin_nontemporal_load(p3 + gi * 3 + 2);
                    sw[r][h] = g < gpr ? ti_h2f(s3[gi]) : 0.0f;
#pragma unroll
                    for (int w = 0; w < 8; w++) qb[r][h][w] = q3_bytes(b0, b1, b2, 4 * w);
                }
            }
        }
        for (int i = 0; i < tot; i++) {
            const int pair = s_list[i];
            const int src = pair / src_div;
            float accv[MOE_R] = {};
#pragma unroll
            for (int h = 0; h < GL; h++) {
                const int g = lane + 64 * h;
                const int gc = g < gpr ? g : gpr - 1;
                const uint4* a4 = reinterpret_cast<const uint4*>(xq + (size_t)src * (K / 4) + gc * 8);
                const uint4 u0 = a4[0], u1 = a4[1];
                const float as = xs[(size_t)src * gpr + gc];
                const int a[8] = {(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
                int asum = 0;
#pragma unroll
                for (int w = 0; w < 8; w++) asum = __builtin_amdgcn_sdot4(a[w], 0x01010101, asum, false);
#pragma unroll
                for (int r = 0; r < MOE_R; r++) {
                    int d = 0;
#pragma unroll
                    for (int w = 0; w < 8; w++) d = __builtin_amdgcn_sdot4((int)qb[r][h][w], a[w], d, false);
                    accv[r] = fmaf((float)(d - 4 * asum), as * sw[r][h], accv[r]);
                }
            }
            const float tot_r = transpose_reduce<64, MOE_R>(accv, lane);
            const int n = row0 + lane / (64 / MOE_R);
            if ((lane % (64 / MOE_R)) == 0 && n < N) y[(size_t)pair * N + n] = tot_r;
        }
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

int ti_quant_act_q8_async(ti_ctx* c, const float* x, uint32_t* xq, float* xs, int32_t* xsum, int groups);

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
    // quantAct8 (lfm25.js:1487-1494): per row, per 32-group int8 into the context's scratch
    int rc = ti_quant_act_q8_async(c, src, c->act_q, c->act_s, nullptr, src_rows * (K / 32));
    if (rc) return rc;
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)nE);
    if (K <= 2048) k_moe_gemm_q3<1><<<grid, 256, 0, c->stream>>>(c->act_q, c->act_s, p3, s3, ridx, y, P, N, K, src_div);
    else k_moe_gemm_q3<2><<<grid, 256, 0, c->stream>>>(c->act_q, c->act_s, p3, s3, ridx, y, P, N, K, src_div);
    TI_LAUNCHED("k_moe_gemm_q3");
    return TI_OK;
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
