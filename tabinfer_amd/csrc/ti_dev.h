// ti_dev.h — device helpers shared by the decode-path kernels (gfx950).
//  int4 x int8 group dots, f32-activation limb dots, the per-32 int8 activation
//  quantizer and the 256-thread RMSNorm reduction, each in the exact arithmetic
//  order the reference uses wherever bits matter.
#pragma once
#include "ti_internal.h"

namespace {

constexpr uint32_t M4 = 0x0F0F0F0Fu;

__device__ __forceinline__ uint32_t even_bytes(uint32_t a0, uint32_t a1) {   // [x0,x2,x4,x6]
    return (a0 & 0xffu) | ((a0 >> 8) & 0xff00u) | ((a1 & 0xffu) << 16) | ((a1 << 8) & 0xff000000u);
}
__device__ __forceinline__ uint32_t odd_bytes(uint32_t a0, uint32_t a1) {    // [x1,x3,x5,x7]
    return ((a0 >> 8) & 0xffu) | ((a0 >> 16) & 0xff00u) | ((a1 << 8) & 0xff0000u) | (a1 & 0xff000000u);
}

// Activation slice of one group for the int8 path.
struct ActQ8 {
    int xe[4], xo[4];
    int corr;      // 8 * sum of the 32 codes
    float s;       // activation group scale
};

// the group's 32 codes (two 16-byte words) and scale, unpacked for group_dot_q8
__device__ __forceinline__ void act_q8_from_words(const uint4 (&u)[2], float s, ActQ8& a) {
    uint32_t w[8] = {u[0].x, u[0].y, u[0].z, u[0].w, u[1].x, u[1].y, u[1].z, u[1].w};
    int sum = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        a.xe[m] = (int)even_bytes(w[2 * m], w[2 * m + 1]);
        a.xo[m] = (int)odd_bytes(w[2 * m], w[2 * m + 1]);
        sum = __builtin_amdgcn_sdot4((int)w[2 * m], 0x01010101, sum, false);
        sum = __builtin_amdgcn_sdot4((int)w[2 * m + 1], 0x01010101, sum, false);
    }
    a.corr = 8 * sum;
    a.s = s;
}

__device__ __forceinline__ void load_act_q8(const uint32_t* __restrict__ xq, const float* __restrict__ xs, int g, ActQ8& a) {
    const uint4* p = reinterpret_cast<const uint4*>(xq + (size_t)g * 8);
    uint4 u0 = p[0], u1 = p[1];
    uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    int sum = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        a.xe[m] = (int)even_bytes(w[2 * m], w[2 * m + 1]);
        a.xo[m] = (int)odd_bytes(w[2 * m], w[2 * m + 1]);
        sum = __builtin_amdgcn_sdot4((int)w[2 * m], 0x01010101, sum, false);
        sum = __builtin_amdgcn_sdot4((int)w[2 * m + 1], 0x01010101, sum, false);
    }
    a.corr = 8 * sum;
    a.s = xs ? xs[g] : 0.0f;
}

// Exact int32 dot of one weight group (16 bytes) with the lane's activation group.
__device__ __forceinline__ int group_dot_q8(const uint4 w, const ActQ8& a) {
    int d = 0;
    d = __builtin_amdgcn_sdot4((int)(w.x & M4), a.xe[0], d, false);
    d = __builtin_amdgcn_sdot4((int)((w.x >> 4) & M4), a.xo[0], d, false);
    d = __builtin_amdgcn_sdot4((int)(w.y & M4), a.xe[1], d, false);
    d = __builtin_amdgcn_sdot4((int)((w.y >> 4) & M4), a.xo[1], d, false);
    d = __builtin_amdgcn_sdot4((int)(w.z & M4), a.xe[2], d, false);
    d = __builtin_amdgcn_sdot4((int)((w.z >> 4) & M4), a.xo[2], d, false);
    d = __builtin_amdgcn_sdot4((int)(w.w & M4), a.xe[3], d, false);
    d = __builtin_amdgcn_sdot4((int)((w.w >> 4) & M4), a.xo[3], d, false);
    return d - a.corr;
}

__device__ __forceinline__ void store_out(float* __restrict__ y, long row, float v, int acc) {
    y[row] = acc ? y[row] + v : v;
}

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Weights are streamed exactly once per call: non-temporal loads keep them from
// displacing the (re-read) activation and scale lines in the caches.
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
    v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint16_t ld_nt(const uint16_t* p) { return __builtin_nontemporal_load(p); }

// Sum R per-lane accumulators across the LPR lanes that share them, leaving the
// total of accumulator (li / (LPR/R)) in every lane: each of the first log2(R)
// butterfly steps hands half of the remaining accumulators to the partner lane
// (lane li ^ o): the lane whose bit o is set keeps the upper half and receives the
// partner's upper half, the other keeps and receives the lower half. Costs R-1 +
// log2(LPR/R) exchanges instead of R*log2(LPR). The exchanges need no per-lane
// selects, which the compiler would otherwise turn into dynamic register-array
// indexing: across 32/16 lanes the permlane swaps deliver exactly (kept, received)
// as their two results; within a row, bank-masked DPP writes the upper lanes' values
// over the lower lanes'. Every sum is kept + received, as a plain xor butterfly forms it.
__device__ __forceinline__ float tr_pair(float lo, float hi, int o) {
    const int l = __builtin_bit_cast(int, lo), h = __builtin_bit_cast(int, hi);
    if (o == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(l, h, false, false);
        return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
    }
    if (o == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(l, h, false, false);
        return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
    }
    if (o == 8) {   // banks 2,3 (lanes 8-15 of a row) hold the upper half; row_ror:8 is xor 8
        const int keep = __builtin_amdgcn_update_dpp(l, h, 0xE4, 0xF, 0xC, false);
        int recv = __builtin_amdgcn_update_dpp(l, l, 0x128, 0xF, 0x3, false);
        recv = __builtin_amdgcn_update_dpp(recv, h, 0x128, 0xF, 0xC, false);
        return __builtin_bit_cast(float, keep) + __builtin_bit_cast(float, recv);
    }
    if (o == 4) {   // banks 1,3 hold the upper half; partner lane +4 (row_shl) below, -4 (row_shr) above
        const int keep = __builtin_amdgcn_update_dpp(l, h, 0xE4, 0xF, 0xA, false);
        int recv = __builtin_amdgcn_update_dpp(l, l, 0x104, 0xF, 0x5, false);
        recv = __builtin_amdgcn_update_dpp(recv, h, 0x114, 0xF, 0xA, false);
        return __builtin_bit_cast(float, keep) + __builtin_bit_cast(float, recv);
    }
    // o = 2, 1: both halves exchanged, the sums selected (no array element is selected)
    const bool up = (threadIdx.x & o) != 0;
    const float slo = lo + ti_xor(lo, o), shi = hi + ti_xor(hi, o);
    return up ? shi : slo;
}

template <int LPR, int R>
__device__ __forceinline__ float transpose_reduce(float (&v)[R], int li) {
    static_assert(R <= LPR || LPR == 1, "R must not exceed the lanes per row");
    (void)li;
    int k = R;
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) {
        if (k > 1) {
#pragma unroll
            for (int i = 0; i < R / 2; i++)
                if (i < k / 2) v[i] = tr_pair(v[i], v[i + k / 2], o);
            k >>= 1;
        } else {
            v[0] += ti_xor(v[0], o);
        }
    }
    return v[0];
}

// ---------------------------------------------------------------------------
// y (+)= W x, f32 activation (lm_head path). Per element: one byte->f32
// convert and one FMA on the unsigned nibble; the -8 offset is removed once per
// group (sum n*x - 8*sum x).
// ---------------------------------------------------------------------------
struct ActF32 {
    float x[32];   // element order of the group: x[0..31]
    float corr;    // 8 * sum x
};

__device__ __forceinline__ void load_act_f32(const float* __restrict__ x, int g, ActF32& a) {
    const float4* p = reinterpret_cast<const float4*>(x + (size_t)g * 32);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float4 t = p[i];
        a.x[4 * i] = t.x; a.x[4 * i + 1] = t.y; a.x[4 * i + 2] = t.z; a.x[4 * i + 3] = t.w;
    }
#pragma unroll
    for (int i = 0; i < 32; i++) s += a.x[i];
    a.corr = 8.0f * s;
}

__device__ __forceinline__ float word_dot_f32(uint32_t p, const float* x8, float acc) {
    uint32_t lo = p & M4, hi = (p >> 4) & M4;
    acc = fmaf((float)(lo & 0xffu), x8[0], acc);
    acc = fmaf((float)(hi & 0xffu), x8[1], acc);
    acc = fmaf((float)((lo >> 8) & 0xffu), x8[2], acc);
    acc = fmaf((float)((hi >> 8) & 0xffu), x8[3], acc);
    acc = fmaf((float)((lo >> 16) & 0xffu), x8[4], acc);
    acc = fmaf((float)((hi >> 16) & 0xffu), x8[5], acc);
    acc = fmaf((float)(lo >> 24), x8[6], acc);
    acc = fmaf((float)(hi >> 24), x8[7], acc);
    return acc;
}

__device__ __forceinline__ float group_dot_f32(const uint4 w, const ActF32& a) {
    float d0 = word_dot_f32(w.x, a.x + 0, 0.0f);
    float d1 = word_dot_f32(w.y, a.x + 8, 0.0f);
    float d2 = word_dot_f32(w.z, a.x + 16, 0.0f);
    float d3 = word_dot_f32(w.w, a.x + 24, 0.0f);
    return ((d0 + d1) + (d2 + d3)) - a.corr;
}

// f32 activation as exact fixed point: per 32-group, x_j = X_j * 2^(ex-22) with
// |X_j| <= 2^22 (ex = exponent of the group absmax), X split into three signed
// int8 limbs X = l2*65536 + l1*256 + l0. Each limb dots with the nibbles through
// v_dot4_i32_i8 exactly; the only approximation is rounding x to 22 bits below its
// group maximum (relative 2^-23), i.e. at the level of f32 rounding itself.
struct ActLimb {
    int e[3][4], o[3][4];   // limb l, weight word m: even / odd element bytes
    int corr[3];            // 8 * sum of limb l
    float S;                // 2^(ex-22)
};

__device__ __forceinline__ void load_act_limbs(const float* __restrict__ x, int g, ActLimb& a) {
    const float4* p = reinterpret_cast<const float4*>(x + (size_t)g * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float4 t = p[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) mx = fmaxf(mx, fabsf(v[j]));
    int ex = 0;
    if (mx > 0.0f) (void)frexpf(mx, &ex);          // mx < 2^ex
    a.S = ldexpf(1.0f, ex - 22);
    int lb[3][32];
#pragma unroll
    for (int j = 0; j < 32; j++) {
        int X = mx > 0.0f ? (int)rintf(ldexpf(v[j], 22 - ex)) : 0;
        int l0 = ((X & 0xff) ^ 0x80) - 0x80;
        int X1 = (X - l0) >> 8;
        int l1 = ((X1 & 0xff) ^ 0x80) - 0x80;
        int l2 = (X1 - l1) >> 8;
        lb[0][j] = l0; lb[1][j] = l1; lb[2][j] = l2;
    }
#pragma unroll
    for (int l = 0; l < 3; l++) {
        int sum = 0;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int* q = lb[l] + 8 * m;
            a.e[l][m] = (int)((uint32_t)(q[0] & 0xff) | ((uint32_t)(q[2] & 0xff) << 8) |
                              ((uint32_t)(q[4] & 0xff) << 16) | ((uint32_t)(q[6] & 0xff) << 24));
            a.o[l][m] = (int)((uint32_t)(q[1] & 0xff) | ((uint32_t)(q[3] & 0xff) << 8) |
                              ((uint32_t)(q[5] & 0xff) << 16) | ((uint32_t)(q[7] & 0xff) << 24));
            sum += q[0] + q[1] + q[2] + q[3] + q[4] + q[5] + q[6] + q[7];
        }
        a.corr[l] = 8 * sum;
    }
}

// sum_j (n_j - 8) * x_j for one 16-byte weight group, through the three limbs
__device__ __forceinline__ float group_dot_limbs(const uint4 w, const ActLimb& a) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    int d[3] = {0, 0, 0};
#pragma unroll
    for (int m = 0; m < 4; m++) {
        int lo = (int)(ws[m] & M4), hi = (int)((ws[m] >> 4) & M4);
#pragma unroll
        for (int l = 0; l < 3; l++) {
            d[l] = __builtin_amdgcn_sdot4(lo, a.e[l][m], d[l], false);
            d[l] = __builtin_amdgcn_sdot4(hi, a.o[l][m], d[l], false);
        }
    }
    int t = (d[2] - a.corr[2]) * 256 + (d[1] - a.corr[1]);     // |t| < 2^23: exact in f32
    return fmaf((float)t, 256.0f, (float)(d[0] - a.corr[0])) * a.S;
}

// ---------------------------------------------------------------------------
// one thread per 32-group. scale = absmax/127, inv = 1/scale (0 if the
// group is zero), q = clamp(round-half-even(v*inv), -127, 127); the per-16
// sums feed the ternary identity. Word w holds elements 4w..4w+3; with COLS,
// elements w, w+8, w+16, w+24 (the order the int3 expert kernels dot in).
// ---------------------------------------------------------------------------
template <bool COLS = false>
__device__ __forceinline__ void q8_group(const float* v, uint32_t* xq, float* xs, int32_t* xsum16) {
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) mx = fmaxf(mx, fabsf(v[j]));
    float scale = mx / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    *xs = scale;
    int q[32];
#pragma unroll
    for (int j = 0; j < 32; j++) {
        float p = v[j] * inv;
        int qi = (int)rintf(p);
        qi = qi < -127 ? -127 : (qi > 127 ? 127 : qi);
        q[j] = qi;
    }
    uint32_t wds[8];
#pragma unroll
    for (int w = 0; w < 8; w++) {
        const int st = COLS ? 8 : 1, e0 = COLS ? w : 4 * w;
        wds[w] = (uint32_t)(q[e0] & 0xff) | ((uint32_t)(q[e0 + st] & 0xff) << 8) |
                 ((uint32_t)(q[e0 + 2 * st] & 0xff) << 16) | ((uint32_t)(q[e0 + 3 * st] & 0xff) << 24);
    }
    uint4* o = reinterpret_cast<uint4*>(xq);
    o[0] = make_uint4(wds[0], wds[1], wds[2], wds[3]);
    o[1] = make_uint4(wds[4], wds[5], wds[6], wds[7]);
    if (xsum16) {
        int a = 0, b = 0;
#pragma unroll
        for (int j = 0; j < 16; j++) { a += q[j]; b += q[16 + j]; }
        xsum16[0] = a;
        xsum16[1] = b;
    }
}

__device__ __forceinline__ void load32(const float* __restrict__ src, float* v) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float4 t = s4[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}

// ---------------------------------------------------------------------------
// RMSNorm: one 256-thread workgroup per row. The sum of squares uses the
// reference's order — 256 strided per-thread partials then a 128..1 tree —
// so the normalized values, and hence the int8 codes, are reproducible.
// inv = 1/sqrt(sum/H + eps) with IEEE division and square root.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float rms_inv_256(const float* __restrict__ x, int H, float eps, float* red) {
    int t = threadIdx.x;
    float s = 0.0f;
    for (int i = t; i < H; i += 256) { float sq = x[i] * x[i]; s = s + sq; }
    float m = ti_tree_sum_256(s, red) / (float)H;
    __syncthreads();   // red is free again for the caller
    m = m + eps;
    return 1.0f / sqrtf(m);
}

// ---- shared by the fused T-token and batch-1 projections ----------------------------
// 8 nibbles of a packed word -> two words of signed bytes (nibble - 8): even
// nibbles (k = 0,2,4,6) and odd nibbles (k = 1,3,5,7)
__device__ __forceinline__ void nib_to_s8(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t e = (w & 0x0F0F0F0Fu) ^ 0x08080808u;           // nibble ^ 8: sign bit at bit 3
    const uint32_t o = ((w >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
    lo = e | (((e & 0x08080808u) >> 3) * 0xF0u);                   // sign-extend 4 -> 8 bits per byte
    hi = o | (((o & 0x08080808u) >> 3) * 0xF0u);
}

// group absmax over the 32/EPT lanes of a contiguous 32-group (after the in-thread max)
template <int EPT>
__device__ __forceinline__ float group_max_contig(float m) {
    uint32_t u = __builtin_bit_cast(uint32_t, m);
    if constexpr (EPT <= 16) u = max(u, (uint32_t)__builtin_amdgcn_update_dpp((int)u, (int)u, 0xB1, 0xF, 0xF, false));
    if constexpr (EPT <= 8) u = max(u, (uint32_t)__builtin_amdgcn_update_dpp((int)u, (int)u, 0x4E, 0xF, 0xF, false));
    if constexpr (EPT <= 4) u = max(u, (uint32_t)__builtin_amdgcn_update_dpp((int)u, (int)u, 0x141, 0xF, 0xF, false));
    if constexpr (EPT <= 2) u = max(u, (uint32_t)__builtin_amdgcn_update_dpp((int)u, (int)u, 0x140, 0xF, 0xF, false));
    if constexpr (EPT <= 1) {
        const auto r = __builtin_amdgcn_permlane16_swap((int)u, (int)u, false, false);
        u = max((uint32_t)r[0], (uint32_t)r[1]);
    }
    return __builtin_bit_cast(float, u);
}

// q8_group's arithmetic for one element, given its group scale
__device__ __forceinline__ int q8_code(float v, float inv) {
    const float p = v * inv;
    int qi = (int)rintf(p);
    return qi < -127 ? -127 : (qi > 127 ? 127 : qi);
}

// SwiGLU of one row: silu(g) * u, silu(g) = g / (1 + e^-g)
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }


// ---- the activation prologue of the norm-fused GEMVs ---------------------------------
// MODE_NORM: rmsnormQ of x (weight nw, eps); MODE_F32: quantQ8 of x; MODE_Q8: given codes.
// A is the kernel's argument block: it supplies x, nw, K, eps and the optional copies
// xq_out / xs_out of the codes (written by workgroup 0).
enum { MODE_Q8 = 0, MODE_F32 = 1, MODE_NORM = 2 };

// Register-resident variant of the prologue for the specialised kernels: thread t
// holds elements t, t+256, ... (EPT of them), loaded before the weights so that one
// memory round trip serves the whole prologue. The sum of squares keeps the
// reference's order (per-thread strided partials, then the 128..1 tree); a 32-group
// is 32 consecutive lanes, whose absmax is a 32-lane butterfly (max is exact in any
// order), so every code and scale equals q8_group's.
template <int EPT, bool FULL>
struct ActRegs {
    // CONTIG: K = 256*EPT (FULL) and EPT divides 32 or is a multiple of it. The quantizer
    // then works on a second, contiguous copy (thread t: elements EPT*t .. EPT*t+EPT-1),
    // so a 32-group spans 32/EPT neighbouring lanes and each thread computes its
    // group's scale once; the strided copy only feeds the sum of squares.
    static constexpr bool CONTIG = FULL && (EPT <= 32 ? (32 % EPT == 0) : (EPT % 32 == 0));
    static constexpr int NC = CONTIG ? EPT : 1;
    float x[EPT];
    uint16_t w[EPT];
    float xc[NC];
    uint16_t wc[NC];
};

template <int MODE, int EPT, bool FULL, class A>
__device__ __forceinline__ void act_regs_load(const A& a, ActRegs<EPT, FULL>& r) {
    const int t = threadIdx.x;
    // unconditional loads (clamped index, value masked after): straight-line code
    // lets the compiler wait for exactly these loads, not the weights behind them
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = t + 256 * i;
        const int ec = e < a.K ? e : a.K - 1;
        r.x[i] = a.x[ec];
        if (MODE == MODE_NORM) r.w[i] = a.nw[ec];
    }
    if constexpr (ActRegs<EPT, FULL>::CONTIG) {   // FULL: K = 256*EPT exactly
        if constexpr (EPT % 4 == 0) {
            const float4* xs4 = reinterpret_cast<const float4*>(a.x + (size_t)EPT * t);
#pragma unroll
            for (int i = 0; i < EPT / 4; i++) {
                const float4 v = xs4[i];
                r.xc[4 * i] = v.x; r.xc[4 * i + 1] = v.y; r.xc[4 * i + 2] = v.z; r.xc[4 * i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < EPT; i++) r.xc[i] = a.x[(size_t)EPT * t + i];
        }
        if (MODE == MODE_NORM) {
#pragma unroll
            for (int i = 0; i < EPT; i++) r.wc[i] = a.nw[(size_t)EPT * t + i];
        }
    }
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        if (t + 256 * i >= a.K) {
            r.x[i] = 0.0f;
            r.w[i] = 0;
        }
    }
}

template <int MODE, int EPT, bool FULL, class A>
__device__ __forceinline__ void act_regs_quant(const A& a, ActRegs<EPT, FULL>& r, uint32_t* s_xq, float* s_xs,
                                               float* red) {
    const int t = threadIdx.x;
    float inv_rms = 0.0f;
    if (MODE == MODE_NORM) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < EPT; i++) {
            float sq = r.x[i] * r.x[i];
            s = s + sq;
        }
        float m = ti_tree_sum_256(s, red) / (float)a.K;
        m = m + a.eps;
        inv_rms = 1.0f / sqrtf(m);
    }
    if constexpr (ActRegs<EPT, FULL>::CONTIG) {
        float v[EPT];
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < EPT; i++) {
            v[i] = r.xc[i];
            if (MODE == MODE_NORM) {
                const float p = v[i] * inv_rms;
                v[i] = p * ti_h2f(r.wc[i]);
            }
        }
        uint8_t* qb = reinterpret_cast<uint8_t*>(s_xq);
        if constexpr (EPT <= 32) {
#pragma unroll
            for (int i = 0; i < EPT; i++) mx = fmaxf(mx, fabsf(v[i]));
            mx = group_max_contig<EPT>(mx);
            const float scale = mx / 127.0f;
            const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
            uint32_t wd[(EPT + 3) / 4] = {};
#pragma unroll
            for (int i = 0; i < EPT; i++) wd[i / 4] |= (uint32_t)(q8_code(v[i], inv) & 0xff) << (8 * (i % 4));
            if constexpr (EPT >= 4) {
#pragma unroll
                for (int k = 0; k < EPT / 4; k++) s_xq[EPT / 4 * t + k] = wd[k];
            } else {
#pragma unroll
                for (int i = 0; i < EPT; i++) qb[EPT * t + i] = (uint8_t)((wd[0] >> (8 * i)) & 0xff);
            }
            if (t % (32 / EPT) == 0) s_xs[EPT * t / 32] = scale;
        } else {   // several whole groups per thread
#pragma unroll
            for (int g = 0; g < EPT / 32; g++) {
                float gm = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; i++) gm = fmaxf(gm, fabsf(v[32 * g + i]));
                const float scale = gm / 127.0f;
                const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    uint32_t wd = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) wd |= (uint32_t)(q8_code(v[32 * g + 4 * k + i], inv) & 0xff) << (8 * i);
                    s_xq[EPT / 4 * t + 8 * g + k] = wd;
                }
                s_xs[EPT / 32 * t + g] = scale;
            }
        }
    } else {
        if (MODE == MODE_NORM) {
#pragma unroll
            for (int i = 0; i < EPT; i++) {
                float p = r.x[i] * inv_rms;
                r.x[i] = p * ti_h2f(r.w[i]);
            }
        }
        uint8_t* qb = reinterpret_cast<uint8_t*>(s_xq);
        // EPT independent chains (group max, two IEEE divisions, rounding) computed
        // without branches so they interleave; only the LDS stores are predicated
        float gsc[EPT];
        int gq[EPT];
#pragma unroll
        for (int i = 0; i < EPT; i++) {
            const float mx = ti_max32_nonneg(fabsf(r.x[i]));
            const float scale = mx / 127.0f;
            const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
            gsc[i] = scale;
            gq[i] = q8_code(r.x[i], inv);
        }
#pragma unroll
        for (int i = 0; i < EPT; i++) {
            const int e = t + 256 * i;
            if (e < a.K) {
                qb[e] = (uint8_t)(gq[i] & 0xff);
                if ((t & 31) == 0) s_xs[e >> 5] = gsc[i];
            }
        }
    }
    __syncthreads();
    if (a.xq_out && blockIdx.x == 0) {
        for (int i = t; i < a.K / 4; i += 256) a.xq_out[i] = s_xq[i];
        for (int g = t; g < a.K / 32; g += 256) a.xs_out[g] = s_xs[g];
    }
}


}  // namespace
