// k_tern2.hip — GEMVs over the reference's on-GPU ternary format:
//  gemvTern2 / gemvTern_only      models/qwen3.js:449-503, 548-556
//  gateupTern2 (+ SiLU)           models/qwen3.js:747-810, 862-870
//
// Weights (quantizeTernaryBf16, :3435-3469, ti_quant_tern_bf16): 16 codes c = w + 1 per u32,
// weight k of a row at bits 8(k&3) + 2((k>>2)&3) of word k/16, so (word >> 2s) & 0x03030303
// holds the codes of weights 16(k/16) + 4s .. + 3 in the byte lanes of v_dot4; one f16 scale
// per 32 weights. The activation is quantQ8's: int8 codes (4 per word), an f32 scale per 32
// and the sums per 16. sum over a group of (c - 1) x = sum c x - sum x, exactly in int32;
// each group then adds f32(scale) * xs * f32(dot) (the reference's product order).
//
// Shape: LPR lanes per row, a lane owning pairs of groups (64 weights: one 16-byte code
// load, one 4-byte load of the two scales) at pair indexes li + LPR j; the lanes of a row
// sum in a butterfly and the first lane stores.
#include "ti_internal.h"

namespace {

constexpr uint32_t T2M = 0x03030303u;

// exact int32 sum over one 32-weight group: codes (two words) dotted with the 32 int8
// activations (eight words), minus the activations' sum
__device__ __forceinline__ int tern2_group(uint32_t w0, uint32_t w1, const uint32_t* a, int xsm) {
    int d = 0;
    d = __builtin_amdgcn_sdot4((int)(w0 & T2M), (int)a[0], d, false);
    d = __builtin_amdgcn_sdot4((int)((w0 >> 2) & T2M), (int)a[1], d, false);
    d = __builtin_amdgcn_sdot4((int)((w0 >> 4) & T2M), (int)a[2], d, false);
    d = __builtin_amdgcn_sdot4((int)((w0 >> 6) & T2M), (int)a[3], d, false);
    d = __builtin_amdgcn_sdot4((int)(w1 & T2M), (int)a[4], d, false);
    d = __builtin_amdgcn_sdot4((int)((w1 >> 2) & T2M), (int)a[5], d, false);
    d = __builtin_amdgcn_sdot4((int)((w1 >> 4) & T2M), (int)a[6], d, false);
    d = __builtin_amdgcn_sdot4((int)((w1 >> 6) & T2M), (int)a[7], d, false);
    return d - xsm;
}

// one pair of groups (2p, 2p + 1) of the activation: 16 code words, two scales, four sums
struct Pair {
    uint32_t a[16];
    float s0, s1;
    int m0, m1;
};

__device__ __forceinline__ void load_pair(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                          const int32_t* __restrict__ xsum, int p, Pair& P) {
    const uint4* q = reinterpret_cast<const uint4*>(xq + (size_t)p * 16);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 v = q[i];
        P.a[4 * i] = v.x; P.a[4 * i + 1] = v.y; P.a[4 * i + 2] = v.z; P.a[4 * i + 3] = v.w;
    }
    const float2 s = reinterpret_cast<const float2*>(xs)[p];
    const int4 m = reinterpret_cast<const int4*>(xsum)[p];
    P.s0 = s.x;
    P.s1 = s.y;
    P.m0 = m.x + m.y;
    P.m1 = m.z + m.w;
}

// the two groups of one weight pair against the activation pair, in f32
__device__ __forceinline__ float pair_dot(const uint4 w, uint32_t sc2, const Pair& P) {
    const int i0 = tern2_group(w.x, w.y, P.a, P.m0);
    const int i1 = tern2_group(w.z, w.w, P.a + 8, P.m1);
    const float t0 = ti_h2f((uint16_t)(sc2 & 0xFFFFu)) * P.s0 * (float)i0;
    const float t1 = ti_h2f((uint16_t)(sc2 >> 16)) * P.s1 * (float)i1;
    return t0 + t1;
}

template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
    return ti_seg_sum<LPR>(v);
}

template <int LPR, int PPL>
__global__ __launch_bounds__(256) void k_gemv_tern2(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                    const int32_t* __restrict__ xsum, const uint4* __restrict__ pack,
                                                    const uint32_t* __restrict__ sc2, float* __restrict__ y, int N, int acc) {
    constexpr int RPW = 64 / LPR, NP = LPR * PPL;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane / LPR, li = lane % LPR;
    const long row = ((long)blockIdx.x * 4 + wave) * RPW + r;
    const long rowc = row < N ? row : N - 1;
    uint4 w[PPL];
    uint32_t s[PPL];
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        w[j] = ti_ld_nt(pack + rowc * NP + li + LPR * j);
        s[j] = sc2[rowc * NP + li + LPR * j];
    }
    const float yold = acc ? y[rowc] : 0.0f;
    float t = 0.0f;
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        Pair P;
        load_pair(xq, xs, xsum, li + LPR * j, P);
        t = t + pair_dot(w[j], s[j], P);
    }
    const float tot = row_sum<LPR>(t);
    if (li == 0 && row < N) y[row] = acc ? yold + tot : tot;
}

// any K % 64 == 0: one wave per row, lanes striding over the pairs
__global__ __launch_bounds__(256) void k_gemv_tern2_generic(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                            const int32_t* __restrict__ xsum, const uint4* __restrict__ pack,
                                                            const uint32_t* __restrict__ sc2, float* __restrict__ y, int N,
                                                            int np, int acc) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    float t = 0.0f;
    for (int p = lane; p < np; p += 64) {
        Pair P;
        load_pair(xq, xs, xsum, p, P);
        t = t + pair_dot(pack[row * np + p], sc2[row * np + p], P);
    }
    const float tot = ti_seg_sum<64>(t);
    if (lane == 0) y[row] = acc ? y[row] + tot : tot;
}

template <int LPR, int PPL>
__global__ __launch_bounds__(256) void k_gateup_tern2(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                      const int32_t* __restrict__ xsum, const uint4* __restrict__ gpack,
                                                      const uint32_t* __restrict__ gsc2, const uint4* __restrict__ upack,
                                                      const uint32_t* __restrict__ usc2, float* __restrict__ swi, int I) {
    constexpr int RPW = 64 / LPR, NP = LPR * PPL;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane / LPR, li = lane % LPR;
    const long row = ((long)blockIdx.x * 4 + wave) * RPW + r;
    const long rowc = row < I ? row : I - 1;
    uint4 gw[PPL], uw[PPL];
    uint32_t gs[PPL], us[PPL];
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const long i = rowc * NP + li + LPR * j;
        gw[j] = ti_ld_nt(gpack + i);
        uw[j] = ti_ld_nt(upack + i);
        gs[j] = gsc2[i];
        us[j] = usc2[i];
    }
    float g = 0.0f, u = 0.0f;
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        Pair P;
        load_pair(xq, xs, xsum, li + LPR * j, P);
        g = g + pair_dot(gw[j], gs[j], P);
        u = u + pair_dot(uw[j], us[j], P);
    }
    g = row_sum<LPR>(g);
    u = row_sum<LPR>(u);
    if (li == 0 && row < I) {
        const float silu = g / (1.0f + expf(-g));
        swi[row] = silu * u;
    }
}

__global__ __launch_bounds__(256) void k_gateup_tern2_generic(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                              const int32_t* __restrict__ xsum, const uint4* __restrict__ gpack,
                                                              const uint32_t* __restrict__ gsc2, const uint4* __restrict__ upack,
                                                              const uint32_t* __restrict__ usc2, float* __restrict__ swi, int I,
                                                              int np) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= I) return;
    float g = 0.0f, u = 0.0f;
    for (int p = lane; p < np; p += 64) {
        Pair P;
        load_pair(xq, xs, xsum, p, P);
        g = g + pair_dot(gpack[row * np + p], gsc2[row * np + p], P);
        u = u + pair_dot(upack[row * np + p], usc2[row * np + p], P);
    }
    g = ti_seg_sum<64>(g);
    u = ti_seg_sum<64>(u);
    if (lane == 0) {
        const float silu = g / (1.0f + expf(-g));
        swi[row] = silu * u;
    }
}

// lanes per row and pairs per lane for np pairs per row; {0, 0}: the generic kernel
struct T2Shape {
    int lpr, ppl;
};
T2Shape t2_shape(int np) {
    if (np % 32 == 0 && np / 32 <= 4) return {32, np / 32};
    if (np % 16 == 0 && np / 16 <= 3) return {16, np / 16};
    return {0, 0};
}

bool t2_args_ok(const void* xq, const void* xs, const void* xsum, const void* pack, const void* sc) {
    return ((uintptr_t)xq & 15) == 0 && ((uintptr_t)xs & 7) == 0 && ((uintptr_t)xsum & 15) == 0 &&
           ((uintptr_t)pack & 15) == 0 && ((uintptr_t)sc & 3) == 0;
}

}  // namespace

extern "C" int ti_gemv_tern2(ti_ctx* c, const uint32_t* xq, const float* xs, const int32_t* xsum, const uint32_t* pack,
                             const uint16_t* scales, float* y, int N, int K, int acc) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(xq && xs && xsum && pack && scales && y, "ti_gemv_tern2: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "ti_gemv_tern2: need N>0 and K%%64==0 (N=%d K=%d)", N, K);
    TI_REQUIRE(t2_args_ok(xq, xs, xsum, pack, scales),
               "ti_gemv_tern2: xq, xsum and pack 16-byte, xs 8-byte, scales 4-byte aligned");
    const int np = K / 64;
    const T2Shape s = t2_shape(np);
    const uint4* p4 = reinterpret_cast<const uint4*>(pack);
    const uint32_t* s2 = reinterpret_cast<const uint32_t*>(scales);
    if (s.lpr) {
        const long rows_per_block = 4L * (64 / s.lpr);
        const long grid = ((long)N + rows_per_block - 1) / rows_per_block;
        TI_REQUIRE(grid < (1L << 31), "ti_gemv_tern2: too many rows");
#define G2(L, P) \
        if (s.lpr == L && s.ppl == P) k_gemv_tern2<L, P><<<(unsigned)grid, 256, 0, c->stream>>>(xq, xs, xsum, p4, s2, y, N, acc);
        G2(32, 1) else G2(32, 2) else G2(32, 3) else G2(32, 4) else G2(16, 1) else G2(16, 2) else G2(16, 3)
#undef G2
        TI_LAUNCHED("k_gemv_tern2");
        return TI_OK;
    }
    k_gemv_tern2_generic<<<(unsigned)(((long)N + 3) / 4), 256, 0, c->stream>>>(xq, xs, xsum, p4, s2, y, N, np, acc);
    TI_LAUNCHED("k_gemv_tern2_generic");
    return TI_OK;
}

extern "C" int ti_gateup_silu_tern2(ti_ctx* c, const uint32_t* xq, const float* xs, const int32_t* xsum,
                                    const uint32_t* gpack, const uint16_t* gscales, const uint32_t* upack,
                                    const uint16_t* uscales, float* swi, int I, int H) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(xq && xs && xsum && gpack && gscales && upack && uscales && swi, "ti_gateup_silu_tern2: null buffer");
    TI_REQUIRE(I > 0 && H > 0 && H % 64 == 0, "ti_gateup_silu_tern2: need I>0 and H%%64==0 (I=%d H=%d)", I, H);
    TI_REQUIRE(t2_args_ok(xq, xs, xsum, gpack, gscales) && t2_args_ok(xq, xs, xsum, upack, uscales),
               "ti_gateup_silu_tern2: xq, xsum and packs 16-byte, xs 8-byte, scales 4-byte aligned");
    const int np = H / 64;
    const T2Shape s = t2_shape(np);
    const uint4 *g4 = reinterpret_cast<const uint4*>(gpack), *u4 = reinterpret_cast<const uint4*>(upack);
    const uint32_t *gs = reinterpret_cast<const uint32_t*>(gscales), *us = reinterpret_cast<const uint32_t*>(uscales);
    if (s.lpr) {
        const long rows_per_block = 4L * (64 / s.lpr);
        const long grid = ((long)I + rows_per_block - 1) / rows_per_block;
        TI_REQUIRE(grid < (1L << 31), "ti_gateup_silu_tern2: too many rows");
#define G2(L, P) \
        if (s.lpr == L && s.ppl == P) k_gateup_tern2<L, P><<<(unsigned)grid, 256, 0, c->stream>>>(xq, xs, xsum, g4, gs, u4, us, swi, I);
        G2(32, 1) else G2(32, 2) else G2(32, 3) else G2(32, 4) else G2(16, 1) else G2(16, 2) else G2(16, 3)
#undef G2
        TI_LAUNCHED("k_gateup_tern2");
        return TI_OK;
    }
    k_gateup_tern2_generic<<<(unsigned)(((long)I + 3) / 4), 256, 0, c->stream>>>(xq, xs, xsum, g4, gs, u4, us, swi, I, np);
    TI_LAUNCHED("k_gateup_tern2_generic");
    return TI_OK;
}
