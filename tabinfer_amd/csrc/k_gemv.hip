// k_gemv.hip — batch-1 int4 GEMVs (HBM-bound; no MFMA):
//  int4 x int8      gemvDP4_only        models/qwen3.js:359-427
//  int4 x f32       gemvQ               models/qwen3.js:276-321
//  gate+up+SiLU     gateUpSiluDP4_only  models/qwen3.js:679-728, 861-877
//
// Mapping (per 64-lane wavefront): a row of K weights is gpr = K/32 groups of
// 16 bytes (32 nibbles + one f16 scale). LPR lanes share a row and each lane
// owns GPL groups (gpr = LPR*GPL), so one wave covers 64/LPR rows per pass and
// every load is one global_load_dwordx4 of a whole quant group. A lane's group
// indices never change across rows, so its slice of the activation is loaded,
// permuted and summed once and then lives in registers. R passes are loaded
// back to back before any arithmetic, to keep several KB in flight per wave.
//
// int8 dot: the nibbles of a word are split into even (p & 0x0F0F0F0F) and odd
// ((p >> 4) & 0x0F0F0F0F) byte lanes and dotted (v_dot4_i32_i8) with the
// activation bytes permuted the same way; the unsigned-nibble offset is removed
// once per group: sum (n-8)*x = sum n*x - 8*sum x. The per-group int32 is exact.
#include "ti_dev.h"

namespace {


// ---------------------------------------------------------------------------
// y (+)= W x, int8 activation
// ---------------------------------------------------------------------------
template <int LPR, int GPL, int R>
__global__ __launch_bounds__(256) void k_gemv_q4_q8(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                    const uint4* __restrict__ pack, const uint16_t* __restrict__ scales,
                                                    float* __restrict__ y, int N, int acc) {
    constexpr int RPP = 64 / LPR;
    constexpr int GPR = LPR * GPL;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, li = lane % LPR;
    const long nwaves = (long)gridDim.x * (blockDim.x >> 6);
    const long nblocks = (N + RPP * R - 1) / (RPP * R);
    long b = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (b >= nblocks) return;
    // every weight/scale load of a block is issued before any arithmetic; rows past
    // N re-read row N-1 (a valid address, result discarded), so no load sits
    // behind a branch
    uint4 wv[2][R][GPL];
    uint16_t sw[2][R][GPL];
    float yold[2];
    constexpr int SPAN = LPR / R;        // lanes holding the same row total
    // raw activation loads first, unpacked after the weight loads are issued: the
    // activation's wait (vmcnt counts in order) then does not include the weights
    uint4 araw[GPL][2];
    float asc[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) {
        const uint4* p = reinterpret_cast<const uint4*>(xq + (size_t)(li + LPR * j) * 8);
        araw[j][0] = p[0];
        araw[j][1] = p[1];
        asc[j] = xs[li + LPR * j];
    }
    auto load = [&](int buf, long blk) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            long row = blk * (RPP * R) + sub + (long)r * RPP;
            row = row < N ? row : N - 1;
#pragma unroll
            for (int j = 0; j < GPL; j++) {
                long gi = row * GPR + li + LPR * j;
                wv[buf][r][j] = ld_nt(pack + gi);
                sw[buf][r][j] = ld_nt(scales + gi);
            }
        }
        // the residual of the row this lane stores, fetched with the weights (not after the dots)
        long orow = blk * (RPP * R) + sub + (long)(li / SPAN) * RPP;
        orow = orow < N ? orow : N - 1;
        yold[buf] = y[orow];
    };
    load(0, b);
    TI_ISSUE_FENCE();
    ActQ8 a[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) act_q8_from_words(araw[j], asc[j], a[j]);
    auto finish = [&](int buf, long blk) {
        float accv[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < GPL; j++) {
                int d = group_dot_q8(wv[buf][r][j], a[j]);
                t = fmaf((float)d, ti_h2f(sw[buf][r][j]) * a[j].s, t);
            }
            accv[r] = t;
        }
        float tot = transpose_reduce<LPR, R>(accv, li);
        const long row = blk * (RPP * R) + sub + (long)(li / SPAN) * RPP;
        if ((li % SPAN) == 0 && row < N) y[row] = acc ? yold[buf] + tot : tot;
    };
    // persistent waves: prefetch block b+nwaves while finishing block b
    for (;;) {
        long nb = b + nwaves;
        if (nb < nblocks) load(1, nb);
        finish(0, b);
        if (nb >= nblocks) break;
        b = nb;
        nb = b + nwaves;
        if (nb < nblocks) load(0, nb);
        finish(1, b);
        if (nb >= nblocks) break;
        b = nb;
    }
}

// Any K % 32 == 0: one wave per row, lanes stride the groups.
__global__ __launch_bounds__(256) void k_gemv_q4_q8_generic(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                            const uint4* __restrict__ pack, const uint16_t* __restrict__ scales,
                                                            float* __restrict__ y, int N, int gpr, int acc) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= N) return;
    float accv = 0.0f;
    for (int g = lane; g < gpr; g += 64) {
        ActQ8 a;
        load_act_q8(xq, xs, g, a);
        long gi = row * gpr + g;
        int d = group_dot_q8(pack[gi], a);
        accv = fmaf((float)d, ti_h2f(scales[gi]) * a.s, accv);
    }
    accv = ti_seg_sum<64>(accv);
    if (lane == 0) store_out(y, row, accv, acc);
}

// ---------------------------------------------------------------------------
// swi = silu(gate x) * (up x)
// ---------------------------------------------------------------------------
template <int LPR, int GPL, int R>
__global__ __launch_bounds__(256) void k_gateup_q4_q8(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                      const uint4* __restrict__ gpack, const uint16_t* __restrict__ gsc,
                                                      const uint4* __restrict__ upack, const uint16_t* __restrict__ usc,
                                                      float* __restrict__ swi, int I) {
    constexpr int RPP = 64 / LPR;
    constexpr int GPR = LPR * GPL;
    const int lane = threadIdx.x & 63;
    const long wave = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int sub = lane / LPR, li = lane % LPR;
    const long row0 = wave * (RPP * R) + sub;
    uint4 gw[R][GPL], uw[R][GPL];
    uint16_t gs[R][GPL], us[R][GPL];
#pragma unroll
    for (int r = 0; r < R; r++) {
        long row = row0 + (long)r * RPP;
        row = row < I ? row : I - 1;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            long gi = row * GPR + li + LPR * j;
            gw[r][j] = ld_nt(gpack + gi);
            uw[r][j] = ld_nt(upack + gi);
            gs[r][j] = ld_nt(gsc + gi);
            us[r][j] = ld_nt(usc + gi);
        }
    }
    ActQ8 a[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) load_act_q8(xq, xs, li + LPR * j, a[j]);
    float ga[R], ua[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float tg = 0.0f, tu = 0.0f;
#pragma unroll
        for (int j = 0; j < GPL; j++) {
            tg = fmaf((float)group_dot_q8(gw[r][j], a[j]), ti_h2f(gs[r][j]) * a[j].s, tg);
            tu = fmaf((float)group_dot_q8(uw[r][j], a[j]), ti_h2f(us[r][j]) * a[j].s, tu);
        }
        ga[r] = tg;
        ua[r] = tu;
    }
    float g = transpose_reduce<LPR, R>(ga, li);
    float u = transpose_reduce<LPR, R>(ua, li);
    constexpr int SPAN = LPR / R;
    const long row = row0 + (long)(li / SPAN) * RPP;
    if ((li % SPAN) == 0 && row < I) {
        float silu = g / (1.0f + expf(-g));
        swi[row] = silu * u;
    }
}

__global__ __launch_bounds__(256) void k_gateup_q4_q8_generic(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                              const uint4* __restrict__ gpack, const uint16_t* __restrict__ gsc,
                                                              const uint4* __restrict__ upack, const uint16_t* __restrict__ usc,
                                                              float* __restrict__ swi, int I, int gpr) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= I) return;
    float ga = 0.0f, ua = 0.0f;
    for (int g = lane; g < gpr; g += 64) {
        ActQ8 a;
        load_act_q8(xq, xs, g, a);
        long gi = row * gpr + g;
        ga = fmaf((float)group_dot_q8(gpack[gi], a), ti_h2f(gsc[gi]) * a.s, ga);
        ua = fmaf((float)group_dot_q8(upack[gi], a), ti_h2f(usc[gi]) * a.s, ua);
    }
    ga = ti_seg_sum<64>(ga);
    ua = ti_seg_sum<64>(ua);
    if (lane == 0) swi[row] = ga / (1.0f + expf(-ga)) * ua;
}


template <int LPR, int GPL, int R>
__global__ __launch_bounds__(256) void k_gemv_q4_f32(const float* __restrict__ x, const uint4* __restrict__ pack,
                                                     const uint16_t* __restrict__ scales, float* __restrict__ y,
                                                     int N, int acc) {
    constexpr int RPP = 64 / LPR;
    constexpr int GPR = LPR * GPL;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, li = lane % LPR;
    const long nwaves = (long)gridDim.x * (blockDim.x >> 6);
    const long nblocks = (N + RPP * R - 1) / (RPP * R);
    long b = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (b >= nblocks) return;
    ActLimb a[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) load_act_limbs(x, li + LPR * j, a[j]);
    uint4 wv[2][R][GPL];
    uint16_t sw[2][R][GPL];
    auto load = [&](int buf, long blk) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            long row = blk * (RPP * R) + sub + (long)r * RPP;
            row = row < N ? row : N - 1;
#pragma unroll
            for (int j = 0; j < GPL; j++) {
                long gi = row * GPR + li + LPR * j;
                wv[buf][r][j] = ld_nt(pack + gi);
                sw[buf][r][j] = ld_nt(scales + gi);
            }
        }
    };
    auto finish = [&](int buf, long blk) {
        float accv[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < GPL; j++) t = fmaf(group_dot_limbs(wv[buf][r][j], a[j]), ti_h2f(sw[buf][r][j]), t);
            accv[r] = t;
        }
        float tot = transpose_reduce<LPR, R>(accv, li);
        constexpr int SPAN = LPR / R;
        const long row = blk * (RPP * R) + sub + (long)(li / SPAN) * RPP;
        if ((li % SPAN) == 0 && row < N) store_out(y, row, tot, acc);
    };
    // persistent waves: prefetch block b+nwaves while finishing block b
    load(0, b);
    for (;;) {
        long nb = b + nwaves;
        if (nb < nblocks) load(1, nb);
        finish(0, b);
        if (nb >= nblocks) break;
        b = nb;
        nb = b + nwaves;
        if (nb < nblocks) load(0, nb);
        finish(1, b);
        if (nb >= nblocks) break;
        b = nb;
    }
}

__global__ __launch_bounds__(256) void k_gemv_q4_f32_generic(const float* __restrict__ x, const uint4* __restrict__ pack,
                                                             const uint16_t* __restrict__ scales, float* __restrict__ y,
                                                             int N, int gpr, int acc) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= N) return;
    float accv = 0.0f;
    for (int g = lane; g < gpr; g += 64) {
        ActF32 a;
        load_act_f32(x, g, a);
        long gi = row * gpr + g;
        accv = fmaf(group_dot_f32(pack[gi], a), ti_h2f(scales[gi]), accv);
    }
    accv = ti_seg_sum<64>(accv);
    if (lane == 0) store_out(y, row, accv, acc);
}

// Debug: exact int32 per (row, group).
__global__ void k_group_dots(const uint32_t* __restrict__ xq, const uint4* __restrict__ pack, int32_t* __restrict__ dots,
                             long total, int gpr) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    int g = (int)(i % gpr);
    ActQ8 a;
    load_act_q8(xq, nullptr, g, a);
    dots[i] = group_dot_q8(pack[i], a);
}

// ---- launch helpers ----------------------------------------------------------
struct Shape {
    int lpr, gpl;
};

// lanes per row = the power-of-two part of gpr (capped at 64); groups per lane = gpr / lanes
Shape pick_shape(int gpr) {
    int lpr = 1;
    while (lpr < 64 && (gpr % (lpr * 2)) == 0) lpr *= 2;
    return {lpr, gpr / lpr};
}

int pick_R(long waves_r1, int lpr) {
    int R = waves_r1 >= 8192 ? 4 : waves_r1 >= 4096 ? 2 : 1;
    while (R > lpr) R >>= 1;
    return R;
}

void grid_for(long waves, unsigned& blocks, unsigned& threads) {
    threads = waves >= 1024 ? 256 : 64;
    long wpb = threads / 64;
    blocks = (unsigned)((waves + wpb - 1) / wpb);
}

// Persistent launches stop at TI_RESIDENT_WAVES waves (256 CUs x 4 SIMDs x 4, what
// fits at the ~88-110 VGPRs of the double-buffered kernels):
// beyond that each wave loops over row blocks with a one-block prefetch.
constexpr long TI_RESIDENT_WAVES = 256 * 4 * 4;
void grid_persistent(long blocks_total, unsigned& blocks, unsigned& threads) {
    long waves = blocks_total < TI_RESIDENT_WAVES ? blocks_total : TI_RESIDENT_WAVES;
    grid_for(waves, blocks, threads);
}

#define GEMV_CASES(X)  \
    X(1, 1) X(1, 3) X(2, 1) X(2, 3) X(4, 1) X(4, 3) X(8, 1) X(8, 3) X(16, 1) X(16, 3) \
    X(32, 1) X(32, 3) X(64, 1) X(64, 2) X(64, 3) X(64, 4) X(64, 6) X(64, 8)

}  // namespace

int ti_gemv_q4_q8_launch(ti_ctx* c, const uint32_t* xq, const float* xs, const uint32_t* pack, const uint16_t* scales,
                         float* y, int N, int K, int acc) {
    int gpr = K / 32;
    Shape s = pick_shape(gpr);
    long rpp = 64 / s.lpr;
    long waves1 = (N + rpp - 1) / rpp;
    int R = pick_R(waves1, s.lpr);
    long waves = (N + rpp * R - 1) / (rpp * R);
    unsigned blocks, threads;
    grid_persistent(waves, blocks, threads);
    const uint4* p4 = reinterpret_cast<const uint4*>(pack);
#define X(L, G)                                                                                                   \
    if (s.lpr == L && s.gpl == G) {                                                                               \
        if (R == 4) k_gemv_q4_q8<L, G, (L >= 4 ? 4 : 1)><<<blocks, threads, 0, c->stream>>>(xq, xs, p4, scales, y, N, acc); \
        else if (R == 2) k_gemv_q4_q8<L, G, (L >= 2 ? 2 : 1)><<<blocks, threads, 0, c->stream>>>(xq, xs, p4, scales, y, N, acc); \
        else k_gemv_q4_q8<L, G, 1><<<blocks, threads, 0, c->stream>>>(xq, xs, p4, scales, y, N, acc);             \
        TI_LAUNCHED("k_gemv_q4_q8");                                                                              \
        return TI_OK;                                                                                             \
    }
    GEMV_CASES(X)
#undef X
    unsigned gb, gt;
    grid_for(N, gb, gt);
    k_gemv_q4_q8_generic<<<gb, gt, 0, c->stream>>>(xq, xs, p4, scales, y, N, gpr, acc);
    TI_LAUNCHED("k_gemv_q4_q8_generic");
    return TI_OK;
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int ti_gemv_q4_q8(ti_ctx* c, const uint32_t* xq, const float* xs, const uint32_t* pack, const uint16_t* scales,
                             float* y, int N, int K, int acc) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(xq && xs && pack && scales && y, "ti_gemv_q4_q8: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "ti_gemv_q4_q8: need N>0 and K a positive multiple of 32 (N=%d K=%d)", N, K);
    TI_REQUIRE(al16(xq) && al16(pack), "ti_gemv_q4_q8: xq and pack must be 16-byte aligned");
    return ti_gemv_q4_q8_launch(c, xq, xs, pack, scales, y, N, K, acc);
}

int ti_gemv_q4_f32_launch(ti_ctx* c, const float* x, const uint32_t* pack, const uint16_t* scales, float* y, int N, int K,
                          int acc) {
    int gpr = K / 32;
    Shape s = pick_shape(gpr);
    long rpp = 64 / s.lpr;
    long waves1 = (N + rpp - 1) / rpp;
    int R = pick_R(waves1, s.lpr);
    long waves = (N + rpp * R - 1) / (rpp * R);
    unsigned blocks, threads;
    grid_persistent(waves, blocks, threads);
    const uint4* p4 = reinterpret_cast<const uint4*>(pack);
#define X(L, G)                                                                                               \
    if (s.lpr == L && s.gpl == G && G <= 3) {                                                                 \
        if (R == 4) k_gemv_q4_f32<L, G, (L >= 4 ? 4 : 1)><<<blocks, threads, 0, c->stream>>>(x, p4, scales, y, N, acc); \
        else if (R == 2) k_gemv_q4_f32<L, G, (L >= 2 ? 2 : 1)><<<blocks, threads, 0, c->stream>>>(x, p4, scales, y, N, acc); \
        else k_gemv_q4_f32<L, G, 1><<<blocks, threads, 0, c->stream>>>(x, p4, scales, y, N, acc);             \
        TI_LAUNCHED("k_gemv_q4_f32");                                                                         \
        return TI_OK;                                                                                         \
    }
    X(1, 1) X(2, 1) X(4, 1) X(8, 1) X(16, 1) X(32, 1) X(64, 1) X(64, 2) X(32, 3) X(64, 3)
#undef X
    unsigned gb, gt;
    grid_for(N, gb, gt);
    k_gemv_q4_f32_generic<<<gb, gt, 0, c->stream>>>(x, p4, scales, y, N, gpr, acc);
    TI_LAUNCHED("k_gemv_q4_f32_generic");
    return TI_OK;
}

extern "C" int ti_gemv_q4_f32(ti_ctx* c, const float* x, const uint32_t* pack, const uint16_t* scales, float* y, int N,
                              int K, int acc) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && pack && scales && y, "ti_gemv_q4_f32: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "ti_gemv_q4_f32: need N>0 and K a positive multiple of 32 (N=%d K=%d)", N, K);
    TI_REQUIRE(al16(x) && al16(pack), "ti_gemv_q4_f32: x and pack must be 16-byte aligned");
    return ti_gemv_q4_f32_launch(c, x, pack, scales, y, N, K, acc);
}

int ti_gateup_launch(ti_ctx* c, const uint32_t* xq, const float* xs, const uint32_t* gpack, const uint16_t* gsc,
                     const uint32_t* upack, const uint16_t* usc, float* swi, int I, int H) {
    int gpr = H / 32;
    Shape s = pick_shape(gpr);
    long rpp = 64 / s.lpr;
    long waves1 = (I + rpp - 1) / rpp;
    int R = waves1 >= 8192 ? 2 : 1;
    while (R > s.lpr) R >>= 1;
    long waves = (I + rpp * R - 1) / (rpp * R);
    unsigned blocks, threads;
    grid_for(waves, blocks, threads);
    const uint4* g4 = reinterpret_cast<const uint4*>(gpack);
    const uint4* u4 = reinterpret_cast<const uint4*>(upack);
#define X(L, G)                                                                                                        \
    if (s.lpr == L && s.gpl == G) {                                                                                    \
        if (R == 2) k_gateup_q4_q8<L, G, (L >= 2 ? 2 : 1)><<<blocks, threads, 0, c->stream>>>(xq, xs, g4, gsc, u4, usc, swi, I); \
        else k_gateup_q4_q8<L, G, 1><<<blocks, threads, 0, c->stream>>>(xq, xs, g4, gsc, u4, usc, swi, I);             \
        TI_LAUNCHED("k_gateup_q4_q8");                                                                                 \
        return TI_OK;                                                                                                  \
    }
    GEMV_CASES(X)
#undef X
    unsigned gb, gt;
    grid_for(I, gb, gt);
    k_gateup_q4_q8_generic<<<gb, gt, 0, c->stream>>>(xq, xs, g4, gsc, u4, usc, swi, I, gpr);
    TI_LAUNCHED("k_gateup_q4_q8_generic");
    return TI_OK;
}

extern "C" int ti_gateup_silu_q4(ti_ctx* c, const uint32_t* xq, const float* xs, const uint32_t* gpack, const uint16_t* gsc,
                                 const uint32_t* upack, const uint16_t* usc, float* swi, int I, int H) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(xq && xs && gpack && gsc && upack && usc && swi, "ti_gateup_silu_q4: null buffer");
    TI_REQUIRE(I > 0 && H > 0 && H % 32 == 0, "ti_gateup_silu_q4: need I>0 and H a positive multiple of 32 (I=%d H=%d)", I, H);
    TI_REQUIRE(al16(xq) && al16(gpack) && al16(upack), "ti_gateup_silu_q4: xq and packs must be 16-byte aligned");
    return ti_gateup_launch(c, xq, xs, gpack, gsc, upack, usc, swi, I, H);
}

extern "C" int ti_group_dots_q4_q8(ti_ctx* c, const uint32_t* xq, const uint32_t* pack, int32_t* dots, int N, int K) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(xq && pack && dots, "ti_group_dots_q4_q8: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "ti_group_dots_q4_q8: bad shape (N=%d K=%d)", N, K);
    long total = (long)N * (K / 32);
    k_group_dots<<<(unsigned)((total + 255) / 256), 256, 0, c->stream>>>(xq, reinterpret_cast<const uint4*>(pack), dots,
                                                                        total, K / 32);
    TI_LAUNCHED("k_group_dots");
    return TI_OK;
}

// linearQ router: the activation scratch lives in the context (allocated once at
// init), like the reference's _dp4/_dp4g buffers.
int ti_quant_act_q8_async(ti_ctx* c, const float* x, uint32_t* xq, float* xs, int32_t* xsum, int groups);
int ti_gemm_q4_q8_launch(ti_ctx* c, const uint32_t* xq, const float* xs, const uint32_t* pack, const uint16_t* scales,
                         float* y, int T, int N, int K, int acc);
int ti_fused_linear_launch(ti_ctx*, const float*, const uint32_t*, const uint16_t*, float*, int, int, int);
int ti_fused_kmax(int lm);

extern "C" int ti_linear_q4(ti_ctx* c, const float* x, const uint32_t* pack, const uint16_t* scales, float* y, int T, int N,
                            int K, int acc) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && pack && scales && y, "ti_linear_q4: null buffer");
    TI_REQUIRE(T > 0 && N > 0 && K > 0 && K % 32 == 0, "ti_linear_q4: bad shape (T=%d N=%d K=%d)", T, N, K);
    TI_REQUIRE(K <= TI_ACT_CAP && T <= TI_ACT_TMAX, "ti_linear_q4: K<=%d and T<=%d required", TI_ACT_CAP, TI_ACT_TMAX);
    TI_REQUIRE(al16(x) && al16(pack), "ti_linear_q4: x and pack must be 16-byte aligned");
    if (T == 1 && N >= 16384) return ti_gemv_q4_f32_launch(c, x, pack, scales, y, N, K, acc);
    if (T == 1 && K <= ti_fused_kmax(0)) return ti_fused_linear_launch(c, x, pack, scales, y, N, K, acc);
    int rc = ti_quant_act_q8_async(c, x, c->act_q, c->act_s, nullptr, T * (K / 32));
    if (rc) return rc;
    if (T == 1) return ti_gemv_q4_q8_launch(c, c->act_q, c->act_s, pack, scales, y, N, K, acc);
    if (ti_tgemm_ok(T, K) && reinterpret_cast<uintptr_t>(scales) % 16 == 0)
        return ti_tgemm_launch(c, TgIn{c->act_q, c->act_s, nullptr, nullptr, 0.0f, nullptr}, 1, &pack, &scales, &y, &N, T, K,
                               acc, nullptr);
    return ti_gemm_q4_q8_launch(c, c->act_q, c->act_s, pack, scales, y, T, N, K, acc);
}
