// k_gemm.hip — T > 1 int4 x int8 GEMM on the matrix cores (gemmDP4A,
// models/qwen3.js:1326-1407; per-token activation quant QUANTQ8T :1210-1231).
//
// y[t][n] (+)= sum_g s_w[n,g] * s_x[t,g] * dot_g(t, n), dot_g the exact int32 dot of
// the 32-element group g. One v_mfma_i32_16x16x32_i8 computes dot_g for a 16-token x
// 16-row tile: K = 32 is exactly one scale group, so every MFMA result is one group's
// int32 partial and is scaled into an f32 accumulator right away, as the reference
// does per group.
//
// Operands (gfx950 16x16x32 i8 layout: lane l feeds row/column l%16 and K slice
// 8*(l/16)..+8; the result row 4*(l/16)+i, column l%16 lands in lane l, element i):
//   A = activations, rows = tokens: 8 int8 codes of token l%16, permuted
//       [x0 x2 x4 x6 | x1 x3 x5 x7] to match B;
//   B = weights, columns = weight rows: one packed word (8 nibbles) of row n0+l%16,
//       split into even/odd nibbles and sign-shifted to int8 (nibble - 8).
// Workgroup = 16 weight rows; its 8 waves take every 8th group and their partials meet
// in LDS. Tokens beyond 16 are further 16-row M tiles of the same
// launch (the weight tile is then re-read from L2).
#include "ti_dev.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int GMAX = 512;       // K <= 16384

// WAVES waves per 16-row tile, each on every WAVES-th group; UNROLL groups per wave have
// their loads in flight together (WAVES * UNROLL groups cover K = 32 * WAVES * UNROLL in
// one batch: 2048 for (8, 8)).
template <int WAVES, int UNROLL>
__global__ __launch_bounds__(64 * WAVES) void k_gemm_q4_q8_mfma(const uint32_t* __restrict__ xq, const float* __restrict__ xs,
                                                               const uint32_t* __restrict__ pack,
                                                               const uint16_t* __restrict__ scales, float* __restrict__ y,
                                                               int T, int N, int K, int acc) {
    constexpr int SX_PER = (16 * GMAX + 64 * WAVES - 1) / (64 * WAVES);
    __shared__ float s_sx[16][GMAX];
    __shared__ float s_part[WAVES][16][17];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int G = K / 32;
    const int m = lane & 15, j = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int row = min(n0 + m, N - 1);
    const uint32_t* prow = pack + (size_t)row * (K / 8);
    const uint16_t* srow = scales + (size_t)row * G;

    for (int t0 = 0; t0 < T; t0 += 16) {
        const int tm = min(16, T - t0);
        // token row of this lane's A operand (rows past T read token t0 and are zeroed by s_sx)
        const int ta = t0 + (m < tm ? m : 0);
        const uint32_t* arow = xq + (size_t)ta * (K / 4);
        uint32_t wq[UNROLL];
        uint2 aq[UNROLL];
        uint16_t sw[UNROLL];
        auto load = [&](int g0) {
#pragma unroll
            for (int u = 0; u < UNROLL; u++) {
                const int g = g0 + WAVES * u;
                const int gc = g < G ? g : G - 1;
                wq[u] = prow[4 * gc + j];
                aq[u] = *reinterpret_cast<const uint2*>(arow + 8 * gc + 2 * j);
                sw[u] = srow[gc];
            }
        };
        load(wave);                            // the first batch is in flight while the scales are staged
        __syncthreads();                       // s_sx / s_part of the previous M tile are consumed
        {   // the tile's activation scales: every load issued before the first store
            float v[SX_PER];
#pragma unroll
            for (int k = 0; k < SX_PER; k++) {
                const int e = tid + k * 64 * WAVES;
                const int t = e / G, g = e % G;
                const int tc = t < tm ? t : 0;
                v[k] = e < 16 * G ? xs[(size_t)(t0 + tc) * G + g] : 0.0f;
            }
#pragma unroll
            for (int k = 0; k < SX_PER; k++) {
                const int e = tid + k * 64 * WAVES;
                const int t = e / G, g = e % G;
                if (e < 16 * G) s_sx[t][g] = t < tm ? v[k] : 0.0f;
            }
        }
        __syncthreads();
        float accv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int g0 = wave; g0 < G; g0 += WAVES * UNROLL) {
            if (g0 != wave) load(g0);
            float sxv[UNROLL][4];
#pragma unroll
            for (int u = 0; u < UNROLL; u++) {
                const int g = g0 + WAVES * u;
                const int gc = g < G ? g : G - 1;
#pragma unroll
                for (int i = 0; i < 4; i++) sxv[u][i] = s_sx[4 * j + i][gc];
            }
            // no branch on g < G here: a guarded use lets the compiler sink the loads into
            // the branch, one memory round trip per group; past G the weight is zeroed
#pragma unroll
            for (int u = 0; u < UNROLL; u++) {
                const int g = g0 + WAVES * u;
                uint32_t blo, bhi;
                nib_to_s8(wq[u], blo, bhi);
                const uint32_t alo = even_bytes(aq[u].x, aq[u].y), ahi = odd_bytes(aq[u].x, aq[u].y);
                const long A = (long)(((uint64_t)ahi << 32) | alo);
                const long B = (long)(((uint64_t)bhi << 32) | blo);
                const v4i z = {0, 0, 0, 0};
                const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, z, 0, 0, 0);
                const float sg = g < G ? ti_h2f(sw[u]) : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) accv[i] = fmaf((float)d[i], sg * sxv[u][i], accv[i]);
            }
        }
        // the waves' partials: lane holds tokens 4j..4j+3 of column m
#pragma unroll
        for (int i = 0; i < 4; i++) s_part[wave][4 * j + i][m] = accv[i];
        __syncthreads();
        if (tid < 256) {
            const int t = tid / 16, c = tid % 16;    // 256 threads = 16 tokens x 16 rows
            const int n = n0 + c;
            if (t < tm && n < N) {
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < WAVES; w++) v += s_part[w][t][c];
                float* yp = y + (size_t)(t0 + t) * N + n;
                *yp = acc ? *yp + v : v;
            }
        }
    }
}

}  // namespace

int ti_gemm_q4_q8_launch(ti_ctx* c, const uint32_t* xq, const float* xs, const uint32_t* pack, const uint16_t* scales,
                         float* y, int T, int N, int K, int acc) {
    if (K % 32 != 0 || K / 32 > GMAX) return ti_fail(TI_ERR_INVALID, "int4 GEMM: K=%d must be a multiple of 32, <= %d", K, GMAX * 32);
    if (T <= 0 || N <= 0) return ti_fail(TI_ERR_INVALID, "int4 GEMM: T=%d N=%d", T, N);
    const unsigned grid = (unsigned)((N + 15) / 16);
    k_gemm_q4_q8_mfma<8, 8><<<grid, 512, 0, c->stream>>>(xq, xs, pack, scales, y, T, N, K, acc);
    TI_LAUNCHED("k_gemm_q4_q8_mfma");
    return TI_OK;
}
