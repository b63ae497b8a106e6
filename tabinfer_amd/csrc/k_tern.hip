// k_tern.hip — ternary (Q2_0_g64) GEMV and its activation quantizer:
//  gemv_tern       native/crates/n2-kernels/src/tern.rs:56-119, 246-338;
//                      cpu/kernel/src/lib.rs:438-544 (B=1) and :331-432 (B=4 batched)
//  quantize_act    tern.rs:196-222 (n2: 127/amax, round half away from zero)
//      quantize        cpu/kernel/src/lib.rs:570-606 (WASM: amax/127, nearest-even)
//
// out[n] = sum_b s[n,b]*dot_b - sum_b s[n,b]*xsum[b], dot_b = sum code*act over the
// 64-code block (codes {0,1,2}); the two sums are kept apart and subtracted once
// per row, as the reference requires. Block layout: 16 bytes, code c at byte c&15,
// bits 2*(c>>4), so plane j ((byte >> 2j) & 3) holds codes 16j..16j+15 and pairs
// with the contiguous activations act[64b+16j .. +16] — one v_dot4_i32_i8 per
// 4 codes, no shuffles.
#include "ti_internal.h"

namespace {

constexpr uint32_t M2 = 0x03030303u;

// the 64 int8 activations of one block (16 dwords) plus its xsum
struct ActT {
    int a[16];
    float xs;
};

__device__ __forceinline__ void load_act_tern(const int8_t* __restrict__ act, const int32_t* __restrict__ xsum, int blk,
                                              ActT& t) {
    const uint4* p = reinterpret_cast<const uint4*>(act + (size_t)blk * 64);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint4 u = p[i];
        t.a[4 * i] = (int)u.x; t.a[4 * i + 1] = (int)u.y; t.a[4 * i + 2] = (int)u.z; t.a[4 * i + 3] = (int)u.w;
    }
    t.xs = xsum ? (float)xsum[blk] : 0.0f;
}

// exact int32 dot of one 64-code block with the activation block
__device__ __forceinline__ int tern_block_dot(const uint4 w, const ActT& t) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    int d = 0;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int m = 0; m < 4; m++) d = __builtin_amdgcn_sdot4((int)((ws[m] >> (2 * j)) & M2), t.a[4 * j + m], d, false);
    return d;
}

// Two phases per tile of TR rows (one wavefront per workgroup):
//  1. lanes compute the exact int32 block dots of the tile (LPR lanes per row, each
//     owning fixed blocks, so its activation blocks live in registers; 16-byte
//     coalesced code loads) and park them in LDS as dots[b][row][block];
//  2. lane (b, r) replays row r's accumulation in the reference's block order —
//     acc += s*dot, sxs += s*xsum, one subtraction — so the f32 result is
//     bit-identical to the reference's scalar kernel (tern.rs:79-119).
template <int LPR, int BPL, int B, int TR>
__global__ __launch_bounds__(64) void k_tern_gemv(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                  const int8_t* __restrict__ act, const int32_t* __restrict__ xsum,
                                                  float* __restrict__ out, int N, int K, long out_stride) {
    constexpr int RPP = 64 / LPR;
    constexpr int NB = LPR * BPL;                // blocks per row
    constexpr int PASSES = TR / RPP;
    constexpr int CH = PASSES < 8 ? PASSES : 8;  // passes whose loads are in flight together
    static_assert(TR % RPP == 0 && TR * B <= 64, "tile shape");
    __shared__ int dots[B][TR][NB + 1];
    const int lane = threadIdx.x;
    const int sub = lane / LPR, li = lane % LPR;
    ActT at[B][BPL];
#pragma unroll
    for (int bb = 0; bb < B; bb++)
#pragma unroll
        for (int j = 0; j < BPL; j++) load_act_tern(act + (size_t)bb * K, nullptr, li + LPR * j, at[bb][j]);
    const long ntiles = (N + TR - 1) / TR;
    for (long tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const long row0 = tile * TR;
#pragma unroll
        for (int pc = 0; pc < PASSES; pc += CH) {
            uint4 cw[CH][BPL];
#pragma unroll
            for (int p = 0; p < CH; p++) {
                long row = row0 + (long)(pc + p) * RPP + sub;
                row = row < N ? row : N - 1;
#pragma unroll
                for (int j = 0; j < BPL; j++) cw[p][j] = ti_ld_nt(codes + row * NB + li + LPR * j);
            }
#pragma unroll
            for (int p = 0; p < CH; p++)
#pragma unroll
                for (int j = 0; j < BPL; j++)
#pragma unroll
                    for (int bb = 0; bb < B; bb++)
                        dots[bb][(pc + p) * RPP + sub][li + LPR * j] = tern_block_dot(cw[p][j], at[bb][j]);
        }
        __syncthreads();
        if (lane < TR * B) {
            const int bb = lane / TR, r = lane % TR;
            const long row = row0 + r;
            if (row < N) {
                const float* srow = scales + row * NB;
                const int32_t* xs = xsum + (size_t)bb * NB;
                float acc = 0.0f, sxs = 0.0f;
                for (int blk = 0; blk < NB; blk++) {
                    const float sc = srow[blk];
                    const float p = sc * (float)dots[bb][r][blk];
                    acc = acc + p;
                    const float q = sc * (float)xs[blk];
                    sxs = sxs + q;
                }
                out[(size_t)bb * out_stride + row] = acc - sxs;
            }
        }
        __syncthreads();
    }
}

// B = 1, the latency-bound decode shapes: LPR lanes per row (32 when the row's block count
// is a multiple of 32, else 16), lane li owning blocks li + LPR j, so a 2048-row matrix
// spreads over 256 workgroups of 4 waves. Every lane forms its blocks' exact int32 dots and
// the two products s*dot and s*xsum (the same IEEE products the reference forms) and parks
// them in LDS; then lane 0 of the row adds the s*dot products and lane 1 the s*xsum
// products, each in block order (tern.rs:79-119's two chains), four per LDS read, and the
// row's result is their difference. A row's products come from its own wave, so the
// hand-off is a wave-level one: LDS operations of a wave complete in program order.
struct TernMats {
    const uint4* codes[3];
    const float* scales[3];
    float* out[3];
    int N[3];
    int blk0[3];      // first workgroup of each matrix
    int nmat;
};

//
// NQE > 0: the input is the residual x (+ add / add_scale) instead of ready codes. Every
// workgroup runs the Bonsai decoder's residual add, RMSNorm and n2 quantizer over the whole
// K = 256 NQE vector itself (NQE consecutive elements per thread; the same inputs and the
// same operations in every workgroup, so every workgroup holds the same codes), keeps the
// codes and block sums in LDS, and workgroup 0 publishes x + add, xn, the codes, the block
// sums and the scale for the kernels after this one. The norm's loads are issued before
// the weights', so its waits do not wait for the weight stream.
//
// SWI: the input is the gate/up pair instead: every workgroup forms the SwiGLU of the scaled
// gate/up over the whole K = 2048 BPL vector (element 8 (tid + 256 k) + i at thread tid, so
// a 64-code block is 8 threads' chunks) and the n2 quantizer of it, and workgroup 0
// publishes the SwiGLU output, the codes, the block sums and the scale.
template <int LPR, int BPL, int NQE, bool SWI = false>
__global__ __launch_bounds__(256) void k_tern_gemv_rw(TernMats m, const int8_t* __restrict__ act,
                                                      const int32_t* __restrict__ xsum, ti_tern_norm nq,
                                                      ti_tern_swiglu sw) {
    constexpr int RW = 64 / LPR, NB = LPR * BPL, RPB = 4 * RW;
    static_assert(NB % 4 == 0, "four products per LDS read");
    static_assert(NQE == 0 || (NB * 64 == 256 * NQE && NQE % 4 == 0 && 64 % NQE == 0), "norm width = K");
    static_assert(!SWI || (NQE == 0 && LPR == 32), "SwiGLU prologue: K = 2048 BPL");
    constexpr bool PRO = NQE > 0 || SWI;
    constexpr int NQA = PRO ? 64 * NB / 4 : 1, NQB = PRO ? NB : 1;
    __shared__ float4 s_pq[4][RW][2][NB / 4];
    __shared__ __align__(16) uint32_t s_act[NQA];
    __shared__ int32_t s_xs[NQB];
    __shared__ float s_red[8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane / LPR, li = lane % LPR;
    // the matrix of this workgroup (uniform: selects, no divergent indexing of the kernargs)
    const int b = blockIdx.x;
    const int mi = (m.nmat > 1 && b >= m.blk0[1]) + (m.nmat > 2 && b >= m.blk0[2]);
    const uint4* codes = mi == 0 ? m.codes[0] : (mi == 1 ? m.codes[1] : m.codes[2]);
    const float* scales = mi == 0 ? m.scales[0] : (mi == 1 ? m.scales[1] : m.scales[2]);
    float* out = mi == 0 ? m.out[0] : (mi == 1 ? m.out[1] : m.out[2]);
    const int N = mi == 0 ? m.N[0] : (mi == 1 ? m.N[1] : m.N[2]);
    const int b0 = mi == 0 ? 0 : (mi == 1 ? m.blk0[1] : m.blk0[2]);
    const long row = (long)(b - b0) * RPB + wave * RW + r;
    const long rowc = row < N ? row : N - 1;
    uint4 cw[BPL];
    float sc[BPL], xs[BPL];
    constexpr int NQR = NQE > 0 ? NQE : 1;
    float nx[NQR], na[NQR], nw[NQR];
    if constexpr (NQE > 0) {
#pragma unroll
        for (int i = 0; i < NQE; i += 4) {
            const float4 x4 = *reinterpret_cast<const float4*>(nq.x + tid * NQE + i);
            const float4 w4 = nq.w ? *reinterpret_cast<const float4*>(nq.w + tid * NQE + i) : make_float4(1.f, 1.f, 1.f, 1.f);
            const float4 a4 = nq.add ? *reinterpret_cast<const float4*>(nq.add + tid * NQE + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            nx[i] = x4.x; nx[i + 1] = x4.y; nx[i + 2] = x4.z; nx[i + 3] = x4.w;
            nw[i] = w4.x; nw[i + 1] = w4.y; nw[i + 2] = w4.z; nw[i + 3] = w4.w;
            na[i] = a4.x; na[i + 1] = a4.y; na[i + 2] = a4.z; na[i + 3] = a4.w;
        }
        TI_ISSUE_FENCE();
    }
    constexpr int SWR = SWI ? 8 * BPL : 1;
    float sg[SWR], su[SWR];
    if constexpr (SWI) {
#pragma unroll
        for (int k = 0; k < BPL; k++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const size_t e = (size_t)8 * (tid + 256 * k) + 4 * h;
                const float4 g4 = *reinterpret_cast<const float4*>(sw.g + e);
                const float4 u4 = *reinterpret_cast<const float4*>(sw.u + e);
                sg[8 * k + 4 * h] = g4.x; sg[8 * k + 4 * h + 1] = g4.y; sg[8 * k + 4 * h + 2] = g4.z; sg[8 * k + 4 * h + 3] = g4.w;
                su[8 * k + 4 * h] = u4.x; su[8 * k + 4 * h + 1] = u4.y; su[8 * k + 4 * h + 2] = u4.z; su[8 * k + 4 * h + 3] = u4.w;
            }
        TI_ISSUE_FENCE();
    }
#pragma unroll
    for (int j = 0; j < BPL; j++) {
        cw[j] = ti_ld_nt(codes + rowc * NB + li + LPR * j);
        sc[j] = scales[rowc * NB + li + LPR * j];
        if constexpr (!PRO) xs[j] = (float)xsum[li + LPR * j];
    }
    const int8_t* av = act;
    if constexpr (SWI) {
        TI_ISSUE_FENCE();
        // ops.rs:110-117 on the scaled gate/up, then quantize_act (tern.rs:206-222)
        const float inv = 1.0f / *sw.gu_scale;
        float mx = 0.0f;
#pragma unroll
        for (int e = 0; e < 8 * BPL; e++) {
            const float gg = sg[e] * inv;
            const float uu = su[e] * inv;
            sg[e] = (gg / (1.0f + expf(-gg))) * uu;
            mx = fmaxf(mx, fabsf(sg[e]));
        }
        mx = ti_wave_max(mx);
        if (lane == 0) s_red[4 + wave] = mx;
        __syncthreads();
        const float amax = fmaxf(fmaxf(s_red[4], s_red[5]), fmaxf(s_red[6], s_red[7]));
        const float qs = amax > 0.0f ? 127.0f / amax : 1.0f;
#pragma unroll
        for (int k = 0; k < BPL; k++) {
            const int ch = tid + 256 * k;                // 8-element chunk; block ch / 8
            uint32_t wd[2];
            int bs = 0;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                uint32_t w = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float rq = roundf(sg[8 * k + 4 * h + i] * qs);
                    rq = fminf(fmaxf(rq, -127.0f), 127.0f);
                    const int q = (int)rq;
                    bs += q;
                    w |= (uint32_t)(q & 0xff) << (8 * i);
                }
                wd[h] = w;
            }
            *reinterpret_cast<uint2*>(&s_act[2 * ch]) = make_uint2(wd[0], wd[1]);
            bs += __shfl_xor(bs, 4);
            bs += __shfl_xor(bs, 2);
            bs += __shfl_xor(bs, 1);
            if ((tid & 7) == 0) s_xs[ch / 8] = bs;
            if (blockIdx.x == 0) {
                *reinterpret_cast<float4*>(sw.swi_out + 8 * ch) = make_float4(sg[8 * k], sg[8 * k + 1], sg[8 * k + 2], sg[8 * k + 3]);
                *reinterpret_cast<float4*>(sw.swi_out + 8 * ch + 4) =
                    make_float4(sg[8 * k + 4], sg[8 * k + 5], sg[8 * k + 6], sg[8 * k + 7]);
                *reinterpret_cast<uint2*>(sw.act_out + 8 * ch) = make_uint2(wd[0], wd[1]);
                if ((tid & 7) == 0) sw.xsum_out[ch / 8] = bs;
            }
        }
        if (blockIdx.x == 0 && tid == 0) *sw.scale_out = qs;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < BPL; j++) xs[j] = (float)s_xs[li + LPR * j];
        av = reinterpret_cast<const int8_t*>(s_act);
    }
    if constexpr (NQE > 0) {
        TI_ISSUE_FENCE();
        constexpr int TPB = 64 / NQE;                    // threads per 64-code block
        const float inv_add = nq.add ? 1.0f / *nq.add_scale : 0.0f;
        float mx = 0.0f;
        if (nq.w) {                                      // uniform: residual add + RMSNorm
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < NQE; i++) {
                if (nq.add) {
                    const float d = na[i] * inv_add;
                    nx[i] = nx[i] + d;
                }
                ss = ss + nx[i] * nx[i];
            }
            ss = ti_wave_sum(ss);
            if (lane == 0) s_red[wave] = ss;
            __syncthreads();
            const float mean = (s_red[0] + s_red[1] + s_red[2] + s_red[3]) / (float)(256 * NQE);
            const float inv = 1.0f / sqrtf(mean + nq.eps);
#pragma unroll
            for (int i = 0; i < NQE; i++) {
                na[i] = nx[i] * inv * nw[i];              // xn
                mx = fmaxf(mx, fabsf(na[i]));
            }
        } else {                                         // the quantizer alone (x as is)
#pragma unroll
            for (int i = 0; i < NQE; i++) {
                na[i] = nx[i];
                mx = fmaxf(mx, fabsf(na[i]));
            }
        }
        mx = ti_wave_max(mx);
        if (lane == 0) s_red[4 + wave] = mx;
        __syncthreads();
        const float amax = fmaxf(fmaxf(s_red[4], s_red[5]), fmaxf(s_red[6], s_red[7]));
        const float qs = amax > 0.0f ? 127.0f / amax : 1.0f;
        uint32_t wd[NQE / 4];
        int bs = 0;
#pragma unroll
        for (int k = 0; k < NQE / 4; k++) {
            uint32_t w = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float rq = roundf(na[4 * k + i] * qs);
                rq = fminf(fmaxf(rq, -127.0f), 127.0f);
                const int q = (int)rq;
                bs += q;
                w |= (uint32_t)(q & 0xff) << (8 * i);
            }
            wd[k] = w;
            s_act[tid * (NQE / 4) + k] = w;
        }
#pragma unroll
        for (int o = TPB / 2; o > 0; o >>= 1) bs += __shfl_xor(bs, o);
        if (tid % TPB == 0) s_xs[tid / TPB] = bs;
        if (blockIdx.x == 0) {
#pragma unroll
            for (int i = 0; i < NQE; i += 4) {
                if (nq.x_out)
                    *reinterpret_cast<float4*>(nq.x_out + tid * NQE + i) = make_float4(nx[i], nx[i + 1], nx[i + 2], nx[i + 3]);
                if (nq.xn_out)
                    *reinterpret_cast<float4*>(nq.xn_out + tid * NQE + i) = make_float4(na[i], na[i + 1], na[i + 2], na[i + 3]);
            }
#pragma unroll
            for (int k = 0; k < NQE / 4; k++) reinterpret_cast<uint32_t*>(nq.act_out)[tid * (NQE / 4) + k] = wd[k];
            if (tid % TPB == 0) nq.xsum_out[tid / TPB] = bs;
            if (tid == 0) *nq.scale_out = qs;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < BPL; j++) xs[j] = (float)s_xs[li + LPR * j];
        av = reinterpret_cast<const int8_t*>(s_act);
    }
    float* sp = reinterpret_cast<float*>(&s_pq[wave][r][0][0]);
    float* sq = reinterpret_cast<float*>(&s_pq[wave][r][1][0]);
#pragma unroll
    for (int j = 0; j < BPL; j++) {
        ActT t;
        const int blk = li + LPR * j;
        load_act_tern(av, nullptr, blk, t);
        sp[blk] = sc[j] * (float)tern_block_dot(cw[j], t);
        sq[blk] = sc[j] * xs[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float v = 0.0f;
    if (li < 2) {
        const float4* pq = &s_pq[wave][r][li][0];
#pragma unroll 6
        for (int i = 0; i < NB / 4; i++) {
            const float4 p = pq[i];
            v = v + p.x;
            v = v + p.y;
            v = v + p.z;
            v = v + p.w;
        }
    }
    const float sxs = __shfl_down(v, 1);
    if (li == 0 && row < N) out[row] = v - sxs;
}

// rows per workgroup of k_tern_gemv_rw for nb blocks per row; 0: no instantiation
static int rw_rows(int nb) {
    if (nb % 32 == 0 && nb / 32 <= 4) return 8;
    if (nb % 16 == 0 && nb / 16 <= 7) return 16;
    return 0;
}

// sets m.blk0 for the kernel's rows per workgroup and launches; false: no kernel for nb
// (with nq: only K = 1024 and 2048, the norm prologue's widths)
static bool rw_launch(ti_ctx* c, TernMats& m, int nb, const int8_t* act, const int32_t* xsum,
                      const ti_tern_norm* nq = nullptr, const ti_tern_swiglu* sw = nullptr) {
    const int rpb = rw_rows(nb);
    if (!rpb) return false;
    long blocks = 0;
    for (int i = 0; i < 3; i++) {
        m.blk0[i] = (int)blocks;
        if (i < m.nmat) blocks += (m.N[i] + rpb - 1) / rpb;
    }
    if (blocks >= (1L << 31)) return false;
    const unsigned grid = (unsigned)blocks;
    const ti_tern_norm nnone = {};
    const ti_tern_swiglu snone = {};
    if (nq) {
        if (nb == 32) { k_tern_gemv_rw<32, 1, 8><<<grid, 256, 0, c->stream>>>(m, act, xsum, *nq, snone); return true; }
        if (nb == 16) { k_tern_gemv_rw<16, 1, 4><<<grid, 256, 0, c->stream>>>(m, act, xsum, *nq, snone); return true; }
        return false;
    }
    if (sw) {
        if (nb == 32) { k_tern_gemv_rw<32, 1, 0, true><<<grid, 256, 0, c->stream>>>(m, act, xsum, nnone, *sw); return true; }
        if (nb == 96) { k_tern_gemv_rw<32, 3, 0, true><<<grid, 256, 0, c->stream>>>(m, act, xsum, nnone, *sw); return true; }
        return false;
    }
#define RW(L, P) \
    if (nb == L * P) { k_tern_gemv_rw<L, P, 0><<<grid, 256, 0, c->stream>>>(m, act, xsum, nnone, snone); return true; }
    RW(32, 1) RW(32, 2) RW(32, 3) RW(32, 4) RW(16, 1) RW(16, 3) RW(16, 5) RW(16, 7)
#undef RW
    return false;
}

// any K % 64 == 0: one lane per row, blocks in order (same arithmetic as above)
__global__ __launch_bounds__(64) void k_tern_gemv_generic(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                          const int8_t* __restrict__ act, const int32_t* __restrict__ xsum,
                                                          float* __restrict__ out, int N, int K, long out_stride) {
    const long row = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= N) return;
    const int nb = K / 64;
    float acc = 0.0f, sxs = 0.0f;
    for (int blk = 0; blk < nb; blk++) {
        ActT t;
        load_act_tern(act, xsum, blk, t);
        const float sc = scales[row * nb + blk];
        const float p = sc * (float)tern_block_dot(codes[row * nb + blk], t);
        acc = acc + p;
        const float q = sc * t.xs;
        sxs = sxs + q;
    }
    out[row] = acc - sxs;
}

__global__ void k_tern_block_dots(const uint4* __restrict__ codes, const int8_t* __restrict__ act, int32_t* __restrict__ dots,
                                  long total, int nb) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    ActT t;
    load_act_tern(act, nullptr, (int)(i % nb), t);
    dots[i] = tern_block_dot(codes[i], t);
}

// ---------------------------------------------------------------------------
// per-tensor int8 activation quant + per-64 sums, one 1024-thread workgroup.
// mode 0 (n2): scale = 127/amax (1 if amax == 0), a = clamp(round-half-away(x*scale))
// mode 1 (WASM): asc = amax/127 (1e-9 if 0), a = clamp(nearest-even(x*(1/asc)))
// The max is order-independent, so the codes are bit-exact.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_quant_act_tern(const float* __restrict__ x, int8_t* __restrict__ act,
                                                         int32_t* __restrict__ xsum, float* __restrict__ scale_out,
                                                         int K, int mode) {
    __shared__ float red[16];
    __shared__ float sh_scale;
    const int t = threadIdx.x;
    float m = 0.0f;
    for (int i = t; i < K; i += 1024) m = fmaxf(m, fabsf(x[i]));
    m = ti_wave_max(m);
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    if (t == 0) {
        float amax = red[0];
        for (int w = 1; w < 16; w++) amax = fmaxf(amax, red[w]);
        float s;
        if (mode == 0) s = amax > 0.0f ? 127.0f / amax : 1.0f;
        else s = amax > 0.0f ? amax / 127.0f : 1e-9f;
        sh_scale = s;
        *scale_out = s;
    }
    __syncthreads();
    const float s = sh_scale;
    const float mul = mode == 0 ? s : 1.0f / s;
    // one wave per 64-block: lane quantizes one element, the wave sums the block
    const int lane = t & 63;
    for (int blk = t >> 6; blk < K / 64; blk += 16) {
        float v = x[blk * 64 + lane] * mul;
        float r = mode == 0 ? roundf(v) : rintf(v);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        int q = (int)r;
        act[blk * 64 + lane] = (int8_t)q;
        const int sum = ti_wave_sum_i(q);
        if (lane == 0) xsum[blk] = sum;
    }
}

struct Shape {
    int lpr, bpl;
};
Shape pick(int nb) {
    int lpr = 1;
    while (lpr < 64 && (nb % (lpr * 2)) == 0) lpr *= 2;
    return {lpr, nb / lpr};
}


}  // namespace

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// launches the tile kernel when the tile is a whole number of row passes;
// returns false otherwise (the caller then splits the batch)
template <int L, int P, int BB, int T>
static bool launch_tile(ti_ctx* c, unsigned grid, const uint4* c4, const float* scales, const int8_t* act,
                        const int32_t* xsum, float* out, int N, int K, long out_stride) {
    if constexpr (T % (64 / L) == 0 && T * BB <= 64) {
        k_tern_gemv<L, P, BB, T><<<grid, 64, 0, c->stream>>>(c4, scales, act, xsum, out, N, K, out_stride);
        return true;
    } else {
        return false;
    }
}

static int tern_launch(ti_ctx* c, float* out, const uint8_t* codes, const float* scales, const int8_t* act,
                       const int32_t* xsum, int N, int K, int B, long out_stride) {
    const uint4* c4 = reinterpret_cast<const uint4*>(codes);
    int nb = K / 64;
    if (B == 1 && N <= (1 << 30) - 16) {
        TernMats m = {};
        m.codes[0] = m.codes[1] = m.codes[2] = c4;
        m.scales[0] = m.scales[1] = m.scales[2] = scales;
        m.out[0] = m.out[1] = m.out[2] = out;
        m.N[0] = m.N[1] = m.N[2] = N;
        m.nmat = 1;
        if (rw_launch(c, m, nb, act, xsum)) {
            TI_LAUNCHED("k_tern_gemv_rw");
            return TI_OK;
        }
    }
    Shape s = pick(nb);
    const int TR = B == 1 ? 64 : (B == 2 ? 32 : 16);
    long ntiles = (N + TR - 1) / TR;
    long maxg = 256L * 8;                       // persistent: up to 8 tiles in flight per CU
    unsigned grid = (unsigned)(ntiles < maxg ? ntiles : maxg);
#define TB(L, P, BB, T) launch_tile<L, P, BB, T>(c, grid, c4, scales, act, xsum, out, N, K, out_stride)
#define TCASE(L, P)                                                        \
    if (s.lpr == L && s.bpl == P) {                                        \
        bool ok = B == 1 ? TB(L, P, 1, 64)                                 \
                : (B == 2 && P <= 2) ? TB(L, P, 2, 32)                     \
                : (B == 4 && P == 1) ? TB(L, P, 4, 16) : false;            \
        if (!ok) goto split;                                               \
        TI_LAUNCHED("k_tern_gemv");                                        \
        return TI_OK;                                                      \
    }
    TCASE(1, 1) TCASE(2, 1) TCASE(4, 1) TCASE(8, 1) TCASE(16, 1) TCASE(32, 1) TCASE(64, 1)
    TCASE(32, 3) TCASE(64, 2) TCASE(64, 3)
#undef TCASE
#undef TB
    if (B == 1) {
        k_tern_gemv_generic<<<(unsigned)((N + 63) / 64), 64, 0, c->stream>>>(c4, scales, act, xsum, out, N, K, out_stride);
        TI_LAUNCHED("k_tern_gemv_generic");
        return TI_OK;
    }
split:
    for (int bb = 0; bb < B; bb++) {
        int rc = tern_launch(c, out + (size_t)bb * out_stride, codes, scales, act + (size_t)bb * K,
                             xsum + (size_t)bb * nb, N, K, 1, out_stride);
        if (rc) return rc;
    }
    return TI_OK;
}

extern "C" int ti_tern_gemv(ti_ctx* c, float* out, const uint8_t* codes, const float* scales, const int8_t* act,
                            const int32_t* xsum, int N, int K) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(out && codes && scales && act && xsum, "ti_tern_gemv: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "ti_tern_gemv: K must be a positive multiple of 64 (N=%d K=%d)", N, K);
    TI_REQUIRE(al16(codes) && al16(act), "ti_tern_gemv: codes and act must be 16-byte aligned");
    return tern_launch(c, out, codes, scales, act, xsum, N, K, 1, N);
}

extern "C" int ti_tern_gemv_multi(ti_ctx* c, const int8_t* act, const int32_t* xsum, int K, int nmat,
                                  const uint8_t* const* codes, const float* const* scales, float* const* outs,
                                  const int* Ns) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(act && xsum && codes && scales && outs && Ns, "ti_tern_gemv_multi: null argument");
    TI_REQUIRE(nmat >= 1 && nmat <= 3, "ti_tern_gemv_multi: nmat must be 1..3 (nmat=%d)", nmat);
    TI_REQUIRE(K > 0 && K % 1024 == 0 && K <= 8192, "ti_tern_gemv_multi: K must be a multiple of 1024, <= 8192 (K=%d)", K);
    TI_REQUIRE(al16(act), "ti_tern_gemv_multi: act must be 16-byte aligned");
    TernMats m = {};
    for (int i = 0; i < 3; i++) {
        const int s = i < nmat ? i : nmat - 1;
        if (i < nmat) {
            TI_REQUIRE(codes[i] && scales[i] && outs[i] && Ns[i] > 0, "ti_tern_gemv_multi: matrix %d: null buffer or N <= 0", i);
            TI_REQUIRE(al16(codes[i]), "ti_tern_gemv_multi: codes[%d] must be 16-byte aligned", i);
        }
        m.codes[i] = reinterpret_cast<const uint4*>(codes[s]);
        m.scales[i] = scales[s];
        m.out[i] = outs[s];
        m.N[i] = Ns[s];
    }
    m.nmat = nmat;
    if (!rw_launch(c, m, K / 64, act, xsum)) return ti_fail(TI_ERR_INVALID, "ti_tern_gemv_multi: no kernel for K=%d", K);
    TI_LAUNCHED("k_tern_gemv_rw");
    return TI_OK;
}

// q/k/v (or gate/up) of the Bonsai decoder with the residual add + RMSNorm + quantizer of
// their input in every workgroup's prologue (k_tern_gemv_rw with NQE > 0): K = 1024 or 2048.
bool ti_tern_norm_ok(int K) { return K == 1024 || K == 2048; }

int ti_tern_gemv_multi_norm(ti_ctx* c, const ti_tern_norm* nq, int K, int nmat, const uint8_t* const* codes,
                            const float* const* scales, float* const* outs, const int* Ns) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(nq && nq->x && nq->act_out && nq->xsum_out && nq->scale_out && (!nq->add || nq->add_scale),
               "ti_tern_gemv_multi_norm: null norm buffer");
    TI_REQUIRE(nq->w || !nq->add, "ti_tern_gemv_multi_norm: a residual add needs the norm");
    TI_REQUIRE(ti_tern_norm_ok(K), "ti_tern_gemv_multi_norm: K must be 1024 or 2048 (K=%d)", K);
    TI_REQUIRE(nq->x_out != nq->x, "ti_tern_gemv_multi_norm: x_out must not alias x");
    TI_REQUIRE(al16(nq->x) && al16(nq->w) && al16(nq->x_out) && al16(nq->xn_out) && al16(nq->act_out) &&
                   (!nq->add || al16(nq->add)), "ti_tern_gemv_multi_norm: vectors must be 16-byte aligned");
    TI_REQUIRE(nmat >= 1 && nmat <= 3 && codes && scales && outs && Ns, "ti_tern_gemv_multi_norm: bad matrices");
    TernMats m = {};
    for (int i = 0; i < 3; i++) {
        const int s = i < nmat ? i : nmat - 1;
        if (i < nmat) {
            TI_REQUIRE(codes[i] && scales[i] && outs[i] && Ns[i] > 0, "ti_tern_gemv_multi_norm: matrix %d: null buffer or N <= 0", i);
            TI_REQUIRE(al16(codes[i]), "ti_tern_gemv_multi_norm: codes[%d] must be 16-byte aligned", i);
        }
        m.codes[i] = reinterpret_cast<const uint4*>(codes[s]);
        m.scales[i] = scales[s];
        m.out[i] = outs[s];
        m.N[i] = Ns[s];
    }
    m.nmat = nmat;
    if (!rw_launch(c, m, K / 64, nullptr, nullptr, nq)) return ti_fail(TI_ERR_INVALID, "ti_tern_gemv_multi_norm: no kernel for K=%d", K);
    TI_LAUNCHED("k_tern_gemv_rw (norm)");
    return TI_OK;
}

// the down projection of the Bonsai decoder with the SwiGLU + quantizer of its input in
// every workgroup's prologue (k_tern_gemv_rw with SWI): K = 2048 or 6144 (the widths the
// decoder's tests cover).
bool ti_tern_swiglu_ok(int K) { return K == 2048 || K == 6144; }

int ti_tern_gemv_swiglu(ti_ctx* c, const ti_tern_swiglu* sw, float* out, const uint8_t* codes, const float* scales, int N,
                        int K) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(sw && sw->g && sw->u && sw->gu_scale && sw->swi_out && sw->act_out && sw->xsum_out && sw->scale_out,
               "ti_tern_gemv_swiglu: null SwiGLU buffer");
    TI_REQUIRE(ti_tern_swiglu_ok(K), "ti_tern_gemv_swiglu: K must be 2048 or 6144 (K=%d)", K);
    TI_REQUIRE(out && codes && scales && N > 0, "ti_tern_gemv_swiglu: null matrix or N <= 0");
    TI_REQUIRE(al16(codes) && al16(sw->g) && al16(sw->u) && al16(sw->swi_out) && al16(sw->act_out),
               "ti_tern_gemv_swiglu: buffers must be 16-byte aligned");
    TernMats m = {};
    for (int i = 0; i < 3; i++) {
        m.codes[i] = reinterpret_cast<const uint4*>(codes);
        m.scales[i] = scales;
        m.out[i] = out;
        m.N[i] = N;
    }
    m.nmat = 1;
    if (!rw_launch(c, m, K / 64, nullptr, nullptr, nullptr, sw)) return ti_fail(TI_ERR_INVALID, "ti_tern_gemv_swiglu: no kernel for K=%d", K);
    TI_LAUNCHED("k_tern_gemv_rw (swiglu)");
    return TI_OK;
}

extern "C" int ti_tern_gemm(ti_ctx* c, float* out, long out_stride, const uint8_t* codes, const float* scales,
                            const int8_t* act, const int32_t* xsum, int N, int K, int B) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(out && codes && scales && act && xsum, "ti_tern_gemm: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 64 == 0 && B > 0 && out_stride >= N, "ti_tern_gemm: bad shape (N=%d K=%d B=%d)", N, K, B);
    TI_REQUIRE(al16(codes) && al16(act), "ti_tern_gemm: codes and act must be 16-byte aligned");
    // batches of 4 share each code unpack (lib.rs gemm_tern_b4); a tail runs as B=2/1
    int done = 0;
    while (done < B) {
        int bb = B - done >= 4 ? 4 : (B - done >= 2 ? 2 : 1);
        int rc = tern_launch(c, out + (size_t)done * out_stride, codes, scales, act + (size_t)done * K,
                             xsum + (size_t)done * (K / 64), N, K, bb, out_stride);
        if (rc) return rc;
        done += bb;
    }
    return TI_OK;
}

extern "C" int ti_tern_block_dots(ti_ctx* c, const uint8_t* codes, const int8_t* act, int32_t* dots, int N, int K) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(codes && act && dots, "ti_tern_block_dots: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "ti_tern_block_dots: bad shape");
    long total = (long)N * (K / 64);
    k_tern_block_dots<<<(unsigned)((total + 255) / 256), 256, 0, c->stream>>>(reinterpret_cast<const uint4*>(codes), act,
                                                                             dots, total, K / 64);
    TI_LAUNCHED("k_tern_block_dots");
    return TI_OK;
}

extern "C" int ti_quant_act_tern(ti_ctx* c, const float* x, int8_t* act, int32_t* xsum, float* scale_out, int K, int mode) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && act && xsum && scale_out, "ti_quant_act_tern: null buffer");
    TI_REQUIRE(K > 0 && K % 64 == 0, "ti_quant_act_tern: K must be a positive multiple of 64 (K=%d)", K);
    TI_REQUIRE(mode == 0 || mode == 1, "ti_quant_act_tern: mode must be 0 (n2) or 1 (wasm)");
    k_quant_act_tern<<<1, 1024, 0, c->stream>>>(x, act, xsum, scale_out, K, mode);
    TI_LAUNCHED("k_quant_act_tern");
    return TI_OK;
}
