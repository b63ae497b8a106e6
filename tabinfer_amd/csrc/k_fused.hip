// k_fused.hip — the batch-1 decode step's GEMVs as single launches.
//
// The reference issues a decode layer as ~13 dispatches (models/qwen3.js:3981-4033):
// rmsnormQ, three projGemv, attention, quantQ8 + gemvDP4 (o_proj), rmsnormQ,
// gateUpSiluDP4, quantQ8 + gemvDP4 (down). On MI355X a graph-launched kernel costs
// ~1.6 us even when empty, more than streaming a 2 MB projection, so here every
// GEMV carries its activation producer in its own prologue:
//
//   k_fgemv  MODE_NORM  rmsnormQ (:569-612) -> int8 -> int4 GEMV over up to three
//                       matrices sharing the activation (q, k, v: :3981-3984)
//            MODE_F32   quantQ8 (:332-358) -> int8 -> GEMV (+ residual): linearQ's
//                       o_proj / down_proj (:1588-1608, :4016, :4033)
//            MODE_Q8    given int8 activation -> GEMV (gemvDP4_only, :422-427)
//            GATEUP     rmsnormQ -> int8 -> gate & up rows -> silu(g)*u (:679-728)
//   k_lmhead            rmsnorm (:60-88) -> f32 GEMV (gemvQ, :276-321) -> argmax
//                       (:2624-2690) -> tok[pos+1], pos += 1 (:4049-4055)
//
// Every workgroup (256 threads) computes the whole activation prologue itself
// into LDS — the RMSNorm reduction in the reference's order (256 strided partial
// sums, then a 128..1 tree), then the per-32 quantizer — so the int8 codes are
// the ones rmsnormQ/quantQ8 produce, bit for bit. The first row block's weight
// loads are issued before the prologue, so its HBM latency overlaps the norm.
// The row engine is the one of the stand-alone GEMVs (k_gemv.hip): LPR lanes
// per row, GPL 16-byte groups per lane, R rows per lane in flight, persistent
// waves with a one-block prefetch.
#include "ti_dev.h"

namespace {

constexpr int FK_MAX = 16384;  // widest int8 activation a fused prologue holds in LDS
constexpr int LM_KMAX = 8192;  // widest f32 activation of the lm_head prologue

struct FSeg {
    const uint4* pack;
    const uint16_t* sc;
    float* y;
    int n;
};

struct FArgs {
    FSeg seg[3];
    int nseg;
    int N;      // rows over all segments
    int K;
    int acc;    // y += W x (residual)
    const float* x;        // MODE_F32 / MODE_NORM source
    const uint16_t* nw;    // MODE_NORM weight (f16)
    float eps;
    const uint32_t* xq;    // MODE_Q8 source
    const float* xs;
    uint32_t* xq_out;      // optional copy of the int8 activation (workgroup 0 writes it)
    float* xs_out;
    const uint4* upack;    // gate/up: the up matrix (seg[0] is gate, its y is swi)
    const uint16_t* usc;
    uint32_t* yq;          // gate/up: swi quantized per 32 (quantQ8) for the down projection
    float* ys;
};

// int8 activation of the whole row into LDS (s_xq: K/4 words, s_xs: K/32 scales)
template <int MODE>
__device__ __forceinline__ void act_prologue(const FArgs& a, uint32_t* s_xq, float* s_xs, float* red) {
    const int K = a.K, ng = K / 32, t = threadIdx.x;
    if (MODE == MODE_Q8) {
        const uint4* src = reinterpret_cast<const uint4*>(a.xq);
        uint4* dst = reinterpret_cast<uint4*>(s_xq);
        for (int i = t; i < K / 16; i += 256) dst[i] = src[i];
        for (int g = t; g < ng; g += 256) s_xs[g] = a.xs[g];
    } else {
        float inv = 0.0f;
        if (MODE == MODE_NORM) inv = rms_inv_256(a.x, K, a.eps, red);
        for (int g = t; g < ng; g += 256) {
            float v[32];
            load32(a.x + (size_t)g * 32, v);
            if (MODE == MODE_NORM) {
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    float p = v[j] * inv;
                    v[j] = p * ti_h2f(a.nw[g * 32 + j]);
                }
            }
            q8_group(v, s_xq + g * 8, s_xs + g, nullptr);
        }
    }
    __syncthreads();
    if (a.xq_out && blockIdx.x == 0) {
        for (int i = t; i < K / 4; i += 256) a.xq_out[i] = s_xq[i];
        for (int g = t; g < ng; g += 256) a.xs_out[g] = s_xs[g];
    }
}

// segment of a global row (the generic kernel: one row per wave)
__device__ __forceinline__ int seg_of(const FArgs& a, long row, long& local) {
    if (row < a.seg[0].n || a.nseg == 1) { local = row; return 0; }
    row -= a.seg[0].n;
    if (row < a.seg[1].n || a.nseg == 2) { local = row; return 1; }
    local = row - a.seg[1].n;
    return 2;
}

__device__ __forceinline__ const uint4* seg_pack(const FArgs& a, int s) {
    return s == 0 ? a.seg[0].pack : (s == 1 ? a.seg[1].pack : a.seg[2].pack);
}
__device__ __forceinline__ const uint16_t* seg_sc(const FArgs& a, int s) {
    return s == 0 ? a.seg[0].sc : (s == 1 ? a.seg[1].sc : a.seg[2].sc);
}
__device__ __forceinline__ float* seg_y(const FArgs& a, int s) {
    return s == 0 ? a.seg[0].y : (s == 1 ? a.seg[1].y : a.seg[2].y);
}

// Segment of a row block. Segment sizes are multiples of the block height (the
// host checks), so a block never straddles two segments and the lookup is
// wave-uniform: the pointers stay in scalar registers, read from the kernel
// arguments with constant offsets (a per-lane lookup would turn into dependent
// vector loads of the argument block before every weight load).
struct BlkSeg {
    const uint4* pack;
    const uint16_t* sc;
    float* y;
    int base;
};
__device__ __forceinline__ BlkSeg blk_seg(const FArgs& a, int row0) {
    // selects, no branches: control flow between the activation loads and the
    // weight loads would make the compiler wait for the weights in the prologue
    const int n0 = a.seg[0].n, n01 = n0 + a.seg[1].n;
    const bool in1 = a.nseg > 1 && row0 >= n0;
    const bool in2 = a.nseg > 2 && row0 >= n01;
    BlkSeg r;
    r.pack = in2 ? a.seg[2].pack : (in1 ? a.seg[1].pack : a.seg[0].pack);
    r.sc = in2 ? a.seg[2].sc : (in1 ? a.seg[1].sc : a.seg[0].sc);
    r.y = in2 ? a.seg[2].y : (in1 ? a.seg[1].y : a.seg[0].y);
    r.base = in2 ? n01 : (in1 ? n0 : 0);
    return r;
}

template <int LPR, int GPL, int R, int MODE, bool GU>
__global__ __launch_bounds__(256) void k_fgemv(FArgs a) {
    __shared__ __align__(16) uint32_t s_xq[FK_MAX / 4];
    __shared__ float s_xs[FK_MAX / 32];
    __shared__ float red[256];
    constexpr int RPP = 64 / LPR;
    constexpr int GPR = LPR * GPL;
    constexpr int SPAN = LPR / R;          // lanes holding the same row total after the reduce
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, li = lane % LPR;
    constexpr int RB = RPP * R;            // rows per wave block
    const int nwaves = gridDim.x * 4;
    const int nblocks = (a.N + RB - 1) / RB;
    int b = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
    const bool active = b < nblocks;

    uint4 wv[2][R][GPL];
    uint16_t sw[2][R][GPL];
    uint4 uv[2][GU ? R : 1][GU ? GPL : 1];
    uint16_t su[2][GU ? R : 1][GU ? GPL : 1];
    float yold[2];
    auto load = [&](int buf, int blk) {
        const BlkSeg sg = blk_seg(a, blk * RB);
#pragma unroll
        for (int r = 0; r < R; r++) {
            int row = blk * RB + sub + r * RPP;
            row = row < a.N ? row : a.N - 1;
            const long local = row - sg.base;
#pragma unroll
            for (int j = 0; j < GPL; j++) {
                long gi = local * GPR + li + LPR * j;
                wv[buf][r][j] = ti_ld_nt(sg.pack + gi);
                sw[buf][r][j] = __builtin_nontemporal_load(sg.sc + gi);
                if constexpr (GU) {
                    uv[buf][r][j] = ti_ld_nt(a.upack + gi);
                    su[buf][r][j] = __builtin_nontemporal_load(a.usc + gi);
                }
            }
        }
        if (!GU) {   // residual: the row this lane will store, fetched with the weights (unused if !acc)
            int row = blk * RB + sub + (li / SPAN) * RPP;
            row = row < a.N ? row : a.N - 1;
            yold[buf] = sg.y[row - sg.base];
        }
    };
    constexpr int EPT = (GPR * 32 + 255) / 256;
    ActRegs<EPT, GPR % 8 == 0> ar;
    if (MODE != MODE_Q8) act_regs_load<MODE>(a, ar);
    load(0, active ? b : 0);   // unconditional (block 0 for idle waves): no branch between the activation and weight loads
    TI_ISSUE_FENCE();
    if (MODE == MODE_Q8) act_prologue<MODE>(a, s_xq, s_xs, red);
    else act_regs_quant<MODE>(a, ar, s_xq, s_xs, red);
    if (!active) return;
    ActQ8 act[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) load_act_q8(s_xq, s_xs, li + LPR * j, act[j]);

    auto finish = [&](int buf, int blk) {
        float ga[R], ua[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float tg = 0.0f, tu = 0.0f;
#pragma unroll
            for (int j = 0; j < GPL; j++) {
                tg = fmaf((float)group_dot_q8(wv[buf][r][j], act[j]), ti_h2f(sw[buf][r][j]) * act[j].s, tg);
                if constexpr (GU) tu = fmaf((float)group_dot_q8(uv[buf][r][j], act[j]), ti_h2f(su[buf][r][j]) * act[j].s, tu);
            }
            ga[r] = tg;
            if (GU) ua[r] = tu;
        }
        float g = transpose_reduce<LPR, R>(ga, li);
        float u = 0.0f;
        if constexpr (GU) u = transpose_reduce<LPR, R>(ua, li);
        const int row = blk * RB + sub + (li / SPAN) * RPP;
        if ((li % SPAN) == 0 && row < a.N) {
            if (GU) {
                a.seg[0].y[row] = silu_mul(g, u);
            } else {
                const BlkSeg sg = blk_seg(a, blk * RB);
                sg.y[row - sg.base] = a.acc ? yold[buf] + g : g;
            }
        }
    };
    for (;;) {
        int nb = b + nwaves;
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

// gate/up + SiLU with the down projection's int8 activation as a by-product: each
// workgroup computes chunks of 32 consecutive rows (wave w: rows 8w..8w+7), so it
// holds whole quantQ8 groups of swi and quantizes them itself (linearQ's quantQ8
// of swi, models/qwen3.js:4033), leaving the down projection a plain int8 GEMV.
template <int LPR, int GPL>
__global__ __launch_bounds__(256) void k_gateup_q8out(FArgs a) {
    __shared__ __align__(16) uint32_t s_xq[FK_MAX / 4];
    __shared__ float s_xs[FK_MAX / 32];
    __shared__ float red[256];
    __shared__ float s_swi[32];
    constexpr int RPP = 64 / LPR;
    constexpr int R = 8 / RPP;                 // 8 rows per wave
    static_assert(R >= 1 && R <= LPR, "gate/up chunk: 8 rows per wave");
    constexpr int GPR = LPR * GPL;
    constexpr int SPAN = LPR / R;
    constexpr int EPT = (GPR * 32 + 255) / 256;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int sub = lane / LPR, li = lane % LPR;
    const int nchunks = (a.N + 31) / 32;
    int ch = blockIdx.x;
    uint4 gw[R][GPL], uw[R][GPL];
    uint16_t gs[R][GPL], us[R][GPL];
    auto load = [&](int chunk) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            int row = chunk * 32 + wave * 8 + sub + r * RPP;
            row = row < a.N ? row : a.N - 1;
#pragma unroll
            for (int j = 0; j < GPL; j++) {
                const long gi = (long)row * GPR + li + LPR * j;
                gw[r][j] = ti_ld_nt(a.seg[0].pack + gi);
                uw[r][j] = ti_ld_nt(a.upack + gi);
                gs[r][j] = __builtin_nontemporal_load(a.seg[0].sc + gi);
                us[r][j] = __builtin_nontemporal_load(a.usc + gi);
            }
        }
    };
    ActRegs<EPT, GPR % 8 == 0> ar;
    act_regs_load<MODE_NORM>(a, ar);
    load(ch < nchunks ? ch : 0);
    TI_ISSUE_FENCE();
    act_regs_quant<MODE_NORM>(a, ar, s_xq, s_xs, red);
    ActQ8 act[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) load_act_q8(s_xq, s_xs, li + LPR * j, act[j]);
    for (; ch < nchunks; ch += gridDim.x) {
        float ga[R], ua[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float tg = 0.0f, tu = 0.0f;
#pragma unroll
            for (int j = 0; j < GPL; j++) {
                tg = fmaf((float)group_dot_q8(gw[r][j], act[j]), ti_h2f(gs[r][j]) * act[j].s, tg);
                tu = fmaf((float)group_dot_q8(uw[r][j], act[j]), ti_h2f(us[r][j]) * act[j].s, tu);
            }
            ga[r] = tg;
            ua[r] = tu;
        }
        const float g = transpose_reduce<LPR, R>(ga, li);
        const float u = transpose_reduce<LPR, R>(ua, li);
        const int rl = wave * 8 + sub + (li / SPAN) * RPP;     // row within the chunk
        const int row = ch * 32 + rl;
        if ((li % SPAN) == 0) {
            const float v = row < a.N ? silu_mul(g, u) : 0.0f;
            if (row < a.N && a.seg[0].y) a.seg[0].y[row] = v;
            s_swi[rl] = v;
        }
        __syncthreads();
        if (wave == 0) {   // quantQ8 of the chunk's 32 values (q8_group's arithmetic); lanes 32..63 mirror 0..31
            const float v = s_swi[lane & 31];
            const float mx = ti_max32_nonneg(fabsf(v));
            const float scale = mx / 127.0f;
            const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
            const float pq = v * inv;
            int qi = (int)rintf(pq);
            qi = qi < -127 ? -127 : (qi > 127 ? 127 : qi);
            const uint32_t word = ti_quad_or((uint32_t)(qi & 0xff) << (8 * (lane & 3)));
            if (lane < 32 && (lane & 3) == 0) a.yq[(size_t)ch * 8 + (lane >> 2)] = word;
            if (lane == 0) a.ys[ch] = scale;
        }
        if (ch + (int)gridDim.x < nchunks) {
            __syncthreads();   // s_swi is rewritten by the next chunk
            load(ch + gridDim.x);
        }
    }
}

// Any K % 32 == 0 without a specialised shape: one wave per row, lanes stride the
// row's groups.
template <int MODE, bool GU>
__global__ __launch_bounds__(256) void k_fgemv_generic(FArgs a) {
    __shared__ __align__(16) uint32_t s_xq[FK_MAX / 4];
    __shared__ float s_xs[FK_MAX / 32];
    __shared__ float red[256];
    act_prologue<MODE>(a, s_xq, s_xs, red);
    const int lane = threadIdx.x & 63;
    const int gpr = a.K / 32;
    for (long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6); row < a.N; row += (long)gridDim.x * 4) {
        long local;
        const int s = GU ? 0 : seg_of(a, row, local);
        if (GU) local = row;
        const uint4* P = seg_pack(a, s);
        const uint16_t* S = seg_sc(a, s);
        float tg = 0.0f, tu = 0.0f;
        for (int g = lane; g < gpr; g += 64) {
            ActQ8 act;
            load_act_q8(s_xq, s_xs, g, act);
            const long gi = local * gpr + g;
            tg = fmaf((float)group_dot_q8(P[gi], act), ti_h2f(S[gi]) * act.s, tg);
            if constexpr (GU) tu = fmaf((float)group_dot_q8(a.upack[gi], act), ti_h2f(a.usc[gi]) * act.s, tu);
        }
        tg = ti_seg_sum<64>(tg);
        if constexpr (GU) tu = ti_seg_sum<64>(tu);
        if (lane == 0) {
            if (GU) {
                a.seg[0].y[row] = silu_mul(tg, tu);
            } else {
                float* y = seg_y(a, s);
                y[local] = a.acc ? y[local] + tg : tg;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// lm_head: final RMSNorm (f32, into LDS) -> f32-activation int4 GEMV (exact limb
// dots, as k_gemv_q4_f32) -> logits; each workgroup reduces its rows' argmax,
// and the last workgroup to finish (device-scope counter) reduces the partials,
// writes tok[pos+1] and advances the device position.
// ---------------------------------------------------------------------------
struct LmArgs {
    const uint4* pack;
    const uint16_t* sc;
    int N, K;
    const float* x;
    const uint16_t* nw;
    float eps;
    float* logits;
    float* part_v;         // per-workgroup argmax partials
    uint32_t* part_i;
    uint32_t* counter;     // zero between launches (the last workgroup resets it)
    uint32_t* hist;        // token history
    int* dpos;             // device position (read, then advanced); may be null
    int out_pos;           // used when dpos is null
    int cap;               // the history holds positions [0, cap]; a step at pos >= cap writes nothing
    const float* rope_tab; // [cap][rope_hd] cos/sin rows; with rope_cur, the row of the new position
    float* rope_cur;       // is copied to rope_cur (the fused attention reads it at a fixed address)
    int rope_hd;
    uint32_t* samp;        // sampling words (TI_SAMP_*) or null: temperature > 0 adds T g to every
                           // logit before the argmax, and the last workgroup advances the seed
};

// argmax over the wave (value, then the reference's tie rank), left in every lane
__device__ __forceinline__ void wave_argmax(float& v, int& i, int N) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = ti_xor(v, o);
        const int i2 = ti_xor_i(i, o);
        ti_amx_take(v, i, v2, i2, N);
    }
}

template <int LPR, int GPL, int R>
__global__ __launch_bounds__(256) void k_lmhead(LmArgs a) {
    constexpr int RPP = 64 / LPR;
    constexpr int GPR = LPR * GPL;
    // LDS sized by this instantiation's K = 32*GPR (not the largest K): every workgroup of
    // the persistent grid stays resident (a workgroup that had to wait for a slot would
    // start its full share of rows late and set the kernel's end)
    __shared__ __align__(16) float s_x[GPR * 32];
    __shared__ ActLimb s_al[GPR];
    __shared__ float red[256];
    __shared__ float bv_s[4];
    __shared__ int bi_s[4];
    __shared__ int last_s;
    constexpr int SPAN = LPR / R;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int sub = lane / LPR, li = lane % LPR;
    const long nwaves = (long)gridDim.x * 4;
    const long nblocks = ((long)a.N + RPP * R - 1) / (RPP * R);
    long b = (long)blockIdx.x * 4 + (tid >> 6);
    const bool active = b < nblocks;
    uint4 wv[2][R][GPL];
    uint16_t sw[2][R][GPL];
    auto load = [&](int buf, long blk) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            long row = blk * (RPP * R) + sub + (long)r * RPP;
            row = row < a.N ? row : a.N - 1;
#pragma unroll
            for (int j = 0; j < GPL; j++) {
                long gi = row * GPR + li + LPR * j;
                wv[buf][r][j] = ti_ld_nt(a.pack + gi);
                sw[buf][r][j] = __builtin_nontemporal_load(a.sc + gi);
            }
        }
    };
    // rmsnorm (models/qwen3.js:60-80): y = (x * inv) * w, x and w loaded once
    constexpr int EPT = (GPR * 32 + 255) / 256;
    float xr[EPT];
    uint16_t wr[EPT];
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        const int e = tid + 256 * i;
        const int ec = e < a.K ? e : a.K - 1;
        xr[i] = a.x[ec];
        wr[i] = a.nw[ec];
    }
    load(0, active ? b : 0);   // unconditional (block 0 for idle waves): no branch between the activation and weight loads
    TI_ISSUE_FENCE();
#pragma unroll
    for (int i = 0; i < EPT; i++) {
        if (tid + 256 * i >= a.K) {
            xr[i] = 0.0f;
            wr[i] = 0;
        }
    }
    {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < EPT; i++) {
            float sq = xr[i] * xr[i];
            s = s + sq;
        }
        float m = ti_tree_sum_256(s, red) / (float)a.K;
        m = m + a.eps;
        const float inv = 1.0f / sqrtf(m);
#pragma unroll
        for (int i = 0; i < EPT; i++) {
            const int e = tid + 256 * i;
            float p = xr[i] * inv;
            if (e < a.K) s_x[e] = p * ti_h2f(wr[i]);
        }
    }
    __syncthreads();
    // the exact three-limb form of each 32-group, computed once per workgroup (one thread
    // per group) and read by every lane that dots with that group
    for (int g = tid; g < GPR; g += 256) load_act_limbs(s_x, g, s_al[g]);
    __syncthreads();
    float best_v = -3.0e38f;
    int best_i = 0x7fffffff;
    float temp = 0.0f;
    uint32_t seed = 0;
    if (a.samp) {
        temp = __uint_as_float(a.samp[TI_SAMP_TEMP]);
        seed = ti_seed_next(a.samp[TI_SAMP_STATE]);
    }
    if (active) {
        ActLimb act[GPL];
#pragma unroll
        for (int j = 0; j < GPL; j++) act[j] = s_al[li + LPR * j];
        auto finish = [&](int buf, long blk) {
            float accv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                float t = 0.0f;
#pragma unroll
                for (int j = 0; j < GPL; j++) t = fmaf(group_dot_limbs(wv[buf][r][j], act[j]), ti_h2f(sw[buf][r][j]), t);
                accv[r] = t;
            }
            float tot = transpose_reduce<LPR, R>(accv, li);
            const long row = blk * (RPP * R) + sub + (long)(li / SPAN) * RPP;
            if ((li % SPAN) == 0 && row < a.N) {
                if (a.logits) a.logits[row] = tot;
                if (temp > 0.0f) {
                    const float g = temp * ti_gumbel((uint32_t)row, seed);
                    tot = tot + g;
                }
                ti_amx_take(best_v, best_i, tot, (int)row, a.N);
            }
        };
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
    // workgroup argmax (ties by the reference's rank): wave butterflies, then the 4 wave winners
    wave_argmax(best_v, best_i, a.N);
    if (lane == 0) {
        bv_s[tid >> 6] = best_v;
        bi_s[tid >> 6] = best_i;
    }
    __syncthreads();
    if (tid == 0) {
        float v = bv_s[0];
        int i = bi_s[0];
#pragma unroll
        for (int w = 1; w < 4; w++) ti_amx_take(v, i, bv_s[w], bi_s[w], a.N);
        ti_pub_store(a.part_v + blockIdx.x, v);
        ti_pub_store(a.part_i + blockIdx.x, (uint32_t)i);
        ti_stores_done();
        last_s = ti_arrive(a.counter) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last_s) return;
    float v = -3.0e38f;
    int i = 0x7fffffff;
    for (int p = tid; p < (int)gridDim.x; p += 256) ti_amx_take(v, i, ti_pub_load(a.part_v + p), (int)ti_pub_load(a.part_i + p), a.N);
    wave_argmax(v, i, a.N);
    __syncthreads();   // every thread has read last_s / the first-stage winners
    if (lane == 0) {
        bv_s[tid >> 6] = v;
        bi_s[tid >> 6] = i;
    }
    __syncthreads();
    if (tid == 0) {
        float vv = bv_s[0];
        int ii = bi_s[0];
#pragma unroll
        for (int w = 1; w < 4; w++) ti_amx_take(vv, ii, bv_s[w], bi_s[w], a.N);
        const int pos = a.dpos ? *a.dpos : a.out_pos - 1;
        last_s = -1;
        if (pos >= 0 && pos < a.cap) {
            a.hist[pos + 1] = (uint32_t)ti_amx_result(vv, ii);
            if (a.dpos) *a.dpos = pos + 1;
            if (temp > 0.0f) a.samp[TI_SAMP_STATE] = seed;   // every workgroup read the state before it arrived
            last_s = pos + 1;
        }
        __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (a.rope_cur && last_s >= 0 && last_s < a.cap && tid < a.rope_hd)
        a.rope_cur[tid] = a.rope_tab[(size_t)last_s * a.rope_hd + tid];
}

// ---- launch shapes -------------------------------------------------------------
struct Shape {
    int lpr, gpl;
};
Shape fshape(int gpr) {
    int lpr = 1;
    while (lpr < 64 && (gpr % (lpr * 2)) == 0) lpr *= 2;
    return {lpr, gpr / lpr};
}

// rows per lane in flight: enough wave-blocks to cover the chip, at most 4
int fpick_R(long N, int lpr) {
    long rpp = 64 / lpr;
    long waves1 = (N + rpp - 1) / rpp;
    int R = waves1 >= 8192 ? 4 : waves1 >= 2048 ? 2 : 1;
    while (R > lpr) R >>= 1;
    return R;
}

// persistent grid: at most 4096 waves (1024 workgroups) resident at once
unsigned fgrid(long nblocks) {
    long waves = nblocks < 4096 ? nblocks : 4096;
    return (unsigned)((waves + 3) / 4);
}

}  // namespace

// shapes with a specialisation: (lpr, gpl) for K = 32*lpr*gpl
#define FGEMV_SHAPES(X) X(32, 1) X(64, 1) X(32, 3) X(64, 3) X(64, 2) X(64, 4) X(16, 1) X(8, 1) X(4, 1) X(2, 1) X(1, 1) \
    X(16, 3) X(8, 3) X(4, 3) X(2, 3) X(1, 3)

template <int MODE, bool GU>
static int fgemv_launch(ti_ctx* c, const FArgs& a) {
    if (a.K % 32 != 0 || a.K > FK_MAX || a.K <= 0)
        return ti_fail(TI_ERR_INVALID, "fused GEMV: K=%d must be a positive multiple of 32 and <= %d", a.K, FK_MAX);
    Shape s = fshape(a.K / 32);
    int R = fpick_R(a.N, s.lpr);
    const int rb = (64 / s.lpr) * R;
    bool aligned = true;
    for (int i = 0; i + 1 < a.nseg; i++) aligned = aligned && a.seg[i].n % rb == 0;
    long nblocks = ((long)a.N + rb - 1) / rb;
    unsigned grid = fgrid(nblocks);
#define X(L, G)                                                                                        \
    if (aligned && s.lpr == L && s.gpl == G) {                                                         \
        if (R == 4) k_fgemv<L, G, (L >= 4 ? 4 : 1), MODE, GU><<<grid, 256, 0, c->stream>>>(a);         \
        else if (R == 2) k_fgemv<L, G, (L >= 2 ? 2 : 1), MODE, GU><<<grid, 256, 0, c->stream>>>(a);    \
        else k_fgemv<L, G, 1, MODE, GU><<<grid, 256, 0, c->stream>>>(a);                               \
        TI_LAUNCHED("k_fgemv");                                                                        \
        return TI_OK;                                                                                  \
    }
    FGEMV_SHAPES(X)
#undef X
    unsigned g2 = (unsigned)((a.N + 3) / 4);
    g2 = g2 < 1024 ? g2 : 1024;
    k_fgemv_generic<MODE, GU><<<g2, 256, 0, c->stream>>>(a);
    TI_LAUNCHED("k_fgemv_generic");
    return TI_OK;
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// widest activation (K) the fused kernels take: GEMVs, lm_head
int ti_fused_kmax(int lm) { return lm ? LM_KMAX : FK_MAX; }

// ---- internal entry points (the decoder and the C ABI below) -------------------
int ti_fused_qkv_launch(ti_ctx* c, const float* x, const uint16_t* nw, float eps, int K, int nmat,
                        const uint32_t* const* packs, const uint16_t* const* scs, float* const* ys, const int* Ns,
                        uint32_t* xq_out, float* xs_out) {
    FArgs a = {};
    a.nseg = nmat;
    a.N = 0;
    for (int i = 0; i < nmat; i++) {
        a.seg[i].pack = reinterpret_cast<const uint4*>(packs[i]);
        a.seg[i].sc = scs[i];
        a.seg[i].y = ys[i];
        a.seg[i].n = Ns[i];
        a.N += Ns[i];
    }
    a.K = K;
    a.x = x;
    a.nw = nw;
    a.eps = eps;
    a.xq_out = xq_out;
    a.xs_out = xs_out;
    return nw ? fgemv_launch<MODE_NORM, false>(c, a) : fgemv_launch<MODE_F32, false>(c, a);
}

int ti_fused_linear_launch(ti_ctx* c, const float* x, const uint32_t* pack, const uint16_t* sc, float* y, int N, int K,
                           int acc) {
    FArgs a = {};
    a.nseg = 1;
    a.seg[0] = {reinterpret_cast<const uint4*>(pack), sc, y, N};
    a.N = N;
    a.K = K;
    a.acc = acc;
    a.x = x;
    return fgemv_launch<MODE_F32, false>(c, a);
}

int ti_fused_gateup_launch(ti_ctx* c, const float* x, const uint16_t* nw, float eps, const uint32_t* gpack,
                           const uint16_t* gsc, const uint32_t* upack, const uint16_t* usc, float* swi, int I, int H,
                           uint32_t* swq, float* sws) {
    FArgs a = {};
    a.nseg = 1;
    a.seg[0] = {reinterpret_cast<const uint4*>(gpack), gsc, swi, I};
    a.N = I;
    a.K = H;
    a.x = x;
    a.nw = nw;
    a.eps = eps;
    a.upack = reinterpret_cast<const uint4*>(upack);
    a.usc = usc;
    a.yq = swq;
    a.ys = sws;
    if (!swq) return fgemv_launch<MODE_NORM, true>(c, a);
    if (I % 32 != 0) return ti_fail(TI_ERR_INVALID, "gate/up: I=%d must be a multiple of 32 to quantize swi", I);
    if (H % 32 != 0 || H > FK_MAX) return ti_fail(TI_ERR_INVALID, "gate/up: H=%d", H);
    Shape s = fshape(H / 32);
    const int nchunks = I / 32;
    const unsigned grid = (unsigned)(nchunks < 1024 ? nchunks : 1024);
#define X(L, G)                                                                          \
    if (s.lpr == L && s.gpl == G) {                                                      \
        k_gateup_q8out<L, G><<<grid, 256, 0, c->stream>>>(a);                            \
        TI_LAUNCHED("k_gateup_q8out");                                                   \
        return TI_OK;                                                                    \
    }
    X(64, 1) X(32, 1) X(16, 1) X(8, 1) X(64, 3) X(32, 3) X(16, 3) X(8, 3) X(64, 2)
#undef X
    return ti_fail(TI_ERR_INVALID, "gate/up: no chunked kernel for H=%d", H);
}

int ti_fused_lmhead_launch(ti_ctx* c, const float* x, const uint16_t* nw, float eps, const uint32_t* pack,
                           const uint16_t* sc, float* logits, int N, int K, uint32_t* hist, int* dpos, int out_pos,
                           int cap, const float* rope_tab, float* rope_cur, int rope_hd, uint32_t* samp) {
    if (K % 32 != 0 || K > LM_KMAX || K <= 0)
        return ti_fail(TI_ERR_INVALID, "lm_head: K=%d must be a positive multiple of 32 and <= %d", K, LM_KMAX);
    LmArgs a = {};
    a.pack = reinterpret_cast<const uint4*>(pack);
    a.sc = sc;
    a.N = N;
    a.K = K;
    a.x = x;
    a.nw = nw;
    a.eps = eps;
    a.logits = logits;
    a.part_v = c->amax_v;
    a.part_i = c->amax_i;
    a.counter = c->sync + TI_SYNC_LMHEAD;
    a.hist = hist;
    a.dpos = dpos;
    a.out_pos = out_pos;
    a.cap = cap;
    a.rope_tab = rope_tab;
    a.rope_cur = rope_cur;
    a.rope_hd = rope_hd;
    a.samp = samp;
    if (rope_cur && (!rope_tab || rope_hd <= 0 || rope_hd > 256))
        return ti_fail(TI_ERR_INVALID, "lm_head: bad rope row arguments");
    Shape s = fshape(K / 32);
    int R = fpick_R(N, s.lpr);
    long nblocks = ((long)N + (64 / s.lpr) * R - 1) / ((64 / s.lpr) * R);
    // half the GEMVs' persistent grid: every workgroup runs the norm and the limbs of the
    // whole activation and leaves one argmax partial, and at 2048 waves those cost less
    // than the streaming they leave to each wave (151936 x 1024: 26.9 -> 24.1 us per
    // launch in a chain; x 2048 unchanged)
    unsigned grid = fgrid(nblocks < 2048 ? nblocks : 2048);
    if (grid > TI_AMAX_PARTS) return ti_fail(TI_ERR_INVALID, "lm_head: %u workgroups > %d partials", grid, TI_AMAX_PARTS);
#define X(L, G)                                                                                     \
    if (s.lpr == L && s.gpl == G && G <= 3) {                                                       \
        if (R == 4) k_lmhead<L, G, (L >= 4 ? 4 : 1)><<<grid, 256, 0, c->stream>>>(a);               \
        else if (R == 2) k_lmhead<L, G, (L >= 2 ? 2 : 1)><<<grid, 256, 0, c->stream>>>(a);          \
        else k_lmhead<L, G, 1><<<grid, 256, 0, c->stream>>>(a);                                     \
        TI_LAUNCHED("k_lmhead");                                                                    \
        return TI_OK;                                                                               \
    }
    X(32, 1) X(64, 1) X(32, 3) X(64, 3) X(64, 2) X(16, 1) X(8, 1) X(4, 1) X(2, 1) X(1, 1)
#undef X
    return ti_fail(TI_ERR_INVALID, "lm_head: no kernel for K=%d", K);
}

// ---- C ABI -----------------------------------------------------------------------
extern "C" int ti_rmsnorm_gemv_q4(ti_ctx* c, const float* x, const uint16_t* norm_w, float eps, int K, int nmat,
                                  const uint32_t* const* packs, const uint16_t* const* scales, float* const* ys,
                                  const int* Ns, uint32_t* xq_out, float* xs_out) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && packs && scales && ys && Ns, "ti_rmsnorm_gemv_q4: null argument");
    TI_REQUIRE(nmat >= 1 && nmat <= 3, "ti_rmsnorm_gemv_q4: 1 to 3 matrices (got %d)", nmat);
    TI_REQUIRE(K > 0 && K % 32 == 0 && K <= FK_MAX, "ti_rmsnorm_gemv_q4: K=%d must be a multiple of 32 in (0, %d]", K, FK_MAX);
    TI_REQUIRE(al16(x), "ti_rmsnorm_gemv_q4: x must be 16-byte aligned");
    TI_REQUIRE((xq_out == nullptr) == (xs_out == nullptr), "ti_rmsnorm_gemv_q4: xq_out and xs_out go together");
    long total = 0;
    for (int i = 0; i < nmat; i++) {
        TI_REQUIRE(packs[i] && scales[i] && ys[i] && Ns[i] > 0, "ti_rmsnorm_gemv_q4: matrix %d: null buffer or N<=0", i);
        TI_REQUIRE(al16(packs[i]), "ti_rmsnorm_gemv_q4: pack %d must be 16-byte aligned", i);
        total += Ns[i];
    }
    TI_REQUIRE(total < (1L << 30), "ti_rmsnorm_gemv_q4: too many rows");
    return ti_fused_qkv_launch(c, x, norm_w, eps, K, nmat, packs, scales, ys, Ns, xq_out, xs_out);
}

extern "C" int ti_rmsnorm_gateup_silu_q4(ti_ctx* c, const float* x, const uint16_t* norm_w, float eps,
                                         const uint32_t* gpack, const uint16_t* gsc, const uint32_t* upack,
                                         const uint16_t* usc, float* swi, int I, int H, uint32_t* swi_q,
                                         float* swi_s) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && norm_w && gpack && gsc && upack && usc, "ti_rmsnorm_gateup_silu_q4: null buffer");
    TI_REQUIRE(swi || swi_q, "ti_rmsnorm_gateup_silu_q4: no output (swi and swi_q both null)");
    TI_REQUIRE((swi_q == nullptr) == (swi_s == nullptr), "ti_rmsnorm_gateup_silu_q4: swi_q and swi_s go together");
    TI_REQUIRE(swi_q || swi, "ti_rmsnorm_gateup_silu_q4: null swi");
    TI_REQUIRE(I > 0 && H > 0 && H % 32 == 0 && H <= FK_MAX, "ti_rmsnorm_gateup_silu_q4: bad shape (I=%d H=%d)", I, H);
    TI_REQUIRE(!swi_q || I % 32 == 0, "ti_rmsnorm_gateup_silu_q4: I=%d must be a multiple of 32 for swi_q", I);
    TI_REQUIRE(al16(x) && al16(gpack) && al16(upack), "ti_rmsnorm_gateup_silu_q4: x and packs must be 16-byte aligned");
    return ti_fused_gateup_launch(c, x, norm_w, eps, gpack, gsc, upack, usc, swi, I, H, swi_q, swi_s);
}

extern "C" int ti_rmsnorm_lm_head_argmax(ti_ctx* c, const float* x, const uint16_t* norm_w, float eps,
                                         const uint32_t* pack, const uint16_t* scales, float* logits, int N, int K,
                                         uint32_t* tok_hist, int out_pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && norm_w && pack && scales && tok_hist, "ti_rmsnorm_lm_head_argmax: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 32 == 0 && K <= LM_KMAX, "ti_rmsnorm_lm_head_argmax: bad shape (N=%d K=%d)", N, K);
    TI_REQUIRE(out_pos >= 1, "ti_rmsnorm_lm_head_argmax: out_pos must be >= 1");
    TI_REQUIRE(al16(x) && al16(pack), "ti_rmsnorm_lm_head_argmax: x and pack must be 16-byte aligned");
    return ti_fused_lmhead_launch(c, x, norm_w, eps, pack, scales, logits, N, K, tok_hist, nullptr, out_pos, out_pos,
                                  nullptr, nullptr, 0, nullptr);
}
