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

enum { MODE_Q8 = 0, MODE_F32 = 1, MODE_NORM = 2 };

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

// segment of a global row (rows past N are clamped by the caller)
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

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

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
    const long nwaves = (long)gridDim.x * 4;
    const long nblocks = ((long)a.N + RPP * R - 1) / (RPP * R);
    long b = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const bool active = b < nblocks;

    uint4 wv[2][R][GPL];
    uint16_t sw[2][R][GPL];
    uint4 uv[2][GU ? R : 1][GU ? GPL : 1];
    uint16_t su[2][GU ? R : 1][GU ? GPL : 1];
    float yold[2];
    auto load = [&](int buf, long blk) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            long row = blk * (RPP * R) + sub + (long)r * RPP;
            row = row < a.N ? row : a.N - 1;
            long local;
            const int s = GU ? 0 : seg_of(a, row, local);
            if (GU) local = row;
            const uint4* P = GU ? a.seg[0].pack : seg_pack(a, s);
            const uint16_t* S = GU ? a.seg[0].sc : seg_sc(a, s);
#pragma unroll
            for (int j = 0; j < GPL; j++) {
                long gi = local * GPR + li + LPR * j;
                wv[buf][r][j] = ti_ld_nt(P + gi);
                sw[buf][r][j] = __builtin_nontemporal_load(S + gi);
                if constexpr (GU) {
                    uv[buf][r][j] = ti_ld_nt(a.upack + gi);
                    su[buf][r][j] = __builtin_nontemporal_load(a.usc + gi);
                }
            }
        }
        if (!GU && a.acc) {   // residual: the row this lane will store, fetched with the weights
            long row = blk * (RPP * R) + sub + (long)(li / SPAN) * RPP;
            row = row < a.N ? row : a.N - 1;
            long local;
            const int s = seg_of(a, row, local);
            yold[buf] = seg_y(a, s)[local];
        }
    };
    if (active) load(0, b);
    act_prologue<MODE>(a, s_xq, s_xs, red);
    if (!active) return;
    ActQ8 act[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) load_act_q8(s_xq, s_xs, li + LPR * j, act[j]);

    auto finish = [&](int buf, long blk) {
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
        const long row = blk * (RPP * R) + sub + (long)(li / SPAN) * RPP;
        if ((li % SPAN) == 0 && row < a.N) {
            if (GU) {
                a.seg[0].y[row] = silu_mul(g, u);
            } else {
                long local;
                const int s = seg_of(a, row, local);
                seg_y(a, s)[local] = a.acc ? yold[buf] + g : g;
            }
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
};

__device__ __forceinline__ void amx_take(float& v, int& i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

template <int LPR, int GPL, int R>
__global__ __launch_bounds__(256) void k_lmhead(LmArgs a) {
    __shared__ __align__(16) float s_x[LM_KMAX];
    __shared__ float red[256];
    __shared__ float bv_s[256];
    __shared__ int bi_s[256];
    __shared__ int last_s;
    constexpr int RPP = 64 / LPR;
    constexpr int GPR = LPR * GPL;
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
    if (active) load(0, b);
    // rmsnorm (models/qwen3.js:60-80): y = (x * inv) * w
    const float inv = rms_inv_256(a.x, a.K, a.eps, red);
    for (int i = tid; i < a.K; i += 256) {
        float p = a.x[i] * inv;
        s_x[i] = p * ti_h2f(a.nw[i]);
    }
    __syncthreads();
    float best_v = -3.0e38f;
    int best_i = 0x7fffffff;
    if (active) {
        ActLimb act[GPL];
#pragma unroll
        for (int j = 0; j < GPL; j++) load_act_limbs(s_x, li + LPR * j, act[j]);
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
                amx_take(best_v, best_i, tot, (int)row);
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
    // workgroup argmax (lowest index wins ties)
    bv_s[tid] = best_v;
    bi_s[tid] = best_i;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) {
            float v = bv_s[tid];
            int i = bi_s[tid];
            amx_take(v, i, bv_s[tid + s], bi_s[tid + s]);
            bv_s[tid] = v;
            bi_s[tid] = i;
        }
        __syncthreads();
    }
    if (tid == 0) {
        a.part_v[blockIdx.x] = bv_s[0];
        a.part_i[blockIdx.x] = (uint32_t)bi_s[0];
        __threadfence();
        unsigned prev = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_s = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!last_s) return;
    __threadfence();
    float v = -3.0e38f;
    int i = 0x7fffffff;
    for (int p = tid; p < (int)gridDim.x; p += 256) {
        float pv = __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t*>(a.part_v) + p, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT));
        int pi = (int)__hip_atomic_load(a.part_i + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        amx_take(v, i, pv, pi);
    }
    bv_s[tid] = v;
    bi_s[tid] = i;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) {
            float vv = bv_s[tid];
            int ii = bi_s[tid];
            amx_take(vv, ii, bv_s[tid + s], bi_s[tid + s]);
            bv_s[tid] = vv;
            bi_s[tid] = ii;
        }
        __syncthreads();
    }
    if (tid == 0) {
        const int pos = a.dpos ? *a.dpos : a.out_pos - 1;
        if (pos >= 0 && pos < a.cap) {
            a.hist[pos + 1] = (uint32_t)bi_s[0];
            if (a.dpos) *a.dpos = pos + 1;
        }
        __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
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
    X(16, 3) X(8, 3) X(4, 3) X(2, 3) X(1, 3) X(64, 6) X(64, 8)

template <int MODE, bool GU>
static int fgemv_launch(ti_ctx* c, const FArgs& a) {
    if (a.K % 32 != 0 || a.K > FK_MAX || a.K <= 0)
        return ti_fail(TI_ERR_INVALID, "fused GEMV: K=%d must be a positive multiple of 32 and <= %d", a.K, FK_MAX);
    Shape s = fshape(a.K / 32);
    int R = fpick_R(a.N, s.lpr);
    long nblocks = ((long)a.N + (64 / s.lpr) * R - 1) / ((64 / s.lpr) * R);
    unsigned grid = fgrid(nblocks);
#define X(L, G)                                                                                        \
    if (s.lpr == L && s.gpl == G) {                                                                    \
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
                           const uint16_t* gsc, const uint32_t* upack, const uint16_t* usc, float* swi, int I, int H) {
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
    return fgemv_launch<MODE_NORM, true>(c, a);
}

int ti_fused_lmhead_launch(ti_ctx* c, const float* x, const uint16_t* nw, float eps, const uint32_t* pack,
                           const uint16_t* sc, float* logits, int N, int K, uint32_t* hist, int* dpos, int out_pos,
                           int cap) {
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
    Shape s = fshape(K / 32);
    int R = fpick_R(N, s.lpr);
    long nblocks = ((long)N + (64 / s.lpr) * R - 1) / ((64 / s.lpr) * R);
    unsigned grid = fgrid(nblocks);
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
                                         const uint16_t* usc, float* swi, int I, int H) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && norm_w && gpack && gsc && upack && usc && swi, "ti_rmsnorm_gateup_silu_q4: null buffer");
    TI_REQUIRE(I > 0 && H > 0 && H % 32 == 0 && H <= FK_MAX, "ti_rmsnorm_gateup_silu_q4: bad shape (I=%d H=%d)", I, H);
    TI_REQUIRE(al16(x) && al16(gpack) && al16(upack), "ti_rmsnorm_gateup_silu_q4: x and packs must be 16-byte aligned");
    return ti_fused_gateup_launch(c, x, norm_w, eps, gpack, gsc, upack, usc, swi, I, H);
}

extern "C" int ti_rmsnorm_lm_head_argmax(ti_ctx* c, const float* x, const uint16_t* norm_w, float eps,
                                         const uint32_t* pack, const uint16_t* scales, float* logits, int N, int K,
                                         uint32_t* tok_hist, int out_pos) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && norm_w && pack && scales && tok_hist, "ti_rmsnorm_lm_head_argmax: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 32 == 0 && K <= LM_KMAX, "ti_rmsnorm_lm_head_argmax: bad shape (N=%d K=%d)", N, K);
    TI_REQUIRE(out_pos >= 1, "ti_rmsnorm_lm_head_argmax: out_pos must be >= 1");
    TI_REQUIRE(al16(x) && al16(pack), "ti_rmsnorm_lm_head_argmax: x and pack must be 16-byte aligned");
    return ti_fused_lmhead_launch(c, x, norm_w, eps, pack, scales, logits, N, K, tok_hist, nullptr, out_pos, out_pos);
}
