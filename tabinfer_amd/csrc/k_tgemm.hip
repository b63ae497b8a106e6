// k_tgemm.hip — the projections of a T-token forward (2 <= T <= 16: the batch-8
// decode step, short prefills) as single launches on the matrix cores.
//
// The reference runs a T-token linear as quantQ8T + gemmDP4A (models/qwen3.js:1210-1231,
// 1326-1407), preceded by an rmsnorm dispatch (:569-612) for q/k/v and gate/up, and
// followed by a SwiGLU dispatch before the down projection. Here each projection is
// one launch:
//
//   TG_NORM   per-token RMSNorm + quantQ8T of x in every workgroup's prologue, then
//             the GEMM over up to three matrices sharing the activation (q, k, v)
//   TG_Q8     the GEMM on int8 activations another kernel produced (o_proj after the
//             attention, down_proj after gate/up), + the residual
//   gate/up   TG_NORM prologue, gate and up rows of one 32-row chunk in one workgroup,
//             silu(g)*u and its per-token quantQ8 (32 rows = one scale group) in the
//             epilogue: the down projection's int8 input, with no f32 round trip
//
// GEMM core. One v_mfma_i32_16x16x32_i8 computes the exact int32 dot of one 32-element
// scale group for 16 tokens x 16 weight rows (lane l feeds row/column l%16, K slice
// 8*(l/16)..+8; result row 4*(l/16)+i, column l%16 in lane l, element i). Operand A =
// activations (row = token), B = weights (column = weight row). Each int32 group dot is
// scaled by s_w[n,g] * s_x[t,g] into an f32 accumulator, as the reference does per group.
//
// Weights are streamed like the batch-1 GEMVs: 16-byte loads, every load of a wave in
// flight before its first use. Lane (m, j) (m = l%16, j = l/16) loads the whole 16-byte
// group g0+j of row m (the four lanes of a row read 64 contiguous bytes); the MFMA wants
// word j of ONE group in the four lanes of a row, so a 4x4 transpose across the lane
// rows (two permlane32 swaps, two permlane16 swaps: no LDS) turns the four loaded groups
// into the B operands of four MFMAs. The 8 scales of a row's 4 groups come as one 8-byte
// load. A wave owns a 16-row block and a 1/KS share of K; the KS partials of a block
// meet in LDS. Tokens past T are computed as padding and never stored.
//
// Activation codes: TG_NORM keeps them in LDS ([T][K/4 + 2] words: the 2-word pad puts
// the 16 token rows of an A-operand read on distinct banks), TG_Q8 loads the A operands
// straight from the producer's [T][K/4] buffer with the weights. Activation scales are
// staged token-minor in LDS ([g][16]): one 16-byte read gives a lane its 4 tokens.
#include "ti_dev.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

enum { TG_Q8 = 0, TG_NORM = 1 };

constexpr int TG_TMAX = 16;

struct TgSeg {
    const uint4* pack;
    const v2u* sc;       // f16 scales, 4 per 8-byte word
    float* y;            // [T][n]
    int n;
};

struct TgArgs {
    TgSeg seg[3];
    int nseg;
    int N;               // rows over all segments
    int K;
    int T;
    int acc;             // y += W x (residual)
    int S;               // LDS row stride of the activation codes, words
    const float* x;      // TG_NORM: [T][K] f32
    const uint16_t* nw;  // TG_NORM: f16 norm weight [K]
    float eps;
    const uint32_t* xq;  // TG_Q8: [T][K/4] codes
    const float* xs;     // TG_Q8: [T][K/32] scales
    const uint4* upack;  // gate/up: the up matrix (seg[0] is gate)
    const v2u* usc;
    uint32_t* yq;        // gate/up: swi codes [T][N/4]
    float* ys;           // gate/up: swi scales [T][N/32]
};

// LDS carve-up (dynamic): codes [T][S] (TG_NORM), scales [G][16], partials [4][16][17],
// norm partial sums [TP][256] (TG_NORM)
__host__ __device__ constexpr int tg_part_floats() { return 4 * 16 * 17; }
__host__ __device__ constexpr int tg_codes_words(int T, int S) { return (T * S + 3) & ~3; }   // keeps s_as 16-byte aligned

// 4x4 transpose of words across the four 16-lane rows: in, lane row j holds words 0..3
// of group j; out, b[u] in lane row j is word j of group u. permlane32_swap(a, b) gives
// {a.lo, b.lo | a.hi, b.hi} by halves, permlane16_swap(a, b) {a.r0, b.r0, a.r2, b.r2 |
// a.r1, b.r1, a.r3, b.r3} by 16-lane rows.
__device__ __forceinline__ void tr4_rows(const uint4 w, uint32_t (&b)[4]) {
    const auto p = __builtin_amdgcn_permlane32_swap(w.x, w.z, false, false);
    const auto q = __builtin_amdgcn_permlane32_swap(w.y, w.w, false, false);
    const auto r0 = __builtin_amdgcn_permlane16_swap(p[0], q[0], false, false);
    const auto r1 = __builtin_amdgcn_permlane16_swap(p[1], q[1], false, false);
    b[0] = r0[0];
    b[1] = r0[1];
    b[2] = r1[0];
    b[3] = r1[1];
}

// sum of a token's 256 per-thread partials in the reference's tree order (red holds them)
__device__ __forceinline__ float tg_tree(const float* red) {
    const int l = threadIdx.x & 63;
    const float a = red[l] + red[l + 128];
    const float b = red[l + 64] + red[l + 192];
    float v = a + b;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = v + ti_xor(v, o);
    return v;
}

// Per-token RMSNorm + quantQ8T of the T x K activation into LDS, K = 256*KU, TP tokens
// per pass. Thread t holds elements t, t+256, ... of each token for the sum of squares
// (the reference's 256 strided partials, then its 128..1 tree), and a contiguous copy,
// elements KU*t .. KU*t+KU-1, for the quantizer: a 32-group spans 32/KU neighbouring
// lanes, each thread computes its group's scale once. Codes and scales equal
// rmsnorm + q8_group's, bit for bit.
template <int KU, int TP>
__device__ __forceinline__ void tg_norm_prologue(const TgArgs& a, uint32_t* s_aq, float* s_as, float* red) {
    constexpr int K = 256 * KU;
    const int t = threadIdx.x, T = a.T, S = a.S;
    uint16_t wc[KU];
#pragma unroll
    for (int i = 0; i < KU; i++) wc[i] = a.nw[KU * t + i];
    for (int p0 = 0; p0 < T; p0 += TP) {
        float xsd[TP][KU], xc[TP][KU];
#pragma unroll
        for (int tp = 0; tp < TP; tp++) {
            const int tok = min(p0 + tp, T - 1);
            const float* xr = a.x + (size_t)tok * K;
#pragma unroll
            for (int i = 0; i < KU; i++) xsd[tp][i] = xr[t + 256 * i];
            if constexpr (KU % 4 == 0) {
                const float4* x4 = reinterpret_cast<const float4*>(xr + KU * t);
#pragma unroll
                for (int i = 0; i < KU / 4; i++) {
                    const float4 v = x4[i];
                    xc[tp][4 * i] = v.x; xc[tp][4 * i + 1] = v.y; xc[tp][4 * i + 2] = v.z; xc[tp][4 * i + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < KU; i++) xc[tp][i] = xr[KU * t + i];
            }
        }
#pragma unroll
        for (int tp = 0; tp < TP; tp++) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < KU; i++) {
                const float sq = xsd[tp][i] * xsd[tp][i];
                s = s + sq;
            }
            red[tp * 256 + t] = s;
        }
        __syncthreads();
#pragma unroll
        for (int tp = 0; tp < TP; tp++) {
            const int tok = p0 + tp;
            float m = tg_tree(red + tp * 256) / (float)K;
            m = m + a.eps;
            const float inv_rms = 1.0f / sqrtf(m);
            float v[KU];
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < KU; i++) {
                const float p = xc[tp][i] * inv_rms;
                v[i] = p * ti_h2f(wc[i]);
                mx = fmaxf(mx, fabsf(v[i]));
            }
            mx = group_max_contig<KU>(mx);
            const float scale = mx / 127.0f;
            const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
            uint32_t wd[(KU + 3) / 4] = {};
#pragma unroll
            for (int i = 0; i < KU; i++) wd[i / 4] |= (uint32_t)(q8_code(v[i], inv) & 0xff) << (8 * (i % 4));
            if (tok < T) {
                if constexpr (KU >= 4) {
#pragma unroll
                    for (int k = 0; k < KU / 4; k++) s_aq[tok * S + KU / 4 * t + k] = wd[k];
                } else {
                    uint8_t* qb = reinterpret_cast<uint8_t*>(s_aq + tok * S);
#pragma unroll
                    for (int i = 0; i < KU; i++) qb[KU * t + i] = (uint8_t)((wd[0] >> (8 * i)) & 0xff);
                }
                if (t % (32 / KU) == 0) s_as[(KU * t / 32) * 16 + tok] = scale;
            }
        }
        __syncthreads();   // codes visible; red free for the next pass
    }
}

// activation scales [T][G] -> LDS [G][16] (TG_Q8): every load issued before the stores
__device__ __forceinline__ void tg_stage_scales(const TgArgs& a, float* s_as) {
    const int G = a.K / 32, n = a.T * G, t = threadIdx.x;
    constexpr int SPT = TG_TMAX * 256 / 256;   // T * G <= 16 * 256
    float v[SPT];
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int e = t + 256 * k;
        v[k] = a.xs[e < n ? e : n - 1];
    }
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int e = t + 256 * k;
        if (e < n) s_as[(e % G) * 16 + e / G] = v[k];
    }
    __syncthreads();
}

// Segment of a 16-row block: selects on wave-uniform values (pointers stay scalar).
struct TgBlk {
    const uint4* pack;
    const v2u* sc;
    float* y;
    int base, n;
};
__device__ __forceinline__ TgBlk tg_blk(const TgArgs& a, int row0) {
    const int n0 = a.seg[0].n, n01 = n0 + a.seg[1].n;
    const bool in1 = a.nseg > 1 && row0 >= n0;
    const bool in2 = a.nseg > 2 && row0 >= n01;
    TgBlk r;
    r.pack = in2 ? a.seg[2].pack : (in1 ? a.seg[1].pack : a.seg[0].pack);
    r.sc = in2 ? a.seg[2].sc : (in1 ? a.seg[1].sc : a.seg[0].sc);
    r.y = in2 ? a.seg[2].y : (in1 ? a.seg[1].y : a.seg[0].y);
    r.base = in2 ? n01 : (in1 ? n0 : 0);
    r.n = in2 ? a.seg[2].n : (in1 ? a.seg[1].n : a.seg[0].n);
    return r;
}

// MODE: TG_NORM / TG_Q8 input. GU: gate/up epilogue (KS = 1, one 32-row chunk per
// workgroup: waves 0,1 gate rows +0/+16, waves 2,3 up rows +0/+16). KS waves share a
// 16-row block, each on NL steps of 4 groups. KU, TP: TG_NORM's prologue shape.
template <int MODE, bool GU, int KS, int NL, int KU, int TP>
__global__ __launch_bounds__(256) void k_tgemm(TgArgs a) {
    static_assert(!GU || KS == 1, "gate/up: one wave per 16-row block");
    extern __shared__ __align__(16) uint32_t s_dyn[];
    const int T = a.T, G = a.K / 32, S = a.S;
    uint32_t* s_aq = s_dyn;
    float* s_as = reinterpret_cast<float*>(s_dyn + (MODE == TG_NORM ? tg_codes_words(T, S) : 0));
    float* s_part = s_as + G * 16;
    float* red = s_part + tg_part_floats();
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m = lane & 15, j = lane >> 4;
    constexpr int BPW = 4 / KS;

    // this wave's block: rows [row0, row0+16) of one matrix, groups [gbase, gbase + 4*NL)
    const int gbase = (wave % KS) * 4 * NL;
    int row0;
    bool valid = true;
    const uint4* P;
    const v2u* SC;
    TgBlk bs;
    if constexpr (GU) {
        row0 = blockIdx.x * 32 + 16 * (wave & 1);
        P = wave < 2 ? a.seg[0].pack : a.upack;
        SC = wave < 2 ? a.seg[0].sc : a.usc;
        bs.base = 0;
        bs.n = a.N;
    } else {
        const int nb = (a.N + 15) / 16;
        int blk = blockIdx.x * BPW + wave / KS;
        valid = blk < nb;
        blk = valid ? blk : nb - 1;
        row0 = blk * 16;
        bs = tg_blk(a, row0);
        P = bs.pack;
        SC = bs.sc;
    }
    const int lrow = min(row0 - bs.base + m, bs.n - 1);
    const int tA = min(m, T - 1);                    // this lane's A-operand token

    uint4 wv[NL];
    v2u sv[NL];
    uint2 aq[MODE == TG_Q8 ? NL : 1][4];
    {
        const uint4* pr = P + (size_t)lrow * G + gbase + j;
        const v2u* sr = SC + ((size_t)lrow * G + gbase) / 4;
#pragma unroll
        for (int s = 0; s < NL; s++) {
            wv[s] = ti_ld_nt(pr + 4 * s);
            sv[s] = __builtin_nontemporal_load(sr + s);
        }
        if constexpr (MODE == TG_Q8) {
            const uint2* ar = reinterpret_cast<const uint2*>(a.xq + (size_t)tA * (a.K / 4)) + 4 * gbase + j;
#pragma unroll
            for (int s = 0; s < NL; s++)
#pragma unroll
                for (int u = 0; u < 4; u++) aq[s][u] = ar[4 * (4 * s + u)];
        }
    }
    // residual rows this thread stores (KS waves of a block: 16*T outputs over 64*KS lanes)
    constexpr int NE = GU ? 1 : (16 * TG_TMAX) / (64 * KS);
    float yold[NE];
    if constexpr (!GU) {
#pragma unroll
        for (int r = 0; r < NE; r++) {
            const int e = (wave % KS) * 64 + lane + r * 64 * KS;
            const int tok = min(e >> 4, T - 1);
            const int lr = min(row0 - bs.base + (e & 15), bs.n - 1);
            yold[r] = a.acc ? bs.y[(size_t)tok * bs.n + lr] : 0.0f;
        }
    }
    TI_ISSUE_FENCE();

    if constexpr (MODE == TG_NORM) tg_norm_prologue<KU, TP>(a, s_aq, s_as, red);
    else tg_stage_scales(a, s_as);

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < NL; s++) {
        uint32_t bw[4];
        tr4_rows(wv[s], bw);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int g = gbase + 4 * s + u;
            uint2 av;
            if constexpr (MODE == TG_Q8) av = aq[s][u];
            else av = *reinterpret_cast<const uint2*>(s_aq + tA * S + 8 * g + 2 * j);
            const uint32_t alo = even_bytes(av.x, av.y), ahi = odd_bytes(av.x, av.y);
            uint32_t blo, bhi;
            nib_to_s8(bw[u], blo, bhi);
            const long A = (long)(((uint64_t)ahi << 32) | alo);
            const long B = (long)(((uint64_t)bhi << 32) | blo);
            const v4i z = {0, 0, 0, 0};
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, z, 0, 0, 0);
            const float4 sx = *reinterpret_cast<const float4*>(s_as + g * 16 + 4 * j);
            const uint32_t sp = (u & 2) ? sv[s].y : sv[s].x;
            const float sw = ti_h2f((uint16_t)((u & 1) ? (sp >> 16) : (sp & 0xffff)));
            acc[0] = fmaf((float)d[0], sw * sx.x, acc[0]);
            acc[1] = fmaf((float)d[1], sw * sx.y, acc[1]);
            acc[2] = fmaf((float)d[2], sw * sx.z, acc[2]);
            acc[3] = fmaf((float)d[3], sw * sx.w, acc[3]);
        }
    }
    // partials: lane (m, j) holds tokens 4j..4j+3 of row m of the wave's block
#pragma unroll
    for (int i = 0; i < 4; i++) s_part[(wave * 16 + 4 * j + i) * 17 + m] = acc[i];
    __syncthreads();

    if constexpr (GU) {
        // silu(g)*u of (token, chunk row) and its quantQ8 over the chunk's 32 rows
        // (q8_group's arithmetic: scale = absmax/127, round-half-even, clamp 127)
        const int r = tid & 31;
        const int ch = blockIdx.x;
        for (int tok = tid >> 5; tok < T; tok += 8) {
            const float gv = s_part[((r >> 4) * 16 + tok) * 17 + (r & 15)];
            const float uv = s_part[((2 + (r >> 4)) * 16 + tok) * 17 + (r & 15)];
            const float v = silu_mul(gv, uv);
            const float mx = ti_max32_nonneg(fabsf(v));
            const float scale = mx / 127.0f;
            const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
            const int qi = q8_code(v, inv);
            const uint32_t word = ti_quad_or((uint32_t)(qi & 0xff) << (8 * (r & 3)));
            if ((r & 3) == 0) a.yq[(size_t)tok * (a.N / 4) + ch * 8 + (r >> 2)] = word;
            if (r == 0) a.ys[(size_t)tok * (a.N / 32) + ch] = scale;
        }
    } else {
        if (!valid) return;
        const int w0 = (wave / KS) * KS;
#pragma unroll
        for (int r = 0; r < NE; r++) {
            const int e = (wave % KS) * 64 + lane + r * 64 * KS;
            const int tok = e >> 4, mm = e & 15;
            const int lr = row0 - bs.base + mm;
            if (tok < T && lr < bs.n) {
                float v = 0.0f;
#pragma unroll
                for (int k = 0; k < KS; k++) v += s_part[((w0 + k) * 16 + tok) * 17 + mm];
                bs.y[(size_t)tok * bs.n + lr] = a.acc ? yold[r] + v : v;
            }
        }
    }
}

// ---- host dispatch ------------------------------------------------------------------
// (KS, NL) per K: NL = K/32 / (4*KS) steps of 4 groups per wave
bool tg_split(int G, int& KS, int& NL) {
    switch (G) {
        case 8: KS = 1; NL = 2; return true;
        case 16: KS = 1; NL = 4; return true;
        case 32: KS = 2; NL = 4; return true;
        case 64: KS = 2; NL = 8; return true;
        case 96: KS = 4; NL = 6; return true;
        case 128: KS = 4; NL = 8; return true;
        case 192: KS = 4; NL = 12; return true;
        case 256: KS = 4; NL = 16; return true;
        default: return false;
    }
}

int tg_ku(int K) {   // TG_NORM prologue: K = 256*KU, KU in {1, 2, 4, 8, 16}
    if (K % 256) return 0;
    const int ku = K / 256;
    return (ku == 1 || ku == 2 || ku == 4 || ku == 8 || ku == 16) ? ku : 0;
}

constexpr int tg_tp(int ku) { return ku >= 16 ? 4 : 8; }

size_t tg_lds(int mode, int T, int K, int ku) {
    const int G = K / 32;
    size_t w = (size_t)G * 16 + tg_part_floats();
    if (mode == TG_NORM) w += (size_t)tg_codes_words(T, K / 4 + 2) + (size_t)tg_tp(ku) * 256;
    return w * 4;
}

template <int MODE, bool GU, int KS, int NL, int KU>
int tg_go(ti_ctx* c, const TgArgs& a, unsigned grid, size_t lds, const char* name) {
    static bool attr = false;
    if (!attr && lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_tgemm<MODE, GU, KS, NL, KU, tg_tp(KU)>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return ti_hip_fail(e, "k_tgemm LDS attribute");
        attr = true;
    }
    k_tgemm<MODE, GU, KS, NL, KU, tg_tp(KU)><<<grid, 256, lds, c->stream>>>(a);
    TI_LAUNCHED(name);
    return TI_OK;
}

}  // namespace

// Which T-token projections take the fused path: 2..16 tokens, K/32 in the split
// table, and (TG_NORM) K = 256 * {1,2,4,8,16}.
bool ti_tgemm_ok(int T, int K, int norm, int gateup) {
    int KS, NL;
    if (T < 2 || T > TG_TMAX || K % 32 || !tg_split(K / 32, KS, NL)) return false;
    if (norm && !tg_ku(K)) return false;
    return !gateup || K / 128 <= 16;                // gate/up runs KS = 1: NL = K/128 <= 16
}

// q/k/v-style: y_s[t][:] = W_s rmsnorm(x[t]) for up to three segments sharing the
// activation (TG_NORM), or y[t][:] (+)= W xq[t] on int8 input (TG_Q8, one segment).
int ti_tgemm_launch(ti_ctx* c, int norm, const float* x, const uint16_t* nw, float eps, const uint32_t* xq,
                    const float* xs, int nseg, const uint32_t* const* packs, const uint16_t* const* scs,
                    float* const* ys, const int* Ns, int T, int K, int acc) {
    TgArgs a = {};
    a.nseg = nseg;
    a.N = 0;
    for (int s = 0; s < nseg; s++) {
        a.seg[s] = {reinterpret_cast<const uint4*>(packs[s]), reinterpret_cast<const v2u*>(scs[s]), ys[s], Ns[s]};
        if (s + 1 < nseg && Ns[s] % 16) return ti_fail(TI_ERR_INVALID, "T-token GEMM: segment rows must be multiples of 16");
        if (reinterpret_cast<uintptr_t>(scs[s]) % 8) return ti_fail(TI_ERR_INVALID, "T-token GEMM: scales must be 8-byte aligned");
        a.N += Ns[s];
    }
    a.K = K;
    a.T = T;
    a.acc = acc;
    a.S = K / 4 + 2;
    a.x = x;
    a.nw = nw;
    a.eps = eps;
    a.xq = xq;
    a.xs = xs;
    int KS, NL;
    if (!ti_tgemm_ok(T, K, norm, 0)) return ti_fail(TI_ERR_INVALID, "T-token GEMM: unsupported T=%d K=%d", T, K);
    tg_split(K / 32, KS, NL);
    const int ku = norm ? tg_ku(K) : 0;
    const unsigned grid = (unsigned)(((a.N + 15) / 16 + 4 / KS - 1) / (4 / KS));
    const size_t lds = tg_lds(norm ? TG_NORM : TG_Q8, T, K, ku);
    if (norm) {
        switch (ku) {
            case 1: return tg_go<TG_NORM, false, 1, 2, 1>(c, a, grid, lds, "k_tgemm_norm");
            case 2: return tg_go<TG_NORM, false, 1, 4, 2>(c, a, grid, lds, "k_tgemm_norm");
            case 4: return tg_go<TG_NORM, false, 2, 4, 4>(c, a, grid, lds, "k_tgemm_norm");
            case 8: return tg_go<TG_NORM, false, 2, 8, 8>(c, a, grid, lds, "k_tgemm_norm");
            case 16: return tg_go<TG_NORM, false, 4, 8, 16>(c, a, grid, lds, "k_tgemm_norm");
        }
    } else {
        switch (K / 32) {
#define TGQ(G_, KS_, NL_) case G_: return tg_go<TG_Q8, false, KS_, NL_, 0>(c, a, grid, lds, "k_tgemm_q8");
            TGQ(8, 1, 2) TGQ(16, 1, 4) TGQ(32, 2, 4) TGQ(64, 2, 8) TGQ(96, 4, 6) TGQ(128, 4, 8) TGQ(192, 4, 12)
            TGQ(256, 4, 16)
#undef TGQ
        }
    }
    return ti_fail(TI_ERR_INVALID, "T-token GEMM: no kernel for K=%d", K);
}

// gate/up: swq[t] = quantQ8(silu(Wg rmsnorm(x[t])) * (Wu rmsnorm(x[t]))), scales sws[t]
int ti_tgemm_gateup_launch(ti_ctx* c, const float* x, const uint16_t* nw, float eps, const uint32_t* gpack,
                           const uint16_t* gsc, const uint32_t* upack, const uint16_t* usc, int I, int H, int T,
                           uint32_t* swq, float* sws) {
    if (!ti_tgemm_ok(T, H, 1, 1) || I % 32) return ti_fail(TI_ERR_INVALID, "T-token gate/up: unsupported T=%d H=%d I=%d", T, H, I);
    if (reinterpret_cast<uintptr_t>(gsc) % 8 || reinterpret_cast<uintptr_t>(usc) % 8)
        return ti_fail(TI_ERR_INVALID, "T-token gate/up: scales must be 8-byte aligned");
    TgArgs a = {};
    a.seg[0] = {reinterpret_cast<const uint4*>(gpack), reinterpret_cast<const v2u*>(gsc), nullptr, I};
    a.nseg = 1;
    a.N = I;
    a.K = H;
    a.T = T;
    a.S = H / 4 + 2;
    a.x = x;
    a.nw = nw;
    a.eps = eps;
    a.upack = reinterpret_cast<const uint4*>(upack);
    a.usc = reinterpret_cast<const v2u*>(usc);
    a.yq = swq;
    a.ys = sws;
    const int ku = tg_ku(H);
    const size_t lds = tg_lds(TG_NORM, T, H, ku);
    const unsigned grid = (unsigned)(I / 32);
    switch (ku) {
        case 1: return tg_go<TG_NORM, true, 1, 2, 1>(c, a, grid, lds, "k_tgemm_gateup");
        case 2: return tg_go<TG_NORM, true, 1, 4, 2>(c, a, grid, lds, "k_tgemm_gateup");
        case 4: return tg_go<TG_NORM, true, 1, 8, 4>(c, a, grid, lds, "k_tgemm_gateup");
        case 8: return tg_go<TG_NORM, true, 1, 16, 8>(c, a, grid, lds, "k_tgemm_gateup");
    }
    return ti_fail(TI_ERR_INVALID, "T-token gate/up: no kernel for H=%d", H);
}
