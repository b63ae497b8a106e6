// k_tgemm.hip — the projections of a T-token forward (2 <= T <= 16: the batch-8
// decode step, short prefills) on the matrix cores.
//
// The reference runs a T-token linear as quantQ8T + gemmDP4A (models/qwen3.js:1210-1231,
// 1326-1407), after an rmsnorm dispatch (:569-612) for q/k/v and gate/up and a SwiGLU
// dispatch before the down projection. Here:
//
//   k_tnorm_q8  per-token RMSNorm + quantQ8T, one workgroup per token (shared by the
//               q/k/v and gate/up projections of a layer; T > 4)
//   k_tgemm     the GEMM on int8 activations (the norm codes, the attention output's,
//               SwiGLU's) over up to three matrices sharing them (q, k, v), with the
//               residual (o_proj, down_proj; K = 6144 as two K halves per block), or
//   gate/up     gate and up rows of one 32-row chunk in one workgroup, silu(g)*u and
//               its per-token quantQ8 (32 rows = one scale group) in the epilogue: the
//               down projection's int8 input, with no f32 round trip.
//   For T <= 4 the residual projections also write the RMSNorm's per-token partial sums
//   (TG_NORM / PART below) and q/k/v and gate/up normalise and quantise x in their
//   prologue from them: every workgroup then quantises all T x K elements, which costs
//   less than the norm launch up to T = 4 and more beyond.
//
// (A first variant computed the sum of squares in every GEMM prologue as well: at T = 8
// each workgroup read the whole T x K f32 activation twice, 24-32 MB of L2 reads per
// projection, and the q/k/v and gate/up kernels took 11 and 16 us against 4.8 + 4.5 and
// 9.8 + 4.5 us for norm kernel + int8 GEMM.)
//
// GEMM core. One v_mfma_i32_16x16x32_i8 computes the exact int32 dot of one 32-element
// scale group for 16 tokens x 16 weight rows (lane l feeds row/column l%16, K slice
// 8*(l/16)..+8; result row 4*(l/16)+i, column l%16 in lane l, element i). Operand A =
// activations (row = token), B = weights (column = weight row). Each int32 group dot is
// scaled by s_w[n,g] * s_x[t,g] into an f32 accumulator, as the reference does per group.
//
// The VALU work per group is what bounds the group loop (a wave64 VALU op takes 4
// cycles; the MFMA is cheap), so everything that can be done once per workgroup is
// taken out of it:
//   - the weight nibbles go into B unsigned (nibble = w + 8, two ANDs and a shift), and
//     the MFMA's accumulator input carries -8 * sum(a) of the group, so the int32 result
//     is the signed dot exactly;
//   - the activation codes are staged in LDS already in B's byte order (per 8-byte K
//     slice: even elements, then odd elements), with the -8*sum(a) terms and the scales
//     token-minor ([g][16]: one 16-byte read gives a lane its 4 tokens).
//
// Weights are streamed like the batch-1 GEMVs: 16-byte loads, all of a wave's loads in
// flight before the first use, issued after the activation loads so that the prologue
// waits for its own data only. Lane (m, j) (m = l%16, j = l/16) loads the whole 16-byte
// group g0+j of row m (a row's four lanes read 64 contiguous bytes); the MFMA wants word
// j of ONE group in a row's four lanes, so a 4x4 transpose across the lane rows (two
// permlane32 swaps, two permlane16 swaps: no LDS) turns four loaded groups into the B
// operands of four MFMAs. A wave owns a 16-row block and a 1/KS share of K; the KS
// partials of a block meet in LDS. Tokens past T are computed as padding, never stored.
#include "ti_dev.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int TG_TMAX = 16;
enum { TG_Q8 = 0, TG_NORM = 1 };

struct TgSeg {
    const uint4* pack;
    const uint4* sc;     // f16 scales, 8 per 16-byte word
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
    int S;               // LDS row stride of the activation codes, words (K/4 + 2)
    const uint32_t* xq;  // [T][K/4] codes
    const float* xs;     // [T][K/32] scales
    const uint4* upack;  // gate/up: the up matrix (seg[0] is gate)
    const uint4* usc;
    uint32_t* yq;        // gate/up: swi codes [T][N/4]
    float* ys;           // gate/up: swi scales [T][N/32]
    // TG_NORM input: the f32 activation, its norm weight and its RMSNorm partial sums
    // ([T][256]: partial t = sum over i of x[t + 256 i]^2, the reference's order)
    const float* x;
    const uint16_t* nw;
    float eps;
    const float* pin;
    // PART epilogue: the output's partial sums ([T][256]) for the next projection's norm;
    // block b owns output rows t + 256 i for 16/pku consecutive t and every i < pku
    float* pout;
    int pku;
    // split-K (SPLIT): K above is one half; kld = the rows' full K (activation and weight
    // row strides). Workgroup 2b + h computes half h of block b, publishes it to sp, and
    // the second of the pair to arrive (counter scnt[b]) adds the halves in order 0, 1
    int kld;
    float* sp;
    uint32_t* scnt;
};

// LDS (dynamic), in words: codes [T][S] (rounded to 4), scales [G][16] f32, -8*sum(a)
// [G][16] i32, partials [W][16][17] f32, per-token 1/rms [16], the residual outputs of the
// workgroup's xnblk = W/KS blocks [xnblk][16][16] (PART; else xnblk = 0)
__host__ __device__ constexpr int tg_codes_words(int T, int S) { return (T * S + 3) & ~3; }
__host__ __device__ constexpr int tg_lds_words(int T, int K, int W, int xnblk) {
    return tg_codes_words(T, K / 4 + 2) + 2 * (K / 32) * 16 + W * 16 * 17 + 16 + xnblk * 256;
}

struct TgLds {
    uint32_t* aq;
    float* as;
    int* corr;
    float* part;
    float* inv;
    float* xn;
};
__device__ __forceinline__ TgLds tg_carve(uint32_t* base, int T, int K, int W) {
    const int G = K / 32;
    TgLds L;
    L.aq = base;
    L.as = reinterpret_cast<float*>(base + tg_codes_words(T, K / 4 + 2));
    L.corr = reinterpret_cast<int*>(L.as + G * 16);
    L.part = reinterpret_cast<float*>(L.corr + G * 16);
    L.inv = L.part + W * 16 * 17;
    L.xn = L.inv + 16;
    return L;
}

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

__device__ __forceinline__ int byte_sum(uint32_t w, int acc) {
    return __builtin_amdgcn_sdot4((int)w, 0x01010101, acc, false);
}

// ---- prologue ------------------------------------------------------------------------
// The producer's [T][K/4] codes and [T][K/32] scales, staged into LDS in B's byte
// order: 16-byte units (two K slices, half a group) per thread, the two halves of a
// group in neighbouring lanes (they add their sums by DPP). UQ, SQ: loads per thread.
template <int UQ, int SQ>
struct Q8Regs {
    uint4 c[UQ];
    float s[SQ];
};

template <int UQ, int SQ, bool SLICE>
__device__ __forceinline__ void tg_q8_load(const TgArgs& a, Q8Regs<UQ, SQ>& r, int nthreads, int part) {
    const int upr = a.K / 16, G = a.K / 32;
    const int units = a.T * upr, ns = a.T * G;
    const uint4* src = reinterpret_cast<const uint4*>(a.xq);
    // UQ / SQ cover 16 tokens; rounds wholly past T are skipped (a workgroup-uniform
    // test, so no load is issued for them), the partial one reads clamped indices.
    // SLICE: the K slice `part` of rows kld wide
#pragma unroll
    for (int k = 0; k < UQ; k++) {
        int u = threadIdx.x + nthreads * k;
        u = u < units ? u : units - 1;
        if (SLICE) u = (u / upr) * (a.kld / 16) + part * upr + u % upr;
        if (nthreads * k < units) r.c[k] = src[u];
    }
#pragma unroll
    for (int k = 0; k < SQ; k++) {
        int e = threadIdx.x + nthreads * k;
        e = e < ns ? e : ns - 1;
        if (SLICE) e = (e / G) * (a.kld / 32) + part * G + e % G;
        if (nthreads * k < ns) r.s[k] = a.xs[e];
    }
}

template <int UQ, int SQ>
__device__ __forceinline__ void tg_q8_stage(const TgArgs& a, const Q8Regs<UQ, SQ>& r, const TgLds& L, int nthreads) {
    const int G = a.K / 32, upr = a.K / 16, units = a.T * upr, ns = a.T * G, S = a.S;
#pragma unroll
    for (int k = 0; k < UQ; k++) {
        if (nthreads * k >= units) break;                 // workgroup-uniform
        const int u = threadIdx.x + nthreads * k;
        const int t = u / upr, c = u % upr, g = c >> 1, h = c & 1;
        const uint4 w = r.c[k];
        int sum = byte_sum(w.w, byte_sum(w.z, byte_sum(w.y, byte_sum(w.x, 0))));
        sum += ti_xor(sum, 1);                       // the other half of the group (u ^ 1)
        if (u < units) {
            uint2* p = reinterpret_cast<uint2*>(L.aq + t * S + 8 * g + 4 * h);
            p[0] = make_uint2(even_bytes(w.x, w.y), odd_bytes(w.x, w.y));
            p[1] = make_uint2(even_bytes(w.z, w.w), odd_bytes(w.z, w.w));
            if (h == 0) L.corr[g * 16 + t] = -8 * sum;
        }
    }
#pragma unroll
    for (int k = 0; k < SQ; k++) {
        const int e = threadIdx.x + nthreads * k;
        if (nthreads * k < ns && e < ns) L.as[(e % G) * 16 + e / G] = r.s[k];
    }
    __syncthreads();
}

// ---- RMSNorm prologue (TG_NORM) ---------------------------------------------------
// The f32 activation x [T][K] (K = 256*KU) with its partial sums from the producing
// projection's epilogue. Each wave: the 1/rms of tokens wave, wave + W, ... from the 256
// partials (the reference's 128..1 tree, as ti_tree_sum_256 adds them), then the quantQ8T
// codes of its own K/W slice of every token (8 consecutive elements per lane, a 32-group
// = 4 lanes), in B's byte order with scales and -8*sum(a): the same codes as rmsnorm +
// q8_group. RX = rounds of 64/(K/(8W)) tokens a lane covers.
template <int RX>
struct NormRegs {
    float4 x[RX][2];
    uint4 w;
    float pt[(TG_TMAX + 3) / 4][4];
};

// Issue order: partial sums (needed first), norm weight, activation; rounds past T are not
// issued (workgroup-uniform tests: a later unconditional load still lets the compiler
// wait for these by count).
template <int RX>
__device__ __forceinline__ void tg_norm_load(const TgArgs& a, NormRegs<RX>& r, int W) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, K = a.K, T = a.T;
    const int lpt = K / (8 * W), tpr = 64 / lpt;
    const int e0 = wave * (K / W) + 8 * (lane % lpt);
#pragma unroll
    for (int k = 0; k < (TG_TMAX + 3) / 4; k++) {
        const int tok = min(wave + W * k, T - 1);
        if (W * k < T) {
#pragma unroll
            for (int i = 0; i < 4; i++) r.pt[k][i] = a.pin[(size_t)tok * 256 + lane + 64 * i];
        }
    }
    r.w = *reinterpret_cast<const uint4*>(a.nw + e0);
#pragma unroll
    for (int q = 0; q < RX; q++) {
        if (q * tpr < T) {
            const int tok = min(q * tpr + lane / lpt, T - 1);
            const float4* xp = reinterpret_cast<const float4*>(a.x + (size_t)tok * K + e0);
            r.x[q][0] = xp[0];
            r.x[q][1] = xp[1];
        }
    }
}

template <int RX>
__device__ __forceinline__ void tg_norm_stage(const TgArgs& a, const NormRegs<RX>& r, const TgLds& L, int W) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, K = a.K, T = a.T, S = a.S;
#pragma unroll
    for (int k = 0; k < (TG_TMAX + 3) / 4; k++) {
        const int tok = wave + W * k;
        if (W * k < T) {
            const float x0 = r.pt[k][0] + r.pt[k][2];    // partials l + l+128
            const float x1 = r.pt[k][1] + r.pt[k][3];    // partials l+64 + l+192
            float v = x0 + x1;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v = v + ti_xor(v, o);
            float mm = v / (float)K;
            mm = mm + a.eps;
            if (lane == 0 && tok < T) L.inv[tok] = 1.0f / sqrtf(mm);
        }
    }
    __syncthreads();
    const int lpt = K / (8 * W), tpr = 64 / lpt;
    const int e0 = wave * (K / W) + 8 * (lane % lpt);
    const uint32_t ww[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
#pragma unroll
    for (int q = 0; q < RX; q++) {
        const int tok = q * tpr + lane / lpt;
        if (q * tpr >= T) break;                         // wave-uniform
        const float inv_rms = L.inv[tok < T ? tok : 0];
        const float xv[8] = {r.x[q][0].x, r.x[q][0].y, r.x[q][0].z, r.x[q][0].w,
                             r.x[q][1].x, r.x[q][1].y, r.x[q][1].z, r.x[q][1].w};
        float v[8], mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float pp = xv[i] * inv_rms;
            v[i] = pp * ti_h2f((uint16_t)((ww[i / 2] >> (16 * (i & 1))) & 0xffff));
            mx = fmaxf(mx, fabsf(v[i]));
        }
        mx = group_max_contig<8>(mx);
        const float scale = mx / 127.0f;
        const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        int qc[8];
#pragma unroll
        for (int i = 0; i < 8; i++) qc[i] = q8_code(v[i], inv);
        uint32_t e = 0, o = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            e |= (uint32_t)(qc[2 * i] & 0xff) << (8 * i);
            o |= (uint32_t)(qc[2 * i + 1] & 0xff) << (8 * i);
        }
        int sum = byte_sum(o, byte_sum(e, 0));
        sum += ti_xor(sum, 1);
        sum += ti_xor(sum, 2);
        if (tok < T) {
            *reinterpret_cast<uint2*>(L.aq + tok * S + e0 / 4) = make_uint2(e, o);
            if ((lane & 3) == 0) {
                L.as[(e0 / 32) * 16 + tok] = scale;
                L.corr[(e0 / 32) * 16 + tok] = -8 * sum;
            }
        }
    }
    __syncthreads();
}

// rounds of the norm prologue for 16 tokens: a round covers 64 / (K / (8W)) tokens, so
// 16 tokens take K / (32 W) rounds (K = 128 KS NL), at least one
constexpr int tg_rx(int W, int KS, int NL) {
    return (4 * KS * NL + W - 1) / W > 0 ? (4 * KS * NL + W - 1) / W : 1;
}

// Segment of a 16-row block: selects on wave-uniform values (pointers stay scalar).
struct TgBlk {
    const uint4* pack;
    const uint4* sc;
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

constexpr int tg_uq(int W, int KS, int NL) { return 2 * NL * KS / W > 0 ? 2 * NL * KS / W : 1; }
constexpr int tg_sq(int W, int KS, int NL) { return (NL * KS + W - 1) / W; }

// W waves per workgroup, KS waves per 16-row block, each on NL steps of 4 groups
// (K = 128*KS*NL). GU: gate/up epilogue (four blocks per workgroup: gate rows +0/+16 of
// the workgroup's 32-row chunk, then up rows +0/+16). IN: TG_Q8 codes or TG_NORM
// (RMSNorm + quantQ8T in the prologue). PART: residual epilogue that also writes the
// output's RMSNorm partial sums (block b owns rows t + 256 i).
template <bool GU, int W, int KS, int NL, int IN, bool PART, bool SPLIT = false, bool DUAL = false>
__global__ __launch_bounds__(64 * W) void k_tgemm(TgArgs a) {
    static_assert(!GU || W / KS == 4, "gate/up: four 16-row blocks per workgroup");
    static_assert(!(GU && PART), "the partial sums come from residual projections");
    static_assert(!SPLIT || (!GU && !PART && IN == TG_Q8 && W == KS), "split-K: one residual block per workgroup");
    static_assert(NL % 2 == 0, "scales are loaded 8 groups at a time");
    extern __shared__ __align__(16) uint32_t s_dyn[];
    const int T = a.T, G = a.K / 32, S = a.S;
    const TgLds L = tg_carve(s_dyn, T, a.K, W);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m = lane & 15, j = lane >> 4;
    constexpr int BPW = W / KS;
    const int part = SPLIT ? blockIdx.x & 1 : 0;         // split-K half
    const int bidx = SPLIT ? blockIdx.x >> 1 : blockIdx.x;
    const int Gld = SPLIT ? a.kld / 32 : G, goff = part * G;   // weight row stride, this half's groups

    // this wave's block: rows [row0, row0+16) of one matrix, groups [gbase, gbase + 4*NL)
    const int gbase = (wave % KS) * 4 * NL;
    int row0;
    bool valid = true;
    const uint4* P;
    const uint4* SC;
    TgBlk bs;
    if constexpr (GU) {   // blocks 0, 1: gate rows +0/+16 of the chunk; 2, 3: up rows
        const int b = wave / KS;
        row0 = blockIdx.x * 32 + 16 * (b & 1);
        P = b < 2 ? a.seg[0].pack : a.upack;
        SC = b < 2 ? a.seg[0].sc : a.usc;
        bs.base = 0;
        bs.n = a.N;
    } else {
        const int nb = (a.N + 15) / 16;
        int blk = bidx * BPW + wave / KS;
        valid = blk < nb;
        blk = valid ? blk : nb - 1;
        row0 = blk * 16;
        bs = tg_blk(a, row0);
        P = bs.pack;
        SC = bs.sc;
    }
    // PART: block b's row for lane m is t + 256 i, t = b*(16/pku) + m % (16/pku), i = m / (16/pku)
    const int tpb = PART ? 16 / a.pku : 16;
    auto out_row = [&](int mm) {
        return PART ? (row0 / 16) * tpb + mm % tpb + 256 * (mm / tpb) : min(row0 - bs.base + mm, bs.n - 1);
    };
    const int lrow = out_row(m);
    const int tA = min(m, T - 1);                    // this lane's A-operand token

    // 1. activation loads first: the prologue then waits for these only
    Q8Regs<IN == TG_Q8 ? tg_uq(W, KS, NL) : 1, IN == TG_Q8 ? tg_sq(W, KS, NL) : 1> qr;
    NormRegs<IN == TG_NORM ? tg_rx(W, KS, NL) : 1> nr;
    if constexpr (IN == TG_Q8) tg_q8_load<tg_uq(W, KS, NL), tg_sq(W, KS, NL), SPLIT>(a, qr, 64 * W, part);
    else tg_norm_load(a, nr, W);
    // 2. the weights and scales of every step
    uint4 wv[NL], sv[NL / 2];
    {
        const uint4* pr = P + (size_t)lrow * Gld + goff + gbase + j;
        const uint4* sr = SC + ((size_t)lrow * Gld + goff + gbase) / 8;
#pragma unroll
        for (int s = 0; s < NL; s++) {
            wv[s] = ti_ld_nt(pr + 4 * s);
            if (s % 2 == 0) sv[s / 2] = ti_ld_nt(sr + s / 2);
        }
    }
    // residual rows this thread stores (KS waves of a block: 16*T outputs over 64*KS lanes)
    constexpr int NE = GU ? 1 : (16 * TG_TMAX + 64 * KS - 1) / (64 * KS);
    float yold[NE];
    if constexpr (!GU) {
#pragma unroll
        for (int r = 0; r < NE; r++) {
            const int e = (wave % KS) * 64 + lane + r * 64 * KS;
            const int tok = min(e >> 4, T - 1);
            const int lr = out_row(e & 15);
            yold[r] = a.acc ? bs.y[(size_t)tok * bs.n + lr] : 0.0f;
        }
    }
    TI_ISSUE_FENCE();

    // 3. prologue: codes in B's byte order, scales, -8*sum(a) into LDS
    if constexpr (IN == TG_Q8) tg_q8_stage(a, qr, L, 64 * W);
    else tg_norm_stage(a, nr, L, W);

    // 4. the group loop
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (DUAL) {
        // T <= 8: one v_mfma_i32_16x16x64_i8 per pair of groups (2p', 2p'+1). Bytes 0-7 of
        // every lane's A and B operands carry the even group's K slice j, bytes 8-15 the odd
        // group's (A and B share their (lane row, byte) -> k pairing, so C sums over both);
        // A rows 0-7 are the tokens of the even group with the odd half zero, rows 8-15 the
        // same tokens of the odd group with the even half zero. Lane (m, j) then holds tokens
        // 4(j&1)..+3 of row m for group 2p' + (j>>1): half the scaling work of one MFMA per
        // group, with no padding rows.
        const int hiA = m >> 3, jh = j >> 1, jt = 4 * (j & 1);
        const uint32_t* arow = L.aq + min(m & 7, T - 1) * S + 8 * hiA + 2 * j;
#pragma unroll
        for (int s = 0; s < NL; s++) {
            uint32_t bw[4];
            tr4_rows(wv[s], bw);
            const uint4 sc4 = sv[s / 2];
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                const int g = gbase + 4 * s + 2 * pp;      // the pair's even group
                const uint2 av = *reinterpret_cast<const uint2*>(arow + 8 * g);
                const v4i cv = *reinterpret_cast<const v4i*>(L.corr + (g + jh) * 16 + jt);
                const float4 sx = *reinterpret_cast<const float4*>(L.as + (g + jh) * 16 + jt);
                const v4i A = hiA ? v4i{0, 0, (int)av.x, (int)av.y} : v4i{(int)av.x, (int)av.y, 0, 0};
                const uint32_t w0 = bw[2 * pp], w1 = bw[2 * pp + 1];
                const v4i B = {(int)(w0 & 0x0F0F0F0Fu), (int)((w0 >> 4) & 0x0F0F0F0Fu), (int)(w1 & 0x0F0F0F0Fu),
                               (int)((w1 >> 4) & 0x0F0F0F0Fu)};
                const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, cv, 0, 0, 0);
                const int h = 4 * (s & 1) + 2 * pp;        // the pair's scales: halves of word h/2 of sc4
                const uint32_t sp = h < 2 ? sc4.x : (h < 4 ? sc4.y : (h < 6 ? sc4.z : sc4.w));
                const float sw = ti_h2f((uint16_t)(sp >> (16 * jh)));
                acc[0] = fmaf((float)d[0], sw * sx.x, acc[0]);
                acc[1] = fmaf((float)d[1], sw * sx.y, acc[1]);
                acc[2] = fmaf((float)d[2], sw * sx.z, acc[2]);
                acc[3] = fmaf((float)d[3], sw * sx.w, acc[3]);
            }
        }
        // lanes j and j ^ 2 hold the same (row, tokens) over the even and odd groups
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = acc[i] + ti_xor(acc[i], 32);
    } else {
#pragma unroll
        for (int s = 0; s < NL; s++) {
            uint32_t bw[4];
            tr4_rows(wv[s], bw);
            const uint4 sc4 = sv[s / 2];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int g = gbase + 4 * s + u;
                const uint2 av = *reinterpret_cast<const uint2*>(L.aq + tA * S + 8 * g + 2 * j);
                const v4i cv = *reinterpret_cast<const v4i*>(L.corr + g * 16 + 4 * j);
                const float4 sx = *reinterpret_cast<const float4*>(L.as + g * 16 + 4 * j);
                const long A = (long)(((uint64_t)av.y << 32) | av.x);
                const uint32_t lo = bw[u] & 0x0F0F0F0Fu, hi = (bw[u] >> 4) & 0x0F0F0F0Fu;
                const long B = (long)(((uint64_t)hi << 32) | lo);
                const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, cv, 0, 0, 0);
                const int h = 4 * (s & 1) + u;             // this group's half in sc4
                const uint32_t sp = h < 2 ? sc4.x : (h < 4 ? sc4.y : (h < 6 ? sc4.z : sc4.w));
                const float sw = ti_h2f((uint16_t)((h & 1) ? (sp >> 16) : (sp & 0xffff)));
                acc[0] = fmaf((float)d[0], sw * sx.x, acc[0]);
                acc[1] = fmaf((float)d[1], sw * sx.y, acc[1]);
                acc[2] = fmaf((float)d[2], sw * sx.z, acc[2]);
                acc[3] = fmaf((float)d[3], sw * sx.w, acc[3]);
            }
        }
    }
    // partials: lane (m, j) holds tokens 4j..4j+3 of row m of the wave's block (DUAL: lanes
    // j >= 2 repeat tokens 0..7 in the slots of tokens 8..15, which T <= 8 never reads)
#pragma unroll
    for (int i = 0; i < 4; i++) L.part[(wave * 16 + 4 * j + i) * 17 + m] = acc[i];
    __syncthreads();

    if constexpr (GU) {
        // silu(g)*u of (token, chunk row) and its quantQ8 over the chunk's 32 rows
        // (q8_group's arithmetic: scale = absmax/127, round-half-even, clamp 127)
        const int r = tid & 31;
        const int ch = blockIdx.x;
        for (int tok = tid >> 5; tok < T; tok += 2 * W) {
            float gv = 0.0f, uv = 0.0f;
#pragma unroll
            for (int k = 0; k < KS; k++) {
                gv += L.part[(((r >> 4) * KS + k) * 16 + tok) * 17 + (r & 15)];
                uv += L.part[(((2 + (r >> 4)) * KS + k) * 16 + tok) * 17 + (r & 15)];
            }
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
        const int w0 = (wave / KS) * KS;
        float* xn = L.xn + (wave / KS) * 256;            // this block's outputs [tok][16] (PART)
        float vr[NE];
#pragma unroll
        for (int r = 0; r < NE; r++) {
            const int e = (wave % KS) * 64 + lane + r * 64 * KS;
            const int tok = e >> 4, mm = e & 15;
            vr[r] = 0.0f;
#pragma unroll
            for (int k = 0; k < KS; k++) vr[r] += L.part[((w0 + k) * 16 + (tok < TG_TMAX ? tok : 0)) * 17 + mm];
        }
        if constexpr (SPLIT) {
            // publish this half (device-scope stores), count the pair; the second to arrive
            // adds the halves in order 0, 1 and stores, then resets the counter
            int& s_second = *reinterpret_cast<int*>(L.inv);   // (the norm slots are unused here)
            const size_t base = (size_t)bidx * 2 * 256;
#pragma unroll
            for (int r = 0; r < NE; r++) {
                const int e = (wave % KS) * 64 + lane + r * 64 * KS;
                if (e < 16 * T) ti_pub_store(a.sp + base + (size_t)part * 256 + e, vr[r]);
            }
            ti_stores_done();
            __syncthreads();
            if (tid == 0) s_second = ti_arrive(a.scnt + bidx) == 1u;
            __syncthreads();
            if (!s_second) return;
#pragma unroll
            for (int r = 0; r < NE; r++) {
                const int e = (wave % KS) * 64 + lane + r * 64 * KS;
                if (e < 16 * T) {
                    const float o = ti_pub_load(a.sp + base + (size_t)(part ^ 1) * 256 + e);
                    vr[r] = part == 0 ? vr[r] + o : o + vr[r];
                }
            }
            if (tid == 0) __hip_atomic_store(a.scnt + bidx, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int r = 0; r < NE; r++) {
            const int e = (wave % KS) * 64 + lane + r * 64 * KS;
            const int tok = e >> 4, mm = e & 15;
            const int lr = PART ? out_row(mm) : row0 - bs.base + mm;
            if (valid && tok < T && lr < bs.n) {
                const float yn = a.acc ? yold[r] + vr[r] : vr[r];
                bs.y[(size_t)tok * bs.n + lr] = yn;
                if (PART) xn[tok * 16 + mm] = yn;
            }
        }
        if constexpr (PART) {   // partial t = sum over i of x[t + 256 i]^2, in i order
            __syncthreads();
            for (int idx = (wave % KS) * 64 + lane; valid && idx < T * tpb; idx += 64 * KS) {
                const int tok = idx / tpb, tl = idx % tpb;
                float sp = 0.0f;
                for (int i = 0; i < a.pku; i++) {
                    const float xv = xn[tok * 16 + tl + tpb * i];
                    const float sq = xv * xv;
                    sp = sp + sq;
                }
                a.pout[(size_t)tok * 256 + (row0 / 16) * tpb + tl] = sp;
            }
        }
    }
}

// Per-token RMSNorm + quantQ8T of a [T][K] activation, one workgroup per token (the
// rmsnorm + quantQ8T dispatches the projections of a T-token forward share): the sum of
// squares in the reference's order (256 strided partials, 128..1 tree), then the
// quantizer on contiguous KU-element runs (a 32-group = 32/KU lanes); codes [T][K/4] and
// scales [T][K/32], bit-exact with rmsnorm + q8_group.
template <int KU>
__global__ __launch_bounds__(256) void k_tnorm_q8(const float* __restrict__ x, const uint16_t* __restrict__ nw, float eps,
                                                  uint32_t* __restrict__ xq, float* __restrict__ xs) {
    constexpr int K = 256 * KU;
    __shared__ float red[256];
    const int t = threadIdx.x;
    const float* xr = x + (size_t)blockIdx.x * K;
    float xsd[KU], xc[KU];
    uint16_t wc[KU];
#pragma unroll
    for (int i = 0; i < KU; i++) {
        xsd[i] = xr[t + 256 * i];
        wc[i] = nw[KU * t + i];
    }
    if constexpr (KU % 4 == 0) {
        const float4* x4 = reinterpret_cast<const float4*>(xr + KU * t);
#pragma unroll
        for (int i = 0; i < KU / 4; i++) {
            const float4 v = x4[i];
            xc[4 * i] = v.x; xc[4 * i + 1] = v.y; xc[4 * i + 2] = v.z; xc[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < KU; i++) xc[i] = xr[KU * t + i];
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < KU; i++) {
        const float sq = xsd[i] * xsd[i];
        s = s + sq;
    }
    float m = ti_tree_sum_256(s, red) / (float)K;
    m = m + eps;
    const float inv_rms = 1.0f / sqrtf(m);
    float v[KU], mx = 0.0f;
#pragma unroll
    for (int i = 0; i < KU; i++) {
        const float p = xc[i] * inv_rms;
        v[i] = p * ti_h2f(wc[i]);
        mx = fmaxf(mx, fabsf(v[i]));
    }
    mx = group_max_contig<KU>(mx);
    const float scale = mx / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    uint32_t wd[(KU + 3) / 4] = {};
#pragma unroll
    for (int i = 0; i < KU; i++) wd[i / 4] |= (uint32_t)(q8_code(v[i], inv) & 0xff) << (8 * (i % 4));
    uint32_t* q = xq + (size_t)blockIdx.x * (K / 4);
    if constexpr (KU >= 4) {
#pragma unroll
        for (int k = 0; k < KU / 4; k++) q[KU / 4 * t + k] = wd[k];
    } else {
        uint8_t* qb = reinterpret_cast<uint8_t*>(q);
#pragma unroll
        for (int i = 0; i < KU; i++) qb[KU * t + i] = (uint8_t)((wd[0] >> (8 * i)) & 0xff);
    }
    if (t % (32 / KU) == 0) xs[(size_t)blockIdx.x * (K / 32) + KU * t / 32] = scale;
}

// The RMSNorm partial sums of a [T][K] activation (K = 256 KU) that no projection
// produced (the embeddings): p[t][u] = sum over i of x[t][u + 256 i]^2, in i order.
__global__ __launch_bounds__(256) void k_tsumsq(const float* __restrict__ x, float* __restrict__ p, int K) {
    const float* xr = x + (size_t)blockIdx.x * K;
    float s = 0.0f;
    for (int i = threadIdx.x; i < K; i += 256) {
        const float sq = xr[i] * xr[i];
        s = s + sq;
    }
    p[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

// ---- host dispatch ------------------------------------------------------------------
// (W, KS, NL) per K = 128*KS*NL: 8 or 12 waves per workgroup (more loads in flight
// per CU: the N = 2048 projections fill only 128 CUs with 16-row blocks; K = 6144 at
// 12 waves measured 8.8 against 9.5 us at 8)
bool tg_split(int G, int& W, int& KS, int& NL) {
    switch (G) {
        case 8: W = 4; KS = 1; NL = 2; return true;
        case 16: W = 4; KS = 2; NL = 2; return true;
        case 32: W = 8; KS = 4; NL = 2; return true;
        case 64: W = 8; KS = 8; NL = 2; return true;
        case 96: W = 12; KS = 12; NL = 2; return true;
        case 128: W = 8; KS = 8; NL = 4; return true;
        case 192: W = 12; KS = 12; NL = 4; return true;
        case 256: W = 8; KS = 8; NL = 8; return true;
        default: return false;
    }
}

int tg_ku(int K) {   // k_tnorm_q8: K = 256*KU, KU in {1, 2, 4, 8, 16}
    if (K % 256) return 0;
    const int ku = K / 256;
    return (ku == 1 || ku == 2 || ku == 4 || ku == 8 || ku == 16) ? ku : 0;
}

template <bool GU, int W, int KS, int NL, int IN, bool PART, bool SPLIT, bool DUAL>
int tg_go1(ti_ctx* c, const TgArgs& a, unsigned grid, const char* name) {
    const size_t lds = (size_t)tg_lds_words(a.T, a.K, W, PART ? W / KS : 0) * 4;
    static bool attr = false;
    if (!attr && lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_tgemm<GU, W, KS, NL, IN, PART, SPLIT, DUAL>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return ti_hip_fail(e, "k_tgemm LDS attribute");
        attr = true;
    }
    k_tgemm<GU, W, KS, NL, IN, PART, SPLIT, DUAL><<<grid, 64 * W, lds, c->stream>>>(a);
    TI_LAUNCHED(name);
    return TI_OK;
}

// T <= 8 takes the pairwise-group MFMA loop (no padding token rows)
template <bool GU, int W, int KS, int NL, int IN, bool PART, bool SPLIT = false>
int tg_go(ti_ctx* c, const TgArgs& a, unsigned grid, const char* name) {
    if (a.T <= 8) return tg_go1<GU, W, KS, NL, IN, PART, SPLIT, true>(c, a, grid, name);
    return tg_go1<GU, W, KS, NL, IN, PART, SPLIT, false>(c, a, grid, name);
}

// dispatch over K for the non-gate/up kernels: (W, KS, NL) from the split table (the
// norm prologue exists for K <= 2048 only)
template <int IN, bool PART>
int tg_dispatch(ti_ctx* c, const TgArgs& a, int nb, const char* name) {
#define TGQ(G_, W_, KS_, NL_) \
    case G_: return tg_go<false, W_, KS_, NL_, IN, PART>(c, a, (unsigned)((nb + W_ / KS_ - 1) / (W_ / KS_)), name);
    if constexpr (IN == TG_NORM) {
        switch (a.K / 32) { TGQ(8, 4, 1, 2) TGQ(16, 4, 2, 2) TGQ(32, 8, 4, 2) TGQ(64, 8, 8, 2) }
    } else {
        switch (a.K / 32) {
            TGQ(8, 4, 1, 2) TGQ(16, 4, 2, 2) TGQ(32, 8, 4, 2) TGQ(64, 8, 8, 2) TGQ(96, 12, 12, 2) TGQ(128, 8, 8, 4)
            TGQ(192, 12, 12, 4) TGQ(256, 8, 8, 8)
        }
    }
#undef TGQ
    return ti_fail(TI_ERR_INVALID, "T-token GEMM: no kernel for K=%d", a.K);
}

}  // namespace

// Which T-token projections take these kernels: 2..16 tokens, K/32 in the split table.
bool ti_tgemm_ok(int T, int K) {
    int W, KS, NL;
    return T >= 2 && T <= TG_TMAX && K % 32 == 0 && tg_split(K / 32, W, KS, NL);
}
bool ti_tnorm_ok(int K) { return tg_ku(K) != 0; }
// the norm prologue: K = 256 * {1,2,4,8}, 8 elements per lane, a 32-group within 4 lanes
bool ti_tgemm_norm_ok(int T, int K) {
    int W, KS, NL;
    if (!ti_tgemm_ok(T, K) || !tg_ku(K) || K > 2048) return false;
    tg_split(K / 32, W, KS, NL);
    const int gw = K / 32 == 8 ? 4 : 8;               // the gate/up kernels' W at this K
    return K % (32 * W) == 0 && K % (32 * gw) == 0;
}
bool ti_tgemm_gateup_ok(int T, int H) {
    const int G = H / 32;
    return ti_tgemm_ok(T, H) && (G == 8 || G == 16 || G == 32 || G == 64 || G == 128);
}

// rmsnorm + quantQ8T of T tokens: xq [T][K/4], xs [T][K/32]; K = 256 * {1,2,4,8,16}
int ti_tnorm_q8_launch(ti_ctx* c, const float* x, const uint16_t* nw, float eps, uint32_t* xq, float* xs, int T, int K) {
    switch (tg_ku(K)) {
#define TN(KU_) case KU_: k_tnorm_q8<KU_><<<T, 256, 0, c->stream>>>(x, nw, eps, xq, xs); TI_LAUNCHED("k_tnorm_q8"); return TI_OK;
        TN(1) TN(2) TN(4) TN(8) TN(16)
#undef TN
    }
    return ti_fail(TI_ERR_INVALID, "T-token norm: no kernel for K=%d", K);
}

// y_s[t][:] (+)= W_s a_t for up to three segments sharing the activation: int8 codes
// (in.xq [T][K/4], in.xs [T][K/32]) or, with in.x set, RMSNorm + quantQ8T of in.x in the
// prologue from the partial sums in.pin. pout: also write the output's partial sums
// (one segment, N = 256 * {1,2,4,8,16}, acc = 1: the residual stream). Scales must be
// 16-byte aligned (K % 256 == 0 keeps every row aligned); segments before the last must
// have a multiple of 16 rows.
int ti_tgemm_launch(ti_ctx* c, const TgIn& in, int nseg, const uint32_t* const* packs, const uint16_t* const* scs,
                    float* const* ys, const int* Ns, int T, int K, int acc, float* pout) {
    TgArgs a = {};
    a.nseg = nseg;
    a.N = 0;
    for (int s = 0; s < nseg; s++) {
        a.seg[s] = {reinterpret_cast<const uint4*>(packs[s]), reinterpret_cast<const uint4*>(scs[s]), ys[s], Ns[s]};
        if (s + 1 < nseg && Ns[s] % 16) return ti_fail(TI_ERR_INVALID, "T-token GEMM: segment rows must be multiples of 16");
        if (reinterpret_cast<uintptr_t>(scs[s]) % 16) return ti_fail(TI_ERR_INVALID, "T-token GEMM: scales must be 16-byte aligned");
        a.N += Ns[s];
    }
    a.K = K;
    a.T = T;
    a.acc = acc;
    a.S = K / 4 + 2;
    a.xq = in.xq;
    a.xs = in.xs;
    a.x = in.x;
    a.nw = in.nw;
    a.eps = in.eps;
    a.pin = in.pin;
    a.pout = pout;
    if (!ti_tgemm_ok(T, K)) return ti_fail(TI_ERR_INVALID, "T-token GEMM: unsupported T=%d K=%d", T, K);
    if (in.x && !ti_tgemm_norm_ok(T, K)) return ti_fail(TI_ERR_INVALID, "T-token GEMM: no norm prologue for T=%d K=%d", T, K);
    if (pout) {
        a.pku = tg_ku(a.N);
        if (nseg != 1 || !acc || !a.pku) return ti_fail(TI_ERR_INVALID, "T-token GEMM: partial sums need one residual segment, N = 256*{1,2,4,8,16}");
    }
    const int nb = (a.N + 15) / 16;
    // K = 6144 residual projections (down at the 1.7B geometry) with at most 128 blocks
    // fill only half the CUs with 16-row blocks: two workgroups per block, each on one
    // half of K (12 waves, 96 groups), the second to finish adding the halves
    if (!in.x && !pout && nseg == 1 && acc && K == 6144 && nb <= TI_TG_SPLIT_BLOCKS) {
        a.K = K / 2;
        a.S = a.K / 4 + 2;
        a.kld = K;
        a.sp = c->tg_part;
        a.scnt = c->sync + TI_SYNC_TGEMM;
        return tg_go<false, 12, 12, 2, TG_Q8, false, true>(c, a, (unsigned)(2 * nb), "k_tgemm");
    }
    a.kld = K;
    if (in.x) return tg_dispatch<TG_NORM, false>(c, a, nb, "k_tgemm");
    return pout ? tg_dispatch<TG_Q8, true>(c, a, nb, "k_tgemm") : tg_dispatch<TG_Q8, false>(c, a, nb, "k_tgemm");
}

// gate/up: swq[t] = quantQ8(silu(Wg a_t) * (Wu a_t)), a_t as for ti_tgemm_launch
int ti_tgemm_gateup_launch(ti_ctx* c, const TgIn& in, const uint32_t* gpack, const uint16_t* gsc, const uint32_t* upack,
                           const uint16_t* usc, int I, int H, int T, uint32_t* swq, float* sws) {
    if (!ti_tgemm_gateup_ok(T, H) || I % 32) return ti_fail(TI_ERR_INVALID, "T-token gate/up: unsupported T=%d H=%d I=%d", T, H, I);
    if (in.x && !ti_tgemm_norm_ok(T, H)) return ti_fail(TI_ERR_INVALID, "T-token gate/up: no norm prologue for H=%d", H);
    if (reinterpret_cast<uintptr_t>(gsc) % 16 || reinterpret_cast<uintptr_t>(usc) % 16)
        return ti_fail(TI_ERR_INVALID, "T-token gate/up: scales must be 16-byte aligned");
    TgArgs a = {};
    a.seg[0] = {reinterpret_cast<const uint4*>(gpack), reinterpret_cast<const uint4*>(gsc), nullptr, I};
    a.nseg = 1;
    a.N = I;
    a.K = H;
    a.T = T;
    a.S = H / 4 + 2;
    a.xq = in.xq;
    a.xs = in.xs;
    a.x = in.x;
    a.nw = in.nw;
    a.eps = in.eps;
    a.pin = in.pin;
    a.upack = reinterpret_cast<const uint4*>(upack);
    a.usc = reinterpret_cast<const uint4*>(usc);
    a.yq = swq;
    a.ys = sws;
    const unsigned grid = (unsigned)(I / 32);
    const char* nm = "k_tgemm_gateup";
    if (in.x) {
        switch (H / 32) {   // 8 waves: 4 blocks x KS = 2 (K/32 = 8 * NL); K = 256: 4 waves
            case 8: return tg_go<true, 4, 1, 2, TG_NORM, false>(c, a, grid, nm);
            case 16: return tg_go<true, 8, 2, 2, TG_NORM, false>(c, a, grid, nm);
            case 32: return tg_go<true, 8, 2, 4, TG_NORM, false>(c, a, grid, nm);
            case 64: return tg_go<true, 8, 2, 8, TG_NORM, false>(c, a, grid, nm);
        }
    } else {
        switch (H / 32) {
            case 8: return tg_go<true, 4, 1, 2, TG_Q8, false>(c, a, grid, nm);
            case 16: return tg_go<true, 8, 2, 2, TG_Q8, false>(c, a, grid, nm);
            case 32: return tg_go<true, 8, 2, 4, TG_Q8, false>(c, a, grid, nm);
            case 64: return tg_go<true, 8, 2, 8, TG_Q8, false>(c, a, grid, nm);
            case 128: return tg_go<true, 8, 2, 16, TG_Q8, false>(c, a, grid, nm);
        }
    }
    return ti_fail(TI_ERR_INVALID, "T-token gate/up: no kernel for H=%d", H);
}

// RMSNorm partial sums of T rows of K = 256 * {1,2,4,8,16} (the embeddings of a forward)
int ti_tsumsq_launch(ti_ctx* c, const float* x, float* p, int T, int K) {
    if (!tg_ku(K)) return ti_fail(TI_ERR_INVALID, "T-token partial sums: K=%d", K);
    k_tsumsq<<<T, 256, 0, c->stream>>>(x, p, K);
    TI_LAUNCHED("k_tsumsq");
    return TI_OK;
}

extern "C" int ti_rmsnorm_q8_t(ti_ctx* c, const float* x, const uint16_t* w, uint32_t* xq, float* xs, int T, int H,
                               float eps) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && w && xq && xs, "ti_rmsnorm_q8_t: null buffer");
    TI_REQUIRE(T > 0 && T < (1 << 20) && tg_ku(H), "ti_rmsnorm_q8_t: need T > 0 and H = 256 * {1,2,4,8,16} (T=%d H=%d)", T, H);
    TI_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0, "ti_rmsnorm_q8_t: x must be 16-byte aligned");
    return ti_tnorm_q8_launch(c, x, w, eps, xq, xs, T, H);
}
