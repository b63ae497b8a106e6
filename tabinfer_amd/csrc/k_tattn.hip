// k_tattn.hip — the attention of a T-token forward (the batch-8 decode step, short
// prefills; head_dim 128, T <= 16, T * G <= 32 query rows per KV head) as one launch per layer.
//
// The reference runs it as ropeQK for q and k (models/qwen3.js:1700-1760), kvQuantWrite
// (:2180-2216), the T-query attention (:2534-2577) and the log-sum-exp combine
// (:2048-2068), then quantQ8T of the output for o_proj (:1210-1231). Here:
//
//  - workgroup (8 waves) = (KV head hk, row tile rt, split); the keys of hk are cut into
//    blocks of 32 and the waves of the NS splits take blocks round robin (gw: blocks gw,
//    gw + 8NS, ..); the T new keys (positions S0 .. S0+T-1) are one more block, computed
//    in the prologue of the workgroup whose wave takes it, which also writes them into
//    the cache (snorm int8, as kvQuantWrite; row tile 0 only) — no other workgroup reads
//    those positions;
//  - a row tile is 16 query rows (t, h) of hk (rows 16 rt ..; more than 16 rows, up to
//    32, take a second tile that streams the keys again): every workgroup RMSNorms +
//    RoPEs its rows (q_norm, the rope row of position S0 + t) and keeps them as f16 hi +
//    lo (q = hi + lo to ~2^-22);
//  - per block, S^T = K Q^T on the matrix cores (v_mfma_f32_16x16x32_f16: K codes are
//    exact in f16, two MFMAs per 32-dim scale group for q's two halves, each group's dot
//    scaled by its key's K scale), causal mask, online softmax per row;
//  - P V on the matrix cores as well: the scores come out of the MFMA with lane (r, j)
//    holding row r at keys 4j..4j+3 of each 16-key half, which is already the A-operand
//    layout of the next MFMA (K index 8j + e <-> key 4j + e, 16 + 4j + e - 4); the V
//    scale of (key, 32-dim group) is folded into P (P'_g = p * vs, again f16 hi + lo);
//    the V operand (8 keys of one dim per lane) comes from the key-major V tile through
//    gfx950's transposing LDS read ds_read_b64_tr_b8 (16 lanes read 8 rows of 16 bytes,
//    lane i receives column i), whose row addresses follow the same key order;
//  - the waves' (m, l, O) merge in LDS into the split's partial; a second small launch
//    (k_attn_tcombine, one workgroup per (KV head, row), every partial load in flight at
//    once) merges the NS partials by log-sum-exp, normalises and writes the output as
//    quantQ8T codes + scales for o_proj (one CU reading every split's partial through
//    device-coherent loads took ~11 us; this takes one memory round trip).
#include "ti_dev.h"

namespace {

typedef ti_h8 h8;
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int HD = 128, NG = HD / 32;
constexpr int TA_ROWS = 16;                  // query rows (t, h) per KV head
constexpr int TA_BLK = 32;                   // keys per wave block
constexpr int TA_KS = 136, TA_VS = 144;      // LDS row strides (bytes): conflict-free operand reads
constexpr int TA_W = 8;                      // waves per workgroup
constexpr int TA_REG = TA_W + 1;             // tile regions: one per wave + the new keys
constexpr int TA_KBYTES = TA_BLK * TA_KS, TA_VBYTES = TA_BLK * TA_VS;
constexpr int TA_MAXS = 32;                  // splits per KV head
constexpr float TA_LOG2E = 1.4426950408889634f;

struct TAttnArgs {
    const float* q;        // [T][nHq*HD] (the q/k/v projections)
    const float* k;        // [T][nKv*HD]
    const float* v;        // [T][nKv*HD]
    const uint16_t* qw;    // q_norm / k_norm weights (f16)
    const uint16_t* kw;
    const float* rope;     // [cap][HD]: cos(pos*theta^(-2i/HD)) at i, sin at HD/2 + i
    uint8_t* kq;           // cache: [pos][kvs][HD] codes (kvs >= nKv slots), [pos][nKv][NG] scales
    float* ks;
    uint8_t* vq;
    float* vs;
    float* po;             // split partials: [nKv][NS][16][HD] and (m, l) [nKv][NS][16][2]
    float* pml;
    int S0, T, nKv, G, NS;
    float eps;
    int RT;                // row tiles: workgroups (hk, rt, split) serve rows 16 rt .. 16 rt + 15
    int kvs;               // code slots per cached position
};

// RMSNorm in the reference's order for a head row held as (element L, element L+64) by
// the 64 lanes (slot j + slot j+64, then an exact 32..1 xor tree), then split-half RoPE
__device__ __forceinline__ void norm_rope(float x0, float x1, float w0, float w1, float c, float s, float eps, float& o0,
                                          float& o1) {
    float v = x0 * x0 + x1 * x1;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = v + ti_xor(v, o);
    float m = v / (float)HD;
    m = m + eps;
    const float inv = 1.0f / sqrtf(m);
    const float t0n = x0 * inv, t1n = x1 * inv;
    const float r0 = t0n * w0, r1 = t1n * w1;
    const float p00 = r0 * c, p01 = (-r1) * s;
    const float p10 = r1 * c, p11 = r0 * s;
    o0 = p00 + p01;
    o1 = p10 + p11;
}

__global__ __launch_bounds__(64 * TA_W) void k_attn_tq8(TAttnArgs a) {
    constexpr int NT = 64 * TA_W;
    __shared__ __align__(16) _Float16 s_qh[TA_ROWS][HD];
    __shared__ __align__(16) _Float16 s_ql[TA_ROWS][HD];
    // K tiles, then V tiles (TA_REG regions each); after the block loop the same bytes
    // hold the waves' O for the merge, then the splits' (m, l)
    __shared__ __align__(16) uint8_t s_tile[TA_REG * (TA_KBYTES + TA_VBYTES)];
    __shared__ __align__(16) float s_ks[TA_REG][TA_BLK][NG];
    __shared__ __align__(16) float s_vs[TA_REG][TA_BLK][NG];
    __shared__ float s_wm[TA_W][TA_ROWS], s_wl[TA_W][TA_ROWS];
    static_assert(TA_W * TA_ROWS * HD * 4 <= TA_REG * (TA_KBYTES + TA_VBYTES), "O merge fits the tiles");

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int NS = a.NS;
    const int split = blockIdx.x % NS, hr = blockIdx.x / NS;
    const int rt = hr % a.RT, hk = hr / a.RT;
    const int rbase = TA_ROWS * rt;                      // this workgroup's first query row
    const int T = a.T, G = a.G, R = T * G, S0 = a.S0;
    const int nq = a.nKv * G * HD, nkv = a.nKv * HD;
    const int nb = (S0 + TA_BLK - 1) / TA_BLK;          // blocks of cached keys
    const int NW = NS * TA_W;
    const int gw = split * TA_W + wave;
    const int tail_gw = nb % NW;                         // the wave that takes the new keys
    const bool tail_wg = tail_gw / TA_W == split;
    // scores in log2 units: the K scales staged in LDS carry 1/(127 sqrt(HD)) * log2(e), so
    // p = 2^(s - m) is one v_exp_f32
    const float qk2 = TA_LOG2E / (127.0f * sqrtf((float)HD));
    uint8_t* kt_base = s_tile;
    uint8_t* vt_base = s_tile + TA_REG * TA_KBYTES;
    constexpr int QPW = TA_ROWS / TA_W, KPW = 2 * TA_ROWS / TA_W;   // prologue rows per wave
    // one block's K, V rows and scales: lane loads rows lane/8 + 8p, 16-byte chunk lane%8
    uint4 kr[4], vr[4];
    float2 ksr, vsr;
    auto load_blk = [&](int k0) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            int key = k0 + (lane >> 3) + 8 * p;
            key = key < S0 ? key : (S0 > 0 ? S0 - 1 : 0);
            const size_t off = ((size_t)key * a.kvs + hk) * HD + 16 * (lane & 7);
            kr[p] = ti_ld_nt(reinterpret_cast<const uint4*>(a.kq + off));
            vr[p] = ti_ld_nt(reinterpret_cast<const uint4*>(a.vq + off));
        }
        int key = k0 + (lane >> 1);
        key = key < S0 ? key : (S0 > 0 ? S0 - 1 : 0);
        const size_t so = ((size_t)key * a.nKv + hk) * NG + 2 * (lane & 1);
        ksr = *reinterpret_cast<const float2*>(a.ks + so);
        vsr = *reinterpret_cast<const float2*>(a.vs + so);
    };

    // ---- prologue loads: the query rows, and (the new keys' workgroup) the 2T new K / V
    // rows, QPW and KPW per wave; lane L holds elements L and L + 64
    float qx[QPW][2], qwv[2], qc[QPW][2];
    float kx[KPW][2], kwv[2], kc[KPW][2];
    qwv[0] = ti_h2f(a.qw[lane]);
    qwv[1] = ti_h2f(a.qw[lane + 64]);
    kwv[0] = ti_h2f(a.kw[lane]);
    kwv[1] = ti_h2f(a.kw[lane + 64]);
#pragma unroll
    for (int i = 0; i < QPW; i++) {
        const int rg = rbase + wave + TA_W * i;
        const int rc = rg < R ? rg : 0;
        const int t = rc / G, h = rc % G;
        const float* src = a.q + (size_t)t * nq + (size_t)(hk * G + h) * HD;
        qx[i][0] = src[lane];
        qx[i][1] = src[lane + 64];
        const float* cs = a.rope + (size_t)(S0 + t) * HD;
        qc[i][0] = cs[lane];
        qc[i][1] = cs[lane + 64];
    }
    {   // unconditional (clamped) loads: straight-line code lets the prologue wait for
        // exactly its own loads, not the key block's issued after them
#pragma unroll
        for (int i = 0; i < KPW; i++) {
            const int jb = wave + TA_W * i;               // job: K rows 0..T-1, then V rows
            const int jc = jb < 2 * T ? jb : 0;
            const bool isv = jc >= T;
            const int t = isv ? jc - T : jc;
            const float* src = (isv ? a.v : a.k) + (size_t)t * nkv + (size_t)hk * HD;
            kx[i][0] = src[lane];
            kx[i][1] = src[lane + 64];
            const float* cs = a.rope + (size_t)(S0 + t) * HD;
            kc[i][0] = cs[lane];
            kc[i][1] = cs[lane + 64];
        }
    }
    // the wave's first block is in flight during the prologue (its loads are issued after
    // the prologue's, so waiting for those does not wait for these)
    load_blk((gw < nb ? gw : 0) * TA_BLK);              // a dummy block (unused) past nb
    TI_ISSUE_FENCE();
    // ---- q rows: RMSNorm + RoPE, f16 hi + lo into LDS (rows past R are zero)
#pragma unroll
    for (int i = 0; i < QPW; i++) {
        const int r = wave + TA_W * i;
        float o0, o1;
        norm_rope(qx[i][0], qx[i][1], qwv[0], qwv[1], qc[i][0], qc[i][1], a.eps, o0, o1);
        if (rbase + r >= R) o0 = o1 = 0.0f;
        const _Float16 h0 = (_Float16)o0, h1 = (_Float16)o1;
        s_qh[r][lane] = h0;
        s_qh[r][lane + 64] = h1;
        s_ql[r][lane] = (_Float16)(o0 - (float)h0);
        s_ql[r][lane + 64] = (_Float16)(o1 - (float)h1);
    }
    // ---- the new keys: K normed + roped, V as is; snorm int8 into the new-key tile (the
    // last region; its rows T..31 are zero) and, after the block loop, into the cache row
    // S0 + t (no other workgroup reads those rows in this launch; a global store here would
    // wait for a slot behind the block loads in flight)
    uint32_t nkw[KPW][2];
    float nks[KPW][2];
    if (tail_wg) {
        uint8_t* kt = kt_base + TA_W * TA_KBYTES;
        uint8_t* vt = vt_base + TA_W * TA_VBYTES;
#pragma unroll
        for (int i = 0; i < KPW; i++) {
            const int jb = wave + TA_W * i;
            if (jb < 2 * T) {                             // wave-uniform
                const bool isv = jb >= T;
                const int t = isv ? jb - T : jb;
                float o0 = kx[i][0], o1 = kx[i][1];
                if (!isv) norm_rope(kx[i][0], kx[i][1], kwv[0], kwv[1], kc[i][0], kc[i][1], a.eps, o0, o1);
                const float mx0 = fmaxf(ti_max32_nonneg(fabsf(o0)), 1e-12f);
                const float mx1 = fmaxf(ti_max32_nonneg(fabsf(o1)), 1e-12f);
                const uint32_t wd0 = ti_quad_or(snorm_code(o0, mx0) << (8 * (lane & 3)));
                const uint32_t wd1 = ti_quad_or(snorm_code(o1, mx1) << (8 * (lane & 3)));
                uint8_t* lt = (isv ? vt + t * TA_VS : kt + t * TA_KS);
                float* lsc = isv ? &s_vs[TA_W][t][0] : &s_ks[TA_W][t][0];
                const float lm = isv ? 1.0f : qk2;
                nkw[i][0] = wd0;
                nkw[i][1] = wd1;
                nks[i][0] = mx0;
                nks[i][1] = mx1;
                if ((lane & 3) == 0) {
                    *reinterpret_cast<uint32_t*>(lt + lane) = wd0;
                    *reinterpret_cast<uint32_t*>(lt + 64 + lane) = wd1;
                }
                if ((lane & 31) == 0) {
                    lsc[lane / 32] = mx0 * lm;
                    lsc[2 + lane / 32] = mx1 * lm;
                }
            }
        }
        for (int e = tid; e < (TA_BLK - T) * (HD / 4); e += NT) {
            const int rr = T + e / (HD / 4), c = e % (HD / 4);
            *reinterpret_cast<uint32_t*>(kt + rr * TA_KS + 4 * c) = 0u;
            *reinterpret_cast<uint32_t*>(vt + rr * TA_VS + 4 * c) = 0u;
        }
        for (int e = tid; e < (TA_BLK - T) * NG; e += NT) {
            s_ks[TA_W][T + e / NG][e % NG] = 0.0f;
            s_vs[TA_W][T + e / NG][e % NG] = 0.0f;
        }
    }
    __syncthreads();

    // ---- B operands of S^T = K Q^T: lane (r, j) = q row r, dims 32g + 8j .. +8
    const int r16 = lane & 15, jq = lane >> 4;
    h8 qh[NG], ql[NG];
#pragma unroll
    for (int g = 0; g < NG; g++) {
        qh[g] = *reinterpret_cast<const h8*>(&s_qh[r16][32 * g + 8 * jq]);
        ql[g] = *reinterpret_cast<const h8*>(&s_ql[r16][32 * g + 8 * jq]);
    }
    const int trow = (rbase + r16) / G;                  // this lane's score row's token
    // per-lane state: score lanes (row r16) the reference maximum and a partial sum of p;
    // O lanes (rows 4jq..4jq+3, dim 16D + r16) the unnormalised outputs
    float m_run = -3.0e38f, l_run = 0.0f;
    f4 O[8];
#pragma unroll
    for (int D = 0; D < 8; D++) O[D] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    uint8_t* kt_w = kt_base + wave * TA_KBYTES;
    uint8_t* vt_w = vt_base + wave * TA_VBYTES;
    auto store_blk = [&]() {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int rr = (lane >> 3) + 8 * p, c = lane & 7;
            uint2* kd = reinterpret_cast<uint2*>(kt_w + rr * TA_KS + 16 * c);
            kd[0] = make_uint2(kr[p].x, kr[p].y);
            kd[1] = make_uint2(kr[p].z, kr[p].w);
            *reinterpret_cast<uint4*>(vt_w + rr * TA_VS + 16 * c) = vr[p];
        }
        *reinterpret_cast<float2*>(&s_ks[wave][lane >> 1][2 * (lane & 1)]) = make_float2(ksr.x * qk2, ksr.y * qk2);
        *reinterpret_cast<float2*>(&s_vs[wave][lane >> 1][2 * (lane & 1)]) = vsr;
    };

    // one block from tile region `reg`: keys valid below `klim` (block-local), and for the
    // new keys (causal) only up to the row's token
    auto process = [&](int reg, int klim, bool causal) {
        const uint8_t* kt = kt_base + reg * TA_KBYTES;
        const uint8_t* vt = vt_base + reg * TA_VBYTES;
        float sc[2][4];
#pragma unroll
        for (int b = 0; b < 2; b++) {
            f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            float4 kg[4];
#pragma unroll
            for (int i = 0; i < 4; i++) kg[i] = *reinterpret_cast<const float4*>(&s_ks[reg][16 * b + 4 * jq + i][0]);
#pragma unroll
            for (int g = 0; g < NG; g++) {
                const uint2 kw2 = *reinterpret_cast<const uint2*>(kt + (16 * b + r16) * TA_KS + 32 * g + 8 * jq);
                const h8 ka = ti_i8x8_h8(kw2.x, kw2.y);
                const f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[g], z, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[g], d, 0, 0, 0);
                const float kgs[4] = {g == 0 ? kg[0].x : g == 1 ? kg[0].y : g == 2 ? kg[0].z : kg[0].w,
                                      g == 0 ? kg[1].x : g == 1 ? kg[1].y : g == 2 ? kg[1].z : kg[1].w,
                                      g == 0 ? kg[2].x : g == 1 ? kg[2].y : g == 2 ? kg[2].z : kg[2].w,
                                      g == 0 ? kg[3].x : g == 1 ? kg[3].y : g == 2 ? kg[3].z : kg[3].w};
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = fmaf(d[i], kgs[i], acc[i]);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kl = 16 * b + 4 * jq + i;
                const bool ok = kl < klim && (!causal || kl <= trow);
                sc[b][i] = ok ? acc[i] : -3.0e38f;
            }
        }
        // online softmax of row r16 (its 32 keys sit in lanes r16 + 16j), base 2. The
        // reference maximum moves only when the block's maximum exceeds it by more than 6
        // (p <= 64, far inside f16 for p * vs), so O is rescaled rarely; the result is
        // unchanged (o and l share the reference)
        float mt = sc[0][0];
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) mt = fmaxf(mt, sc[b][i]);
        mt = fmaxf(mt, ti_xor(mt, 16));
        mt = fmaxf(mt, ti_xor(mt, 32));
        const bool bump = mt > m_run + 6.0f;
        const float mn = bump ? mt : m_run;
        const float corr = bump ? __builtin_amdgcn_exp2f(m_run - mn) : 1.0f;
        m_run = mn;
        float p[2][4], ps = 0.0f;
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[b][i] = sc[b][i] > -1.0e38f ? __builtin_amdgcn_exp2f(sc[b][i] - mn) : 0.0f;
                ps += p[b][i];
            }
        l_run = fmaf(l_run, corr, ps);
        if (__any(bump)) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float ci = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (4 * jq + i),
                                                                                        __builtin_bit_cast(int, corr)));
#pragma unroll
                for (int D = 0; D < 8; D++) O[D][i] *= ci;
            }
        }
        // P'_g = p * vs(key, g) as f16 hi + lo, A operands: K index 8jq + 4b + i
        h8 ph[NG], pl[NG];
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 vg = *reinterpret_cast<const float4*>(&s_vs[reg][16 * b + 4 * jq + i][0]);
                const float vv[4] = {vg.x, vg.y, vg.z, vg.w};
#pragma unroll
                for (int g = 0; g < NG; g++) {
                    const float pv = p[b][i] * vv[g];
                    const _Float16 hi = (_Float16)pv;
                    ph[g][4 * b + i] = hi;
                    pl[g][4 * b + i] = (_Float16)(pv - (float)hi);
                }
            }
        // V operands through the transposing read: lanes 2rr, 2rr+1 of a 16-lane group
        // address key(8jq + rr) (rr < 4: 4jq + rr; else 16 + 4jq + rr - 4), 8-byte halves
        // of the dim block; lane i of the group receives dim 16D + i of the 8 keys
        const int rr = r16 >> 1;
        const int kv_row = rr < 4 ? 4 * jq + rr : 16 + 4 * jq + (rr - 4);
        const uint8_t* vrow = vt + kv_row * TA_VS + 8 * (r16 & 1);
#pragma unroll
        for (int D = 0; D < 8; D++) {
            const v2i vb = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (__attribute__((address_space(3))) v2i*)(vrow + 16 * D));
            const h8 vh = ti_i8x8_h8((uint32_t)vb.x, (uint32_t)vb.y);
            O[D] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[D >> 1], vh, O[D], 0, 0, 0);
            O[D] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[D >> 1], vh, O[D], 0, 0, 0);
        }
    };

    // ---- this wave's blocks of cached keys, the next block's loads in flight during the
    // current one (LDS tile reuse is ordered: one wave's LDS accesses complete in order)
    int blk = gw;
    while (blk < nb) {
        store_blk();
        const int k0 = blk * TA_BLK;
        blk += NW;
        if (blk < nb) load_blk(blk * TA_BLK);
        process(wave, S0 - k0, false);
    }
    if (gw == tail_gw) process(TA_W, T, true);
    if (tail_wg && rt == 0) {   // the new keys into the cache (one row tile writes them)
#pragma unroll
        for (int i = 0; i < KPW; i++) {
            const int jb = wave + TA_W * i;
            if (jb < 2 * T) {                             // wave-uniform
                const bool isv = jb >= T;
                const int t = isv ? jb - T : jb;
                const size_t row = (size_t)(S0 + t) * a.nKv + hk, crow = (size_t)(S0 + t) * a.kvs + hk;
                uint32_t* gq = reinterpret_cast<uint32_t*>((isv ? a.vq : a.kq) + crow * HD);
                float* gs = (isv ? a.vs : a.ks) + row * NG;
                if ((lane & 3) == 0) {
                    gq[lane / 4] = nkw[i][0];
                    gq[16 + lane / 4] = nkw[i][1];
                }
                if ((lane & 31) == 0) {
                    gs[lane / 32] = nks[i][0];
                    gs[2 + lane / 32] = nks[i][1];
                }
            }
        }
    }

    // ---- merge the waves into the split's partial (plain stores: the combine kernel
    // that reads them runs after this launch)
    float l16 = l_run;
    l16 += ti_xor(l16, 16);
    l16 += ti_xor(l16, 32);
    __syncthreads();                                     // tiles free: they become s_om
    float (*s_om)[TA_ROWS][HD] = reinterpret_cast<float (*)[TA_ROWS][HD]>(s_tile);
    if (jq == 0) {
        s_wm[wave][r16] = m_run;
        s_wl[wave][r16] = l16;
    }
#pragma unroll
    for (int D = 0; D < 8; D++)
#pragma unroll
        for (int i = 0; i < 4; i++) s_om[wave][4 * jq + i][16 * D + r16] = O[D][i];
    __syncthreads();
    constexpr int DPT = TA_ROWS * HD / NT;               // outputs per thread (4)
    static_assert(DPT == 4, "one float4 of the partial per thread");
    const int row = tid / (HD / DPT), d0 = DPT * (tid % (HD / DPT));
    float M = s_wm[0][row];
#pragma unroll
    for (int w = 1; w < TA_W; w++) M = fmaxf(M, s_wm[w][row]);
    float e[TA_W], L = 0.0f;
#pragma unroll
    for (int w = 0; w < TA_W; w++) {
        e[w] = __builtin_amdgcn_exp2f(s_wm[w][row] - M);
        L = fmaf(s_wl[w][row], e[w], L);
    }
    float o[DPT];
#pragma unroll
    for (int k = 0; k < DPT; k++) {
        o[k] = 0.0f;
#pragma unroll
        for (int w = 0; w < TA_W; w++) o[k] = fmaf(s_om[w][row][d0 + k], e[w], o[k]);
    }
    const size_t pr = (((size_t)hk * a.RT + rt) * NS + split) * TA_ROWS + row;
    *reinterpret_cast<float4*>(a.po + pr * HD + d0) = make_float4(o[0], o[1], o[2], o[3]);
    if (d0 == 0) *reinterpret_cast<float2*>(a.pml + pr * 2) = make_float2(M, L);
}

// The split merge of k_attn_tq8: workgroup = (KV head, query row (t, h)), thread = dim.
// O = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s (max and sums in log2 units, as the
// attention kernel keeps them), then quantQ8T of 32 consecutive dims = 32 lanes.
struct TCombArgs {
    const float* po;
    const float* pml;
    uint32_t* oq;          // [T][nHq*HD/4]
    float* os;             // [T][nHq*HD/32]
    int NS, nKv, G, R, RT;
};

__global__ __launch_bounds__(HD) void k_attn_tcombine(TCombArgs c) {
    __shared__ float s_e[TA_MAXS];
    __shared__ float s_L;
    const int hk = blockIdx.x / c.R, row = blockIdx.x % c.R, d = threadIdx.x;
    const int NS = c.NS;
    const size_t pbase = ((size_t)hk * c.RT + row / TA_ROWS) * NS;   // this row's tile's splits
    float ov[TA_MAXS];
#pragma unroll
    for (int s = 0; s < TA_MAXS; s++)   // every load at once; splits past NS repeat the last one
        ov[s] = c.po[((pbase + (s < NS ? s : NS - 1)) * TA_ROWS + row % TA_ROWS) * HD + d];
    if (d < 64) {   // wave 0: lane s holds split s's (m, l); the split weights 2^(m_s - M)
        const bool in = d < NS;
        const float2 ml = *reinterpret_cast<const float2*>(c.pml + ((pbase + (in ? d : 0)) * TA_ROWS + row % TA_ROWS) * 2);
        const float m = in ? ml.x : -3.0e38f;
        float M = m;
#pragma unroll
        for (int o2 = 32; o2 > 0; o2 >>= 1) M = fmaxf(M, ti_xor(M, o2));
        const float ew = in ? __builtin_amdgcn_exp2f(m - M) : 0.0f;
        float L = in ? ml.y * ew : 0.0f;
#pragma unroll
        for (int o2 = 32; o2 > 0; o2 >>= 1) L += ti_xor(L, o2);
        if (d < TA_MAXS) s_e[d] = ew;
        if (d == 0) s_L = L;
    }
    __syncthreads();
    float o = 0.0f;
#pragma unroll
    for (int s = 0; s < TA_MAXS; s++) o = fmaf(ov[s], s_e[s], o);
    const float res = o * (1.0f / (127.0f * s_L));
    const float mx = ti_max32_nonneg(fabsf(res));
    const float scale = mx / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const uint32_t word = ti_quad_or((uint32_t)(q8_code(res, inv) & 0xff) << (8 * (d & 3)));
    const int t = row / c.G, h = row % c.G;
    const size_t e = (size_t)t * c.nKv * c.G * HD + (size_t)(hk * c.G + h) * HD + d;
    if ((d & 3) == 0) c.oq[e / 4] = word;
    if ((d & 31) == 0) c.os[e / 32] = scale;
}

}  // namespace

// Whether the T-token attention takes this kernel: head_dim 128, T*G <= 32 query rows
// per KV head (two row tiles of 16), T <= 16 new keys.
bool ti_tattn_ok(int T, int nHq, int nKv, int hd) {
    return hd == HD && nKv > 0 && nHq % nKv == 0 && T >= 1 && T <= 16 && T * (nHq / nKv) <= 2 * TA_ROWS;
}

// T new tokens at positions S0 .. S0+T-1 of one layer: q, k, v are the projections
// ([T][nHq*HD], [T][nKv*HD]), rope the model's rotary table; writes the new K/V rows
// into the cache and the output's quantQ8T codes/scales (oq [T][nHq*HD/4], os [T][nHq*HD/32]).
int ti_tattn_launch(ti_ctx* c, const float* q, const float* k, const float* v, const uint16_t* qw, const uint16_t* kw,
                    const float* rope, uint32_t* kq, float* ks, uint32_t* vq, float* vs, int S0, int T, int nHq, int nKv,
                    int hd, float eps, uint32_t* oq, float* os, int kvs) {
    if (kvs < nKv) return ti_fail(TI_ERR_INVALID, "T-token attention: %d code slots per position < %d KV heads", kvs, nKv);
    if (!ti_tattn_ok(T, nHq, nKv, hd)) return ti_fail(TI_ERR_INVALID, "T-token attention: unsupported T=%d heads %d/%d hd=%d", T, nHq, nKv, hd);
    const int nb = (S0 + TA_BLK - 1) / TA_BLK;
    // about 2048 waves (8 per CU) over the KV heads and row tiles, at most TA_MAXS
    // splits, none without a block (a second row tile streams the keys again: 32 rows
    // would need twice the O registers of a wave)
    const int R = T * (nHq / nKv), RT = (R + TA_ROWS - 1) / TA_ROWS;
    int NS = (2048 / TA_W + nKv * RT - 1) / (nKv * RT);
    const int need = (nb + 1 + TA_W - 1) / TA_W;
    if (NS > need) NS = need;
    if (NS > TA_MAXS) NS = TA_MAXS;
    if (NS < 1) NS = 1;
    TAttnArgs a = {q, k, v, qw, kw, rope, reinterpret_cast<uint8_t*>(kq), ks, reinterpret_cast<uint8_t*>(vq), vs,
                   c->attn_po, c->attn_ml, S0, T, nKv, nHq / nKv, NS, eps, RT, kvs};
    k_attn_tq8<<<nKv * RT * NS, 64 * TA_W, 0, c->stream>>>(a);
    TI_LAUNCHED("k_attn_tq8");
    TCombArgs cb = {c->attn_po, c->attn_ml, oq, os, NS, nKv, nHq / nKv, R, RT};
    k_attn_tcombine<<<nKv * R, HD, 0, c->stream>>>(cb);
    TI_LAUNCHED("k_attn_tcombine");
    return TI_OK;
}
