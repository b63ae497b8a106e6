// ti_internal.h — shared host/device helpers for libtabinfer (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include "ti_host.h"

// ---- host-side error plumbing (ti_fail, TI_REQUIRE: ti_host.h) -----------------
int ti_hip_fail(hipError_t e, const char* what);

#define TI_HIP(call) do { hipError_t _e = (call); if (_e != hipSuccess) return ti_hip_fail(_e, #call); } while (0)
#define TI_LAUNCHED(name) do { hipError_t _e = hipGetLastError(); if (_e != hipSuccess) return ti_hip_fail(_e, name); } while (0)

struct ti_ctx {
    int device;
    int cus;              // compute units of the device
    int qkv_separate;     // TI_DECODE_QKV_SEPARATE set at ti_init: the decode step's q/k/v GEMV
                          // and attention as two launches (same results; for A/B checks)
    int qkv_polls;        // rounds a wave polls for its q/k/v rows before computing them itself
                          // (TI_DECODE_QKV_POLLS at ti_init; 0 takes that path at once, for tests)
    hipStream_t stream;
    hipEvent_t ev[64];
    int capturing;
    // persistent scratch (allocated at init, never reallocated, so calls may be
    // captured into graphs): int8 activation for the linearQ router, split-KV
    // partials, argmax partials.
    uint32_t* act_q;      // [TI_ACT_CAP/4 * TI_ACT_TMAX]
    float* act_s;         // [TI_ACT_CAP/32 * TI_ACT_TMAX]
    int32_t* act_sum;     // [TI_ACT_CAP/16]
    float* attn_po;       // split-KV partial outputs
    float* attn_ml;       // split-KV (m, l)
    float* amax_v;        // argmax partial values
    uint32_t* amax_i;     // argmax partial indices
    uint32_t* moe_cnt;    // MoE counting sort: counts / offsets / fill / sorted index
    uint32_t* moe_off;
    uint32_t* moe_fill;
    uint32_t* moe_sidx;
    float* tg_part;       // split-K halves of the T-token projections ([TI_TG_SPLIT_BLOCKS][2][256])
    uint64_t* qkv_pub;    // q/k/v rows handed between the workgroups of a decode attention
                          // launch that computes them (value | epoch << 32; TI_QKV_PUB_WORDS)
    // device-scope counters of "last workgroup finishes the reduction" kernels;
    // zero between launches (each kernel's last workgroup resets its own)
    uint32_t* sync;
};

struct ti_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
    int device;
};

// Scratch capacities (elements). Activation rows up to 65536 wide, up to 256
// tokens for the batched path; split-KV partials for (query rows x splits) <= 512 x 512.
#define TI_ACT_CAP 65536
#define TI_ACT_TMAX 256
#define TI_ATTN_HEADS_MAX 64
#define TI_ATTN_ROWS_MAX 4096     // T * nHq of one attention call (a 256-token prefill of 16 heads)
#define TI_ATTN_SPLITS_MAX 512
#define TI_ATTN_ROWSPLITS (512 * 512)   // (T * nHq) x splits of one call: the partials' capacity
#define TI_ATTN_HD_MAX 128
#define TI_AMAX_PARTS 1024
#define TI_MOE_P_MAX 8192
#define TI_MOE_E_MAX 256
#define TI_SYNC_WORDS (TI_SYNC_ATTN + TI_ATTN_COUNTERS * TI_SYNC_ATTN_STRIDE)
#define TI_SYNC_LMHEAD 0          // lm_head argmax
#define TI_SYNC_BONSAI 1          // Bonsai attention merge: the head workgroups' arrivals
#define TI_SYNC_ATTN 1024         // fused attention: one counter per KV head (up to 64), each on its
#define TI_SYNC_ATTN_STRIDE 64    //   own 256-byte line (atomics on one line serialise at the memory side)
#define TI_ATTN_COUNTERS 64
#define TI_SYNC_TGEMM 512         // split-K T-token projections: one counter per 16-row block
#define TI_TG_SPLIT_BLOCKS 128    // (blocks of one split-K launch, at most)
#define TI_SYNC_DUMMY 256         // 256 words never written: a valid read target for unused inputs
#define TI_SYNC_ATTN_EPOCH 1      // word of a KV head's counter line: the epoch of its q/k/v hand-off
#define TI_QKV_PUB_WORDS 16384    // KV heads x (query heads per KV head + 2) x head_dim, at most

// ---- the T-token forward (2 <= T <= 16) ---------------------------------------------
// Input of a T-token projection: int8 codes (xq [T][K/4], xs [T][K/32]) or, with x set,
// the f32 activation x [T][K] that the kernel RMS-normalises (weight nw, eps) and
// quantises itself, from its partial sums pin [T][256] (p[t][u] = sum over i of
// x[t][u + 256 i]^2: what a residual projection's epilogue or ti_tsumsq_launch writes).
struct TgIn {
    const uint32_t* xq;
    const float* xs;
    const float* x;
    const uint16_t* nw;
    float eps;
    const float* pin;
};
// The residual add + RMSNorm + n2 quantizer run in the prologue of the ternary projections
// that consume it (k_tern.hip): x_out = x + add * (1 / *add_scale) (x alone without add),
// xn_out = x_out * (1 / sqrt(mean(x_out^2) + eps)) * w, codes act_out (127 / amax, rounded
// half away from zero), 64-block sums xsum_out, the quantizer's 127 / amax in *scale_out.
// x_out must not alias x: other workgroups of the launch still read x. Without w the
// prologue is the quantizer of x alone (no add; x_out, xn_out may be null).
struct ti_tern_norm {
    const float* x;
    const float* add;
    const float* add_scale;
    const float* w;
    float eps;
    float* x_out;
    float* xn_out;
    int8_t* act_out;
    int32_t* xsum_out;
    float* scale_out;
};
// The SwiGLU of the scaled gate/up and its n2 quantizer in the down projection's prologue:
// swi = silu(g / *gu_scale) * (u / *gu_scale), codes, block sums, scale as above.
struct ti_tern_swiglu {
    const float* g;
    const float* u;
    const float* gu_scale;
    float* swi_out;
    int8_t* act_out;
    int32_t* xsum_out;
    float* scale_out;
};
bool ti_tern_swiglu_ok(int K);
int ti_tern_gemv_swiglu(ti_ctx* c, const ti_tern_swiglu* sw, float* out, const uint8_t* codes, const float* scales, int N,
                        int K);
bool ti_tern_norm_ok(int K);
int ti_tern_gemv_multi_norm(ti_ctx* c, const ti_tern_norm* nq, int K, int nmat, const uint8_t* const* codes,
                            const float* const* scales, float* const* outs, const int* Ns);
bool ti_tgemm_ok(int T, int K);
bool ti_tgemm_norm_ok(int T, int K);
bool ti_tnorm_ok(int K);
bool ti_tgemm_gateup_ok(int T, int H);
int ti_tnorm_q8_launch(ti_ctx* c, const float* x, const uint16_t* nw, float eps, uint32_t* xq, float* xs, int T, int K);
int ti_tsumsq_launch(ti_ctx* c, const float* x, float* p, int T, int K);
int ti_tgemm_launch(ti_ctx* c, const TgIn& in, int nseg, const uint32_t* const* packs, const uint16_t* const* scs,
                    float* const* ys, const int* Ns, int T, int K, int acc, float* pout);
int ti_tgemm_gateup_launch(ti_ctx* c, const TgIn& in, const uint32_t* gpack, const uint16_t* gsc, const uint32_t* upack,
                           const uint16_t* usc, int I, int H, int T, uint32_t* swq, float* sws);
bool ti_tattn_ok(int T, int nHq, int nKv, int hd);
int ti_tattn_launch(ti_ctx* c, const float* q, const float* k, const float* v, const uint16_t* qw, const uint16_t* kw,
                    const float* rope, uint32_t* kq, float* ks, uint32_t* vq, float* vs, int S0, int T, int nHq, int nKv,
                    int hd, float eps, uint32_t* oq, float* os, int kvs);

// ---- device helpers -----------------------------------------------------------
// f16 bits -> f32 (exact).
__device__ __forceinline__ float ti_h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// Non-temporal 16-byte load (streamed data: weights, KV) — global_load_dwordx4 ... nt.
typedef unsigned int ti_v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ti_ld_nt(const uint4* p) {
    ti_v4u v = __builtin_nontemporal_load(reinterpret_cast<const ti_v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 8 int8 codes (two words, byte e = element e) -> 8 f16 values, exactly: the biased byte
// (code + 128) under an 0x64 high byte is the f16 1024 + code + 128 (one v_perm_b32 per
// two codes; selector bytes 0-3 pick the second operand's bytes, 4-7 the first's), and a
// packed f16 subtraction removes the 1152.
typedef _Float16 ti_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 ti_h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void ti_i8x4_h2x2(uint32_t w, ti_h2& a, ti_h2& b) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);   // [u0, 64, u1, 64]
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);   // [u2, 64, u3, 64]
    const ti_h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    a = __builtin_bit_cast(ti_h2, p0) - bias;
    b = __builtin_bit_cast(ti_h2, p1) - bias;
}
__device__ __forceinline__ ti_h8 ti_i8x8_h8(uint32_t lo, uint32_t hi) {
    ti_h2 a, b, c, d;
    ti_i8x4_h2x2(lo, a, b);
    ti_i8x4_h2x2(hi, c, d);
    const uint4 w = make_uint4(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                               __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d));
    return __builtin_bit_cast(ti_h8, w);
}

// Keep every memory operation issued so far above this point: the scheduler may
// otherwise sink a kernel's weight loads below the wait for its activation loads,
// which serialises two memory round trips that were meant to overlap.
#define TI_ISSUE_FENCE() __builtin_amdgcn_sched_barrier(0)
// cache policy of a buffer load/store (gfx950): sc1 = agent scope, as the agent-scope
// atomic loads and stores of the hand-offs (the access misses the non-coherent caches)
#define TI_CPOL_SC1 16

// ---- lane exchange as VALU operations ------------------------------------------------
// ti_xor(v, o): the value held by lane (lane ^ o), o in {1, 2, 4, 8, 16, 32}, without
// an LDS round trip (__shfl_xor lowers to ds_bpermute, ~100+ cycles each, and a chain
// of them serialises a reduction). DPP within a 16-lane row: quad_perm for 1 and 2,
// row_shl/row_shr:4 picked by lane bit 2, row_ror:8; across rows the gfx950 permlane
// swaps: permlane16_swap(v, v) yields {rows 0,0,2,2 ; rows 1,1,3,3} and
// permlane32_swap(v, v) yields {halves 0,0 ; halves 1,1} (lane layouts checked on
// the device). `o` must be a compile-time constant after unrolling.
__device__ __forceinline__ int ti_xor_i(int v, int o) {
    const int lane = threadIdx.x & 63;
    switch (o) {
        case 1: return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);
        case 2: return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);
        case 4: {
            const int up = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xF, 0xF, false);   // lane + 4
            const int dn = __builtin_amdgcn_update_dpp(v, v, 0x114, 0xF, 0xF, false);   // lane - 4
            return (lane & 4) ? dn : up;
        }
        case 8: return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xF, 0xF, false);
        case 16: {
            const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
            return (lane & 16) ? (int)r[0] : (int)r[1];
        }
        default: {
            const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
            return (lane & 32) ? (int)r[0] : (int)r[1];
        }
    }
}
__device__ __forceinline__ float ti_xor(float v, int o) {
    return __builtin_bit_cast(float, ti_xor_i(__builtin_bit_cast(int, v), o));
}
__device__ __forceinline__ uint32_t ti_xor(uint32_t v, int o) { return (uint32_t)ti_xor_i((int)v, o); }
__device__ __forceinline__ int ti_xor(int v, int o) { return ti_xor_i(v, o); }

// Whole-wave butterflies with the offsets spelled out (32, 16, 8, 4, 2, 1). A loop over the
// offset is not always unrolled (inside an unrolled outer loop the compiler may keep it),
// and ti_xor of a run-time offset is a chain of branches: these stay straight-line.
__device__ __forceinline__ int ti_wave_sum_i(int v) {
    v += ti_xor_i(v, 32); v += ti_xor_i(v, 16); v += ti_xor_i(v, 8);
    v += ti_xor_i(v, 4); v += ti_xor_i(v, 2); v += ti_xor_i(v, 1);
    return v;
}
__device__ __forceinline__ float ti_wave_sum(float v) {
    v += ti_xor(v, 32); v += ti_xor(v, 16); v += ti_xor(v, 8);
    v += ti_xor(v, 4); v += ti_xor(v, 2); v += ti_xor(v, 1);
    return v;
}
__device__ __forceinline__ float ti_wave_max(float v) {
    v = fmaxf(v, ti_xor(v, 32)); v = fmaxf(v, ti_xor(v, 16)); v = fmaxf(v, ti_xor(v, 8));
    v = fmaxf(v, ti_xor(v, 4)); v = fmaxf(v, ti_xor(v, 2)); v = fmaxf(v, ti_xor(v, 1));
    return v;
}

// Wavefront-64 butterfly sum over lanes that share the same (lane / width): pairs at
// distance width/2 first, down to 1 (every lane of a segment ends with the same sum).
template <int WIDTH>
__device__ __forceinline__ float ti_seg_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += ti_xor(v, o);
    return v;
}

// Maximum of a non-negative float over each aligned group of 32 lanes, returned in
// every lane. Max is exact in any order, so the pairing may differ from xor: after
// quads agree, row_half_mirror and row_mirror pair each lane with the other half of
// its 8- and 16-lane block. Compared as unsigned bit patterns (valid for x >= 0).
__device__ __forceinline__ float ti_max32_nonneg(float x) {
    uint32_t m = __builtin_bit_cast(uint32_t, x);
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0xB1, 0xF, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x4E, 0xF, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x141, 0xF, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x140, 0xF, 0xF, false));
    const auto r = __builtin_amdgcn_permlane16_swap((int)m, (int)m, false, false);
    m = max((uint32_t)r[0], (uint32_t)r[1]);
    return __builtin_bit_cast(float, m);
}

// OR of a word over each aligned quad of lanes, in every lane of the quad (packs four
// lanes' bytes into one word).
__device__ __forceinline__ uint32_t ti_quad_or(uint32_t v) {
    v |= (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false);
    v |= (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false);
    return v;
}

// Total of one float per thread over a 256-thread workgroup, in the association of
// the tree `for st = 128..1: red[t] += red[t + st]` (rmsnormQ's order), returned in
// every thread with one barrier: levels 128 and 64 combine the four waves' partials
// read back from LDS, levels 32..1 are an exact xor butterfly (lane t < st adds lane
// t + st, as the tree does; the partner lane computes the same sum). `red` holds 256
// floats and must not be reused before the caller's next barrier.
__device__ __forceinline__ float ti_tree_sum_256(float s, float* red) {
    const int t = threadIdx.x, l = t & 63;
    red[t] = s;
    __syncthreads();
    const float a = red[l] + red[l + 128];
    const float b = red[l + 64] + red[l + 192];
    float v = a + b;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = v + ti_xor(v, o);
    return v;
}

// snorm int8 of the KV cache (pack4x8snorm): code = floor(0.5 + 127*clamp(x/mx, -1, 1)),
// evaluated exactly (double) on the f32 quotient; mx = max(1e-12, max|x|) of the 32-group.
__device__ __forceinline__ uint32_t snorm_code(float x, float mx) {
    float e = x / mx;
    e = e > 1.0f ? 1.0f : (e < -1.0f ? -1.0f : e);
    return (uint32_t)((int)floor(0.5 + 127.0 * (double)e) & 0xff);
}

// ---- argmax tie order of the reference (models/qwen3.js:2624-2690) ----------------------
// The reference's argmax keeps, per thread, the first strict maximum of a strided scan and
// then folds the threads' slots in a shared-memory tree where slot l takes slot l+s only if
// strictly greater (s = n/2 .. 1). Among equal maxima that tree favours the slot whose
// number, read with its bits reversed, is smallest (slot 0 beats 1 at the last level, 0
// beats 2 one level up, ...). Index i of an N-logit argmax therefore ranks as
//   N >= 16384 (64 workgroups x 256 threads, then 64 partials):
//       (bitrev6(workgroup (i >> 8) & 63), bitrev8(thread i & 255), i >> 14)
//   N <  16384 (one workgroup of 256 threads): (bitrev8(thread i & 255), i >> 8)
// and the smaller rank wins a tie. Only logits above -3e38 are candidates (NaN never is);
// with none the answer is index 0. Merging (value, index) pairs with ti_amx_take is
// associative and commutative, so any reduction order gives the reference's index.
__device__ __forceinline__ uint32_t ti_amx_rank(uint32_t i, int N) {
    if (N >= 16384)
        return ((__builtin_bitreverse32((i >> 8) & 63u) >> 26) << 26) | ((__builtin_bitreverse32(i & 255u) >> 24) << 18) |
               (i >> 14);
    return ((__builtin_bitreverse32(i & 255u) >> 24) << 6) | (i >> 8);
}
// keep (v, i) or take (v2, i2); start from (-3e38, any index)
__device__ __forceinline__ void ti_amx_take(float& v, int& i, float v2, int i2, int N) {
    if (v2 > v || (v2 == v && v > -3.0e38f && ti_amx_rank((uint32_t)i2, N) < ti_amx_rank((uint32_t)i, N))) {
        v = v2;
        i = i2;
    }
}
// the answer of a finished reduction
__device__ __forceinline__ int ti_amx_result(float v, int i) { return v > -3.0e38f ? i : 0; }

// ---- Gumbel-max temperature sampling (models/qwen3.js:2713-2740) -------------------
// argmax(logit + T g), g = -log(-log(u)), is a sample of softmax(logits / T). u comes from
// the PCG hash (the 32-bit pcg_hash of Jarzynski and Olano, "Hash Functions for GPU
// Rendering", 2020) of the index mixed with the step's seed: 24 bits plus one half,
// over 2^24, so u is in (0, 1) and exact in f32. The seed stream advances by the LCG
// s' = 1664525 s + 1013904223 (mod 2^32) once per sampled step, before use.
__host__ __device__ __forceinline__ uint32_t ti_pcg(uint32_t v) {
    const uint32_t s = v * 747796405u + 2891336453u;
    const uint32_t w = ((s >> ((s >> 28u) + 4u)) ^ s) * 277803737u;
    return (w >> 22u) ^ w;
}
__host__ __device__ __forceinline__ uint32_t ti_seed_next(uint32_t s) { return s * 1664525u + 1013904223u; }
__device__ __forceinline__ float ti_gumbel(uint32_t i, uint32_t seed) {
    const uint32_t h = ti_pcg(i ^ (seed * 2654435761u));
    const float u = ((float)(h >> 8u) + 0.5f) / 16777216.0f;
    return -logf(-logf(u));
}
// the sampling words a decoder keeps on the device: [0] temperature (f32; <= 0: greedy),
// [1] the seed stream's state (the last seed used)
#define TI_SAMP_TEMP 0
#define TI_SAMP_STATE 1
#define TI_SEED_INIT 0x9E3779B9u

// ---- cross-workgroup hand-off without cache maintenance ----------------------------
// The "last workgroup finishes the reduction" kernels publish a few words per
// workgroup. A device-scope fence on gfx950 writes back and invalidates the whole
// XCD L2 (buffer_wbl2/buffer_inv), which costs microseconds when every workgroup
// does it; instead the published words are written and read with device-scope
// atomic stores/loads (sc1: they bypass the non-coherent XCD L2), and the writer
// waits for its stores to be acknowledged (vmcnt(0)) before bumping the counter.
__device__ __forceinline__ void ti_pub_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ti_pub_store(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ti_pub_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ti_pub_load(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 8-byte words (a value and the epoch it belongs to) as one naturally aligned access each
__device__ __forceinline__ void ti_pub_store(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ti_pub_load(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// all of this thread's prior memory operations acknowledged (gfx9 encoding of
// s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15))
__device__ __forceinline__ void ti_stores_done() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// bump a completion counter; returns the previous count
__device__ __forceinline__ uint32_t ti_arrive(uint32_t* counter) {
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
