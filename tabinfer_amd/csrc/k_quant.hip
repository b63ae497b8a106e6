// k_quant.hip — quantizers of the decode path (all integer outputs bit-exact):
//  int4 weight quantizer     models/qwen3.js:3405-3426 (JS f64 semantics)
//  ternary weight format     models/qwen3.js:3435-3469
//  per-32 int8 activation    models/qwen3.js:332-358, 1210-1231
//  fused RMSNorm + int8      models/qwen3.js:569-612
//     plain RMSNorm             models/qwen3.js:60-80
// Built with -ffp-contract=off: every f32/f64 expression rounds once per
// operation in the written order, which is what makes these bit-exact.
#include "ti_dev.h"

// ---------------------------------------------------------------------------
// one thread per (row, 32-group). The reference runs this in JavaScript at
// load time, so the arithmetic is f64 (JS numbers), with its own f32->f16
// rounding (ties away from zero) and Math.round (ties toward +inf).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_to_f16_q3(float v) {
    uint32_t x = __float_as_uint(v);
    uint32_t sign = (x >> 16) & 0x8000u;
    int exp = (int)((x >> 23) & 0xffu);
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xff) return sign | (mant ? 0x7e00u : 0x7c00u);
    int e = exp - 127 + 15;
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = mant | 0x800000u;
        int shift = 14 - e;
        uint32_t half = m >> shift;
        if ((m >> (shift - 1)) & 1u) half += 1;
        return sign | half;
    }
    uint32_t half = ((uint32_t)e << 10) | (mant >> 13);
    if ((mant >> 12) & 1u) half += 1;
    return sign | half;
}

__device__ __forceinline__ double f16_exact(uint32_t h) {
    return (double)ti_h2f((uint16_t)h);
}

__global__ __launch_bounds__(256) void k_quant_int4_bf16(const uint16_t* __restrict__ w,
                                                         uint32_t* __restrict__ pack,
                                                         uint16_t* __restrict__ scales,
                                                         long ngroups) {
    long gi = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= ngroups) return;
    // a row's groups are contiguous, so group gi covers elements [32gi, 32gi+32)
    const uint4* src = reinterpret_cast<const uint4*>(w + gi * 32);
    uint32_t u[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint4 v = src[i];
        u[4 * i] = v.x; u[4 * i + 1] = v.y; u[4 * i + 2] = v.z; u[4 * i + 3] = v.w;
    }
    float f[32];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        f[2 * i] = __uint_as_float(u[i] << 16);
        f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
    double maxabs = 0.0;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        double a = fabs((double)f[j]);
        if (a > maxabs) maxabs = a;
    }
    double scale = maxabs > 0.0 ? maxabs / 7.0 : 1e-8;
    uint32_t sbits = f32_to_f16_q3((float)scale);
    scales[gi] = (uint16_t)sbits;
    double inv = 1.0 / f16_exact(sbits);          // +inf when the scale rounds to 0
    uint32_t words[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 32; j++) {
        double p = (double)f[j] * inv;
        uint32_t nib;
        if (p != p) {
            nib = 0u;                               // JS: (NaN + 8) & 0xF == 0
        } else {
            double q;
            if (isinf(p)) {
                q = p;
            } else {
                double fl = floor(p);
                q = (p - fl >= 0.5) ? fl + 1.0 : fl; // Math.round: ties toward +inf
            }
            if (q < -8.0) q = -8.0; else if (q > 7.0) q = 7.0;
            nib = (uint32_t)((int)q + 8) & 0xFu;
        }
        words[j >> 3] |= nib << (4 * (j & 7));
    }
    uint4 o; o.x = words[0]; o.y = words[1]; o.z = words[2]; o.w = words[3];
    reinterpret_cast<uint4*>(pack)[gi] = o;
}

extern "C" int ti_quant_int4_bf16(ti_ctx* c, const uint16_t* w, uint32_t* pack, uint16_t* scales, int N, int K) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(w && pack && scales, "ti_quant_int4_bf16: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "ti_quant_int4_bf16: need N>0, K>0, K%%32==0 (N=%d K=%d)", N, K);
    long ng = (long)N * (K / 32);
    long blocks = (ng + 255) / 256;
    TI_REQUIRE(blocks < (1L << 31), "ti_quant_int4_bf16: too large");
    k_quant_int4_bf16<<<(unsigned)blocks, 256, 0, c->stream>>>(w, pack, scales, ng);
    TI_LAUNCHED("k_quant_int4_bf16");
    return TI_OK;
}


// ---------------------------------------------------------------------------
// quantizeTernaryBf16 (models/qwen3.js:3435-3469), one thread per (row, 32-group): the
// group's scale is its largest bf16 magnitude (bits & 0x7FFF compared as integers), in
// f16 by the reference's f32 -> f16 rounding; code = 1 for a zero, 0 for a negative, 2
// for a positive weight, at bits 8(k&3) + 2((k>>2)&3) of word k/16. A nonzero magnitude
// more than 2 bf16 ULPs below its group's maximum means the tensor is not ternary (the
// reference's null, after which its loader quantizes to int4): *not_ternary gets 1.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quant_tern_bf16(const uint16_t* __restrict__ w, uint32_t* __restrict__ pack,
                                                         uint16_t* __restrict__ scales, uint32_t* __restrict__ not_ternary,
                                                         long ngroups) {
    const long gi = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= ngroups) return;
    const uint4* src = reinterpret_cast<const uint4*>(w + gi * 32);
    uint32_t u[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint4 v = src[i];
        u[4 * i] = v.x; u[4 * i + 1] = v.y; u[4 * i + 2] = v.z; u[4 * i + 3] = v.w;
    }
    uint32_t mx = 0;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const uint32_t m = (u[j >> 1] >> (16 * (j & 1))) & 0x7FFFu;
        mx = m > mx ? m : mx;
    }
    bool bad = false;
    uint32_t words[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const uint32_t bits = (u[j >> 1] >> (16 * (j & 1))) & 0xFFFFu, m = bits & 0x7FFFu;
        if (m != 0u && mx - m > 2u) bad = true;
        const uint32_t c = m == 0u ? 1u : ((bits & 0x8000u) ? 0u : 2u);
        words[j >> 4] |= c << (((j & 3) << 3) + ((j >> 2) & 3) * 2);
    }
    reinterpret_cast<uint2*>(pack)[gi] = make_uint2(words[0], words[1]);
    scales[gi] = (uint16_t)f32_to_f16_q3(__uint_as_float(mx << 16));
    if (bad) __hip_atomic_fetch_or(not_ternary, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

extern "C" int ti_quant_tern_bf16(ti_ctx* c, const uint16_t* w, uint32_t* pack, uint16_t* scales, int N, int K,
                                  uint32_t* not_ternary) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(w && pack && scales && not_ternary, "ti_quant_tern_bf16: null buffer");
    TI_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "ti_quant_tern_bf16: need N>0, K>0, K%%64==0 (N=%d K=%d)", N, K);
    TI_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)pack & 7) == 0, "ti_quant_tern_bf16: w 16-byte, pack 8-byte aligned");
    const long ng = (long)N * (K / 32);
    const long blocks = (ng + 255) / 256;
    TI_REQUIRE(blocks < (1L << 31), "ti_quant_tern_bf16: too large");
    k_quant_tern_bf16<<<(unsigned)blocks, 256, 0, c->stream>>>(w, pack, scales, not_ternary, ng);
    TI_LAUNCHED("k_quant_tern_bf16");
    return TI_OK;
}

__global__ __launch_bounds__(64) void k_quant_act_q8(const float* __restrict__ x, uint32_t* __restrict__ xq,
                                                     float* __restrict__ xs, int32_t* __restrict__ xsum, int ng) {
    int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= ng) return;
    float v[32];
    load32(x + (size_t)g * 32, v);
    q8_group(v, xq + (size_t)g * 8, xs + g, xsum ? xsum + (size_t)g * 2 : nullptr);
}

int ti_quant_act_q8_async(ti_ctx* c, const float* x, uint32_t* xq, float* xs, int32_t* xsum, int groups) {
    k_quant_act_q8<<<(groups + 63) / 64, 64, 0, c->stream>>>(x, xq, xs, xsum, groups);
    TI_LAUNCHED("k_quant_act_q8");
    return TI_OK;
}

extern "C" int ti_quant_act_q8(ti_ctx* c, const float* x, uint32_t* xq, float* xs, int32_t* xsum, int K) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && xq && xs, "ti_quant_act_q8: null buffer");
    TI_REQUIRE(K > 0 && K % 32 == 0, "ti_quant_act_q8: K must be a positive multiple of 32 (K=%d)", K);
    return ti_quant_act_q8_async(c, x, xq, xs, xsum, K / 32);
}

extern "C" int ti_quant_act_q8_t(ti_ctx* c, const float* x, uint32_t* xq, float* xs, int T, int K) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && xq && xs, "ti_quant_act_q8_t: null buffer");
    TI_REQUIRE(T > 0 && K > 0 && K % 32 == 0, "ti_quant_act_q8_t: need T>0 and K%%32==0 (T=%d K=%d)", T, K);
    long ng = (long)T * (K / 32);
    TI_REQUIRE(ng < (1L << 30), "ti_quant_act_q8_t: too large");
    return ti_quant_act_q8_async(c, x, xq, xs, nullptr, (int)ng);
}


__global__ __launch_bounds__(256) void k_rmsnorm_q8(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                    uint32_t* __restrict__ xq, float* __restrict__ xs,
                                                    int32_t* __restrict__ xsum, int H, float eps) {
    __shared__ float red[256];
    float inv = rms_inv_256(x, H, eps, red);
    int ng = H / 32;
    for (int g = threadIdx.x; g < ng; g += 256) {
        float v[32];
        load32(x + (size_t)g * 32, v);
#pragma unroll
        for (int j = 0; j < 32; j++) {
            float a = v[j] * inv;
            v[j] = a * ti_h2f(w[g * 32 + j]);
        }
        q8_group(v, xq + (size_t)g * 8, xs + g, xsum ? xsum + (size_t)g * 2 : nullptr);
    }
}

extern "C" int ti_rmsnorm_q8(ti_ctx* c, const float* x, const uint16_t* w, uint32_t* xq, float* xs,
                             int32_t* xsum, int H, float eps) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && w && xq && xs, "ti_rmsnorm_q8: null buffer");
    TI_REQUIRE(H > 0 && H % 32 == 0, "ti_rmsnorm_q8: H must be a positive multiple of 32 (H=%d)", H);
    k_rmsnorm_q8<<<1, 256, 0, c->stream>>>(x, w, xq, xs, xsum, H, eps);
    TI_LAUNCHED("k_rmsnorm_q8");
    return TI_OK;
}

__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                 float* __restrict__ y, int H, float eps) {
    __shared__ float red[256];
    const float* xr = x + (size_t)blockIdx.x * H;
    float inv = rms_inv_256(xr, H, eps, red);
    float* yr = y + (size_t)blockIdx.x * H;
    for (int i = threadIdx.x; i < H; i += 256) { float a = xr[i] * inv; yr[i] = a * ti_h2f(w[i]); }
}

extern "C" int ti_rmsnorm(ti_ctx* c, const float* x, const uint16_t* w, float* y, int T, int H, float eps) {
    TI_CHECK_CTX(c);
    TI_REQUIRE(x && w && y, "ti_rmsnorm: null buffer");
    TI_REQUIRE(T > 0 && H > 0, "ti_rmsnorm: need T>0, H>0");
    k_rmsnorm<<<T, 256, 0, c->stream>>>(x, w, y, H, eps);
    TI_LAUNCHED("k_rmsnorm");
    return TI_OK;
}
