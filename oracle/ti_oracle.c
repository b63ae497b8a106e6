/*
 * ti_oracle.c — CPU restatement of the reference's arithmetic for the quantized
 * decode hot path. TEST INFRASTRUCTURE ONLY: the checker for tests/, smoke() and
 * bench.py's cpu_baseline leg; nothing in the product library uses it.
 *
 * Built with gcc -O2 -ffp-contract=off on x86-64 (SSE arithmetic, IEEE single
 * with round-to-nearest-even, no fused multiply-add), so every f32 expression
 * below rounds exactly once per operation, in the written order.
 *
 * Every function names the reference file:line it follows (paths relative to
 * the reference repository root).
 */
#include "ti_oracle.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------- */
/* f16 conversions                                                           */
/* ------------------------------------------------------------------------- */

/* models/qwen3.js:3357-3374 (identical: models/lfm25.js:448). Normal numbers
 * round half away from zero by adding 1 when mantissa bit 12 is set; the +1
 * carries into the exponent. Subnormals shift the implicit-one mantissa. */
uint16_t or_f32_to_f16_q3(float v) {
    uint32_t x = f2u(v);
    uint32_t sign = (x >> 16) & 0x8000u;
    int exp = (int)((x >> 23) & 0xffu);
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | (mant ? 0x7e00u : 0x7c00u));
    int e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = mant | 0x800000u;
        int shift = 14 - e;
        uint32_t half = m >> shift;
        if ((m >> (shift - 1)) & 1u) half += 1;
        return (uint16_t)(sign | half);
    }
    uint32_t half = ((uint32_t)e << 10) | (mant >> 13);
    if ((mant >> 12) & 1u) half += 1;
    return (uint16_t)(sign | half);
}

/* engine/webgpu-engine.js:217-236. Rounds by adding 0x1000 before the shift and
 * ORs the mantissa into (e<<10): a mantissa carry (value 0x400) is OR-ed, not
 * added, so for odd e the carry is lost. Restated as written. */
uint16_t or_f32_to_f16_eng(float v) {
    uint32_t x = f2u(v);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x007fffffu;
    int exp = (int)((x >> 23) & 0xffu);
    if (exp == 255) return (uint16_t)(sign | (mant ? 0x7e00u : 0x7c00u));
    int e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant = (mant | 0x00800000u) >> (1 - e);
        return (uint16_t)(sign | ((mant + 0x00001000u) >> 13));
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | ((mant + 0x00001000u) >> 13));
}

/* models/qwen3.js:3397-3400: exact value of an f16 bit pattern. */
double or_f16_to_f32(uint16_t h) {
    int s = (h & 0x8000) >> 15, e = (h & 0x7c00) >> 10, f = h & 0x03ff;
    double sg = s ? -1.0 : 1.0;
    if (e == 0) return sg * ldexp((double)f / 1024.0, -14);
    if (e == 31) return f ? NAN : sg * INFINITY;
    return sg * ldexp(1.0 + (double)f / 1024.0, e - 15);
}

/* models/qwen3.js:3409: bf16 bits -> f32 by u16 << 16. */
float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* JS Math.round: nearest integer, ties toward +infinity; NaN/Inf pass through. */
static double js_round(double x) {
    if (!isfinite(x)) return x;
    double f = floor(x);
    return (x - f >= 0.5) ? f + 1.0 : f;
}
/* JS ToInt32 (for the `(q + 8) & 0xF` of a possibly-NaN q). */
static int32_t js_toint32(double x) {
    if (!isfinite(x)) return 0;
    double t = trunc(x);
    double m = fmod(t, 4294967296.0);
    if (m < 0) m += 4294967296.0;
    uint32_t u = (uint32_t)m;
    return (int32_t)u;
}

/* ------------------------------------------------------------------------- */
/* int4 group quantizer, models/qwen3.js:3405-3426 (= lfm25.js:454-477)  */
/* ------------------------------------------------------------------------- */
void or_quant_int4_bf16(const uint16_t* w, int N, int K, uint32_t* pack, uint16_t* scales) {
    const int G = 32, wpr = K / 8, gpr = K / G;
    memset(pack, 0, (size_t)N * wpr * 4);
    for (int n = 0; n < N; n++) {
        const uint16_t* row = w + (size_t)n * K;
        for (int g = 0; g < gpr; g++) {
            double maxabs = 0;                      /* JS number; values are f32 */
            for (int j = 0; j < G; j++) {
                double v = fabs((double)or_bf16_to_f32(row[g * G + j]));
                if (v > maxabs) maxabs = v;         /* NaN never wins `>` */
            }
            double scale = maxabs > 0 ? maxabs / 7.0 : 1e-8;
            /* f32ToF16 stores into a Float32Array first: RNE f64 -> f32 */
            uint16_t sBits = or_f32_to_f16_q3((float)scale);
            scales[(size_t)n * gpr + g] = sBits;
            double inv = 1.0 / or_f16_to_f32(sBits);  /* +Inf when sBits == 0 */
            for (int j = 0; j < G; j++) {
                int k = g * G + j;
                double q = js_round((double)or_bf16_to_f32(row[k]) * inv);
                if (q < -8) q = -8; else if (q > 7) q = 7;   /* NaN passes both */
                uint32_t nib = (uint32_t)js_toint32(q + 8) & 0xFu;
                pack[(size_t)n * wpr + (k >> 3)] |= nib << (4 * (k & 7));
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* per-32 int8 activation quant, models/qwen3.js:332-358                  */
/* scale = absmax/127 (f32), inv = 1/scale (0 if scale == 0),                */
/* q = clamp(round_even(v*inv), -127, 127); xsum per 16.                      */
/* ------------------------------------------------------------------------- */
static void q8_group(const float* v, uint32_t* xq, float* xs, int32_t* xsum16) {
    float mx = 0.0f;
    for (int j = 0; j < 32; j++) { float a = fabsf(v[j]); if (a > mx) mx = a; }
    float scale = mx / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    *xs = scale;
    int q[32];
    for (int j = 0; j < 32; j++) {
        float p = v[j] * inv;
        int qi = (int)rintf(p);
        if (qi < -127) qi = -127; if (qi > 127) qi = 127;
        q[j] = qi;
    }
    for (int w = 0; w < 8; w++) {
        uint32_t word = 0;
        for (int b = 0; b < 4; b++) word |= ((uint32_t)(q[w * 4 + b] & 0xff)) << (8 * b);
        xq[w] = word;
    }
    if (xsum16) {
        int32_t a = 0, b = 0;
        for (int j = 0; j < 16; j++) a += q[j];
        for (int j = 16; j < 32; j++) b += q[j];
        xsum16[0] = a; xsum16[1] = b;
    }
}

void or_quant_act_q8(const float* x, int K, uint32_t* xq, float* xs, int32_t* xsum) {
    for (int g = 0; g < K / 32; g++)
        q8_group(x + g * 32, xq + g * 8, xs + g, xsum ? xsum + g * 2 : NULL);
}

/* models/qwen3.js:1210-1231: the same per (token, group). */
void or_quant_act_q8_t(const float* x, int T, int K, uint32_t* xq, float* xs) {
    for (int t = 0; t < T; t++)
        or_quant_act_q8(x + (size_t)t * K, K, xq + (size_t)t * (K / 4), xs + (size_t)t * (K / 32), NULL);
}

/* ------------------------------------------------------------------------- */
/* fused RMSNorm + int8 quant, models/qwen3.js:569-612                    */
/* sum of squares: 256 strided per-thread partials (s = s + v*v, two          */
/* roundings), then the 128..1 tree; inv = 1/sqrt(sum/H + eps) with IEEE     */
/* sqrt and division (the browser's inverseSqrt is only specified to 2 ULP;  */
/* this build pins the correctly rounded form). v = (x*inv)*w.               */
/* ------------------------------------------------------------------------- */
static float rms_inv_256(const float* x, int H, float eps) {
    float red[256];
    for (int t = 0; t < 256; t++) {
        float s = 0.0f;
        for (int i = t; i < H; i += 256) { float sq = x[i] * x[i]; s = s + sq; }
        red[t] = s;
    }
    for (int st = 128; st > 0; st >>= 1)
        for (int t = 0; t < st; t++) red[t] = red[t] + red[t + st];
    float m = red[0] / (float)H;
    m = m + eps;
    return 1.0f / sqrtf(m);
}

void or_rmsnorm_q8(const float* x, const uint16_t* w, int H, float eps,
                   uint32_t* xq, float* xs, int32_t* xsum) {
    float inv = rms_inv_256(x, H, eps);
    float v[32];
    for (int g = 0; g < H / 32; g++) {
        for (int j = 0; j < 32; j++) {
            int i = g * 32 + j;
            float t = x[i] * inv;
            v[j] = t * (float)or_f16_to_f32(w[i]);
        }
        q8_group(v, xq + g * 8, xs + g, xsum + g * 2);
    }
}

/* models/qwen3.js:60-80: one 256-thread workgroup per row, same reduction. */
void or_rmsnorm(const float* x, const uint16_t* w, int T, int H, float eps, float* y) {
    for (int t = 0; t < T; t++) {
        const float* xr = x + (size_t)t * H;
        float inv = rms_inv_256(xr, H, eps);
        for (int i = 0; i < H; i++) { float a = xr[i] * inv; y[(size_t)t * H + i] = a * (float)or_f16_to_f32(w[i]); }
    }
}

/* ------------------------------------------------------------------------- */
/* GEMV oracles in f64 from the quantized operands                  */
/* ------------------------------------------------------------------------- */
static inline int nib_at(const uint32_t* rowp, int k) { return (int)((rowp[k >> 3] >> (4 * (k & 7))) & 0xFu) - 8; }
static inline int i8_at(const uint32_t* xq, int k) { return (int)(int8_t)((xq[k >> 2] >> (8 * (k & 3))) & 0xFFu); }

void or_group_dots_q4_q8(const uint32_t* xq, const uint32_t* pack, int N, int K, int32_t* dots) {
    int gpr = K / 32, wpr = K / 8;
    for (int n = 0; n < N; n++) {
        const uint32_t* rp = pack + (size_t)n * wpr;
        for (int g = 0; g < gpr; g++) {
            int32_t d = 0;
            for (int j = 0; j < 32; j++) { int k = g * 32 + j; d += nib_at(rp, k) * i8_at(xq, k); }
            dots[(size_t)n * gpr + g] = d;
        }
    }
}

/* models/qwen3.js:359-400: y[n] = sum_g f16(s_w)*s_x[g]*dot_g */
void or_gemv_q4_q8(const uint32_t* xq, const float* xs, const uint32_t* pack,
                   const uint16_t* scales, int N, int K, double* y) {
    int gpr = K / 32, wpr = K / 8;
    for (int n = 0; n < N; n++) {
        const uint32_t* rp = pack + (size_t)n * wpr;
        double acc = 0;
        for (int g = 0; g < gpr; g++) {
            long d = 0;
            for (int j = 0; j < 32; j++) { int k = g * 32 + j; d += nib_at(rp, k) * i8_at(xq, k); }
            acc += or_f16_to_f32(scales[(size_t)n * gpr + g]) * (double)xs[g] * (double)d;
        }
        y[n] = acc;
    }
}

/* quantizeTernaryBf16 (models/qwen3.js:3435-3469), literally: a pre-check of the first
 * rows (an early exit only: the full pass applies the same test), then per 32-group the
 * largest magnitude (bf16 bits & 0x7FFF as integers) is the scale (bf16 -> f16 through
 * the f32 -> f16 rounding of :3357-3374), each weight's code is 1 for a zero magnitude,
 * else 0 for a set sign bit and 2 otherwise, at bits 8(k&3) + 2((k>>2)&3) of word k/16;
 * any nonzero magnitude more than TOL = 2 below its group's maximum returns 0. */
int or_quant_tern_bf16(const uint16_t* u16, int N, int K, uint32_t* pack, uint16_t* scales) {
    const int G = 32, TOL = 2;
    if (K % 64 != 0) return 0;
    const int wpr = K / 16, gpr = K / G;
    const int pre = N < 4 ? N : 4;
    for (int n = 0; n < pre; n++)
        for (int g = 0; g < gpr; g++) {
            int mx = 0;
            for (int j = 0; j < G; j++) { int m = u16[(size_t)n * K + g * G + j] & 0x7FFF; if (m > mx) mx = m; }
            for (int j = 0; j < G; j++) { int m = u16[(size_t)n * K + g * G + j] & 0x7FFF; if (m != 0 && mx - m > TOL) return 0; }
        }
    memset(pack, 0, (size_t)N * wpr * 4);
    for (int n = 0; n < N; n++) {
        const uint16_t* rU = u16 + (size_t)n * K;
        uint32_t* rP = pack + (size_t)n * wpr;
        for (int g = 0; g < gpr; g++) {
            int mx = 0;
            for (int j = 0; j < G; j++) { int m = rU[g * G + j] & 0x7FFF; if (m > mx) mx = m; }
            uint32_t fb = (uint32_t)mx << 16;
            float f;
            memcpy(&f, &fb, 4);
            scales[(size_t)n * gpr + g] = or_f32_to_f16_q3(f);
            for (int j = 0; j < G; j++) {
                int k = g * G + j, bits = rU[k], m = bits & 0x7FFF;
                if (m != 0 && mx - m > TOL) return 0;
                uint32_t c = m == 0 ? 1u : ((bits & 0x8000) ? 0u : 2u);
                rP[k >> 4] |= c << (((k & 3) << 3) + ((k >> 2) & 3) * 2);
            }
        }
    }
    return 1;
}

/* the code of weight k in a row of the ternary format, minus 1: the weight's sign */
static int tern2_w(const uint32_t* rp, int k) {
    return (int)((rp[k >> 4] >> (((k & 3) << 3) + ((k >> 2) & 3) * 2)) & 3u) - 1;
}

/* gemvTern2 (models/qwen3.js:449-503): y[n] = sum_g f16(s[n,g]) * xs[g] * (sum_j w x) over
 * 32-groups; the group sum is the reference's sum c x - sum x, exact. */
void or_gemv_tern2(const uint32_t* xq, const float* xs, const uint32_t* pack, const uint16_t* scales,
                   int N, int K, double* y) {
    const int gpr = K / 32, wpr = K / 16;
    for (int n = 0; n < N; n++) {
        const uint32_t* rp = pack + (size_t)n * wpr;
        double acc = 0;
        for (int g = 0; g < gpr; g++) {
            long d = 0;
            for (int j = 0; j < 32; j++) { int k = g * 32 + j; d += tern2_w(rp, k) * i8_at(xq, k); }
            acc += or_f16_to_f32(scales[(size_t)n * gpr + g]) * (double)xs[g] * (double)d;
        }
        y[n] = acc;
    }
}

/* gateupTern2 (models/qwen3.js:747-810): swi = silu(g) * u */
void or_gateup_silu_tern2(const uint32_t* xq, const float* xs, const uint32_t* gpack, const uint16_t* gsc,
                          const uint32_t* upack, const uint16_t* usc, int I, int H, double* swi) {
    double* g = (double*)malloc(sizeof(double) * (size_t)I);
    double* u = (double*)malloc(sizeof(double) * (size_t)I);
    or_gemv_tern2(xq, xs, gpack, gsc, I, H, g);
    or_gemv_tern2(xq, xs, upack, usc, I, H, u);
    for (int i = 0; i < I; i++) swi[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
    free(g);
    free(u);
}

/* models/qwen3.js:276-313: y[n] = sum_k f16(s)*(nib-8)*x[k], x f32 */
void or_gemv_q4_f32(const float* x, const uint32_t* pack, const uint16_t* scales,
                    int N, int K, double* y) {
    int gpr = K / 32, wpr = K / 8;
    for (int n = 0; n < N; n++) {
        const uint32_t* rp = pack + (size_t)n * wpr;
        double acc = 0;
        for (int g = 0; g < gpr; g++) {
            double d = 0;
            for (int j = 0; j < 32; j++) { int k = g * 32 + j; d += (double)nib_at(rp, k) * (double)x[k]; }
            acc += or_f16_to_f32(scales[(size_t)n * gpr + g]) * d;
        }
        y[n] = acc;
    }
}

/* models/qwen3.js:679-728: swi = silu(g)*u, silu(g) = g/(1+exp(-g)) */
void or_gateup_silu_q4(const uint32_t* xq, const float* xs,
                       const uint32_t* gpack, const uint16_t* gsc,
                       const uint32_t* upack, const uint16_t* usc,
                       int I, int H, double* swi) {
    double* g = (double*)malloc(sizeof(double) * I);
    double* u = (double*)malloc(sizeof(double) * I);
    or_gemv_q4_q8(xq, xs, gpack, gsc, I, H, g);
    or_gemv_q4_q8(xq, xs, upack, usc, I, H, u);
    for (int i = 0; i < I; i++) swi[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
    free(g); free(u);
}

/* models/qwen3.js:1326-1388: Y[t,n] = sum_g dot_g(t,n) * xs[t,g] * f16(s_w[n,g]) */
void or_gemm_q4_q8(const uint32_t* xq, const float* xs, const uint32_t* pack,
                   const uint16_t* scales, int T, int N, int K, double* y) {
    for (int t = 0; t < T; t++)
        or_gemv_q4_q8(xq + (size_t)t * (K / 4), xs + (size_t)t * (K / 32), pack, scales, N, K, y + (size_t)t * N);
}

/* ------------------------------------------------------------------------- */
/* KV snorm int8, models/qwen3.js:2180-2210 / 2280-2295                       */
/* mx = max(1e-12, max|x|) over 32; code = floor(0.5 + 127*clamp(x/mx,-1,1)) */
/* (the WGSL pack4x8snorm formula, evaluated exactly on the f32 quotient).   */
/* ------------------------------------------------------------------------- */
static inline int snorm_code(float x, float mx) {
    float e = x / mx;
    if (e > 1.0f) e = 1.0f;
    if (e < -1.0f) e = -1.0f;
    return (int)floor(0.5 + 127.0 * (double)e);
}

void or_kv_quant(const float* x, int n, uint32_t* q, float* s) {
    for (int g = 0; g < n / 32; g++) {
        float mx = 1e-12f;
        for (int j = 0; j < 32; j++) { float a = fabsf(x[g * 32 + j]); if (a > mx) mx = a; }
        s[g] = mx;
        for (int w = 0; w < 8; w++) {
            uint32_t word = 0;
            for (int b = 0; b < 4; b++) word |= ((uint32_t)(snorm_code(x[g * 32 + w * 4 + b], mx) & 0xff)) << (8 * b);
            q[g * 8 + w] = word;
        }
    }
}

/* unpack4x8snorm: max(code/127, -1), times the group scale */
double or_snorm_dequant(uint32_t word, int byte, float scale) {
    int c = (int)(int8_t)((word >> (8 * byte)) & 0xffu);
    double v = (double)c / 127.0;
    if (v < -1.0) v = -1.0;
    return v * (double)scale;
}

/* ------------------------------------------------------------------------- */
/* QK RMSNorm + split-half RoPE + KV write, models/qwen3.js:2228-2296     */
/* RMSNorm over hd: thread j holds x_j^2, tree from 64 down (128 threads).    */
/* RoPE angle: the reference evaluates pos*pow(theta,-2i/hd) and sin/cos in   */
/* f32 WGSL builtins (accurate only on [-pi,pi]); this build evaluates the    */
/* angle and sin/cos in f64 and rounds to f32 (pinned by the n2 ops.rs        */
/* known-answer tests). out = rk*c + rot*s (two products, one sum, f32).      */
/* ------------------------------------------------------------------------- */
void or_rope_norm_row(const float* x, const uint16_t* w, int hd, int pos,
                      float theta, float eps, int apply_norm, float* out) {
    float rk[256];
    if (apply_norm) {
        float red[128];
        for (int j = 0; j < 128; j++) red[j] = (j < hd) ? x[j] * x[j] : 0.0f;
        for (int st = 64; st > 0; st >>= 1)
            for (int j = 0; j < st; j++) red[j] = red[j] + red[j + st];
        float m = red[0] / (float)hd;
        m = m + eps;
        float inv = 1.0f / sqrtf(m);
        for (int j = 0; j < hd; j++) { float a = x[j] * inv; rk[j] = a * (float)or_f16_to_f32(w[j]); }
    } else {
        for (int j = 0; j < hd; j++) rk[j] = x[j];
    }
    int half = hd / 2;
    for (int j = 0; j < hd; j++) {
        int fi = j < half ? j : j - half;
        double ang = (double)pos * pow((double)theta, -2.0 * (double)fi / (double)hd);
        float c = (float)cos(ang), s = (float)sin(ang);
        float partner = j < half ? rk[j + half] : rk[j - half];
        float rot = j < half ? -partner : partner;
        float a = rk[j] * c, b = rot * s;
        out[j] = a + b;
    }
}

void or_attn_prep_q8(const float* q, const float* k, const float* v,
                     const uint16_t* qw, const uint16_t* kw,
                     int nHq, int nKv, int hd, int pos, float theta, float eps,
                     float* qr, uint32_t* kq, float* ks, uint32_t* vq, float* vs) {
    float row[256];
    for (int h = 0; h < nHq; h++) or_rope_norm_row(q + h * hd, qw, hd, pos, theta, eps, 1, qr + h * hd);
    for (int h = 0; h < nKv; h++) {
        or_rope_norm_row(k + h * hd, kw, hd, pos, theta, eps, 1, row);
        or_kv_quant(row, hd, kq + h * (hd / 4), ks + h * (hd / 32));
        or_kv_quant(v + h * hd, hd, vq + h * (hd / 4), vs + h * (hd / 32));
    }
}

/* ------------------------------------------------------------------------- */
/* decode attention, models/qwen3.js:2077-2164 + 2048-2068.           */
/* The split-KV online softmax with an exact LSE merge equals one softmax    */
/* over all S keys; the oracle evaluates that directly in f64.               */
/* ------------------------------------------------------------------------- */
static void attn_one(const float* qrow, const uint32_t* kq, const float* ks,
                     const uint32_t* vq, const float* vs, int nkeys, int nKv, int hd, int hk,
                     double* out) {
    int kv4 = nKv * hd / 4, kvg = nKv * hd / 32;
    double scale = 1.0 / sqrt((double)hd);
    double* sc = (double*)malloc(sizeof(double) * (nkeys > 0 ? nkeys : 1));
    double m = -INFINITY;
    for (int t = 0; t < nkeys; t++) {
        const uint32_t* kr = kq + (size_t)t * kv4 + hk * (hd / 4);
        const float* kscale = ks + (size_t)t * kvg + hk * (hd / 32);
        double d = 0;
        for (int i = 0; i < hd; i++) d += (double)qrow[i] * or_snorm_dequant(kr[i >> 2], i & 3, kscale[i >> 5]);
        sc[t] = d * scale;
        if (sc[t] > m) m = sc[t];
    }
    double den = 0;
    for (int i = 0; i < hd; i++) out[i] = 0;
    for (int t = 0; t < nkeys; t++) {
        double w = exp(sc[t] - m);
        den += w;
        const uint32_t* vr = vq + (size_t)t * kv4 + hk * (hd / 4);
        const float* vscale = vs + (size_t)t * kvg + hk * (hd / 32);
        for (int i = 0; i < hd; i++) out[i] += w * or_snorm_dequant(vr[i >> 2], i & 3, vscale[i >> 5]);
    }
    for (int i = 0; i < hd; i++) out[i] /= den;
    free(sc);
}

void or_attn_decode_q8(const float* qr, const uint32_t* kq, const float* ks,
                       const uint32_t* vq, const float* vs,
                       int S, int nHq, int nKv, int hd, double* out) {
    int grp = nHq / nKv;
    for (int hq = 0; hq < nHq; hq++)
        attn_one(qr + hq * hd, kq, ks, vq, vs, S, nKv, hd, hq / grp, out + hq * hd);
}

/* The same arithmetic as attn_one for every query head of KV heads [hk0, hk1) and T
 * causal queries (query t attends keys [0, pos0+t]), with each KV head's keys and values
 * dequantized once (the sums run in attn_one's order, so the results are bit-identical
 * to or_attn_causal_q8's for those heads). Disjoint head ranges may run in parallel. */
void or_attn_causal_q8_kvheads(const float* qr, const uint32_t* kq, const float* ks,
                               const uint32_t* vq, const float* vs,
                               int T, int pos0, int nHq, int nKv, int hd, int hk0, int hk1, double* out) {
    int grp = nHq / nKv, kv4 = nKv * hd / 4, kvg = nKv * hd / 32, S = pos0 + T;
    double scale = 1.0 / sqrt((double)hd);
    double* K = (double*)malloc(sizeof(double) * (size_t)S * hd);
    double* V = (double*)malloc(sizeof(double) * (size_t)S * hd);
    double* sc = (double*)malloc(sizeof(double) * (size_t)S);
    for (int hk = hk0; hk < hk1; hk++) {
        for (int t = 0; t < S; t++)
            for (int i = 0; i < hd; i++) {
                K[(size_t)t * hd + i] = or_snorm_dequant(kq[(size_t)t * kv4 + hk * (hd / 4) + (i >> 2)], i & 3,
                                                         ks[(size_t)t * kvg + hk * (hd / 32) + (i >> 5)]);
                V[(size_t)t * hd + i] = or_snorm_dequant(vq[(size_t)t * kv4 + hk * (hd / 4) + (i >> 2)], i & 3,
                                                         vs[(size_t)t * kvg + hk * (hd / 32) + (i >> 5)]);
            }
        for (int q = 0; q < T; q++)
            for (int hq = hk * grp; hq < (hk + 1) * grp; hq++) {
                const float* qrow = qr + ((size_t)q * nHq + hq) * hd;
                double* o = out + ((size_t)q * nHq + hq) * hd;
                int nkeys = pos0 + q + 1;
                double m = -INFINITY;
                for (int t = 0; t < nkeys; t++) {
                    double d = 0;
                    for (int i = 0; i < hd; i++) d += (double)qrow[i] * K[(size_t)t * hd + i];
                    sc[t] = d * scale;
                    if (sc[t] > m) m = sc[t];
                }
                double den = 0;
                for (int i = 0; i < hd; i++) o[i] = 0;
                for (int t = 0; t < nkeys; t++) {
                    double w = exp(sc[t] - m);
                    den += w;
                    for (int i = 0; i < hd; i++) o[i] += w * V[(size_t)t * hd + i];
                }
                for (int i = 0; i < hd; i++) o[i] /= den;
            }
    }
    free(K);
    free(V);
    free(sc);
}

/* models/qwen3.js:2534-2577 (causal, T queries at positions pos0..pos0+T-1) */
void or_attn_causal_q8(const float* qr, const uint32_t* kq, const float* ks,
                       const uint32_t* vq, const float* vs,
                       int T, int pos0, int nHq, int nKv, int hd, double* out) {
    int grp = nHq / nKv;
    for (int t = 0; t < T; t++)
        for (int hq = 0; hq < nHq; hq++)
            attn_one(qr + ((size_t)t * nHq + hq) * hd, kq, ks, vq, vs, pos0 + t + 1, nKv, hd, hq / grp,
                     out + ((size_t)t * nHq + hq) * hd);
}

/* ------------------------------------------------------------------------- */
/* decode-step glue: embed gather (models/qwen3.js:1621-1633), argmax         */
/* (models/qwen3.js:2624-2690)                                                */
/* ------------------------------------------------------------------------- */
void or_embed(const int32_t* ids, const uint16_t* emb, int T, int H, float* y) {
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) y[(size_t)t * H + h] = (float)or_f16_to_f32(emb[(size_t)ids[t] * H + h]);
}

/* pcg (models/qwen3.js:2725): the 32-bit PCG hash (one LCG step, then the random
 * xorshift and multiply of PCG-RXS-M-XS). */
uint32_t or_pcg(uint32_t v) {
    uint32_t s = v * 747796405u + 2891336453u;
    uint32_t w = ((s >> ((s >> 28u) + 4u)) ^ s) * 277803737u;
    return (w >> 22u) ^ w;
}

/* the per-step seed update of gumbelNoise (models/qwen3.js:2735) */
uint32_t or_seed_next(uint32_t s) { return s * 1664525u + 1013904223u; }

/* GUMBEL_WGSL (models/qwen3.js:2722-2732), in f32 as the shader computes it:
 * h = pcg(i ^ seed * 2654435761), u = (f32(h >> 8) + 0.5) / 2^24 (in (0, 1), exact),
 * logits[i] = logits[i] + temp * (-log(-log(u))). */
void or_gumbel_noise(float* logits, int N, uint32_t seed, float temp) {
    for (int i = 0; i < N; i++) {
        uint32_t h = or_pcg((uint32_t)i ^ (seed * 2654435761u));
        float u = ((float)(h >> 8u) + 0.5f) / 16777216.0f;
        float g = -logf(-logf(u));
        float d = temp * g;
        logits[i] = logits[i] + d;
    }
}

/* The shared-memory tree of the argmax kernels over nthr per-thread (max, index) slots:
 * for s = nthr/2 .. 1, slot l < s takes slot l+s only if strictly greater
 * (models/qwen3.js:2642, 2664, 2677). Each thread's slot holds the first strict maximum
 * of its strided scan, from (-3e38, 0) (:2640, 2662). */
static void amx_tree(int nthr, float* sv, uint32_t* si) {
    for (int s = nthr / 2; s > 0; s /= 2)
        for (int l = 0; l < s; l++)
            if (sv[l + s] > sv[l]) { sv[l] = sv[l + s]; si[l] = si[l + s]; }
}

/* argmaxKernel (models/qwen3.js:2681-2690): N < 16384 runs the one-workgroup kernel
 * (256 threads striding by 256, :2626-2645); larger N the two-stage pair (64
 * workgroups of 256 threads over interleaved slices striding by 64*256, then one
 * 64-thread workgroup over the partials, :2651-2679). Evaluated literally, so ties
 * resolve as the reference's trees resolve them (not to the lowest index). */
int or_argmax(const float* logits, int N) {
    enum { WG = 256, WGS = 64 };
    float sv[WG];
    uint32_t si[WG];
    if (N < 16384) {
        for (int t = 0; t < WG; t++) {
            float bv = -3.0e38f; uint32_t bi = 0;
            for (int i = t; i < N; i += WG) if (logits[i] > bv) { bv = logits[i]; bi = (uint32_t)i; }
            sv[t] = bv; si[t] = bi;
        }
        amx_tree(WG, sv, si);
        return (int)si[0];
    }
    float pv[WGS];
    uint32_t pi[WGS];
    for (int w = 0; w < WGS; w++) {
        for (int t = 0; t < WG; t++) {
            float bv = -3.0e38f; uint32_t bi = 0;
            for (long i = (long)w * WG + t; i < N; i += (long)WGS * WG)
                if (logits[i] > bv) { bv = logits[i]; bi = (uint32_t)i; }
            sv[t] = bv; si[t] = bi;
        }
        amx_tree(WG, sv, si);
        pv[w] = sv[0]; pi[w] = si[0];
    }
    amx_tree(WGS, pv, pi);
    return (int)pi[0];
}

/* ------------------------------------------------------------------------- */
/* ternary, native/crates/n2-kernels/src/tern.rs                      */
/* ------------------------------------------------------------------------- */
#define TG 64
#define TBPB 16

/* tern.rs:131-160 (= native/tools/pack_bin.py:19-29) */
void or_tern_pack(const float* w, int N, int K, uint8_t* codes, float* scales) {
    int nb = K / TG;
    memset(codes, 0, (size_t)N * K / 4);
    for (int r = 0; r < N; r++)
        for (int b = 0; b < nb; b++) {
            const float* g = w + (size_t)r * K + b * TG;
            float s = 0.0f;
            for (int c = 0; c < TG; c++) s = fmaxf(s, fabsf(g[c]));
            scales[(size_t)r * nb + b] = s;
            float thr = s * 0.5f;
            for (int c = 0; c < TG; c++) {
                float v = g[c];
                uint8_t code = fabsf(v) < thr ? 1 : (v < 0.0f ? 0 : 2);
                codes[(size_t)r * (K / 4) + b * TBPB + (c % TBPB)] |= (uint8_t)(code << (2 * (c / TBPB)));
            }
        }
}

/* tern.rs:206-222: scale = 127/amax (1 if amax == 0); round half away from 0 */
float or_tern_quant_act_n2(const float* x, int K, int8_t* act, int32_t* xsum) {
    float amax = 0.0f;
    for (int i = 0; i < K; i++) amax = fmaxf(amax, fabsf(x[i]));
    float scale = amax > 0.0f ? 127.0f / amax : 1.0f;
    for (int i = 0; i < K; i++) {
        float r = roundf(x[i] * scale);
        if (r < -127.0f) r = -127.0f; if (r > 127.0f) r = 127.0f;
        act[i] = (int8_t)r;
    }
    for (int b = 0; b < K / TG; b++) { int32_t s = 0; for (int j = 0; j < TG; j++) s += act[b * TG + j]; xsum[b] = s; }
    return scale;
}

/* cpu/kernel/src/lib.rs:570-606: asc = amax/127 (1e-9 if 0), q = nearest-even(x*(1/asc)) */
float or_tern_quant_act_wasm(const float* x, int K, int8_t* act, int32_t* xsum) {
    float amax = 0.0f;
    for (int i = 0; i < K; i++) amax = fmaxf(amax, fabsf(x[i]));
    float asc = amax > 0.0f ? amax / 127.0f : 1e-9f;
    float inv = 1.0f / asc;
    for (int i = 0; i < K; i++) {
        float r = rintf(x[i] * inv);
        int q = (int)r;
        if (q < -127) q = -127; if (q > 127) q = 127;
        act[i] = (int8_t)q;
    }
    for (int b = 0; b < K / TG; b++) { int32_t s = 0; for (int j = 0; j < TG; j++) s += act[b * TG + j]; xsum[b] = s; }
    return asc;
}

static inline int32_t tern_dot_block(const uint8_t* blk, const int8_t* ab) {
    int32_t dot = 0;
    for (int j = 0; j < 4; j++)
        for (int i = 0; i < TBPB; i++) dot += (int32_t)((blk[i] >> (2 * j)) & 3) * (int32_t)ab[j * TBPB + i];
    return dot;
}

/* tern.rs:79-119: acc += s*dot, sxs += s*xsum per block, out = acc - sxs */
void or_tern_gemv_scalar(const uint8_t* codes, const float* scales, const int8_t* act,
                         const int32_t* xsum, int N, int K, float* out) {
    int nb = K / TG, bpr = K / 4;
    for (int r = 0; r < N; r++) {
        float acc = 0.0f, sxs = 0.0f;
        for (int b = 0; b < nb; b++) {
            int32_t dot = tern_dot_block(codes + (size_t)r * bpr + b * TBPB, act + b * TG);
            float s = scales[(size_t)r * nb + b];
            float p = s * (float)dot; acc = acc + p;
            float q = s * (float)xsum[b]; sxs = sxs + q;
        }
        out[r] = acc - sxs;
    }
}

/* tern.rs:166-189: dequantize, f32 product, f64 accumulate */
void or_tern_gemv_dequant(const uint8_t* codes, const float* scales, const int8_t* act,
                          int N, int K, float* out) {
    int nb = K / TG;
    for (int r = 0; r < N; r++) {
        double acc = 0;
        for (int kk = 0; kk < K; kk++) {
            int b = kk / TG, c = kk % TG;
            uint8_t raw = codes[(size_t)r * (K / 4) + b * TBPB + (c % TBPB)];
            int code = (raw >> (2 * (c / TBPB))) & 3;
            float w = (float)(code - 1) * scales[(size_t)r * nb + b];
            float p = w * (float)act[kk];
            acc += (double)p;
        }
        out[r] = (float)acc;
    }
}

void or_tern_block_dots(const uint8_t* codes, const int8_t* act, int N, int K, int32_t* dots) {
    int nb = K / TG, bpr = K / 4;
    for (int r = 0; r < N; r++)
        for (int b = 0; b < nb; b++)
            dots[(size_t)r * nb + b] = tern_dot_block(codes + (size_t)r * bpr + b * TBPB, act + b * TG);
}

/* tern.rs:356-389 Rng (xorshift64, high 32 bits) and fixture(); the n2-cli
 * fixture (main.rs:93-114) is the same generator seeded 0x9E3779B97F4A7C15. */
static uint32_t xs_next(uint64_t* s) {
    uint64_t x = *s;
    x ^= x << 13; x ^= x >> 7; x ^= x << 17;
    *s = x;
    return (uint32_t)(x >> 32);
}
void or_n2_fixture(int N, int K, uint64_t seed, uint8_t* codes, float* scales,
                   int8_t* act, int32_t* xsum, float* w_out, float* x_out) {
    uint64_t s = seed;
    float* w = (float*)malloc(sizeof(float) * (size_t)N * K);
    for (size_t i = 0; i < (size_t)N * K; i++) {
        switch (xs_next(&s) % 5) {
            case 0: w[i] = -1.0f; break;
            case 1: w[i] = 1.0f; break;
            case 2: w[i] = 0.0f; break;
            case 3: w[i] = 0.2f; break;
            default: w[i] = -0.9f; break;
        }
    }
    or_tern_pack(w, N, K, codes, scales);
    float* x = (float*)malloc(sizeof(float) * K);
    for (int i = 0; i < K; i++) { float a = (float)(xs_next(&s) % 2001) / 1000.0f; x[i] = a - 1.0f; }
    or_tern_quant_act_n2(x, K, act, xsum);
    if (w_out) memcpy(w_out, w, sizeof(float) * (size_t)N * K);
    if (x_out) memcpy(x_out, x, sizeof(float) * K);
    free(w); free(x);
}

/* ------------------------------------------------------------------------- */
/* int3 MoE, models/lfm25.js                                          */
/* ------------------------------------------------------------------------- */

/* lfm25.js:833-856: int4 -> int3 cascade requant into three bitplanes. */
void or_requant43(const uint32_t* pack4, const uint16_t* sc4, int rows, int K,
                  uint32_t* p3, uint16_t* s3) {
    int gpr = K / 32; long nG = (long)rows * gpr;
    for (long gi = 0; gi < nG; gi++) {
        int q4[32]; int m = 0;
        for (int wI = 0; wI < 4; wI++) {
            uint32_t word = pack4[gi * 4 + wI];
            for (int i = 0; i < 8; i++) {
                int q = (int)((word >> (4 * i)) & 15u) - 8;
                q4[wI * 8 + i] = q;
                int a = q < 0 ? -q : q; if (a > m) m = a;
            }
        }
        if (m == 0) { s3[gi] = or_f32_to_f16_eng(0.0f); p3[gi * 3] = 0; p3[gi * 3 + 1] = 0; p3[gi * 3 + 2] = 0xFFFFFFFFu; continue; }
        double ratio = 4.0 / (double)m;
        double s3d = or_f16_to_f32(sc4[gi]) * (double)m / 4.0;   /* JS left-to-right, f64 */
        s3[gi] = or_f32_to_f16_eng((float)s3d);                  /* Float32Array store, then engine f32ToF16 */
        uint32_t b0 = 0, b1 = 0, b2 = 0;
        for (int i = 0; i < 32; i++) {
            double q = js_round((double)q4[i] * ratio);
            if (q > 3) q = 3; else if (q < -4) q = -4;
            uint32_t st = (uint32_t)((int)q + 4);
            b0 |= (st & 1u) << i; b1 |= ((st >> 1) & 1u) << i; b2 |= ((st >> 2) & 1u) << i;
        }
        p3[gi * 3] = b0; p3[gi * 3 + 1] = b1; p3[gi * 3 + 2] = b2;
    }
}

/* lfm25.js:111-141: sigmoid (f32), top-k of score+bias by strict `>`
 * (lowest index wins ties), weights = s/(sum + 1e-6). */
void or_router(const float* logits, const float* bias, int T, int nE, int topk, int32_t* idx, float* wt) {
    float sc[256], sel[256];
    for (int t = 0; t < T; t++) {
        for (int e = 0; e < nE; e++) {
            float l = logits[t * nE + e];
            float s = 1.0f / (1.0f + expf(-l));
            sc[e] = s; sel[e] = s + bias[e];
        }
        float sum = 0.0f;
        for (int k = 0; k < topk; k++) {
            int best = 0; float bv = -1.0e30f;
            for (int j = 0; j < nE; j++) if (sel[j] > bv) { bv = sel[j]; best = j; }
            sel[best] = -2.0e30f;
            idx[t * topk + k] = best;
            wt[t * topk + k] = sc[best];
            sum = sum + sc[best];
        }
        for (int k = 0; k < topk; k++) wt[t * topk + k] = wt[t * topk + k] / (sum + 1e-6f);
    }
}

static inline int q3_at(const uint32_t* planes, int i) {
    return (int)(((planes[0] >> i) & 1u) | (((planes[1] >> i) & 1u) << 1) | (((planes[2] >> i) & 1u) << 2)) - 4;
}

/* lfm25.js:1924-1974: y[k*N+n] = sum_g f16(s)*sum_i (stored-4)*x */
void or_moe_gemv_q3(const float* x, const uint32_t* p3, const uint16_t* s3,
                    const int32_t* idx, int pairs, int N, int K,
                    int in_stride, int xdiv, double* y) {
    int gpr = K / 32;
    for (int k = 0; k < pairs; k++) {
        int e = idx[k];
        const float* xr = x + (size_t)(k / xdiv) * in_stride;
        for (int n = 0; n < N; n++) {
            long row = (long)e * N + n;
            double acc = 0;
            for (int g = 0; g < gpr; g++) {
                const uint32_t* pl = p3 + (row * gpr + g) * 3;
                double d = 0;
                for (int i = 0; i < 32; i++) d += (double)q3_at(pl, i) * (double)xr[g * 32 + i];
                acc += or_f16_to_f32(s3[row * gpr + g]) * d;
            }
            y[(size_t)k * N + n] = acc;
        }
    }
}

/* lfm25.js:1541-1622: pair p reads activation row p/src_div (int8 per group) */
void or_moe_gemm_q3(const uint32_t* xq, const float* xs, const uint32_t* p3, const uint16_t* s3,
                    const int32_t* ridx, int P, int N, int K, int src_div, double* y) {
    int gpr = K / 32;
    for (int p = 0; p < P; p++) {
        int e = ridx[p], src = p / src_div;
        const uint32_t* aq = xq + (size_t)src * (K / 4);
        const float* as = xs + (size_t)src * gpr;
        for (int n = 0; n < N; n++) {
            long row = (long)e * N + n;
            double acc = 0;
            for (int g = 0; g < gpr; g++) {
                const uint32_t* pl = p3 + (row * gpr + g) * 3;
                long d = 0;
                for (int i = 0; i < 32; i++) d += q3_at(pl, i) * i8_at(aq, g * 32 + i);
                acc += (double)d * (double)as[g] * or_f16_to_f32(s3[row * gpr + g]);
            }
            y[(size_t)p * N + n] = acc;
        }
    }
}

/* lfm25.js:1982-1995 */
void or_moe_combine(float* x, const float* o, const float* wt, int H, int K, int T) {
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            float s = 0.0f;
            for (int k = 0; k < K; k++) { float p = wt[t * K + k] * o[((size_t)t * K + k) * H + h]; s = s + p; }
            x[(size_t)t * H + h] = x[(size_t)t * H + h] + s;
        }
}

/* ------------------------------------------------------------------------- */
/* The Bonsai-1.7B forward's f32 glue, native/crates/n2-core/src/ops.rs and    */
/* model.rs:349-501, in the reference's own f32 arithmetic and order (every sum */
/* sequential from index 0, no fused multiply-adds: the Makefile builds with   */
/* -ffp-contract=off).                                                          */
/* ------------------------------------------------------------------------- */

/* ops.rs:14-22: out = x * (1 / sqrt(mean(x^2) + eps)) * w */
void or_n2_rmsnorm(const float* x, const float* w, int n, float eps, float* out) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    const float mean = ss / (float)n;
    const float inv = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* ops.rs:29-40: the same over each head of t[n_heads * head_dim], in place */
void or_n2_rmsnorm_heads(float* t, const float* w, int n_heads, int head_dim, float eps) {
    for (int h = 0; h < n_heads; h++) {
        float* x = t + (size_t)h * head_dim;
        float ss = 0.0f;
        for (int i = 0; i < head_dim; i++) ss += x[i] * x[i];
        const float mean = ss / (float)head_dim;
        const float inv = 1.0f / sqrtf(mean + eps);
        for (int i = 0; i < head_dim; i++) x[i] = x[i] * inv * w[i];
    }
}

/* ops.rs:79-90: table[i] = cos, table[half + i] = sin of pos * theta^(-2i/head_dim) (f32) */
void or_n2_rope_table(int head_dim, int pos, float theta, float* table) {
    const int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        const float e = -((float)(2 * i)) / (float)head_dim;
        const float inv = powf(theta, e);
        const float ang = (float)pos * inv;
        table[i] = cosf(ang);
        table[half + i] = sinf(ang);
    }
}

/* ops.rs:93-107: split-half rotation of every head with a table, in place */
void or_n2_rope_with_table(float* t, int n_heads, int head_dim, const float* table) {
    const int half = head_dim / 2;
    for (int h = 0; h < n_heads; h++) {
        float* x = t + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            const float x0 = x[i], x1 = x[half + i];
            x[i] = x0 * table[i] - x1 * table[half + i];
            x[half + i] = x1 * table[i] + x0 * table[half + i];
        }
    }
}

/* ops.rs:110-117 */
void or_n2_swiglu(const float* gate, const float* up, int n, float* out) {
    for (int i = 0; i < n; i++) {
        const float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

/* model.rs:421-447 with ops.rs:120-135: GQA attention of q[n_heads * head_dim] (normed,
 * roped) over the f32 cache k/v[S][n_kv * head_dim]; scores scaled by 1/sqrt(head_dim),
 * softmax max-subtracted, out = sum_p w_p v_p */
void or_n2_attention(const float* q, const float* kc, const float* vc, int S, int n_heads, int n_kv, int head_dim,
                     float* out) {
    const int kv_dim = n_kv * head_dim, qpk = n_heads / n_kv;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* sc = (float*)malloc(sizeof(float) * (size_t)(S > 0 ? S : 1));
    for (int h = 0; h < n_heads; h++) {
        const int kvh = h / qpk;
        const float* qh = q + (size_t)h * head_dim;
        for (int p = 0; p < S; p++) {
            const float* kh = kc + (size_t)p * kv_dim + (size_t)kvh * head_dim;
            float dot = 0.0f;
            for (int i = 0; i < head_dim; i++) dot += kh[i] * qh[i];
            sc[p] = dot * scale;
        }
        float mx = -INFINITY;
        for (int p = 0; p < S; p++) mx = fmaxf(mx, sc[p]);
        float sum = 0.0f;
        for (int p = 0; p < S; p++) { sc[p] = expf(sc[p] - mx); sum += sc[p]; }
        const float inv = 1.0f / sum;
        for (int p = 0; p < S; p++) sc[p] *= inv;
        float* o = out + (size_t)h * head_dim;
        for (int i = 0; i < head_dim; i++) o[i] = 0.0f;
        for (int p = 0; p < S; p++) {
            const float* vh = vc + (size_t)p * kv_dim + (size_t)kvh * head_dim;
            for (int i = 0; i < head_dim; i++) o[i] += sc[p] * vh[i];
        }
    }
    free(sc);
}

/* ops.rs:138-149: index of the largest element, the lowest index on ties (start -inf, 0) */
int or_n2_argmax(const float* x, int n) {
    int best = 0;
    float bv = -INFINITY;
    for (int i = 0; i < n; i++) if (x[i] > bv) { bv = x[i]; best = i; }
    return best;
}
