/*
 * tern_avx2.c — restatement of the reference's native CPU ternary GEMV,
 * native/crates/n2-kernels/src/tern.rs:246-338 (avx2::gemv_tern), in C with the
 * same instruction plan: two 64-code blocks per 256-bit step (block b in the low
 * 128-bit lane, b+1 in the high lane), vpmaddubsw + vpmaddwd per 2-bit plane,
 * a lane-split scale vector, a separate scalar sum of s*xsum, one horizontal
 * sum and one subtraction per row, and the scalar tail for an odd block count.
 *
 * TEST INFRASTRUCTURE ONLY: this is the CPU baseline that bench.py times and the
 * tests check against or_tern_gemv_scalar; the product library never uses it.
 */
#include "ti_oracle.h"
#include <immintrin.h>
#include <pthread.h>
#include <string.h>

int or_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") ? 1 : 0;
}

__attribute__((target("avx2")))
static float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x55));
    return _mm_cvtss_f32(s);
}

__attribute__((target("avx2")))
static void rows_avx2(const uint8_t* codes, const float* scales, const int8_t* act,
                      const int32_t* xsum, int r0, int r1, int K, float* out) {
    const int G = 64, BPB = 16;
    int nblocks = K / G, bpr = K / 4, pairs = nblocks / 2;
    const __m256i m3 = _mm256_set1_epi8(3);
    const __m256i ones = _mm256_set1_epi16(1);
    for (int row = r0; row < r1; row++) {
        const uint8_t* rc = codes + (size_t)row * bpr;
        const float* rs = scales + (size_t)row * nblocks;
        __m256 facc = _mm256_setzero_ps();
        float sxs = 0.0f;
        for (int p = 0; p < pairs; p++) {
            int b = p * 2;
            __m256i raw = _mm256_loadu_si256((const __m256i*)(rc + b * BPB));
            __m256i iacc = _mm256_setzero_si256();
#define PLANE(J, SH) do { \
                __m256i pl = _mm256_and_si256(_mm256_srli_epi16(raw, SH), m3); \
                __m128i lo = _mm_loadu_si128((const __m128i*)(act + b * G + (J) * BPB)); \
                __m128i hi = _mm_loadu_si128((const __m128i*)(act + (b + 1) * G + (J) * BPB)); \
                __m256i a = _mm256_inserti128_si256(_mm256_castsi128_si256(lo), hi, 1); \
                __m256i prod = _mm256_maddubs_epi16(pl, a); \
                iacc = _mm256_add_epi32(iacc, _mm256_madd_epi16(prod, ones)); \
            } while (0)
            PLANE(0, 0); PLANE(1, 2); PLANE(2, 4); PLANE(3, 6);
#undef PLANE
            float s0 = rs[b], s1 = rs[b + 1];
            __m256 sv = _mm256_insertf128_ps(_mm256_castps128_ps256(_mm_set1_ps(s0)), _mm_set1_ps(s1), 1);
            facc = _mm256_add_ps(facc, _mm256_mul_ps(_mm256_cvtepi32_ps(iacc), sv));
            float t0 = s0 * (float)xsum[b]; sxs = sxs + t0;
            float t1 = s1 * (float)xsum[b + 1]; sxs = sxs + t1;
        }
        float acc = hsum256(facc);
        for (int b = pairs * 2; b < nblocks; b++) {
            const uint8_t* blk = rc + b * BPB;
            const int8_t* ab = act + b * G;
            int32_t dot = 0;
            for (int j = 0; j < 4; j++)
                for (int i = 0; i < BPB; i++) dot += (int32_t)((blk[i] >> (2 * j)) & 3) * (int32_t)ab[j * BPB + i];
            float s = rs[b];
            float pa = s * (float)dot; acc = acc + pa;
            float pb = s * (float)xsum[b]; sxs = sxs + pb;
        }
        out[row] = acc - sxs;
    }
}

void or_tern_gemv_avx2(const uint8_t* codes, const float* scales, const int8_t* act,
                       const int32_t* xsum, int N, int K, float* out) {
    rows_avx2(codes, scales, act, xsum, 0, N, K, out);
}

/* ---- a persistent thread pool over a GEMV set --------------------------------------
 * The reference's multi-worker CPU engine splits each GEMV's rows statically over its
 * workers and meets at a barrier before the next one (cpu/cpukern-fwd-worker.js:1-4);
 * this pool does the same with threads created once (or_tern_pool_start), so a timed
 * pass pays no thread creation. The calling thread is worker 0. */
static struct {
    int n;                              /* workers including the caller; 0 = not started */
    pthread_t th[256];
    pthread_mutex_t mu;
    pthread_cond_t cv;
    pthread_barrier_t bar;
    unsigned gen;                       /* bumped per pass; workers run one pass per bump */
    int quit;
    const or_tern_mat* mats;
    int nmat;
} P;

static void pass_rows(int w) {
    for (int m = 0; m < P.nmat; m++) {
        const or_tern_mat* t = &P.mats[m];
        const int r0 = (int)((long)t->N * w / P.n), r1 = (int)((long)t->N * (w + 1) / P.n);
        if (r0 < r1) rows_avx2(t->codes, t->scales, t->act, t->xsum, r0, r1, t->K, t->out);
        pthread_barrier_wait(&P.bar);
    }
}

static void* worker(void* arg) {
    const int w = (int)(long)arg;
    unsigned seen = 0;
    for (;;) {
        pthread_mutex_lock(&P.mu);
        while (P.gen == seen && !P.quit) pthread_cond_wait(&P.cv, &P.mu);
        seen = P.gen;
        const int quit = P.quit;
        pthread_mutex_unlock(&P.mu);
        if (quit) return NULL;
        pass_rows(w);
    }
}

int or_tern_pool_start(int nthreads) {
    if (P.n) or_tern_pool_stop();
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_mutex_init(&P.mu, NULL);
    pthread_cond_init(&P.cv, NULL);
    pthread_barrier_init(&P.bar, NULL, (unsigned)nthreads);
    P.gen = 0;
    P.quit = 0;
    P.n = nthreads;
    for (int w = 1; w < nthreads; w++)
        if (pthread_create(&P.th[w], NULL, worker, (void*)(long)w) != 0) return -1;
    return nthreads;
}

void or_tern_pool_stop(void) {
    if (!P.n) return;
    pthread_mutex_lock(&P.mu);
    P.quit = 1;
    pthread_cond_broadcast(&P.cv);
    pthread_mutex_unlock(&P.mu);
    for (int w = 1; w < P.n; w++) pthread_join(P.th[w], NULL);
    pthread_barrier_destroy(&P.bar);
    pthread_cond_destroy(&P.cv);
    pthread_mutex_destroy(&P.mu);
    P.n = 0;
}

void or_tern_pool_run(const or_tern_mat* mats, int nmat) {
    if (!P.n) or_tern_pool_start(1);
    P.mats = mats;
    P.nmat = nmat;
    pthread_mutex_lock(&P.mu);
    P.gen++;
    pthread_cond_broadcast(&P.cv);
    pthread_mutex_unlock(&P.mu);
    pass_rows(0);                 /* the last barrier of the pass: every worker is done */
}

/* the same set on the calling thread alone, matrix after matrix (the reference's
 * single-threaded configuration, native/crates/n2-cli/src/main.rs:377) */
void or_tern_set_serial(const or_tern_mat* mats, int nmat) {
    for (int m = 0; m < nmat; m++)
        rows_avx2(mats[m].codes, mats[m].scales, mats[m].act, mats[m].xsum, 0, mats[m].N, mats[m].K, mats[m].out);
}

void or_tern_gemv_avx2_mt(const uint8_t* codes, const float* scales, const int8_t* act,
                          const int32_t* xsum, int N, int K, float* out, int nthreads) {
    if (nthreads <= 1) { rows_avx2(codes, scales, act, xsum, 0, N, K, out); return; }
    if (P.n != nthreads) or_tern_pool_start(nthreads);
    or_tern_mat m = {codes, scales, act, xsum, out, N, K};
    or_tern_pool_run(&m, 1);
}
