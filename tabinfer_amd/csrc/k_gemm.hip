// k_gemm.hip — T>1 int4 x int8 GEMM (gemmDP4A, models/qwen3.js:1326-1407).
#include "ti_internal.h"

int ti_gemv_q4_q8_launch(ti_ctx* c, const uint32_t* xq, const float* xs, const uint32_t* pack, const uint16_t* scales,
                         float* y, int N, int K, int acc);

// One GEMV per token over the per-token int8 rows (exact same arithmetic as
// the T=1 path).
int ti_gemm_q4_q8_launch(ti_ctx* c, const uint32_t* xq, const float* xs, const uint32_t* pack, const uint16_t* scales,
                         float* y, int T, int N, int K, int acc) {
    for (int t = 0; t < T; t++) {
        int rc = ti_gemv_q4_q8_launch(c, xq + (size_t)t * (K / 4), xs + (size_t)t * (K / 32), pack, scales,
                                      y + (size_t)t * N, N, K, acc);
        if (rc) return rc;
    }
    return TI_OK;
}
