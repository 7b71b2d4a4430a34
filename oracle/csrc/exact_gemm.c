/* Order-exact restatement of the prefill MFMA GEMM (test infrastructure only):
 * Y[t][r] = sum_k X[t][k] W[r][k] with K ascending, each output one accumulator chain of the
 * model in mfma_model.h (the kernels' K order: every 16-wide K slice is one MFMA step).
 * Compiled with -ffp-contract=off. */
#include "mfma_model.h"

/* y[t][r] (FP32) = MFMA-order sum over k of x[t][k] * w[r][k]; w [m][k], x [tokens][k] BF16
 * bits; k a multiple of 8. */
void plamo_oracle_mfma_gemm(const uint16_t* w, const uint16_t* x, float* y, int64_t m, int64_t k, int64_t tokens) {
    bfdec* wd = (bfdec*)malloc(sizeof(bfdec) * (size_t)(m * k));
    bfdec* xd = (bfdec*)malloc(sizeof(bfdec) * (size_t)(tokens * k));
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m * k; ++i) wd[i] = bf_decode(w[i]);
    for (int64_t i = 0; i < tokens * k; ++i) xd[i] = bf_decode(x[i]);
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t t = 0; t < tokens; ++t) y[t * m + r] = mfma_dot(wd + r * k, xd + t * k, k, 0.0f);
    free(wd);
    free(xd);
}

/* One MFMA-order chain continuing from `acc`: products a[i] * b[i], i = 0 .. n-1 in groups of 8
 * (attention: scores over head dimensions, P.V over a tile's keys). */
float plamo_oracle_mfma_chain(const uint16_t* a, const uint16_t* b, int64_t n, float acc) {
    bfdec ad[256], bd[256];
    float r = acc;
    for (int64_t c = 0; c < n; c += 256) {
        const int64_t len = n - c < 256 ? n - c : 256;
        for (int64_t i = 0; i < len; ++i) {
            ad[i] = bf_decode(a[c + i]);
            bd[i] = bf_decode(b[c + i]);
        }
        r = mfma_dot(ad, bd, len, r);
    }
    return r;
}
