/* Order-exact GEMV restatement for the CPU oracle (test infrastructure only).
 *
 * y[r] = sum over the 64 lanes of a wave: lane l accumulates w[r][c]*x[c] for its columns
 * c = it*512 + l*8 + j (it ascending, j = 0..7) in that order, then the 64 lane sums are
 * combined by an XOR butterfly with offsets 32,16,8,4,2,1 -- the reduction tree of the
 * decode GEMV kernel.  BF16 x BF16 products are exact in FP32, so each step is one
 * correctly rounded FP32 addition.  Compiled with -ffp-contract=off. */
#include <stdint.h>

void plamo_oracle_gemv(const float* w, const float* x, float* y, int64_t m, int64_t n) {
    const int64_t its = n / 512;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r) {
        float acc[64];
        const float* row = w + r * n;
        for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
        for (int64_t it = 0; it < its; ++it)
            for (int l = 0; l < 64; ++l) {
                const int64_t c = it * 512 + l * 8;
                float a = acc[l];
                for (int j = 0; j < 8; ++j) {
                    const float p = row[c + j] * x[c + j];
                    a = a + p;
                }
                acc[l] = a;
            }
        for (int o = 32; o > 0; o >>= 1) {
            float next[64];
            for (int l = 0; l < 64; ++l) next[l] = acc[l] + acc[l ^ o];
            for (int l = 0; l < 64; ++l) acc[l] = next[l];
        }
        y[r] = acc[0];
    }
}
