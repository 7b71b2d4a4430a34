/* Order-exact GEMV restatement for the CPU oracle (test infrastructure only).
 *
 * y[r] = sum over the 64 lanes of a wave: lane l accumulates w[r][c]*x[c] for its columns
 * c = it*512 + l*8 + j (it ascending, j = 0..7) as four v_dot2_f32_bf16 steps per column
 * block (pairs j = 0-1, 2-3, 4-5, 6-7, in that order; each step folds its two exact
 * products into the accumulator as mfma_model.h states), then the 64 lane sums are combined
 * by an XOR butterfly with offsets 32,16,8,4,2,1 (correctly rounded FP32 additions) -- the
 * reduction tree of the decode GEMV kernel.  w and x hold BF16 values in FP32.
 * Compiled with -ffp-contract=off. */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "mfma_model.h"

static inline uint16_t hi16(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    return (uint16_t)(u >> 16);
}

void plamo_oracle_gemv(const float* w, const float* x, float* y, int64_t m, int64_t n) {
    const int64_t its = n / 512;
    uint16_t* xb = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n);
    for (int64_t c = 0; c < n; ++c) xb[c] = hi16(x[c]);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r) {
        float acc[64];
        const float* row = w + r * n;
        for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
        for (int64_t it = 0; it < its; ++it)
            for (int l = 0; l < 64; ++l) {
                const int64_t c = it * 512 + l * 8;
                float a = acc[l];
                for (int j = 0; j < 8; j += 2)
                    a = dot2_bits(hi16(row[c + j]), hi16(row[c + j + 1]), xb[c + j], xb[c + j + 1], a);
                acc[l] = a;
            }
        for (int o = 32; o > 0; o >>= 1) {
            float next[64];
            for (int l = 0; l < 64; ++l) next[l] = acc[l] + acc[l ^ o];
            for (int l = 0; l < 64; ++l) acc[l] = next[l];
        }
        y[r] = acc[0];
    }
    free(xb);
}

/* One v_dot2_f32_bf16 chain per output: acc_i <- dot2(a[s][i], b[s][i], acc_i) for s = 0 ..
 * steps-1, a and b BF16 pairs (low half first) laid out [steps][n]; every intermediate
 * accumulator is written to out [steps][n].  fast = 0: the general fold (dot2_group);
 * fast = 1: dot2_bits, the form plamo_oracle_gemv uses. */
void plamo_oracle_dot2_chain(const uint32_t* a, const uint32_t* b, const float* c, float* out, int64_t n,
                             int64_t steps, int32_t fast) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float acc = c[i];
        for (int64_t s = 0; s < steps; ++s) {
            const uint32_t u = a[s * n + i], v = b[s * n + i];
            if (fast) {
                acc = dot2_bits((uint16_t)(u & 0xffffu), (uint16_t)(u >> 16), (uint16_t)(v & 0xffffu),
                                (uint16_t)(v >> 16), acc);
            } else {
                const bfdec wd[2] = {bf_decode((uint16_t)(u & 0xffffu)), bf_decode((uint16_t)(u >> 16))};
                const bfdec xd[2] = {bf_decode((uint16_t)(v & 0xffffu)), bf_decode((uint16_t)(v >> 16))};
                acc = dot2_group(wd, xd, acc);
            }
            out[s * n + i] = acc;
        }
    }
}

/* Decode attention scores (before the scale): q [16][128] and k [n][128] BF16 bits ->
 * out [16][n].  Each score is four chains over dims 32c .. 32c+31, each a v_dot2_f32_bf16
 * chain over the dim pairs (32c + 2i, 32c + 2i + 1) in order from 0, summed as
 * (c0 + c1) + (c2 + c3) -- the decode attention kernel's order. */
void plamo_oracle_attn_scores(const uint16_t* q, const uint16_t* k, int64_t n, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < n; ++j) {
        const uint16_t* kr = k + j * 128;
        for (int h = 0; h < 16; ++h) {
            const uint16_t* qr = q + h * 128;
            float c[4];
            for (int cc = 0; cc < 4; ++cc) {
                float a = 0.0f;
                for (int i = 0; i < 16; ++i) {
                    const int d = 32 * cc + 2 * i;
                    a = dot2_bits(qr[d], qr[d + 1], kr[d], kr[d + 1], a);
                }
                c[cc] = a;
            }
            out[h * n + j] = (c[0] + c[1]) + (c[2] + c[3]);
        }
    }
}

/* Decode attention P.V of one 64-key partition: e [16][64] FP32 probabilities (unnormalised),
 * v [nk][128] BF16 bits -> out [16][128].  Per head and dim, keys 0..31 and 32..63 are two
 * chains of fused multiply-adds in key order from 0 (keys past nk are absent), then the two
 * halves are added -- the decode attention kernel's order. */
void plamo_oracle_attn_pv(const float* e, const uint16_t* v, int64_t nk, float* out) {
    for (int h = 0; h < 16; ++h)
        for (int d = 0; d < 128; ++d) {
            float half[2] = {0.0f, 0.0f};
            for (int hf = 0; hf < 2; ++hf)
                for (int64_t j = 32 * hf; j < 32 * hf + 32 && j < nk; ++j) {
                    const uint32_t u = (uint32_t)v[j * 128 + d] << 16;
                    float vf;
                    memcpy(&vf, &u, 4);
                    half[hf] = fmaf(e[h * 64 + j], vf, half[hf]);
                }
            out[h * 128 + d] = half[0] + half[1];
        }
}
