/* Order-exact restatement of the prefill flash-attention kernel (test infrastructure only).
 *
 * The attention of Runtime.swift:389-444 (scores scaled by 1/sqrt(128) before the maximum,
 * softmax over the visible keys, roundbf(sum p v)) in the exact arithmetic of the gfx950
 * kernel flash_prefill_kernel:
 *
 *   Query blocks of 8 tokens; keys klo .. khi of a block (klo = 0 on global layers, else the
 *   window start of the block's first token) in 64-key tiles, the tiles of a block split over
 *   parts = min(3, ceil(tiles / 11)) contiguous ranges (tile j0 = part * tiles / parts).
 *   Keys of local layers are rotated with coordinate key - base, base = max(0, c - 2047) for
 *   the block's 16-token chunk start c.  Per query and part, tile by tile:
 *     s_k   = MFMA chain over the 128 dimensions in order (mfma_model.h), from 0;
 *     x_k   = s_k * (1/sqrt(128) * log2(e)) in FP32, or -inf for a key the query cannot see;
 *     m'    = max(m, max_k x_k); base ms = m' (0 while nothing is visible);
 *     alpha = exp2_det(m - ms); l_h = l_h * alpha for the two half-lane sums h;
 *     e_k   = exp2_det(x_k - ms), added to l_h in lane order (h = key bit 2; keys of a lane
 *             taken as tile 32r + 8(i/4) + 4h + i%4 for r = 0, 1 and i = 0 .. 15);
 *     o_d   = o_d * alpha, then for each 16-key step s the MFMA chain over the products
 *             v_kd * hi_k (keys 16s + {0-3, 8-11}, then {4-7, 12-15}) and v_kd * lo_k (same
 *             two groups), hi = bf16(e), lo = bf16(e - hi);
 *   l = l_0 + l_1.  One part: out = bf16(o / l).  With a QSA mask, keys of unselected complete
 *   blocks of four are invisible like masked ones.  Several: M = max of the parts' m in part
 *   order, w = exp2_det(m_q - M), l = sum l_q * w and o = sum o_q * w in part order (every
 *   product and sum rounded), out = bf16(o / l).
 * Compiled with -ffp-contract=off. */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "mfma_model.h"

enum { FT = 8, FK = 64, WINDOW = 2048, CHUNK = 16, PARTS = 3, PART_TILES = 11, HEADS = 16, HD = 128 };

static inline float bf(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t bits16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static inline float roundbf(float x) { return bf(bits16(x)); }

/* The device exp2_det: rint split, degree-6 Taylor polynomial of 2^f with fused multiply-adds,
 * exact scale; 0 below -64. */
float plamo_oracle_exp2_det(float x) {
    if (!(x >= -64.0f)) return 0.0f;
    const float k = rintf(x);
    const float f = x - k;
    float p = 1.54035304e-04f;
    p = fmaf(p, f, 1.33335581e-03f);
    p = fmaf(p, f, 9.61812911e-03f);
    p = fmaf(p, f, 5.55041087e-02f);
    p = fmaf(p, f, 2.40226507e-01f);
    p = fmaf(p, f, 6.93147182e-01f);
    p = fmaf(p, f, 1.0f);
    return ldexpf(p, (int)k);
}

typedef struct {
    float m, l;
    float o[HD];
} part_state;

/* One query (token position qpos, head vector q) over tiles j0 .. j1 of its block. */
/* QSA: key kp is seen when its block is the query's unfinished one or selected in `mask`
 * (bit b of word b / 32); null mask: every key. */
static inline int qsa_seen(const uint32_t* mask, uint32_t qpos, uint32_t kp) {
    if (!mask) return 1;
    const uint32_t b = kp >> 2;
    return b >= (qpos + 1) / 4 || ((mask[b >> 5] >> (b & 31)) & 1u);
}

static void flash_part(const bfdec* qd, const bfdec* kd, const uint16_t* vt, uint32_t klo, uint32_t qpos, int full,
                       const uint32_t* mask, int j0, int j1, part_state* st) {
    const float sc = 0.08838834764831845f * 1.4426950408889634f;
    float m = -INFINITY, ls[2] = {0.0f, 0.0f};
    float* o = st->o;
    for (int d = 0; d < HD; ++d) o[d] = 0.0f;
    for (int j = j0; j < j1; ++j) {
        const uint32_t k0 = klo + (uint32_t)j * FK;
        const bfdec* kt = kd + (size_t)(j * FK) * HD;
        const uint16_t* vj = vt + (size_t)(j * FK) * HD;
        float x[FK], e[FK];
        float mt = -INFINITY;
        for (int c = 0; c < FK; ++c) {
            const uint32_t kp = k0 + (uint32_t)c;
            const int vis = kp <= qpos && (full || kp + (uint32_t)(WINDOW - 1) >= qpos) && qsa_seen(mask, qpos, kp);
            const float s = mfma_dot(kt + (size_t)c * HD, qd, HD, 0.0f);
            x[c] = vis ? s * sc : -INFINITY;
            mt = fmaxf(mt, x[c]);
        }
        const float mn = fmaxf(m, mt);
        const float ms = mn == -INFINITY ? 0.0f : mn;
        const float alpha = plamo_oracle_exp2_det(m - ms);
        ls[0] = ls[0] * alpha;
        ls[1] = ls[1] * alpha;
        for (int c = 0; c < FK; ++c) e[c] = plamo_oracle_exp2_det(x[c] - ms);
        for (int h = 0; h < 2; ++h)
            for (int r = 0; r < 2; ++r)
                for (int i = 0; i < 16; ++i) ls[h] = ls[h] + e[32 * r + 8 * (i >> 2) + 4 * h + (i & 3)];
        m = mn;
        bfdec ph[FK], pl[FK];
        for (int c = 0; c < FK; ++c) {
            const uint16_t hb = bits16(e[c]);
            ph[c] = bf_decode(hb);
            pl[c] = bf_decode(bits16(e[c] - bf(hb)));
        }
        for (int d = 0; d < HD; ++d) {
            float acc = o[d] * alpha;
            for (int s = 0; s < 4; ++s) {
                static const int grp[2][8] = {{0, 1, 2, 3, 8, 9, 10, 11}, {4, 5, 6, 7, 12, 13, 14, 15}};
                bfdec va[32], pa[32];
                for (int half = 0; half < 2; ++half)
                    for (int g = 0; g < 2; ++g)
                        for (int i = 0; i < 8; ++i) {
                            const int c = 16 * s + grp[g][i];
                            va[16 * half + 8 * g + i] = bf_decode(vj[(size_t)c * HD + d]);
                            pa[16 * half + 8 * g + i] = half ? pl[c] : ph[c];
                        }
                acc = mfma_dot(va, pa, 32, acc);
            }
            o[d] = acc;
        }
    }
    st->m = m;
    st->l = ls[0] + ls[1];
}

/* q: [tokens][16][128] normalised rotated queries; keys, values: [capacity][128] with position
 * p in slot p % capacity (global keys rotated, local keys unrotated); lcos, lsin: the local
 * RoPE table [rows][64] (local layers only); out: [tokens][2048].  All BF16 bits. */
void plamo_oracle_flash(const uint16_t* q, const uint16_t* keys, const uint16_t* values, const uint16_t* lcos,
                        const uint16_t* lsin, int64_t capacity, int64_t p0, int64_t tokens, int32_t full,
                        uint16_t* out, const uint32_t* qsa_mask, int64_t qsa_words) {
    const int nqb = (int)((tokens + FT - 1) / FT);
    for (int qb = 0; qb < nqb; ++qb) {
        const int t0 = qb * FT;
        const int t1 = (int)(t0 + FT < tokens ? t0 + FT : tokens);
        const uint32_t chunk = (uint32_t)p0 + (uint32_t)(t0 / CHUNK) * CHUNK;
        const uint32_t base = full ? 0u : (chunk > WINDOW - 1 ? chunk - (WINDOW - 1) : 0u);
        const uint32_t plo = (uint32_t)(p0 + t0), khi = (uint32_t)(p0 + t1 - 1);
        const uint32_t klo = full ? 0u : (plo > WINDOW - 1 ? plo - (WINDOW - 1) : 0u);
        const int ntiles = (int)((khi + 1 - klo + FK - 1) / FK);
        const int np = (ntiles + PART_TILES - 1) / PART_TILES;
        const int parts = np < PARTS ? np : PARTS;
        const size_t nk = (size_t)ntiles * FK;
        bfdec* kd = (bfdec*)malloc(sizeof(bfdec) * nk * HD);
        uint16_t* vt = (uint16_t*)calloc(nk * HD, sizeof(uint16_t));
        for (size_t c = 0; c < nk; ++c) {
            const uint32_t kp = klo + (uint32_t)c;
            uint16_t row[HD];
            if (kp > khi) {
                memset(row, 0, sizeof(row));
            } else {
                const uint16_t* kr = keys + (size_t)(kp % (uint64_t)capacity) * HD;
                memcpy(vt + c * HD, values + (size_t)(kp % (uint64_t)capacity) * HD, HD * sizeof(uint16_t));
                if (full) {
                    memcpy(row, kr, sizeof(row));
                } else {
                    const uint16_t* cr = lcos + (size_t)(kp - base) * 64;
                    const uint16_t* sr = lsin + (size_t)(kp - base) * 64;
                    for (int d = 0; d < 64; ++d) {
                        const float a = bf(kr[d]), b = bf(kr[d + 64]), co = bf(cr[d]), si = bf(sr[d]);
                        row[d] = bits16(roundbf(a * co) + roundbf(-b * si));
                        row[d + 64] = bits16(roundbf(b * co) + roundbf(a * si));
                    }
                }
            }
            for (int d = 0; d < HD; ++d) kd[c * HD + d] = bf_decode(row[d]);
        }
        const int nq = (t1 - t0) * HEADS;
#pragma omp parallel for schedule(dynamic, 1)
        for (int w = 0; w < nq; ++w) {
            const int t = t0 + w / HEADS, h = w % HEADS;
            const uint32_t qpos = (uint32_t)(p0 + t);
            bfdec qd[HD];
            for (int d = 0; d < HD; ++d) qd[d] = bf_decode(q[((size_t)t * HEADS + h) * HD + d]);
            part_state ps[PARTS];
            const uint32_t* mask = qsa_mask ? qsa_mask + (size_t)t * (size_t)qsa_words : 0;
            for (int pt = 0; pt < parts; ++pt)
                flash_part(qd, kd, vt, klo, qpos, full, mask, pt * ntiles / parts, (pt + 1) * ntiles / parts, &ps[pt]);
            float o[HD], l;
            if (parts == 1) {
                l = ps[0].l;
                memcpy(o, ps[0].o, sizeof(o));
            } else {
                float M = -INFINITY;
                for (int pt = 0; pt < parts; ++pt) M = fmaxf(M, ps[pt].m);
                l = 0.0f;
                for (int d = 0; d < HD; ++d) o[d] = 0.0f;
                for (int pt = 0; pt < parts; ++pt) {
                    const float wq = plamo_oracle_exp2_det(ps[pt].m - M);
                    l = l + ps[pt].l * wq;
                    for (int d = 0; d < HD; ++d) o[d] = o[d] + ps[pt].o[d] * wq;
                }
            }
            uint16_t* orow = out + (size_t)t * HEADS * HD + (size_t)h * HD;
            for (int d = 0; d < HD; ++d) orow[d] = bits16(o[d] / l);
        }
        free(kd);
        free(vt);
    }
}
