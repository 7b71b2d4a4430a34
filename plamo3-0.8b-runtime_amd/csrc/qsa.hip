// QSA block indexers on gfx950 (Kernels.metal:564-702, Runtime.swift:380-418): on the global
// layers, each query attends only to its budget/4 best blocks of four keys plus the keys of
// its unfinished block, once it sees more complete blocks than that.
//
//   qsa_prep_kernel    queries of the indexer (4 heads: RMSNorm with q_norm + 1, global RoPE at
//                      the query's position) and each token's raw key (qsa_query)
//   qsa_pool_kernel    the block key of every block a forward completes: the mean of its four
//                      raw keys, RMSNorm with k_norm + 1, global RoPE at the block's first
//                      position (qsa_pool)
//   qsa_scores_kernel  score(query, block) = sum over heads of max(0, q_h . k_b) / sqrt(128)
//                      for the blocks complete at the query's position (qsa_scores)
//   qsa_select_kernel  the budget/4 best blocks (ties to the lower index) as a bitmap; every
//                      block when the query sees no more than that (qsa_select)
// The attention kernels then mask the keys of unselected blocks (qsa_gather + attention over
// the gathered keys in the reference: the same key set).
#include <hip/hip_runtime.h>

#include "common.h"
#include "device.h"
#include "kernels.h"

namespace plamo {
using namespace dev;

namespace {

constexpr float QSA_SCALE = 0.08838834764831845f;  // 1 / sqrt(128)

__device__ __forceinline__ uint32_t row_pos(const QsaParams& p, int t) {
    return p.state ? p.state->pos[0] + uint32_t(t) : p.p0 + uint32_t(t);
}

// RMSNorm of a 128-dim head held as (dim l, dim l + 64) in lane l of a wave, gain
// roundbf(bf(w) + 1), then global RoPE with the table word (BF16 cos | sin << 16):
// ss = a*a + b*b, the wave's XOR butterfly, r = 1 / sqrt(ss / 128 + 1e-6),
// z = roundbf(roundbf(v * r) * g) (Kernels.metal:574-577,590-594),
// (za, zb) -> (roundbf(roundbf(za c) + roundbf(-zb s)), roundbf(roundbf(zb c) + roundbf(za s)))
// (Kernels.metal:261-274).
__device__ __forceinline__ void norm_rope(float a, float b, const uint16_t* w, uint32_t rope, float& ra, float& rb) {
#pragma clang fp contract(off)
    const int l = int(threadIdx.x & 63);
    const float ss = wave_sum(a * a + b * b);
    const float r = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
    const float za = roundbf(roundbf(a * r) * roundbf(bf(w[l]) + 1.0f));
    const float zb = roundbf(roundbf(b * r) * roundbf(bf(w[l + 64]) + 1.0f));
    const float c = lo(rope), s = hi(rope);
    ra = roundbf(roundbf(za * c) + roundbf(-zb * s));
    rb = roundbf(roundbf(zb * c) + roundbf(za * s));
}

// Token t = blockIdx.x: wave h normalises and rotates query head h (BF16 out), threads
// 0..127 copy the raw key (projection columns 512..639) to raw[pos].
__global__ __launch_bounds__(256) void qsa_prep_kernel(const QsaParams p) {
    const int t = int(blockIdx.x), tid = int(threadIdx.x), l = tid & 63, h = tid >> 6;
    if (p.state && (p.state->stopped || p.state->rows == 0)) return;
    const uint32_t pos = row_pos(p, t);
    const uint16_t* x = p.proj + size_t(t) * QSA_PROJ;
    float ra, rb;
    norm_rope(bf(x[h * HEAD_DIM + l]), bf(x[h * HEAD_DIM + 64 + l]), p.q_norm, p.global_rope[size_t(pos) * 64 + l],
              ra, rb);
    uint16_t* q = p.queries + size_t(t) * (4 * HEAD_DIM) + h * HEAD_DIM;
    q[l] = uint16_t(bits(ra));
    q[l + 64] = uint16_t(bits(rb));
    if (tid < HEAD_DIM) p.raw[size_t(pos) * HEAD_DIM + tid] = x[4 * HEAD_DIM + tid];
}

// Blocks first .. first + gridDim.x - 1 with blockIdx.x < count (one wave each): the blocks
// the forward completes, (p0 + n) / 4 - p0 / 4 of them (Runtime.swift:385-388).
__global__ __launch_bounds__(64) void qsa_pool_kernel(const QsaParams p) {
#pragma clang fp contract(off)
    const int l = int(threadIdx.x);
    uint32_t first, count;
    if (p.state) {
        if (p.state->stopped || p.state->rows == 0) return;
        const uint32_t pos = p.state->pos[0];
        first = pos / 4;
        count = (pos + 1) / 4 - first;
    } else {
        first = p.p0 / 4;
        count = (p.p0 + uint32_t(p.tokens)) / 4 - first;
    }
    if (blockIdx.x >= count) return;
    const uint32_t b = first + blockIdx.x;
    const uint16_t* k = p.raw + size_t(4 * b) * HEAD_DIM;
    // roundbf((((k0 + k1) + k2) + k3) / 4) (Kernels.metal:588)
    auto mean = [&](int d) {
        return roundbf((((bf(k[d]) + bf(k[HEAD_DIM + d])) + bf(k[2 * HEAD_DIM + d])) + bf(k[3 * HEAD_DIM + d])) / 4.0f);
    };
    float ra, rb;
    norm_rope(mean(l), mean(l + 64), p.k_norm, p.global_rope[size_t(4 * b) * 64 + l], ra, rb);
    p.pooled[size_t(b) * HEAD_DIM + l] = uint16_t(bits(ra));
    p.pooled[size_t(b) * HEAD_DIM + l + 64] = uint16_t(bits(rb));
}

// Lane = block b = blockIdx.x * 64 + lane, token t = blockIdx.y.  Each head's dot product is
// one v_dot2_f32_bf16 chain over the 64 dim pairs in order from 0; the score is
// ((((0 + max(d0, 0)) + max(d1, 0)) + max(d2, 0)) + max(d3, 0)) * (1 / sqrt(128))
// (Kernels.metal:606-613).  Blocks not complete at the query's position are not scored.
__global__ __launch_bounds__(64) void qsa_scores_kernel(const QsaParams p) {
#pragma clang fp contract(off)
    __shared__ __align__(16) uint32_t qs[4 * HEAD_DIM / 2];
    const int t = int(blockIdx.y), l = int(threadIdx.x);
    if (p.state && (p.state->stopped || p.state->rows == 0)) return;
    const uint32_t complete = (row_pos(p, t) + 1) / 4;
    const uint32_t b = blockIdx.x * 64 + uint32_t(l);
    if (blockIdx.x * 64 >= complete) return;
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(p.queries + size_t(t) * (4 * HEAD_DIM));
#pragma unroll
    for (int i = 0; i < 4; ++i) qs[l + 64 * i] = qw[l + 64 * i];
    __syncthreads();
    if (b >= complete) return;
    const uint4* kr = reinterpret_cast<const uint4*>(p.pooled + size_t(b) * HEAD_DIM);
    uint4 kv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) kv[i] = kr[i];
    float score = 0.f;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint4 qv = *reinterpret_cast<const uint4*>(&qs[h * 64 + 4 * i]);
            acc = dot2bf(qv.x, kv[i].x, acc);
            acc = dot2bf(qv.y, kv[i].y, acc);
            acc = dot2bf(qv.z, kv[i].z, acc);
            acc = dot2bf(qv.w, kv[i].w, acc);
        }
        score = score + fmaxf(acc, 0.0f);
    }
    p.scores[size_t(t) * p.blocks + b] = score * QSA_SCALE;
}

// Inclusive prefix sum of one value per thread over a 256-thread workgroup (wave scans with
// lane shuffles, then the wave totals through LDS); `total` gets the sum of all 256.
// Integer sums: the order does not matter.
__device__ __forceinline__ uint32_t block_scan(uint32_t v, uint32_t* waves, uint32_t& total) {
    const int lane = int(threadIdx.x & 63), w = int(threadIdx.x >> 6);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(v, o, 64);
        if (lane >= o) v += y;
    }
    if (lane == 63) waves[w] = v;
    __syncthreads();
    uint32_t before = 0;
    total = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t x = waves[i];
        before += i < w ? x : 0u;
        total += x;
    }
    __syncthreads();  // waves[] is free again
    return v + before;
}

// Token t = blockIdx.x: visible = pos + 1 keys, complete = visible / 4 blocks, chosen =
// min(complete, budget / 4).  With chosen == complete every block is selected; otherwise
// the chosen blocks of largest value max(score, 0) (as FP32 bits: nonnegative floats order
// as integers), ties to the lower index (Kernels.metal:618-682): a radix search, 8 bits per
// pass from the top, for the chosen-th largest value v (each pass: a histogram of the next
// digit among the values matching the digits found so far; thread t holds digit 255 - t,
// and the one whose prefix sum from the top first reaches the remaining rank is the digit),
// then every block above v and the first (chosen - above) blocks equal to v in index order
// (thread i owns a contiguous run of blocks; its ties start after the prefix sum of the
// earlier runs' ties).  Output: bit b of mask word b / 32 (words up to p.words).
__global__ __launch_bounds__(256) void qsa_select_kernel(const QsaParams p) {
    __shared__ uint32_t hist[256], words[MAX_CONTEXT / 4 / 32], waves[4];
    __shared__ uint32_t s_prefix, s_rank;
    const int t = int(blockIdx.x), tid = int(threadIdx.x);
    if (p.state && (p.state->stopped || p.state->rows == 0)) return;
    const uint32_t visible = row_pos(p, t) + 1, complete = visible / 4;
    const uint32_t chosen = min(complete, uint32_t(p.budget) / 4);
    uint32_t* out = p.mask + size_t(t) * p.words;
    const float* sc = p.scores + size_t(t) * p.blocks;
    for (uint32_t i = uint32_t(tid); i < p.words; i += 256) words[i] = 0;
    __syncthreads();
    if (chosen == complete) {
        for (uint32_t b = uint32_t(tid); b < complete; b += 256) atomicOr(&words[b >> 5], 1u << (b & 31));
    } else if (chosen > 0) {
        auto value = [&](uint32_t b) { const float s = sc[b]; return __float_as_uint(s > 0.f ? s : 0.f); };
        if (tid == 0) { s_prefix = 0; s_rank = chosen; }
        for (int shift = 24; shift >= 0; shift -= 8) {
            hist[tid] = 0;
            __syncthreads();  // also orders the last pass's s_prefix / s_rank before these reads
            const uint32_t prefix = s_prefix, rank = s_rank;
            const uint32_t mask = shift == 24 ? 0u : ~0u << (shift + 8);
            for (uint32_t b = uint32_t(tid); b < complete; b += 256) {
                const uint32_t v = value(b);
                if ((v & mask) == prefix) atomicAdd(&hist[(v >> shift) & 255u], 1u);
            }
            __syncthreads();
            const uint32_t c = hist[255 - tid], d = uint32_t(255 - tid);
            uint32_t total;
            const uint32_t incl = block_scan(c, waves, total);
            // count above digit d: incl - c; exactly one thread sees the rank inside its bin
            if (incl - c < rank && rank <= incl) {
                s_prefix = prefix | (d << shift);
                s_rank = rank - (incl - c);
            }
        }
        __syncthreads();
        const uint32_t v = s_prefix;
        const uint32_t run = (complete + 255) / 256, b0 = uint32_t(tid) * run, b1 = min(b0 + run, complete);
        uint32_t above = 0, eq = 0;
        for (uint32_t b = b0; b < b1; ++b) {
            const uint32_t x = value(b);
            above += x > v;
            eq += x == v;
        }
        uint32_t total_above, total_eq;
        block_scan(above, waves, total_above);
        const uint32_t eq_incl = block_scan(eq, waves, total_eq);
        const uint32_t allowance = chosen - total_above;
        uint32_t seen = eq_incl - eq;  // ties in the runs of threads before this one
        for (uint32_t b = b0; b < b1; ++b) {
            const uint32_t x = value(b);
            bool take = x > v;
            if (x == v) { take = seen < allowance; ++seen; }
            if (take) atomicOr(&words[b >> 5], 1u << (b & 31));
        }
    }
    __syncthreads();
    for (uint32_t i = uint32_t(tid); i < p.words; i += 256) out[i] = words[i];
}

bool qsa_shape_ok(const QsaParams& p) {
    return p.tokens >= 1 && p.words <= uint32_t(MAX_CONTEXT / 4 / 32) && p.words * 32 >= p.blocks;
}

}  // namespace

void launch_qsa_select(const QsaParams& p, hipStream_t s) {
    if (!qsa_shape_ok(p) || p.state || p.budget < 0 || uint64_t(p.p0) + uint64_t(p.tokens) > 4ull * p.blocks + 3)
        throw Error(E_INVAL, "QSA select: bad shape");
    hipLaunchKernelGGL(qsa_select_kernel, dim3(p.tokens), dim3(256), 0, s, p);
}

void launch_qsa(const QsaParams& p, int max_blocks, hipStream_t s) {
    if (!qsa_shape_ok(p)) throw Error(E_INVAL, "QSA: bad shape");
    hipLaunchKernelGGL(qsa_prep_kernel, dim3(p.tokens), dim3(256), 0, s, p);
    // decode: at most one block completes per step; a chunk completes up to (n + 3) / 4
    const int pools = p.state ? 1 : (p.tokens + 3) / 4 + 1;
    hipLaunchKernelGGL(qsa_pool_kernel, dim3(pools), dim3(64), 0, s, p);
    hipLaunchKernelGGL(qsa_scores_kernel, dim3((max_blocks + 63) / 64, p.tokens), dim3(64), 0, s, p);
    hipLaunchKernelGGL(qsa_select_kernel, dim3(p.tokens), dim3(256), 0, s, p);
}

}  // namespace plamo
