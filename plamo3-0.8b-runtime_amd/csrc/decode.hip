// Decode-step kernels for gfx950 (CDNA4, wave64).
//
//   gemv_kernel       BF16 / .p12 GEMV for 1..4 activation rows with fused prologues
//                     (embedding gather + RMSNorm; post-norm + residual + next norm) and
//                     epilogues (BF16 rounding; SwiGLU; BF16 logits + sampler + argmax).
//                     Replaces linear / project3 / project4 / norm / swiglu / argmax
//                     (Kernels.metal:46-114,202-210,704-729; Batch.metal:171-221).
//   attn_decode       split-K (flash-decoding) attention over the ring or global KV with
//                     fused q/k RMSNorm, RoPE and KV write; the last workgroup merges.
//                     Replaces qkv / matrix_rotary / softmax / attend / attention /
//                     attention_merge and the mapped batch variants
//                     (Kernels.metal:223-562; Batch.metal:1-168).
//   step_begin        per-step bookkeeping of the device-driven token loop and the
//                     sampler history (counts, no-repeat-n-gram ban).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "device.h"
#include "kernels.h"

namespace plamo {
using namespace dev;

namespace {

// ------------------------------------------------------------------------ step timeline
#ifdef PLAMO_TIMELINE
__device__ uint64_t g_timeline[TIMELINE_TAGS * TIMELINE_BLOCKS * 2];
// Thread 0 of each workgroup stores the workgroup's first and last stamp when it ends.
struct TimelineScope {
    uint64_t t0;
    uint32_t tag;
    __device__ explicit TimelineScope(uint32_t t) : t0(__builtin_amdgcn_s_memrealtime()), tag(t) {}
    __device__ ~TimelineScope() {
        if (threadIdx.x != 0 || tag >= uint32_t(TIMELINE_TAGS)) return;
        const uint32_t b = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        if (b >= uint32_t(TIMELINE_BLOCKS)) return;
        const size_t i = (size_t(tag) * TIMELINE_BLOCKS + b) * 2;
        g_timeline[i] = t0;
        g_timeline[i + 1] = __builtin_amdgcn_s_memrealtime();
    }
};
#define PLAMO_TIMELINE_SCOPE(tag) TimelineScope timeline_scope_(tag)
#else
#define PLAMO_TIMELINE_SCOPE(tag) (void)0
#endif

// Weight rows per wave group: four for one activation row; with four rows the
// arithmetic per weight byte quadruples, so groups shrink to spread it over more waves
// (SwiGLU: one gate and one up row, three groups for each of a CU's eight waves).  The
// one-row .p12 down projection takes one row per group: 384 workgroups instead of 192
// hide its block decode behind more waves (.p12 step 0.542 -> 0.524 ms; plain rows keep two).
template <int N, int MAXR, int EPI, bool PACKED>
constexpr int gemv_u() {
    if constexpr (EPI == EPI_SWIGLU) return MAXR == 1 ? 4 : 2;
    else if constexpr (N >= 6144) return MAXR == 1 ? (PACKED ? 1 : 2) : 1;
    else return MAXR == 1 ? (N == ATTN ? 2 : 4) : 2;
}

// Waves per workgroup.  Four-row kernels with a norm prologue or 6144-wide rows run eight
// waves: each half of the workgroup stages two of the rows (every row with the same
// ownership of elements by its 256 threads, so the same sums), and one workgroup per CU
// does the prologue once for twice the waves.
__host__ __device__ constexpr int gemv_waves(int n, int maxr, int epi) {
    (void)epi;
    return maxr > 1 && (n == HIDDEN || n == INTER) ? 8 : 4;
}

// ---------------------------------------------------------------------------- prologues
// Staged activation rows in LDS: BF16, row-major, so the 8 columns a lane owns are one
// 16-byte read at 16-byte lane strides (no bank conflicts), in the pair form v_dot2 takes.
// (Four 6144-wide rows take 48 KB.)

// Stage the BF16 activation rows into LDS.  Values are BF16-exact FP32 (every producer
// rounds), so the BF16 copy is lossless.  The prologue is split into its loads
// (stage_load) and its arithmetic (stage_finish) so the kernel can request the first
// weights in between: the vector-memory counter is in order, and inputs requested before
// the weights can be consumed while the weights are still in flight.  A group of 256
// threads stages rows q0 .. q0+RQ-1 (thread t owns the same elements of every row).
template <int N, int RQ, int PRO>
struct Staged {
    static constexpr int V = (N + 1023) / 1024;  // PLAIN: float4 per thread and row
    static constexpr int V16 = (N + 2047) / 2048; // PLAIN16: 8 BF16 per thread and row
    static constexpr int E = HIDDEN / 256;       // norm prologues: elements per thread (6t .. 6t+5)
    float4 v[PRO == PRO_PLAIN ? RQ : 1][V];
    uint4 h[PRO == PRO_PLAIN16 || PRO == PRO_MERGE ? RQ : 1][V16];
    float4 mo[PRO == PRO_MERGE ? int(MERGE_IN_O) : 1][2];  // MERGE: partition outputs, 8 dims
    float2 ml[PRO == PRO_MERGE ? int(MERGE_IN_O) : 1];     // MERGE: partition (m, l) of the head
    uint32_t pos;                                          // MERGE: the row's position
    float2 a[PRO == PRO_RESID ? RQ : 1][E / 2];   // RESID: projection output
    float2 r[PRO == PRO_RESID ? RQ : 1][E / 2];   // RESID: residual stream
    uint32_t a16[PRO == PRO_RESID16 ? RQ : 1][E / 2];  // RESID16: projection output (BF16 pairs)
    uint32_t r16[PRO == PRO_RESID16 ? RQ : 1][E / 2];  // RESID16: residual stream (BF16 pairs)
    uint32_t emb[PRO == PRO_EMBED ? RQ : 1][E / 2];  // EMBED: embedding row (BF16 pairs)
    uint32_t gp[E / 2], gn[E / 2];                 // norm weights (BF16 pairs)

    // Holds the wave here until every prologue input has arrived (each register is named
    // as an input of an empty asm statement, so the compiler waits for its load), without
    // consuming them: requests issued after this call are not queued ahead of the inputs.
    __device__ __forceinline__ void wait_arrived() const {
        if constexpr (PRO == PRO_PLAIN16) {
#pragma unroll
            for (int qi = 0; qi < RQ; ++qi)
#pragma unroll
                for (int k = 0; k < V16; ++k) asm volatile("" ::"v"(h[qi][k].x), "v"(h[qi][k].y), "v"(h[qi][k].z), "v"(h[qi][k].w));
        } else if constexpr (PRO == PRO_RESID16 || PRO == PRO_RESID || PRO == PRO_EMBED) {
#pragma unroll
            for (int k = 0; k < E / 2; ++k) asm volatile("" ::"v"(gn[k]));
#pragma unroll
            for (int qi = 0; qi < RQ; ++qi)
#pragma unroll
                for (int k = 0; k < E / 2; ++k) {
                    if constexpr (PRO == PRO_RESID16) asm volatile("" ::"v"(a16[qi][k]), "v"(r16[qi][k]), "v"(gp[k]));
                    else if constexpr (PRO == PRO_RESID) asm volatile("" ::"v"(a[qi][k].x), "v"(a[qi][k].y), "v"(r[qi][k].x), "v"(r[qi][k].y), "v"(gp[k]));
                    else asm volatile("" ::"v"(emb[qi][k]));
                }
        }
    }
};

// Unconditional loads (rows past rb re-read row rb-1, columns past N re-read the last
// four), kept raw: converting them here would make the compiler wait for each one.
// rb: rows the input buffers hold.
template <int N, int RQ, int PRO>
__device__ __forceinline__ void stage_load(const GemvParams& p, int rb, int q0, Staged<N, RQ, PRO>& S) {
    const int tid = threadIdx.x & 255;
    constexpr int V = Staged<N, RQ, PRO>::V, V16 = Staged<N, RQ, PRO>::V16, E = Staged<N, RQ, PRO>::E;
    if constexpr (PRO == PRO_PLAIN) {
#pragma unroll
        for (int qi = 0; qi < RQ; ++qi) {
            const int q = q0 + qi, qq = q < rb ? q : rb - 1;
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const int e = (tid + 256 * k) * 4;
                S.v[qi][k] = *reinterpret_cast<const float4*>(p.in + qq * N + (e < N ? e : N - 4));
            }
        }
    } else if constexpr (PRO == PRO_PLAIN16) {
#pragma unroll
        for (int qi = 0; qi < RQ; ++qi) {
            const int q = q0 + qi, qq = q < rb ? q : rb - 1;
#pragma unroll
            for (int k = 0; k < V16; ++k) {
                const int e = (tid + 256 * k) * 8;
                S.h[qi][k] = *reinterpret_cast<const uint4*>(p.in16 + qq * N + (e < N ? e : N - 8));
            }
        }
    } else if constexpr (PRO == PRO_MERGE) {
        // thread t: dims 8t .. 8t+7 = dims 8(t % 16) .. of head t / 16.  Both sources are
        // requested: the attention output, and the first MERGE_IN_O partitions of the head
        // (indices past the buffer's partitions re-read the last one); which one is used
        // depends on the row's position, known only when the step state arrives.
        static_assert(N == ATTN && RQ == 1 && V16 == 1, "one-row o projection");
        S.h[0][0] = *reinterpret_cast<const uint4*>(p.in16 + tid * 8);
        const uint32_t h = uint32_t(tid) >> 4, d0 = (uint32_t(tid) & 15u) * 8;
#pragma unroll
        for (uint32_t k = 0; k < MERGE_IN_O; ++k) {
            const uint32_t kk = k < p.parts ? k : p.parts - 1;
            const float* o = p.part_o + (size_t(kk) * HEADS + h) * HEAD_DIM + d0;
            S.mo[k][0] = *reinterpret_cast<const float4*>(o);
            S.mo[k][1] = *reinterpret_cast<const float4*>(o + 4);
            S.ml[k] = make_float2(p.part_m[kk * HEADS + h], p.part_l[kk * HEADS + h]);
        }
    } else {
        static_assert(N == HIDDEN && E == 6, "norm prologue is 1536 wide");
        const int e0 = tid * E;
        const uint32_t* gn32 = reinterpret_cast<const uint32_t*>(p.g_next + e0);
#pragma unroll
        for (int k = 0; k < E / 2; ++k) S.gn[k] = gn32[k];
        if constexpr (PRO == PRO_EMBED) {
#pragma unroll
            for (int qi = 0; qi < RQ; ++qi) {
                const int q = q0 + qi, qq = q < rb ? q : rb - 1;
                int tok = p.state->token[qq];  // the embedding prologue always runs with a step state
                tok = (tok < 0 || tok >= VOCAB) ? 0 : tok;  // loop guards stop before this
                const uint32_t* row = reinterpret_cast<const uint32_t*>(p.embed + size_t(tok) * HIDDEN + e0);
#pragma unroll
                for (int k = 0; k < E / 2; ++k) S.emb[qi][k] = row[k];
            }
        } else {
            const uint32_t* gp32 = reinterpret_cast<const uint32_t*>(p.g_post + e0);
#pragma unroll
            for (int k = 0; k < E / 2; ++k) S.gp[k] = gp32[k];
#pragma unroll
            for (int qi = 0; qi < RQ; ++qi) {
                const int q = q0 + qi, qq = q < rb ? q : rb - 1;
#pragma unroll
                for (int k = 0; k < E / 2; ++k) {
                    if constexpr (PRO == PRO_RESID16) {
                        S.a16[qi][k] = *reinterpret_cast<const uint32_t*>(p.in16 + qq * HIDDEN + e0 + 2 * k);
                        S.r16[qi][k] = *reinterpret_cast<const uint32_t*>(p.resid16_in + qq * HIDDEN + e0 + 2 * k);
                    } else {
                        S.a[qi][k] = *reinterpret_cast<const float2*>(p.in + qq * HIDDEN + e0 + 2 * k);
                        S.r[qi][k] = *reinterpret_cast<const float2*>(p.resid_in + qq * HIDDEN + e0 + 2 * k);
                    }
                }
            }
        }
    }
}

// 1 / sqrt(mean square + eps) of rows q0 .. q0+RQ-1 from the four wave partials in red:
// with several rows, lane i computes row q0 + i (one sequence for all rows) and the scales
// are read back from those lanes.
template <int RQ>
__device__ __forceinline__ void row_scales(const float* red, int q0, float (&rs)[RQ]) {
    const auto scale = [&](int q) {
        const float total = (red[q * 4] + red[q * 4 + 1]) + (red[q * 4 + 2] + red[q * 4 + 3]);
        return 1.0f / sqrtf(total / float(HIDDEN) + 1e-6f);
    };
    if constexpr (RQ == 1) {
        rs[0] = scale(q0);
    } else {
        static_assert((RQ & (RQ - 1)) == 0, "rows per group: a power of two");
        const float r = scale(q0 + int(threadIdx.x & (RQ - 1)));
#pragma unroll
        for (int qi = 0; qi < RQ; ++qi) rs[qi] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(r), qi));
    }
}

// Every LDS row is written: rows past the step's hold re-read buffer rows or zeros, so the
// main loop can run all MAXR rows without branches (their results are never stored).
template <int N, int MAXR, int RQ, int PRO>
__device__ __forceinline__ void stage_finish(const GemvParams& p, int rows, int q0, const Staged<N, RQ, PRO>& S,
                                             uint16_t* xs, float* red) {
    const int tid = threadIdx.x & 255;
    constexpr int V = Staged<N, RQ, PRO>::V, V16 = Staged<N, RQ, PRO>::V16, E = Staged<N, RQ, PRO>::E;
    if constexpr (PRO == PRO_PLAIN) {
#pragma unroll
        for (int qi = 0; qi < RQ; ++qi) {
            const int q = q0 + qi;
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const int e = (tid + 256 * k) * 4;
                if (e >= N) continue;
                const uint32_t lo2 = (bits(S.v[qi][k].x) & 0xffffu) | (bits(S.v[qi][k].y) << 16);
                const uint32_t hi2 = (bits(S.v[qi][k].z) & 0xffffu) | (bits(S.v[qi][k].w) << 16);
                *reinterpret_cast<uint2*>(&xs[q * N + e]) = make_uint2(lo2, hi2);
            }
        }
    } else if constexpr (PRO == PRO_MERGE) {
        // The attention kernel's merge (same operations, same partition order): M = max m_p,
        // w_p = exp(m_p - M), den = sum l_p w_p, num = sum o_p w_p, out = bf16(num / den).
#pragma clang fp contract(off)
        const uint32_t count = p.merge_full ? S.pos + 1 : (S.pos > uint32_t(WINDOW - 1) ? uint32_t(WINDOW) : S.pos + 1);
        const uint32_t nparts = (count + KEYS_PER_PART - 1) / KEYS_PER_PART;
        float v[8];
        if (nparts >= 2 && nparts <= MERGE_IN_O) {
            float M = NEG_INF;
#pragma unroll
            for (uint32_t k = 0; k < MERGE_IN_O; ++k)
                if (k < nparts) M = fmaxf(M, S.ml[k].x);
            float num[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, den = 0.f;
#pragma unroll
            for (uint32_t k = 0; k < MERGE_IN_O; ++k) {
                if (k >= nparts) break;
                const float w = exp_det(S.ml[k].x - M);
                den = den + S.ml[k].y * w;
                const float o[8] = {S.mo[k][0].x, S.mo[k][0].y, S.mo[k][0].z, S.mo[k][0].w,
                                    S.mo[k][1].x, S.mo[k][1].y, S.mo[k][1].z, S.mo[k][1].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) num[j] = num[j] + o[j] * w;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = roundbf(num[j] / den);
        } else {
            const uint4 hw = S.h[0][0];
            const uint32_t w4[4] = {hw.x, hw.y, hw.z, hw.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = lo(w4[j]);
                v[2 * j + 1] = hi(w4[j]);
            }
        }
        *reinterpret_cast<uint4*>(&xs[tid * 8]) = make_uint4(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]),
                                                            pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7]));
    } else if constexpr (PRO == PRO_PLAIN16) {
#pragma unroll
        for (int qi = 0; qi < RQ; ++qi) {
            const int q = q0 + qi;
#pragma unroll
            for (int k = 0; k < V16; ++k) {
                const int e = (tid + 256 * k) * 8;
                if (e >= N) continue;
                *reinterpret_cast<uint4*>(&xs[q * N + e]) = S.h[qi][k];
            }
        }
    } else {
        const int wq = tid >> 6;  // this thread's wave within its group of four
        float xv[RQ][E];
        float ss[RQ];
        if constexpr (PRO == PRO_EMBED) {
#pragma unroll
            for (int qi = 0; qi < RQ; ++qi)
#pragma unroll
                for (int k = 0; k < E / 2; ++k) {
                    xv[qi][2 * k] = (q0 + qi < rows) ? lo(S.emb[qi][k]) : 0.f;
                    xv[qi][2 * k + 1] = (q0 + qi < rows) ? hi(S.emb[qi][k]) : 0.f;
                }
        } else {
            // z = roundbf(roundbf(p*r) * roundbf(bf(w)+offset)); x = roundbf(x + z)
            // (Kernels.metal:59-72, full == 1)
            float pv[RQ][E], rv[RQ][E], gp[E];
#pragma unroll
            for (int k = 0; k < E / 2; ++k) {
                gp[2 * k] = lo(S.gp[k]);
                gp[2 * k + 1] = hi(S.gp[k]);
            }
#pragma unroll
            for (int qi = 0; qi < RQ; ++qi)
#pragma unroll
                for (int k = 0; k < E / 2; ++k) {
                    if constexpr (PRO == PRO_RESID16) {
                        pv[qi][2 * k] = lo(S.a16[qi][k]);
                        pv[qi][2 * k + 1] = hi(S.a16[qi][k]);
                        rv[qi][2 * k] = lo(S.r16[qi][k]);
                        rv[qi][2 * k + 1] = hi(S.r16[qi][k]);
                    } else {
                        pv[qi][2 * k] = S.a[qi][k].x;
                        pv[qi][2 * k + 1] = S.a[qi][k].y;
                        rv[qi][2 * k] = S.r[qi][k].x;
                        rv[qi][2 * k + 1] = S.r[qi][k].y;
                    }
                }
#pragma unroll
            for (int qi = 0; qi < RQ; ++qi) {
                ss[qi] = 0.f;
#pragma unroll
                for (int k = 0; k < E; ++k) ss[qi] += pv[qi][k] * pv[qi][k];
            }
#pragma unroll
            for (int qi = 0; qi < RQ; ++qi) {
                ss[qi] = wave_sum(ss[qi]);
                if ((tid & 63) == 0) red[(q0 + qi) * 4 + wq] = ss[qi];
            }
            __syncthreads();
            // BF16 roundings two at a time (packed RNE conversion, identical to `roundbf`)
            float g[E];
#pragma unroll
            for (int k = 0; k < E; k += 2) round_bf16x2(gp[k] + p.post_offset, gp[k + 1] + p.post_offset, g[k], g[k + 1]);
            float rs[RQ];
            row_scales<RQ>(red, q0, rs);
#pragma unroll
            for (int qi = 0; qi < RQ; ++qi) {
                const int q = q0 + qi;
                const float r = rs[qi];
#pragma unroll
                for (int k = 0; k < E; k += 2) {
                    float t0, t1, z0, z1, x0, x1;
                    round_bf16x2(pv[qi][k] * r, pv[qi][k + 1] * r, t0, t1);
                    round_bf16x2(t0 * g[k], t1 * g[k + 1], z0, z1);
                    round_bf16x2(rv[qi][k] + z0, rv[qi][k + 1] + z1, x0, x1);
                    xv[qi][k] = (q < rows) ? x0 : 0.f;
                    xv[qi][k + 1] = (q < rows) ? x1 : 0.f;
                }
            }
            red += MAXR * 4;  // the next norm's partials go to the second half (no barrier)
        }
        // next norm with +1 offset (Kernels.metal:76-89)
        float gn[E];
#pragma unroll
        for (int k = 0; k < E / 2; ++k) round_bf16x2(lo(S.gn[k]) + 1.0f, hi(S.gn[k]) + 1.0f, gn[2 * k], gn[2 * k + 1]);
#pragma unroll
        for (int qi = 0; qi < RQ; ++qi) {
            ss[qi] = 0.f;
#pragma unroll
            for (int k = 0; k < E; ++k) ss[qi] += xv[qi][k] * xv[qi][k];
            ss[qi] = wave_sum(ss[qi]);
            if ((tid & 63) == 0) red[(q0 + qi) * 4 + wq] = ss[qi];
        }
        __syncthreads();
        float rs[RQ];
        row_scales<RQ>(red, q0, rs);
#pragma unroll
        for (int qi = 0; qi < RQ; ++qi) {
            const int q = q0 + qi;
            const float r = rs[qi];
#pragma unroll
            for (int k = 0; k < E; k += 2) {
                const int i = tid * E + k;
                float t0, t1;
                round_bf16x2(xv[qi][k] * r, xv[qi][k + 1] * r, t0, t1);
                const uint32_t xn2 = pack_bf16(t0 * gn[k], t1 * gn[k + 1]);  // the two BF16 results
                *reinterpret_cast<uint32_t*>(&xs[q * HIDDEN + i]) = xn2;
                if (blockIdx.x == 0 && q < rows) {
                    if constexpr (PRO == PRO_RESID) {
                        p.resid_out[q * HIDDEN + i] = xv[qi][k];
                        p.resid_out[q * HIDDEN + i + 1] = xv[qi][k + 1];
                    } else {  // BF16-exact residual: the BF16 pair is lossless
                        *reinterpret_cast<uint32_t*>(&p.resid16_out[q * HIDDEN + i]) = pack_bf16(xv[qi][k], xv[qi][k + 1]);
                    }
                    if (p.hidden) {
                        const size_t hrow = p.state ? size_t(p.state->lane[q]) : size_t(q);
                        p.hidden[hrow * HIDDEN + i] = lo(xn2);
                        p.hidden[hrow * HIDDEN + i + 1] = hi(xn2);
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------------- weight loads
// Lane `lane` owns columns it*512 + lane*8 .. +8 of a row: inside .p12 block it*4+lane/16
// at offset (lane%16)*8.  Plain and packed therefore feed identical words to dot8, so
// packed results are bit-identical to plain ones.
// A lane's weight words as requested, decoded only when used (decoding at request time
// would make the compiler wait for each load).  .p12: a 128-weight block is 256 raw bytes
// (tag 0) or 128 sign/mantissa bytes + 64 exponent-nibble bytes; two branch-free loads
// cover both layouts and stay inside the block.
template <bool PACKED>
struct WRaw {
    uint4 v;
};
// Weight streams are read once per step: non-temporal loads, so they do not displace the
// activations, KV rows and .p12 tables from the caches.
__device__ __forceinline__ uint4 stream_load16(const void* p) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const v4 v = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 stream_load8(const void* p) {
    typedef uint32_t v2 __attribute__((ext_vector_type(2)));
    const v2 v = __builtin_nontemporal_load(reinterpret_cast<const v2*>(p));
    return make_uint2(v[0], v[1]);
}
template <>
struct WRaw<true> {
    uint2 a;       // raw: weights 0..3; packed: the 8 sign/mantissa bytes
    uint2 b;       // raw: weights 4..7; packed: the exponent codes of this lane and its pair
    uint32_t tag;  // block minimum - 107 (0: raw block)
};

// Plain weight requests for U rows x IT column steps.
template <int N, int U, int IT>
__device__ __forceinline__ void request_plain(const GemvParams& p, const int (&wrow)[U], int lane,
                                              WRaw<false> (&r)[U][IT]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int it = 0; it < IT; ++it)
            r[u][it].v = stream_load16(p.w + size_t(wrow[u]) * N + it * 512 + lane * 8);
}

// .p12 requests come in two halves: the block-table entries of U rows x IT column steps,
// then (once they arrived) the payload at the offsets they hold.  The kernel issues the
// table half one group ahead, so only a wave's first group waits for two round trips.
template <int N, int U, int IT>
__device__ __forceinline__ void request_table(const GemvParams& p, const int (&wrow)[U], int lane,
                                              uint32_t (&e)[U][IT]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int it = 0; it < IT; ++it) e[u][it] = p.table[size_t(wrow[u]) * (N / 128) + it * 4 + (lane >> 4)];
}

template <int U, int IT>
__device__ __forceinline__ void request_payload(const GemvParams& p, const uint32_t (&e)[U][IT], int lane,
                                                WRaw<true> (&r)[U][IT]) {
    const int sub = lane & 15;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const uint8_t* blk = reinterpret_cast<const uint8_t*>(p.w) + (e[u][it] & ~63u);
            const uint32_t tag = e[u][it] & 63u;
            // two naturally aligned 8-byte loads, branch-free: a raw block's 16 bytes, or
            // (packed) this lane's 8 sign/mantissa bytes and the 8 exponent-code bytes of its
            // lane pair (the two lanes of a pair read the same word)
            r[u][it].a = stream_load8(blk + (tag ? sub * 8 : sub * 16));
            r[u][it].b = stream_load8(blk + (tag ? 128 + (sub & ~1) * 4 : sub * 16 + 8));
            r[u][it].tag = tag;
        }
}

// Lane `lane` owns columns it*512 + lane*8 .. +8 of a row: inside .p12 block it*4+lane/16
// at offset (lane%16)*8.  Plain and packed therefore feed identical words to dot8, so
// packed results are bit-identical to plain ones.
template <bool PACKED>
__device__ __forceinline__ uint4 decode_w(const WRaw<PACKED>& r) {
    if constexpr (!PACKED) return r.v;
    else {
        if (!r.tag) return make_uint4(r.a.x, r.a.y, r.b.x, r.b.y);
        const uint32_t nib = (threadIdx.x & 1u) ? r.b.y : r.b.x;  // lane parity = sub parity
        return p12_decode8(r.a, nib, r.tag);
    }
}

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);  // Kernels.metal:716
}

template <int O>
__device__ __forceinline__ void best_step(float& bv, uint32_t& bi) {
    const float v = xor_lane<O>(bv);
    const uint32_t i = xor_lane<O>(bi);
    if (better(v, i, bv, bi)) { bv = v; bi = i; }
}
// First maximum over the wavefront (the selection is order-independent).
__device__ __forceinline__ void wave_best(float& bv, uint32_t& bi) {
    best_step<32>(bv, bi);
    best_step<16>(bv, bi);
    best_step<8>(bv, bi);
    best_step<4>(bv, bi);
    best_step<2>(bv, bi);
    best_step<1>(bv, bi);
}

struct Controls {
    bool on;
    int ngram;
    float penalty, frequency, presence;
};

// Sampler.select adjustments of one logit (Sampler.swift:11-24), FP32, no contraction.
__device__ __forceinline__ float sampled(float l, int32_t count, bool banned, const Controls& c) {
#pragma clang fp contract(off)
    if (count > 0) {
        if (c.penalty != 1.0f) l = l > 0.0f ? l / c.penalty : l * c.penalty;
        if (c.presence != 0.0f) l = l - c.presence;
        if (c.frequency != 0.0f) {
            const float f = c.frequency * float(count);
            l = l - f;
        }
    }
    return banned ? NEG_INF : l;
}

// ------------------------------------------------------------------------------- GEMV
template <int N, bool PACKED, int MAXR, int PRO, int EPI, bool STATE>
__global__ __launch_bounds__(64 * gemv_waves(N, MAXR, EPI)) void gemv_kernel(const GemvParams p) {
    PLAMO_TIMELINE_SCOPE(p.tag);
    constexpr int NWV = gemv_waves(N, MAXR, EPI);
    constexpr int IT = N / 512;
    constexpr int U = gemv_u<N, MAXR, EPI, PACKED>();
    constexpr int H = U / 2;  // SwiGLU: gate rows (and up rows) per group
    __shared__ __align__(16) uint16_t xs[MAXR * N];
    __shared__ float red[MAXR * 4 * 2];  // norm partials: post-norm half, next-norm half
    __shared__ float cand_v[MAXR * NWV];
    __shared__ uint32_t cand_i[MAXR * NWV];

    const StepState* st = p.state;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // prologue groups of 256 threads: with eight waves, each half stages half of the rows
    constexpr int NH = NWV / 4, RQ = MAXR / NH > 0 ? MAXR / NH : 1;
    static_assert(MAXR % NH == 0 || MAXR == 1, "rows split evenly over the prologue groups");
    const int q0 = (wave >> 2) * RQ;
    const int groups = p.m / U;
    // Request order = consumption order: step state, prologue inputs, first weights.  The
    // state is read through a lane-dependent address (lane_mask is 0, so every lane reads
    // the same words): that makes it a vector load, first in the in-order vector-memory
    // queue, instead of a scalar load whose wait would also cover the kernel arguments the
    // weight addresses need.
    auto rows_of = [&](int g, int (&wrow)[U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (EPI == EPI_SWIGLU) wrow[u] = (u < H) ? H * g + u : INTER + H * g + (u - H);
            else wrow[u] = g * U + u;
        }
    };
    // Software pipelined over the wave's row groups: the next group's weights are in flight
    // while the current group is reduced and written.  The first group's weights do not
    // depend on the previous kernel, so they are requested before the activation prologue.
    // Four-row kernels: each workgroup takes an equal run of consecutive row groups, its
    // waves in turn (every CU does the same work when groups do not divide evenly over the
    // waves).  One row: groups dealt over the whole grid.
    int g, gend, stride;
    if constexpr (MAXR > 1) {
        const int per = (groups + int(gridDim.x) - 1) / int(gridDim.x);
        gend = min(int(blockIdx.x) * per + per, groups);
        stride = NWV;
        g = int(blockIdx.x) * per + wave;
    } else {
        gend = groups;
        stride = int(gridDim.x) * NWV;
        g = int(blockIdx.x) * NWV + wave;
    }
    // .p12: the first group's block-table entries go out before anything else, so their
    // round trip overlaps the state and prologue loads (unconditional: a wave without a
    // group re-reads the last one, and the compiler counts the requests in flight exactly)
    uint32_t tab[PACKED ? U : 1][PACKED ? IT : 1];
    if constexpr (PACKED) {
        int wrow[U];
        rows_of(g < groups ? g : groups - 1, wrow);
        request_table<N, U, IT>(p, wrow, lane, tab);
    }
    uint32_t stopped = 0, srows = 0, spos = 0;
    if constexpr (STATE) {
        const StepState* sv = st + (threadIdx.x & p.lane_mask);
        stopped = sv->stopped;
        srows = sv->rows;
        if constexpr (PRO == PRO_MERGE) spos = sv->pos[0];
    }
    Staged<N, RQ, PRO> S;
    stage_load<N, RQ, PRO>(p, p.rows < MAXR ? p.rows : MAXR, q0, S);
    float best_v[MAXR];
    uint32_t best_i[MAXR];
#pragma unroll
    for (int q = 0; q < MAXR; ++q) { best_v[q] = NEG_INF; best_i[q] = 0xffffffffu; }

    // Waves of the LM head and of the four-row kernels walk several groups: their next
    // group's table words are requested one group ahead.  The other launches give every wave
    // one group (gemv_blocks), and keep no table registers live past the first payload.
    constexpr bool PIPE_TABLE = MAXR > 1 || EPI == EPI_LOGITS;
    WRaw<PACKED> wr[U][IT];
    if constexpr (PACKED) {
        // the payload as soon as the table arrived (the prologue loads issued after the table
        // may still be in flight), then the next group's table
        request_payload<U, IT>(p, tab, lane, wr);
        if (PIPE_TABLE && g + stride < gend) {
            int wrow[U];
            rows_of(g + stride, wrow);
            request_table<N, U, IT>(p, wrow, lane, tab);
        }
    } else {
        // Four-row kernels: the prologue inputs (four rows, each workgroup's norms) are the
        // critical path; weights requested behind them would be queued ahead of the inputs of
        // other workgroups, so the first weights wait for this wave's inputs (batch 4
        // 5448 -> 5636 tok/s).  One-row kernels request them at once (their prologue is short,
        // and waiting costs 10 us per step).
        if constexpr (MAXR > 1) S.wait_arrived();
        int wrow[U];
        rows_of(g < groups ? g : groups - 1, wrow);
        request_plain<N, U, IT>(p, wrow, lane, wr);
    }
    // A stopped device loop runs the kernel with no rows (an early return here would let
    // the compiler sink every request above below a wait for the state).
    int rows = p.rows;
    if constexpr (STATE) rows = stopped ? 0 : int(srows);
    Controls ctl{false, 0, 1.0f, 0.0f, 0.0f};
    // logits rows land in the slot of the row's lane (lane-indexed outputs need no copies)
    uint32_t orow[MAXR];
#pragma unroll
    for (int q = 0; q < MAXR; ++q) orow[q] = uint32_t(q);
    if constexpr (EPI == EPI_LOGITS && STATE) {
        if (st->sampling) ctl = Controls{true, st->ngram, st->penalty, st->frequency, st->presence};
#pragma unroll
        for (int q = 0; q < MAXR; ++q) orow[q] = st->lane[q];
    }
    uint32_t orow_packed = 0;  // lanes are below 4: one byte each
#pragma unroll
    for (int q = 0; q < MAXR; ++q) orow_packed |= (orow[q] & 0xffu) << (8 * q);
    S.pos = spos;
    stage_finish<N, MAXR, RQ, PRO>(p, rows, q0, S, xs, red);
    __syncthreads();
    auto decode_all = [&](const WRaw<PACKED> (&cur)[U][IT], uint4 (&w)[U][IT]) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int it = 0; it < IT; ++it) w[u][it] = decode_w<PACKED>(cur[u][it]);
    };
    // One row group with its weights `w`.
    auto group = [&](const int g, const uint4 (&w)[U][IT]) {
        int wrow[U];
        rows_of(g, wrow);
        float acc[U][MAXR];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int q = 0; q < MAXR; ++q) acc[u][q] = 0.f;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
#pragma unroll
            for (int q = 0; q < MAXR; ++q) {
                if (MAXR > 1 && q >= rows) break;
                const uint4 xv = *reinterpret_cast<const uint4*>(&xs[q * N + it * 512 + lane * 8]);
#pragma unroll
                for (int u = 0; u < U; ++u) acc[u][q] = dot8(w[u][it], xv, acc[u][q]);
            }
        }
        if constexpr (EPI == EPI_ROUND || EPI == EPI_BF16 || EPI == EPI_SWIGLU || EPI == EPI_RAW) {
            // Reduce-scatter: lane holds the sum of value idx = u * MAXR + q, idx = lane >> S
            // (the gate/up split is the top bit of idx, so a SwiGLU gate lane finds its up
            // sum 32 lanes away).  Lane (idx << S) writes output (row q, weight row u).
            constexpr int K = U * MAXR, S = 6 - log2_pow2(K);
            float vals[K];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int q = 0; q < MAXR; ++q) vals[u * MAXR + q] = acc[u][q];
            const float t = wave_sum_scatter<K>(vals);
            const int idx = lane >> S, u = idx / MAXR, q = idx % MAXR;
            const bool writer = (lane & ((1 << S) - 1)) == 0 && q < rows;
            if constexpr (EPI == EPI_SWIGLU) {
                // gates = roundbf(g), ups = roundbf(u); y = roundbf(roundbf(g/(1+exp(-g))) * u)
                // (Kernels.metal:202-210)
                const float upv = xor_lane<32>(t);
                if (writer && u < H) {
                    const float gt = roundbf(t);
                    const float up = roundbf(upv);
                    p.out16[size_t(q) * INTER + H * g + u] = uint16_t(bits(roundbf(gt / (1.0f + exp_det(-gt))) * up));
                }
            } else {
                int r = wrow[0];
#pragma unroll
                for (int uu = 1; uu < U; ++uu)
                    if (uu == u) r = wrow[uu];
                if (writer) {
                    if constexpr (EPI == EPI_ROUND) p.out[size_t(q) * p.m + r] = roundbf(t);
                    else if constexpr (EPI == EPI_RAW) p.out[size_t(q) * p.m + r] = t;
                    else p.out16[size_t(q) * p.m + r] = uint16_t(bits(t));
                }
            }
        } else {  // EPI_LOGITS
            // Same reduce-scatter: lane holds the logit of value idx = lane >> S (weight row
            // u = idx / MAXR of row q = idx % MAXR), written by lane idx << S; every lane keeps
            // the first maximum of the values it held (its q never changes).
            constexpr int K = U * MAXR, S = 6 - log2_pow2(K);
            float vals[K];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int q = 0; q < MAXR; ++q) vals[u * MAXR + q] = acc[u][q];
            const float t = wave_sum_scatter<K>(vals);
            const int idx = lane >> S, u = idx / MAXR, q = idx % MAXR;
            if (q < rows) {
                const int r = g * U + u;                                   // rows_of for logits
                const uint32_t oq = (orow_packed >> (8 * q)) & 0xffu;     // lane of row q
                const uint32_t b = bits(t);
                if ((lane & ((1 << S) - 1)) == 0) p.out16[size_t(oq) * VOCAB + r] = uint16_t(b);
                float v = bf(b);
                if (ctl.on) {
                    const int32_t c = p.bufs.counts[size_t(q) * VOCAB + r];
                    const bool ban = ctl.ngram > 1 &&
                                     ((p.bufs.banned[size_t(q) * (VOCAB / 32) + (uint32_t(r) >> 5)] >> (r & 31)) & 1u);
                    v = sampled(v, c, ban, ctl);
                }
                if (better(v, uint32_t(r), best_v[0], best_i[0])) { best_v[0] = v; best_i[0] = uint32_t(r); }
            }
        }
    };
    if constexpr (!PACKED) {
        // plain weights: two request buffers in turn (the next group's requests land in the
        // other buffer, so no register copies between groups)
        WRaw<PACKED> wb[U][IT];
        for (; g < gend; g += 2 * stride) {
            const int g1 = g + stride, g2 = g1 + stride;
            int nrow[U];
            if (g1 < gend) {
                rows_of(g1, nrow);
                request_plain<N, U, IT>(p, nrow, lane, wb);
            }
            uint4 w[U][IT];
            decode_all(wr, w);
            group(g, w);
            if (g1 >= gend) break;
            if (g2 < gend) {
                rows_of(g2, nrow);
                request_plain<N, U, IT>(p, nrow, lane, wr);
            }
            decode_all(wb, w);
            group(g1, w);
        }
    } else {
        // .p12: decode, then request the next group's payload into the same buffer (fewer
        // registers than two buffers of payload, table words and tags) from the table words
        // requested one group earlier, and the table of the group after it
        for (; g < gend; g += stride) {
            uint4 w[U][IT];
            decode_all(wr, w);
            const int gn = g + stride;
            if (gn < gend) {
                if constexpr (!PIPE_TABLE) {
                    int nrow[U];
                    rows_of(gn, nrow);
                    request_table<N, U, IT>(p, nrow, lane, tab);
                }
                request_payload<U, IT>(p, tab, lane, wr);
                if (PIPE_TABLE && gn + stride < gend) {
                    int nrow[U];
                    rows_of(gn + stride, nrow);
                    request_table<N, U, IT>(p, nrow, lane, tab);
                }
            }
            group(g, w);
        }
    }

    if constexpr (EPI == EPI_LOGITS) {
        // block partial; head_merge_kernel reduces the partials of every block.  Lanes with
        // the same row q differ in the weight-row bits of the lane index (and in the low S
        // bits, which hold copies): first maximum over the weight-row bits, then lane q << S
        // holds the wave's best for row q.
        constexpr int K = U * MAXR, S = 6 - log2_pow2(K), QB = S + log2_pow2(MAXR);
        float bv = best_v[0];
        uint32_t bi = best_i[0];
        if constexpr (QB <= 5) best_step<32>(bv, bi);
        if constexpr (QB <= 4) best_step<16>(bv, bi);
        if constexpr (QB <= 3) best_step<8>(bv, bi);
        if constexpr (QB <= 2) best_step<4>(bv, bi);
        if constexpr (QB <= 1) best_step<2>(bv, bi);
        if constexpr (QB <= 0) best_step<1>(bv, bi);
        if ((lane & ((1 << S) - 1)) == 0 && (lane >> QB) == 0) {
            const int q = lane >> S;
            cand_v[q * NWV + wave] = bv;
            cand_i[q * NWV + wave] = bi;
        }
        __syncthreads();
        if (tid < MAXR && tid < rows) {
            const int q = tid;
            float bv = cand_v[q * NWV];
            uint32_t bi = cand_i[q * NWV];
            for (int k = 1; k < NWV; ++k)
                if (better(cand_v[q * NWV + k], cand_i[q * NWV + k], bv, bi)) { bv = cand_v[q * NWV + k]; bi = cand_i[q * NWV + k]; }
            p.bufs.head_v[q * HEAD_BLOCKS + blockIdx.x] = bv;
            p.bufs.head_i[q * HEAD_BLOCKS + blockIdx.x] = bi;
        }
    }
}

// First maximum over the LM-head block partials (Kernels.metal:704-729 semantics: ties to
// the lowest index, NaN never wins, none -> 0xffffffff; Sampler.select defaults to 0), then
// the device side of the token loop: feed the token back and advance the position.
// The step state travels as one parallel copy into LDS and back: the single-workgroup
// bookkeeping kernels then pay one memory round trip instead of one per dependent field.
constexpr int STATE_WORDS = int(sizeof(StepState) / 4);
static_assert(sizeof(StepState) % 4 == 0 && STATE_WORDS <= 256, "state copy: one word per thread");
__device__ __forceinline__ void state_in(StepState& ls, const StepState* st) {
    if (threadIdx.x < STATE_WORDS)
        reinterpret_cast<uint32_t*>(&ls)[threadIdx.x] = reinterpret_cast<const uint32_t*>(st)[threadIdx.x];
}
__device__ __forceinline__ void state_out(StepState* st, const StepState& ls) {
    if (threadIdx.x < STATE_WORDS)
        reinterpret_cast<uint32_t*>(st)[threadIdx.x] = reinterpret_cast<const uint32_t*>(&ls)[threadIdx.x];
}

__device__ void begin_step(StepState& ls, const DecodeBuffers& b, int* s_stop);

__global__ __launch_bounds__(256) void head_merge_kernel(DecodeBuffers b, int blocks, int begin_next) {
    PLAMO_TIMELINE_SCOPE(TL_HEAD_MERGE);
    __shared__ float cv[ROWS * 4];
    __shared__ uint32_t ci[ROWS * 4];
    __shared__ StepState ls;
    __shared__ int s_stop;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
    // every row's partials requested together with the state (rows past the step's are not used)
    constexpr int PER = HEAD_BLOCKS / 256;
    float pv[ROWS][PER];
    uint32_t pi[ROWS][PER];
#pragma unroll
    for (int q = 0; q < ROWS; ++q)
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int k = tid + 256 * j;
            pv[q][j] = k < blocks ? b.head_v[q * HEAD_BLOCKS + k] : NEG_INF;
            pi[q][j] = k < blocks ? b.head_i[q * HEAD_BLOCKS + k] : 0xffffffffu;
        }
    state_in(ls, b.state);
    __syncthreads();
    if (ls.stopped) return;
    const int rows = int(ls.rows);
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        if (q >= rows) break;
        float bv = NEG_INF;
        uint32_t bi = 0xffffffffu;
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (better(pv[q][j], pi[q][j], bv, bi)) { bv = pv[q][j]; bi = pi[q][j]; }
        wave_best(bv, bi);
        if (lane == 0) { cv[q * 4 + wave] = bv; ci[q * 4 + wave] = bi; }
    }
    __syncthreads();
    if (tid < rows && tid < ROWS) {
        const int q = tid;
        float bv = cv[q * 4];
        uint32_t bi = ci[q * 4];
        for (int k = 1; k < 4; ++k)
            if (better(cv[q * 4 + k], ci[q * 4 + k], bv, bi)) { bv = cv[q * 4 + k]; bi = ci[q * 4 + k]; }
        if (ls.sampling && bi == 0xffffffffu) bi = 0;  // Sampler.select default index (Sampler.swift:26)
        ls.next[q] = bi;
        if (ls.loop) {
            ls.token[q] = int32_t(bi);
            ls.pos[q] += 1;
        }
        if (ls.quad) {
            const uint32_t ln = ls.lane[q];
            ls.lnext[ln] = int32_t(bi);
            ls.lpos[ln] += 1;
            if (bi >= uint32_t(VOCAB)) { ls.stopped = 1; ls.reason = 3; }  // invalid prediction
        }
    }
    __syncthreads();
    // device loops: the next step's bookkeeping (emit, stop, lane pass, sampler history)
    if (begin_next && (ls.loop || ls.quad) && !ls.stopped) begin_step(ls, b, &s_stop);
    state_out(b.state, ls);
}

// ---------------------------------------------------------------------- decode attention
constexpr int KP = KEYS_PER_PART;
constexpr int HG = 4;                // heads per workgroup (HEADS / HG head groups per partition)
constexpr int KS = 68;               // padded LDS row of rotated keys: 64 BF16 pairs + 4 words

// Workgroup (partition x, head group y, row z): keys x*64 .. x*64+63 of the row's visible
// keys for heads 4y .. 4y+3.  All four head groups rotate the same keys; only group 0
// writes the newest key and value to the cache.
template <bool FULL>
__global__ __launch_bounds__(256) void attn_decode_kernel(const AttnParams p) {
#pragma clang fp contract(off)  // fixed rounding sequence, reproduced by the CPU oracle
    PLAMO_TIMELINE_SCOPE(p.tag);
    __shared__ __align__(16) uint32_t qs[HG * HEAD_DIM / 2];  // BF16 pairs (dims 2i, 2i + 1)
    __shared__ __align__(16) uint32_t ks[KP * KS];            // BF16 pairs
    __shared__ __align__(16) uint16_t vs[KP * HEAD_DIM];
    __shared__ __align__(16) float ps[HG * KP];
    __shared__ __align__(16) float knew[HEAD_DIM];
    __shared__ float l_s[HG];
    __shared__ float den_s[HG];
    __shared__ int s_last;

    const StepState* st = p.state;
    // workgroup -> (partition, head group): the four head groups of a partition share
    // id % 8, so they run on one XCD and read its keys and values through one L2 (ids of
    // partitions past p.parts return below)
    const uint32_t wid = blockIdx.x;
    const uint32_t part = (wid >> 5) * 8u + (wid & 7u);
    const int q = int(blockIdx.z + p.row0), hg = int((wid >> 3) & 3u);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
    // ---- loads that do not depend on the step state go out before it arrives: the group's
    //      queries and norm weights (threads 0..63), the newest key (64..79) and value (128..)
    const float* x = p.qkv + size_t(q) * QKV;
    const int hl = tid >> 4, sq = tid & 15;                 // local q head (threads 0..63), pair group
    float4 qlo = make_float4(0.f, 0.f, 0.f, 0.f), qhi = qlo;
    uint2 glo = make_uint2(0, 0), ghi = glo;
    if (tid < HG * 16) {
        const int h = hg * HG + hl;
        qlo = *reinterpret_cast<const float4*>(x + h * HEAD_DIM + sq * 4);
        qhi = *reinterpret_cast<const float4*>(x + h * HEAD_DIM + 64 + sq * 4);
        glo = *reinterpret_cast<const uint2*>(p.q_norm + sq * 4);
        ghi = *reinterpret_cast<const uint2*>(p.q_norm + 64 + sq * 4);
    }
    float4 klo = make_float4(0.f, 0.f, 0.f, 0.f), khi = klo;
    uint2 kgl = make_uint2(0, 0), kgh = kgl;
    if (tid >= 64 && tid < 80) {
        const int t = tid - 64;
        klo = *reinterpret_cast<const float4*>(x + ATTN + t * 4);
        khi = *reinterpret_cast<const float4*>(x + ATTN + 64 + t * 4);
        kgl = *reinterpret_cast<const uint2*>(p.k_norm + t * 4);
        kgh = *reinterpret_cast<const uint2*>(p.k_norm + 64 + t * 4);
    }
    const float vnew = tid >= 128 ? x[QKV - HEAD_DIM + (tid - 128)] : 0.f;
    // Row geometry.  Visible keys are the absolute positions first..pos (window 2048 on the
    // local layers); key r sits at ring slot (first + r) % capacity.  Local keys rotate
    // with coordinate r and the query with pos - first: a decode step is a 16-token chunk
    // of one token, whose RoPE base max(0, pos - 2047) is `first` (Runtime.swift:389,
    // Kernels.metal:251,283-284).
    if (st->stopped || q >= int(st->rows)) return;
    const uint32_t pos = st->pos[q];
    const uint32_t lanei = st->kv_shared ? 0u : st->lane[q];
    const uint32_t first = FULL ? 0u : (pos > uint32_t(WINDOW - 1) ? pos - uint32_t(WINDOW - 1) : 0u);
    const uint32_t qcoord = FULL ? pos : pos - first;
    const uint32_t count = pos + 1 - first;
    const uint32_t k0 = part * KP;
    const uint32_t cap = p.capacity;
    const uint32_t start = first % cap;
    uint16_t* K = p.keys + size_t(lanei) * cap * HEAD_DIM;
    uint16_t* V = p.values + size_t(lanei) * cap * HEAD_DIM;
    // A local-layer row whose window starts at 0 rotates every key with its own position:
    // those rotations are cached (keys_rot, written with each key), so the keys are read
    // rotated and only the newest one is rotated here.
    const bool prerot = !FULL && p.keys_rot != nullptr && first == 0;
    uint16_t* KR = prerot ? p.keys_rot + size_t(lanei) * p.rot_rows * HEAD_DIM : nullptr;
    const size_t pslot = size_t(q) * p.parts + part;
    // partition results travel between workgroups with sc1 stores and loads (no cache fences)
    const uint32_t pstats = uint32_t(ROWS) * p.parts * HEADS;
    const __amdgpu_buffer_rsrc_t mview = buffer_view(p.part_m, pstats * 4u);
    const __amdgpu_buffer_rsrc_t lview = buffer_view(p.part_l, pstats * 4u);
    const __amdgpu_buffer_rsrc_t oview = buffer_view(p.part_o, pstats * HEAD_DIM * 4u);
    const uint32_t nparts = (count + KP - 1) / KP;
    if (part >= nparts) return;  // partitions past the visible keys take no ticket
    const uint32_t newest = count - 1;
    const bool has_new = newest >= k0 && newest < k0 + KP;

    // ---- every other independent global load
    uint4 qr = make_uint4(0, 0, 0, 0);
    if (tid < HG * 16)
        qr = *reinterpret_cast<const uint4*>((FULL ? p.global_rope : p.local_rope) + size_t(qcoord) * 64 + sq * 4);
    const int kj = tid >> 2, ksub = tid & 3;                // key, pair group (16 pairs)
    const uint32_t kr = k0 + kj;
    uint4 ka[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    uint4 kb[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    uint4 vv[4] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    uint4 rr[4] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    if (kr < count && kr != newest) {
        uint32_t phys = start + kr;
        phys = phys >= cap ? phys - cap : phys;  // visible keys (<= capacity) wrap at most once
        const uint16_t* krow = (prerot ? KR : K) + size_t(phys) * HEAD_DIM;  // phys == kr when prerot
        ka[0] = *reinterpret_cast<const uint4*>(krow + ksub * 16);
        ka[1] = *reinterpret_cast<const uint4*>(krow + ksub * 16 + 8);
        kb[0] = *reinterpret_cast<const uint4*>(krow + 64 + ksub * 16);
        kb[1] = *reinterpret_cast<const uint4*>(krow + 64 + ksub * 16 + 8);
        const uint16_t* vrow = V + size_t(phys) * HEAD_DIM + ksub * 32;  // 32 of the 128 values
#pragma unroll
        for (int i = 0; i < 4; ++i) vv[i] = *reinterpret_cast<const uint4*>(vrow + 8 * i);
    }
    if (!FULL && !prerot && kr < count) {
        const uint4* rrow = reinterpret_cast<const uint4*>(p.local_rope + size_t(kr) * 64 + ksub * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) rr[i] = rrow[i];
    }
    // ---- queries of the group: norm and RoPE in registers
    if (tid < HG * 16) {
        float z[8];
        head_norm8(qlo, qhi, glo, ghi, z);
        const uint32_t c4[4] = {qr.x, qr.y, qr.z, qr.w};
        float ra[4] = {z[0], z[1], z[2], z[3]}, rb[4] = {z[4], z[5], z[6], z[7]};
#pragma unroll
        for (int j = 0; j < 4; j += 2) rope_pair_x2f(ra[j], rb[j], c4[j], ra[j + 1], rb[j + 1], c4[j + 1]);
        // BF16-exact values: the pairs are lossless
        uint32_t* qrow = qs + hl * (HEAD_DIM / 2);
        *reinterpret_cast<uint2*>(qrow + sq * 2) = make_uint2(pack_bf16(ra[0], ra[1]), pack_bf16(ra[2], ra[3]));
        *reinterpret_cast<uint2*>(qrow + 32 + sq * 2) = make_uint2(pack_bf16(rb[0], rb[1]), pack_bf16(rb[2], rb[3]));
    }
    // ---- the newest key: k norm, RoPE at pos for global layers, KV write (Kernels.metal:253-257)
    if (has_new && tid >= 64 && tid < 80) {
        const int t = tid - 64;
        float z[8];
        head_norm8(klo, khi, kgl, kgh, z);
        const size_t slot = size_t(pos % cap) * HEAD_DIM;
        if (FULL) {
            const uint4 gr = *reinterpret_cast<const uint4*>(p.global_rope + size_t(pos) * 64 + t * 4);
            const uint32_t c4[4] = {gr.x, gr.y, gr.z, gr.w};
#pragma unroll
            for (int j = 0; j < 4; j += 2) rope_pair_x2f(z[j], z[4 + j], c4[j], z[j + 1], z[4 + j + 1], c4[j + 1]);
        }
        float zr[8];
        if (prerot) {  // the newest key at its own position (coordinate pos - first = pos)
            const uint4 lr = *reinterpret_cast<const uint4*>(p.local_rope + size_t(pos) * 64 + t * 4);
            const uint32_t c4[4] = {lr.x, lr.y, lr.z, lr.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) zr[j] = z[j];
#pragma unroll
            for (int j = 0; j < 4; j += 2) rope_pair_x2f(zr[j], zr[4 + j], c4[j], zr[j + 1], zr[4 + j + 1], c4[j + 1]);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) zr[j] = z[j];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (hg == 0) {
                K[slot + t * 4 + j] = uint16_t(bits(z[j]));
                K[slot + 64 + t * 4 + j] = uint16_t(bits(z[4 + j]));
                if (prerot) {
                    KR[size_t(pos) * HEAD_DIM + t * 4 + j] = uint16_t(bits(zr[j]));
                    KR[size_t(pos) * HEAD_DIM + 64 + t * 4 + j] = uint16_t(bits(zr[4 + j]));
                }
            }
            knew[t * 4 + j] = zr[j];
            knew[64 + t * 4 + j] = zr[4 + j];
        }
    }
    if (has_new && tid >= 128) {
        const int d = tid - 128;
        const uint32_t bv = bits(vnew);
        if (hg == 0) V[size_t(pos % cap) * HEAD_DIM + d] = uint16_t(bv);
        vs[int(newest - k0) * HEAD_DIM + d] = uint16_t(bv);
    }
    // the newest key and value rows are read by other threads below; the queries only after
    // the next barrier (has_new is the same for the whole workgroup)
    if (has_new) __syncthreads();
    // ---- keys: (newest from LDS) rotate with coordinate r, stage BF16 pairs in LDS: thread
    //      (kj, ksub) holds dims ksub*16 .. +16 (words aw) and 64 + ksub*16 .. +16 (words bw)
    {
        uint32_t aw[8] = {ka[0].x, ka[0].y, ka[0].z, ka[0].w, ka[1].x, ka[1].y, ka[1].z, ka[1].w};
        uint32_t bw[8] = {kb[0].x, kb[0].y, kb[0].z, kb[0].w, kb[1].x, kb[1].y, kb[1].z, kb[1].w};
        if (kr == newest) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                aw[i] = pack_bf16(knew[ksub * 16 + 2 * i], knew[ksub * 16 + 2 * i + 1]);
                bw[i] = pack_bf16(knew[64 + ksub * 16 + 2 * i], knew[64 + ksub * 16 + 2 * i + 1]);
            }
        }
        if (!FULL && !prerot && kr < count) {
            const uint32_t rw[16] = {rr[0].x, rr[0].y, rr[0].z, rr[0].w, rr[1].x, rr[1].y, rr[1].z, rr[1].w,
                                     rr[2].x, rr[2].y, rr[2].z, rr[2].w, rr[3].x, rr[3].y, rr[3].z, rr[3].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) rope_pair_x2(aw[i], bw[i], rw[2 * i], rw[2 * i + 1], aw[i], bw[i]);
        }
        uint32_t* krow = ks + kj * KS;
        *reinterpret_cast<uint4*>(krow + ksub * 8) = make_uint4(aw[0], aw[1], aw[2], aw[3]);
        *reinterpret_cast<uint4*>(krow + ksub * 8 + 4) = make_uint4(aw[4], aw[5], aw[6], aw[7]);
        *reinterpret_cast<uint4*>(krow + 32 + ksub * 8) = make_uint4(bw[0], bw[1], bw[2], bw[3]);
        *reinterpret_cast<uint4*>(krow + 32 + ksub * 8 + 4) = make_uint4(bw[4], bw[5], bw[6], bw[7]);
        if (kr != newest) {  // the newest V row was staged before the barrier
#pragma unroll
            for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(vs + kj * HEAD_DIM + ksub * 32 + 8 * i) = vv[i];
        }
    }
    __syncthreads();
    // ---- scores: wave w = local head w, lane = key.  Each score is four ordered 32-dim
    //      chains (dims 32c .. 32c+31, v_dot2_f32_bf16 over the dim pairs in order) summed as
    //      (c0 + c1) + (c2 + c3).
    {
        const int j = lane, w = wave;
        // validity first: with the QSA mask's branch and load after the score chains, the
        // compiler holds every operand of the chains at once (135 instead of 75 VGPRs)
        bool valid = k0 + j < count;
        if (FULL && p.qsa_mask) {
            // QSA: key k = position k; the blocks of four keys complete at this position must be
            // selected, the unfinished block is always seen (Kernels.metal:618-700)
            const uint32_t b = (k0 + uint32_t(j)) >> 2;
            valid = valid && (b >= (pos + 1) / 4 || ((p.qsa_mask[size_t(q) * p.qsa_words + (b >> 5)] >> (b & 31)) & 1u));
        }
        float sc[4] = {0.f, 0.f, 0.f, 0.f};
        const uint32_t* krow = ks + j * KS;
        const uint32_t* qrow = qs + w * (HEAD_DIM / 2);
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint4 kd = *reinterpret_cast<const uint4*>(krow + 16 * c + i);
                const uint4 qd = *reinterpret_cast<const uint4*>(qrow + 16 * c + i);
                sc[c] = dot2bf(qd.x, kd.x, sc[c]);
                sc[c] = dot2bf(qd.y, kd.y, sc[c]);
                sc[c] = dot2bf(qd.z, kd.z, sc[c]);
                sc[c] = dot2bf(qd.w, kd.w, sc[c]);
            }
        }
        const float dot = (sc[0] + sc[1]) + (sc[2] + sc[3]);
        const float s = valid ? dot * SCALE : NEG_INF;
        const float m = wave_max(s);
        const float e = valid ? exp_det(s - m) : 0.f;
        const float l = wave_sum(e);
        ps[w * KP + j] = e;
        if (lane == 0) {
            l_s[w] = l;
            if (nparts > 1) {
                buffer_store4_sc1(mview, uint32_t(pslot * HEADS + hg * HG + w) * 4u, __float_as_uint(m));
                buffer_store4_sc1(lview, uint32_t(pslot * HEADS + hg * HG + w) * 4u, __float_as_uint(l));
            }
        }
    }
    // P.V reads only what its own wave wrote above (the probabilities and l of head w; the V
    // rows were staged before the last barrier): a wave-level fence orders it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- unnormalised P.V: wave w = local head w; lanes 0..31 take keys 0..31 and lanes
    //      32..63 keys 32..63, lane l owning dims 4(l % 32) .. +3 (one 8-byte value read per
    //      key).  Per dim: two ordered chains of fused multiply-adds (keys 0..31, keys 32..63),
    //      added at the end (lanes 0..31 add the partner lane's chain to their own)
    {
        const int hl = wave, hf = lane >> 5, d4 = (lane & 31) * 4;
        const float* pr = ps + hl * KP + hf * (KP / 2);
        const uint16_t* vb = vs + hf * (KP / 2) * HEAD_DIM + d4;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
        for (int j = 0; j < KP / 2; j += 4) {
            uint2 vw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) vw[i] = *reinterpret_cast<const uint2*>(vb + (j + i) * HEAD_DIM);
            const float4 pp = *reinterpret_cast<const float4*>(pr + j);
            const float pw[4] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[0] = fmaf(pw[i], lo(vw[i].x), o[0]);
                o[1] = fmaf(pw[i], hi(vw[i].x), o[1]);
                o[2] = fmaf(pw[i], lo(vw[i].y), o[2]);
                o[3] = fmaf(pw[i], hi(vw[i].y), o[3]);
            }
        }
        float of[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) of[k] = o[k] + xor_lane<32>(o[k]);  // lanes 0..31: first half + second
        const int h = hg * HG + hl;
        if (lane < 32) {
            if (nparts == 1) {  // one partition: the merge reduces to o / l (exp(0) == 1 exactly)
                const float l = l_s[hl];
#pragma unroll
                for (int k = 0; k < 4; ++k) p.out16[size_t(q) * ATTN + h * HEAD_DIM + d4 + k] = uint16_t(bits(of[k] / l));
            } else {
                buffer_store16_sc1(oview, uint32_t((pslot * HEADS + h) * HEAD_DIM + d4) * 4u,
                                   make_uint4(__float_as_uint(of[0]), __float_as_uint(of[1]), __float_as_uint(of[2]),
                                              __float_as_uint(of[3])));
            }
        }
    }
    if (nparts == 1) return;
    if (p.merge_in_o && nparts <= MERGE_IN_O) return;  // the o projection's prologue merges
    if (p.defer != 0 && nparts > p.defer) return;  // attn_merge_kernel merges this row
    // ticket: the last workgroup of this (row, head group) merges the partitions; every
    // wave's partition stores have completed before the ticket is taken
    wait_stores();
    __syncthreads();
    uint32_t* ticket = p.tickets + q * (HEADS / HG) + hg;
    if (tid == 0) {
        const uint32_t prev = atomicAdd(ticket, 1u);
        s_last = prev == nparts - 1;
    }
    __syncthreads();
    if (!s_last) return;
    const size_t row0 = size_t(q) * p.parts;
    // per head: M = max_p m_p, w_p = exp(m_p - M), den = sum_p l_p w_p (partition order);
    // then each (h, d) sums o_p w_p in partition order.  Partition statistics are staged in
    // LDS (the key tile is free now) with all loads in flight together.
    float* mm = reinterpret_cast<float*>(ks);          // [np][HG]
    float* wl = mm + (KP * KS) / 2;                    // [np][HG]: l, then the weights
    const uint32_t np = nparts <= uint32_t(KP * KS / 2 / HG) ? nparts : uint32_t(KP * KS / 2 / HG);
    // up to 64 partitions one entry per thread; more: eight entries per thread in flight
    if (np * HG <= 256) {
        if (uint32_t(tid) < np * HG) {
            const uint32_t k = uint32_t(tid) / HG, h = hg * HG + uint32_t(tid) % HG;
            mm[tid] = __uint_as_float(buffer_load4_sc1(mview, uint32_t((row0 + k) * HEADS + h) * 4u));
            wl[tid] = __uint_as_float(buffer_load4_sc1(lview, uint32_t((row0 + k) * HEADS + h) * 4u));
        }
    } else
    for (uint32_t i0 = tid; i0 < np * HG; i0 += 256 * 8) {
        float mv[8], lv[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            const uint32_t i = i0 + 256 * j;
            if (i < np * HG) {
                const uint32_t k = i / HG, h = hg * HG + i % HG;
                mv[j] = __uint_as_float(buffer_load4_sc1(mview, uint32_t((row0 + k) * HEADS + h) * 4u));
                lv[j] = __uint_as_float(buffer_load4_sc1(lview, uint32_t((row0 + k) * HEADS + h) * 4u));
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            const uint32_t i = i0 + 256 * j;
            if (i < np * HG) {
                mm[i] = mv[j];
                wl[i] = lv[j];
            }
        }
    }
    // thread -> dim d = tid & 127 of local heads (tid >> 7) and (tid >> 7) + 2.  The outputs
    // of the first F partitions are requested together with the statistics (only those that
    // exist); the rest go in chunks of PRE, chunk c + 1 requested while chunk c is summed
    // (loads past the last partition re-read it, so every chunk issues the same number of
    // requests and the wait before the sums counts exactly).
    const int d = tid & 127, hb = tid >> 7;
    constexpr uint32_t F = 8, PRE = 32;
    float ovf[F][2];
    auto load_one = [&](uint32_t k, float (&dst)[2]) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            dst[i] = __uint_as_float(
                buffer_load4_sc1(oview, uint32_t(((row0 + k) * HEADS + hg * HG + hb + 2 * i) * HEAD_DIM + d) * 4u));
    };
    auto load_chunk = [&](uint32_t c0, float (&dst)[PRE][2]) {
#pragma unroll
        for (uint32_t j = 0; j < PRE; ++j) load_one(c0 + j < nparts ? c0 + j : nparts - 1, dst[j]);
    };
    // Global layers merge only rows of up to F partitions here (every caller hands longer
    // rows to attn_merge_kernel); a longer one would take the memory path below, which has
    // the same operations in the same order, so the chunked loop is left out of that kernel.
    const bool staged = nparts == np && (!FULL || nparts <= F);
    if (staged) {
#pragma unroll
        for (uint32_t j = 0; j < F; ++j)
            if (j < nparts) load_one(j, ovf[j]);
    }
    __syncthreads();
    if (staged) {
        // M per head; then every weight exp(m_p - M) in parallel (in place of m_p); then each
        // thread forms den for its own two heads (partition order) while summing o_p w_p
        // M per head: up to 16 partitions one thread per head; more: wave w takes local head w
        // (a maximum has no rounding, so any order gives the same M)
        static_assert(HG == 4, "one wave per local head");
        if (nparts <= 16) {
            if (tid < HG) {
                float M = NEG_INF;
                for (uint32_t k = 0; k < nparts; ++k) M = fmaxf(M, mm[k * HG + tid]);
                l_s[tid] = M;
            }
        } else {
            float M = NEG_INF;
            for (uint32_t k = uint32_t(lane); k < nparts; k += 64) M = fmaxf(M, mm[k * HG + wave]);
            M = fmaxf(M, xor_lane<32>(M));
            M = fmaxf(M, xor_lane<16>(M));
            M = fmaxf(M, xor_lane<8>(M));
            M = fmaxf(M, xor_lane<4>(M));
            M = fmaxf(M, xor_lane<2>(M));
            M = fmaxf(M, xor_lane<1>(M));
            if (lane == 0) l_s[wave] = M;
        }
        __syncthreads();
        for (uint32_t i = tid; i < np * HG; i += 256) mm[i] = exp_det(mm[i] - l_s[i % HG]);
        __syncthreads();
        float num[2] = {0.f, 0.f}, den[2] = {0.f, 0.f};
        float ovp[PRE][2];
        if constexpr (!FULL)
            if (F < nparts) load_chunk(F, ovp);
#pragma unroll
        for (uint32_t k = 0; k < F; ++k) {
            if (k >= nparts) break;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float w = mm[k * HG + hb + 2 * i];
                num[i] = num[i] + ovf[k][i] * w;
                den[i] = den[i] + wl[k * HG + hb + 2 * i] * w;
            }
        }
        for (uint32_t c0 = F; !FULL && c0 < nparts; c0 += PRE) {
            const bool more = c0 + PRE < nparts;
            float nxt[PRE][2];
            if (more) load_chunk(c0 + PRE, nxt);
#pragma unroll
            for (uint32_t j = 0; j < PRE; ++j) {
                const uint32_t k = c0 + j;
                if (k >= nparts) break;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const float w = mm[k * HG + hb + 2 * i];
                    num[i] = num[i] + ovp[j][i] * w;
                    den[i] = den[i] + wl[k * HG + hb + 2 * i] * w;
                }
            }
            if (more) {
#pragma unroll
                for (uint32_t j = 0; j < PRE; ++j) {
                    ovp[j][0] = nxt[j][0];
                    ovp[j][1] = nxt[j][1];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
            p.out16[size_t(q) * ATTN + (hg * HG + hb + 2 * i) * HEAD_DIM + d] = uint16_t(bits(num[i] / den[i]));
    } else {  // more partitions than LDS holds (or a global row past F): read them from memory
        if (tid < HG) {
            const int h = hg * HG + tid;
            float M = NEG_INF, den = 0.f;
            auto pm = [&](uint32_t k) { return __uint_as_float(buffer_load4_sc1(mview, uint32_t((row0 + k) * HEADS + h) * 4u)); };
            auto pl = [&](uint32_t k) { return __uint_as_float(buffer_load4_sc1(lview, uint32_t((row0 + k) * HEADS + h) * 4u)); };
            for (uint32_t k = 0; k < nparts; ++k) M = fmaxf(M, pm(k));
            for (uint32_t k = 0; k < nparts; ++k) den = den + pl(k) * exp_det(pm(k) - M);
            den_s[tid] = den;
            l_s[tid] = M;
        }
        __syncthreads();
        float num[2] = {0.f, 0.f};
        for (uint32_t k = 0; k < nparts; ++k)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int h = hg * HG + hb + 2 * i;
                const float ov = __uint_as_float(buffer_load4_sc1(oview, uint32_t(((row0 + k) * HEADS + h) * HEAD_DIM + d) * 4u));
                const float mk = __uint_as_float(buffer_load4_sc1(mview, uint32_t((row0 + k) * HEADS + h) * 4u));
                num[i] = num[i] + ov * exp_det(mk - l_s[hb + 2 * i]);
            }
#pragma unroll
        for (int i = 0; i < 2; ++i)
            p.out16[size_t(q) * ATTN + (hg * HG + hb + 2 * i) * HEAD_DIM + d] = uint16_t(bits(num[i] / den_s[hb + 2 * i]));
    }
    if (tid == 0) atomicExch(ticket, 0u);  // ready for the next launch
}

// Partition merge of rows with more than p.defer partitions (long contexts),
// one workgroup per (32 dims of a head, head, row).  Past MERGE_BLOCK partitions the sums
// run as blocks of MERGE_BLOCK partitions in parallel, added in block order.  The workgroup's slice of every partition
// output is staged in LDS with all of its loads in flight together (one workgroup keeping a
// few partitions in flight would take tens of microseconds at 500 partitions), then 32
// threads sum in partition order.  Same arithmetic in the same order as the attention
// kernel's own merge: M = max_p m_p, w_p = exp(m_p - M), den = sum l_p w_p, num = sum o_p w_p.
__global__ __launch_bounds__(256) void attn_merge_kernel(const AttnParams p) {
#pragma clang fp contract(off)  // fixed rounding sequence, reproduced by the CPU oracle
    PLAMO_TIMELINE_SCOPE(p.tag + 1);
    constexpr uint32_t MAXP = uint32_t(MAX_CONTEXT / KP);
    static_assert(MAXP <= 512, "two statistics per thread");
    __shared__ __align__(16) float os[MAXP * 32];
    __shared__ float ws[MAXP], lsh[MAXP];
    __shared__ float red[4];
    // block sums of the merge: MERGE_BLOCK partitions per block, one block per wave
    constexpr uint32_t MB = uint32_t(MERGE_BLOCK), NB = MAXP / MB;
    static_assert(MAXP % MB == 0 && NB <= 4, "one wave per block");
    __shared__ float bnum[NB * 32], bden[NB * 32];
    const StepState* st = p.state;
    const int q = blockIdx.z, h = blockIdx.y, d0 = blockIdx.x * 32;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t row0 = size_t(q) * p.parts;
    const uint32_t pstats = uint32_t(ROWS) * p.parts * HEADS;
    const __amdgpu_buffer_rsrc_t mview = buffer_view(p.part_m, pstats * 4u);
    const __amdgpu_buffer_rsrc_t lview = buffer_view(p.part_l, pstats * 4u);
    const __amdgpu_buffer_rsrc_t oview = buffer_view(p.part_o, pstats * HEAD_DIM * 4u);
    // every load first: statistics of partitions tid and tid + 256, then the output slice
    // (eight threads per partition, 16 bytes each).  The first EARLY partitions of the buffer
    // are requested before the step state arrives (their addresses do not depend on it; a
    // local layer's partitions all fall there); entries past the row's partitions are never
    // used.  The rest follow once the state gives the row's partition count.
    constexpr uint32_t EARLY = 64;
    const uint32_t early = p.parts < EARLY ? p.parts : EARLY;
    constexpr int OPT = int(MAXP) / 32;  // output loads per thread
    static_assert(EARLY <= 256 && EARLY % 32 == 0, "early statistics: one per thread of the first slot");
    float mv[2] = {NEG_INF, NEG_INF}, lv[2] = {0.f, 0.f};
    uint4 ov[OPT];
    const int sub4 = (tid & 7) * 4;
    if (uint32_t(tid) < early) {
        mv[0] = __uint_as_float(buffer_load4_sc1(mview, uint32_t((row0 + tid) * HEADS + h) * 4u));
        lv[0] = __uint_as_float(buffer_load4_sc1(lview, uint32_t((row0 + tid) * HEADS + h) * 4u));
    }
#pragma unroll
    for (int j = 0; j < int(EARLY / 32); ++j) {
        const uint32_t k = uint32_t((tid >> 3) + 32 * j);
        if (k < early)
            ov[j] = buffer_load16_sc1(oview, uint32_t(((row0 + k) * HEADS + h) * HEAD_DIM + d0 + sub4) * 4u);
    }
    if (st->stopped || q >= int(st->rows)) return;
    // keys 0 .. pos on global layers, the last WINDOW of them on local layers
    const uint32_t count = p.window && st->pos[q] + 1 > p.window ? p.window : st->pos[q] + 1;
    const uint32_t nparts = (count + KP - 1) / KP;
    if (nparts <= p.defer || nparts > MAXP || nparts > p.parts) return;  // merged in the attention kernel
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t k = uint32_t(tid + 256 * j);
        if (k >= early && k < nparts) {
            mv[j] = __uint_as_float(buffer_load4_sc1(mview, uint32_t((row0 + k) * HEADS + h) * 4u));
            lv[j] = __uint_as_float(buffer_load4_sc1(lview, uint32_t((row0 + k) * HEADS + h) * 4u));
        }
    }
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
        const uint32_t k = uint32_t((tid >> 3) + 32 * j);
        if (k >= early && k < nparts)
            ov[j] = buffer_load16_sc1(oview, uint32_t(((row0 + k) * HEADS + h) * HEAD_DIM + d0 + sub4) * 4u);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
        if (uint32_t(tid + 256 * j) >= nparts) mv[j] = NEG_INF;  // early entries past the row's partitions
    // M: a maximum has no rounding, so any order gives the same value
    float M = fmaxf(mv[0], mv[1]);
    M = fmaxf(M, xor_lane<32>(M));
    M = fmaxf(M, xor_lane<16>(M));
    M = fmaxf(M, xor_lane<8>(M));
    M = fmaxf(M, xor_lane<4>(M));
    M = fmaxf(M, xor_lane<2>(M));
    M = fmaxf(M, xor_lane<1>(M));
    if (lane == 0) red[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t k = uint32_t(tid + 256 * j);
        if (k < nparts) {
            ws[k] = exp_det(mv[j] - M);
            lsh[k] = lv[j];
        }
    }
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
        const uint32_t k = uint32_t((tid >> 3) + 32 * j);
        if (k < nparts) *reinterpret_cast<uint4*>(&os[k * 32 + sub4]) = ov[j];
    }
    __syncthreads();
    // num = sum_k o_k w_k, den = sum_k l_k w_k: lanes 0..31 of wave b sum partitions
    // b*MB .. b*MB + MB - 1 in order (a chain of at most MB dependent sums instead of one of
    // nparts; the partition index stays wave-uniform), then 32 threads add the block sums in
    // block order.  With one block this is the partition-order sum of the attention kernel's
    // own merge.
    const uint32_t nblk = (nparts + MB - 1) / MB;
    if (uint32_t(wave) < nblk && lane < 32) {
        float bn = 0.f, bd = 0.f;
        const uint32_t k0 = uint32_t(wave) * MB, k1 = min(k0 + MB, nparts);
#pragma unroll 8  // eight partitions' LDS reads per round trip
        for (uint32_t k = k0; k < k1; ++k) {
            const float w = ws[k];
            bn = bn + os[k * 32 + lane] * w;
            bd = bd + lsh[k] * w;
        }
        if (nblk == 1) {  // one block: 0 + bn is bn, so the block sum is the result
            p.out16[size_t(q) * ATTN + h * HEAD_DIM + d0 + lane] = uint16_t(bits(bn / bd));
            return;
        }
        bnum[wave * 32 + lane] = bn;
        bden[wave * 32 + lane] = bd;
    }
    if (nblk == 1) return;
    __syncthreads();
    if (tid < 32) {
        float num = 0.f, den = 0.f;
        for (uint32_t b = 0; b < nblk; ++b) {
            num = num + bnum[b * 32 + tid];
            den = den + bden[b * 32 + tid];
        }
        p.out16[size_t(q) * ATTN + h * HEAD_DIM + d0 + tid] = uint16_t(bits(num / den));
    }
}

// ------------------------------------------------------------------------- step begin
// Device side of the token loop (Main.swift:278-287) and of the sampler history
// (Main.swift:237-244; Sampler.swift:11-24,54-70), on the state copy `ls` in LDS; every
// thread of the 256-thread workgroup calls it.  A device loop runs it before each step's
// layers: once before the first replay (step_begin_kernel) and then at the end of every
// step, after the head merge fed the prediction back (head_merge_kernel), so the replayed
// loop graph has no separate bookkeeping kernel.
__device__ void begin_step(StepState& ls, const DecodeBuffers& b, int* s_stop) {
    const int tid = threadIdx.x;
    if (tid == 0) {
        *s_stop = 0;
        if (ls.quad) {
            // decodeBatch's lane pass (BatchDecode.swift:16-31): a lane stops at its limit or
            // on token 1 / 16, otherwise emits its prediction and, below the limit, feeds it
            // back; running lanes are packed into rows in lane order (Batch.swift:130-146).
            uint32_t rows = 0, last = ls.last;
            for (uint32_t ln = 0; ln < ls.lanes && ln < uint32_t(ROWS); ++ln) {
                if (ln > last) break;
                if (ls.lreason[ln]) continue;
                const int32_t nx = ls.lnext[ln];
                uint32_t reason = 0;
                if (ls.lcount[ln] == ls.llimit[ln]) reason = 2;
                else if (nx == 1 || nx == 16) reason = 1;
                else {
                    b.out_ids[size_t(ln) * ls.out_stride + ls.lcount[ln]] = nx;
                    ls.lcount[ln] += 1;
                    if (ls.lcount[ln] == ls.llimit[ln]) reason = 2;
                    else {
                        ls.lane[rows] = ln;
                        ls.pos[rows] = ls.lpos[ln];
                        ls.token[rows] = nx;
                        ++rows;
                    }
                }
                if (reason) {
                    ls.lreason[ln] = reason;
                    if (ls.trunc_stop && reason == 2 && ln < last) last = ln;
                }
            }
            ls.last = last;
            ls.rows = rows;
            if (!rows) { ls.stopped = 1; *s_stop = 1; }
        } else if (ls.loop) {
            const int32_t tok = ls.token[0];
            if (ls.stop_enabled && (tok == 1 || tok == 16)) {
                ls.stopped = 1; ls.reason = 1; *s_stop = 1;
            } else if (tok < 0 || tok >= VOCAB) {
                ls.stopped = 1; ls.reason = 3; *s_stop = 1;
            } else {
                b.out_ids[ls.produced] = tok;
                ls.produced += 1;
                if (ls.sampling && ls.hist_len[0] < b.hist_cap) {
                    b.history[ls.hist_len[0]] = tok;
                    ls.hist_len[0] += 1;
                }
                if (ls.produced >= ls.max_tokens) { ls.stopped = 1; ls.reason = 2; *s_stop = 1; }
            }
        }
    }
    __syncthreads();
    if (!*s_stop && ls.sampling) {
        for (uint32_t q = 0; q < ls.rows; ++q) {
            const int32_t* hist = b.history + size_t(q) * b.hist_cap;
            const uint32_t len = ls.hist_len[q];
            if (tid == 0) {
                for (uint32_t i = ls.counted[q]; i < len; ++i) {
                    const int32_t id = hist[i];
                    if (id >= 0 && id < VOCAB) b.counts[size_t(q) * VOCAB + id] += 1;
                }
                ls.counted[q] = len;
            }
            if (ls.ngram > 1) {
                uint32_t* ban = b.banned + size_t(q) * (VOCAB / 32);
                for (int i = tid; i < VOCAB / 32; i += 256) ban[i] = 0;
                __syncthreads();
                const int n = ls.ngram, span = n - 1;
                if (int(len) >= n) {
                    const int last = int(len) - span;
                    for (int s = tid; s < last; s += 256) {
                        bool match = true;
                        for (int k = 0; k < span && match; ++k) match = hist[s + k] == hist[last + k];
                        if (match) {
                            const int32_t id = hist[s + span];
                            if (id >= 0 && id < VOCAB) atomicOr(&ban[id >> 5], 1u << (id & 31));
                        }
                    }
                }
            }
            __syncthreads();
        }
    }
    __syncthreads();
}

__global__ __launch_bounds__(256) void step_begin_kernel(DecodeBuffers b) {
    PLAMO_TIMELINE_SCOPE(TL_STEP_BEGIN);
    __shared__ StepState ls;
    __shared__ int s_stop;
    state_in(ls, b.state);
    __syncthreads();
    if (ls.stopped) return;
    begin_step(ls, b, &s_stop);
    state_out(b.state, ls);
}

// ---------------------------------------------------------------- kernel-level helpers
__global__ __launch_bounds__(512) void argmax_kernel(const void* x, uint32_t* out, int n, int bf16) {
    __shared__ float mv[8];
    __shared__ uint32_t mi[8];
    const int row = blockIdx.x, tid = threadIdx.x;
    float bv = NEG_INF;
    uint32_t bi = 0xffffffffu;
    for (int i = tid; i < n; i += 512) {
        const float v = bf16 ? bf(static_cast<const uint16_t*>(x)[size_t(row) * n + i])
                             : static_cast<const float*>(x)[size_t(row) * n + i];
        if (better(v, uint32_t(i), bv, bi)) { bv = v; bi = uint32_t(i); }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float v = __shfl_xor(bv, o, 64);
        const uint32_t i = __shfl_xor(bi, o, 64);
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    if ((tid & 63) == 0) { mv[tid >> 6] = bv; mi[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int k = 1; k < 8; ++k)
            if (better(mv[k], mi[k], bv, bi)) { bv = mv[k]; bi = mi[k]; }
        out[row] = bi;
    }
}

// Sampler.select (Sampler.swift:9-32) for the known-answer tests: one workgroup.
__global__ __launch_bounds__(256) void select_kernel(float* logits, int n, const int32_t* hist, int len, float penalty,
                                                     int ngram, float frequency, float presence, int32_t* out) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    __shared__ float mv[4];
    __shared__ uint32_t mi[4];
    if (penalty != 1.0f || presence != 0.0f || frequency != 0.0f) {
        for (int id = tid; id < n; id += 256) {
            int c = 0;
            for (int k = 0; k < len; ++k) c += hist[k] == id;
            if (c == 0) continue;
            float l = logits[id];
            if (penalty != 1.0f) l = l > 0.0f ? l / penalty : l * penalty;
            if (presence != 0.0f) l = l - presence;
            if (frequency != 0.0f) {
                const float f = frequency * float(c);
                l = l - f;
            }
            logits[id] = l;
        }
        __syncthreads();
    }
    if (ngram > 1 && len >= ngram) {
        const int span = ngram - 1, last = len - span;
        for (int s = tid; s < last; s += 256) {
            bool match = true;
            for (int k = 0; k < span && match; ++k) match = hist[s + k] == hist[last + k];
            if (match) {
                const int32_t id = hist[s + span];
                if (id >= 0 && id < n) logits[id] = NEG_INF;
            }
        }
        __syncthreads();
    }
    float bv = NEG_INF;
    uint32_t bi = 0xffffffffu;
    for (int i = tid; i < n; i += 256)
        if (logits[i] > bv) { bv = logits[i]; bi = uint32_t(i); }  // strict: first max, NaN never wins
    for (int o = 32; o > 0; o >>= 1) {
        const float v = __shfl_xor(bv, o, 64);
        const uint32_t i = __shfl_xor(bi, o, 64);
        if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
    }
    if ((tid & 63) == 0) { mv[tid >> 6] = bv; mi[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int k = 1; k < 4; ++k)
            if (mv[k] > bv || (mv[k] == bv && mi[k] < bi)) { bv = mv[k]; bi = mi[k]; }
        *out = bi == 0xffffffffu ? 0 : int32_t(bi);
    }
}

// One thread per 8 weights (count is a whole number of 128-weight blocks), decoded by the
// same p12_decode8 as the GEMV and GEMM loads.
// ------------------------------------------------------------------------------------ MTP
// Input of the MTP adapter (Runtime.swift:493-494): the final normalised hidden row of the
// last output, then the embedding row of the first draft token, as 3072 floats.
__global__ __launch_bounds__(256) void mtp_input_kernel(const float* hidden, const uint16_t* embed, int token,
                                                         float* out) {
    for (int i = threadIdx.x; i < HIDDEN; i += 256) {
        out[i] = hidden[i];
        out[HIDDEN + i] = bf(embed[size_t(token) * HIDDEN + i]);
    }
}

// The adapter's activation, down projection and residual (mtp_activate, linear, mtp_add;
// Kernels.metal:347-356, Runtime.swift:498-501): a_j = roundbf(u_j / (1 + exp(-u_j))) of the
// up projection's 256 outputs, then row r: y = roundbf(W_r . a), out_r = roundbf(x_r + y)
// with x the hidden half of the input.  One wave per row; lane l owns columns 4l .. 4l+3:
// two v_dot2_f32_bf16 steps over the column pairs in order, then the wave's XOR butterfly.
__global__ __launch_bounds__(256) void mtp_down_kernel(const float* up, const float* x, const uint16_t* w,
                                                        float* out) {
#pragma clang fp contract(off)  // fixed rounding sequence, reproduced by the CPU oracle
    __shared__ uint32_t as[MTP_RANK / 2];  // activations as BF16 pairs (BF16-exact values)
    const int tid = threadIdx.x;
    if (tid < MTP_RANK / 2) {
        const float u0 = up[2 * tid], u1 = up[2 * tid + 1];
        as[tid] = pack_bf16(roundbf(u0 / (1.0f + exp_det(-u0))), roundbf(u1 / (1.0f + exp_det(-u1))));
    }
    __syncthreads();
    const int lane = tid & 63, r = int(blockIdx.x) * 4 + (tid >> 6);
    if (r >= HIDDEN) return;
    const uint2 wv = *reinterpret_cast<const uint2*>(w + size_t(r) * MTP_RANK + lane * 4);
    float acc = dot2bf(wv.x, as[2 * lane], 0.f);
    acc = dot2bf(wv.y, as[2 * lane + 1], acc);
    const float t = wave_sum(acc);
    if (lane == 0) out[r] = roundbf(x[r] + roundbf(t));
}

__global__ void unpack_kernel(const uint8_t* payload, const uint32_t* table, uint16_t* out, int64_t count) {
    const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
    if (i >= count) return;
    const uint32_t entry = table[i / 128];
    const uint8_t* blk = payload + (entry & ~63u);
    const uint32_t tag = entry & 63u, sub = uint32_t(i % 128) / 8;
    const uint4 w = tag == 0 ? *reinterpret_cast<const uint4*>(blk + sub * 16)
                             : p12_decode8(*reinterpret_cast<const uint2*>(blk + sub * 8),
                                           *reinterpret_cast<const uint32_t*>(blk + 128 + sub * 4), tag);
    *reinterpret_cast<uint4*>(out + i) = w;
}

// Scratch of the allocation-free decode attention entry point: a file-scope device array, one
// copy per GPU, held until the process ends.  Host code uses the address hipGetSymbolAddress
// returns for the current device (the array's name is not a device address on the host).
static __device__ __align__(256) uint8_t scratch[attn_workspace_bytes(STATIC_ATTN_PARTS)];
static_assert(sizeof(StepState) <= 256, "step state fits its workspace slot");

}  // namespace

void* static_attn_scratch() {
    constexpr int MAX_DEVICES = 64;
    static std::mutex mu;
    static void* ptr[MAX_DEVICES] = {};
    int dev = 0;
    PLAMO_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) throw Error(E_DEVICE, "device index out of range");
    std::lock_guard<std::mutex> lk(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        PLAMO_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        ptr[dev] = p;
    }
    return ptr[dev];
}

namespace {

struct AttnStateArgs {
    int32_t pos[ROWS];
    int32_t rows;
};
__global__ __launch_bounds__(64) void attn_state_kernel(StepState* st, uint32_t* tickets, AttnStateArgs a) {
    const int tid = threadIdx.x;
    uint32_t* w = reinterpret_cast<uint32_t*>(st);
    for (int i = tid; i < STATE_WORDS; i += 64) w[i] = 0;
    if (tid < ROWS * HEADS / HG) tickets[tid] = 0;
    __syncthreads();
    if (tid == 0) {
        st->rows = uint32_t(a.rows);
        st->penalty = 1.0f;
        for (int q = 0; q < ROWS; ++q) {
            st->lane[q] = uint32_t(q);
            st->pos[q] = q < a.rows ? uint32_t(a.pos[q]) : 0u;
        }
    }
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, size_t n) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

template <int N, bool PACKED, int MAXR>
void gemv_dispatch_epi(Prologue pro, Epilogue epi, const GemvParams& p, int blocks, hipStream_t s) {
    const dim3 grid(blocks), block(64 * gemv_waves(N, MAXR, epi));
#define PLAMO_GEMV(PRO, EPI) hipLaunchKernelGGL((gemv_kernel<N, PACKED, MAXR, PRO, EPI, true>), grid, block, 0, s, p)
#define PLAMO_GEMV_NOSTATE(PRO, EPI) \
    hipLaunchKernelGGL((gemv_kernel<N, PACKED, MAXR, PRO, EPI, false>), grid, block, 0, s, p)
    if (!p.state) {  // kernel-level entry points: plain rows, no step state
        if (pro == PRO_PLAIN && epi == EPI_ROUND) PLAMO_GEMV_NOSTATE(PRO_PLAIN, EPI_ROUND);
        else if (pro == PRO_PLAIN && epi == EPI_BF16) PLAMO_GEMV_NOSTATE(PRO_PLAIN, EPI_BF16);
        else if (pro == PRO_PLAIN && epi == EPI_RAW) PLAMO_GEMV_NOSTATE(PRO_PLAIN, EPI_RAW);
        else throw Error(E_INVAL, "unsupported GEMV variant");
        return;
    }
    if (pro == PRO_PLAIN16) {
        if (epi == EPI_BF16) PLAMO_GEMV(PRO_PLAIN16, EPI_BF16);
        else throw Error(E_INVAL, "unsupported GEMV variant");
        return;
    }
    if (pro == PRO_MERGE) {
        if constexpr (N == ATTN && MAXR == 1) {
            if (epi == EPI_BF16) PLAMO_GEMV(PRO_MERGE, EPI_BF16);
            else throw Error(E_INVAL, "unsupported GEMV variant");
        } else {
            throw Error(E_INVAL, "the merging prologue is the one-row o projection's");
        }
        return;
    }
    if constexpr (N == HIDDEN) {
        if (pro == PRO_EMBED && epi == EPI_ROUND) PLAMO_GEMV(PRO_EMBED, EPI_ROUND);
        else if (pro == PRO_RESID16 && epi == EPI_ROUND) PLAMO_GEMV(PRO_RESID16, EPI_ROUND);
        else if (pro == PRO_RESID16 && epi == EPI_BF16) PLAMO_GEMV(PRO_RESID16, EPI_BF16);  // QSA indexer
        else if (pro == PRO_RESID16 && epi == EPI_SWIGLU) PLAMO_GEMV(PRO_RESID16, EPI_SWIGLU);
        else if (pro == PRO_RESID16 && epi == EPI_LOGITS) PLAMO_GEMV(PRO_RESID16, EPI_LOGITS);
        else if (pro == PRO_RESID && epi == EPI_LOGITS) PLAMO_GEMV(PRO_RESID, EPI_LOGITS);
        else if (pro == PRO_PLAIN && epi == EPI_LOGITS) PLAMO_GEMV(PRO_PLAIN, EPI_LOGITS);
        else throw Error(E_INVAL, "unsupported GEMV variant");
    } else {
        throw Error(E_INVAL, "unsupported GEMV variant");
    }
#undef PLAMO_GEMV
#undef PLAMO_GEMV_NOSTATE
}

template <int N>
void gemv_dispatch_n(bool packed, int maxr, Prologue pro, Epilogue epi, const GemvParams& p, int blocks,
                     hipStream_t s) {
    if (packed) {
        if (maxr == 1) gemv_dispatch_epi<N, true, 1>(pro, epi, p, blocks, s);
        else gemv_dispatch_epi<N, true, 4>(pro, epi, p, blocks, s);
    } else {
        if (maxr == 1) gemv_dispatch_epi<N, false, 1>(pro, epi, p, blocks, s);
        else gemv_dispatch_epi<N, false, 4>(pro, epi, p, blocks, s);
    }
}

}  // namespace

int gemv_group_rows(int n, int maxr, Epilogue epi, bool packed) {
    if (epi == EPI_SWIGLU) return maxr == 1 ? 4 : 2;
    if (n >= 6144) return maxr == 1 ? (packed ? 1 : 2) : 1;
    return maxr == 1 ? (n == ATTN ? 2 : 4) : 2;
}

int gemv_blocks(int n, int maxr, Epilogue epi, int m, bool packed) {
    const int groups = m / gemv_group_rows(n, maxr, epi, packed);
    const int nw = gemv_waves(n, maxr, epi);
    const int b = (groups + nw - 1) / nw;  // one group per wave
    // Multi-row kernels: at most two workgroups per CU, each wave walking several groups
    // (weights of the next in flight), so the activation prologue every workgroup
    // recomputes is paid twice per CU instead of four to six times.
    return maxr > 1 ? std::min(b, 2048 / nw) : b;
}

void launch_gemv(int n, bool packed, int maxr, Prologue pro, Epilogue epi, const GemvParams& p, int blocks,
                 hipStream_t s) {
    if (n == HIDDEN) gemv_dispatch_n<HIDDEN>(packed, maxr, pro, epi, p, blocks, s);
    else if (n == ATTN) gemv_dispatch_n<ATTN>(packed, maxr, pro, epi, p, blocks, s);
    else if (n == INTER) gemv_dispatch_n<INTER>(packed, maxr, pro, epi, p, blocks, s);
    else if (n == MTP_IN && !packed && maxr == 1 && !p.state) {  // the MTP adapter's up projection
        const dim3 grid(blocks), block(64 * gemv_waves(MTP_IN, 1, EPI_ROUND));
        if (pro != PRO_PLAIN || epi != EPI_ROUND) throw Error(E_INVAL, "unsupported GEMV variant");
        hipLaunchKernelGGL((gemv_kernel<MTP_IN, false, 1, PRO_PLAIN, EPI_ROUND, false>), grid, block, 0, s, p);
    } else throw Error(E_INVAL, "GEMV input width must be 1536, 2048, 3072 or 6144");
}

void launch_attention(bool full, const AttnParams& p, int rows, hipStream_t s) {
    const dim3 grid(32 * ((p.parts + 7) / 8), 1, rows), block(256);
    if (full) hipLaunchKernelGGL(attn_decode_kernel<true>, grid, block, 0, s, p);
    else hipLaunchKernelGGL(attn_decode_kernel<false>, grid, block, 0, s, p);
}

void launch_attention_merge(const AttnParams& p, int rows, hipStream_t s) {
    if (p.parts > uint32_t(MAX_CONTEXT / KEYS_PER_PART)) throw Error(E_INVAL, "attention merge: too many partitions");
    hipLaunchKernelGGL(attn_merge_kernel, dim3(HEAD_DIM / 32, HEADS, rows), dim3(256), 0, s, p);
}

void launch_head_merge(const DecodeBuffers& b, int blocks, bool begin_next, hipStream_t s) {
    hipLaunchKernelGGL(head_merge_kernel, dim3(1), dim3(256), 0, s, b, blocks, begin_next ? 1 : 0);
}

void launch_step_begin(const DecodeBuffers& b, hipStream_t s) {
    hipLaunchKernelGGL(step_begin_kernel, dim3(1), dim3(256), 0, s, b);
}

void launch_argmax(const void* x, uint32_t* out, int n, int rows, bool bf16, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(512), 0, s, x, out, n, bf16 ? 1 : 0);
}

void launch_select(float* logits, int n, const int32_t* history, int hist, float penalty, int ngram, float frequency,
                   float presence, int32_t* out, hipStream_t s) {
    hipLaunchKernelGGL(select_kernel, dim3(1), dim3(256), 0, s, logits, n, history, hist, penalty, ngram, frequency,
                       presence, out);
}

void launch_mtp_input(const float* hidden, const uint16_t* embed, int token, float* out, hipStream_t s) {
    hipLaunchKernelGGL(mtp_input_kernel, dim3(1), dim3(256), 0, s, hidden, embed, token, out);
}

void launch_mtp_down(const float* up, const float* x, const uint16_t* w, float* out, hipStream_t s) {
    hipLaunchKernelGGL(mtp_down_kernel, dim3(HIDDEN / 4), dim3(256), 0, s, up, x, w, out);
}

void launch_unpack(const uint8_t* payload, const uint32_t* table, uint16_t* out, int64_t count, hipStream_t s) {
    if (count <= 0) return;
    if (count % 128) throw Error(E_INVAL, "unpack: count must be a whole number of 128-weight blocks");
    hipLaunchKernelGGL(unpack_kernel, dim3(unsigned((count / 8 + 255) / 256)), dim3(256), 0, s, payload, table, out, count);
}

void launch_attn_state(StepState* st, uint32_t* tickets, const int32_t* pos, int rows, hipStream_t s) {
    AttnStateArgs a{};
    for (int q = 0; q < ROWS; ++q) a.pos[q] = q < rows ? pos[q] : 0;
    a.rows = rows;
    hipLaunchKernelGGL(attn_state_kernel, dim3(1), dim3(64), 0, s, st, tickets, a);
}

void launch_fill_u32(uint32_t* p, uint32_t value, size_t count, hipStream_t s) {
    if (!count) return;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(unsigned((count + 255) / 256)), dim3(256), 0, s, p, value, count);
}

void timeline_copy(uint64_t* out, size_t words, bool clear) {
#ifdef PLAMO_TIMELINE
    const size_t n = size_t(TIMELINE_TAGS) * TIMELINE_BLOCKS * 2;
    if (out && words < n) throw Error(E_INVAL, "timeline buffer too small");
    void* dev = nullptr;
    PLAMO_HIP(hipGetSymbolAddress(&dev, HIP_SYMBOL(g_timeline)));
    if (out) PLAMO_HIP(hipMemcpy(out, dev, n * sizeof(uint64_t), hipMemcpyDeviceToHost));
    if (clear) PLAMO_HIP(hipMemset(dev, 0, n * sizeof(uint64_t)));
#else
    (void)out;
    (void)words;
    (void)clear;
    throw Error(E_INVAL, "this library was built without the step timeline (make timeline)");
#endif
}

}  // namespace plamo
