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

#include "common.h"
#include "device.h"
#include "kernels.h"

namespace plamo {
using namespace dev;

namespace {

// ---------------------------------------------------------------------------- prologues
// Stage the BF16 activation rows into LDS.  Values are BF16-exact FP32 (every producer
// rounds), so the BF16 copy is lossless.
template <int N, int MAXR, int PRO>
__device__ __forceinline__ void stage_rows(const GemvParams& p, int rows, uint16_t* xs, float* red) {
    const int tid = threadIdx.x;
    if constexpr (PRO == PRO_PLAIN) {
        for (int q = 0; q < MAXR; ++q) {
            if (q >= rows) break;
            for (int i = tid; i < N; i += 256) xs[q * N + i] = uint16_t(bits(p.in[q * N + i]));
        }
    } else {
        static_assert(N == HIDDEN, "norm prologue is 1536 wide");
        constexpr int E = HIDDEN / 256;  // 6 elements per thread
        float xv[MAXR][E];
        float ss[MAXR];
        if constexpr (PRO == PRO_EMBED) {
#pragma unroll
            for (int q = 0; q < MAXR; ++q) {
                int tok = (q < rows && p.state) ? p.state->token[q] : 0;
                tok = (tok < 0 || tok >= VOCAB) ? 0 : tok;  // loop guards stop before this
#pragma unroll
                for (int k = 0; k < E; ++k)
                    xv[q][k] = (q < rows) ? bf(p.embed[size_t(tok) * HIDDEN + tid + 256 * k]) : 0.f;
            }
        } else {
            // z = roundbf(roundbf(p*r) * roundbf(bf(w)+offset)); x = roundbf(x + z)
            // (Kernels.metal:59-72, full == 1)
            float pv[MAXR][E];
#pragma unroll
            for (int q = 0; q < MAXR; ++q) {
                ss[q] = 0.f;
#pragma unroll
                for (int k = 0; k < E; ++k) {
                    pv[q][k] = (q < rows) ? p.in[q * HIDDEN + tid + 256 * k] : 0.f;
                    ss[q] += pv[q][k] * pv[q][k];
                }
            }
#pragma unroll
            for (int q = 0; q < MAXR; ++q) {
                ss[q] = wave_sum(ss[q]);
                if ((tid & 63) == 0) red[q * 4 + (tid >> 6)] = ss[q];
            }
            __syncthreads();
#pragma unroll
            for (int q = 0; q < MAXR; ++q) {
                const float total = (red[q * 4] + red[q * 4 + 1]) + (red[q * 4 + 2] + red[q * 4 + 3]);
                const float r = 1.0f / sqrtf(total / float(HIDDEN) + 1e-6f);
#pragma unroll
                for (int k = 0; k < E; ++k) {
                    const int i = tid + 256 * k;
                    const float g = roundbf(bf(p.g_post[i]) + p.post_offset);
                    const float z = roundbf(roundbf(pv[q][k] * r) * g);
                    xv[q][k] = (q < rows) ? roundbf(p.resid_in[q * HIDDEN + i] + z) : 0.f;
                }
            }
            __syncthreads();
        }
        // next norm with +1 offset (Kernels.metal:76-89)
#pragma unroll
        for (int q = 0; q < MAXR; ++q) {
            ss[q] = 0.f;
#pragma unroll
            for (int k = 0; k < E; ++k) ss[q] += xv[q][k] * xv[q][k];
            ss[q] = wave_sum(ss[q]);
            if ((tid & 63) == 0) red[q * 4 + (tid >> 6)] = ss[q];
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < MAXR; ++q) {
            if (q >= rows) break;
            const float total = (red[q * 4] + red[q * 4 + 1]) + (red[q * 4 + 2] + red[q * 4 + 3]);
            const float r = 1.0f / sqrtf(total / float(HIDDEN) + 1e-6f);
#pragma unroll
            for (int k = 0; k < E; ++k) {
                const int i = tid + 256 * k;
                const float g = roundbf(bf(p.g_next[i]) + 1.0f);
                const float xn = roundbf(roundbf(xv[q][k] * r) * g);
                xs[q * HIDDEN + i] = uint16_t(bits(xn));
                if (blockIdx.x == 0) {
                    p.resid_out[q * HIDDEN + i] = xv[q][k];
                    if (p.hidden) p.hidden[q * HIDDEN + i] = xn;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------- weight loads
// Lane `lane` owns columns it*512 + lane*8 .. +8 of a row: inside .p12 block it*4+lane/16
// at offset (lane%16)*8.  Plain and packed therefore feed identical words to dot8, so
// packed results are bit-identical to plain ones.
template <int N, bool PACKED>
__device__ __forceinline__ uint4 load_w(const GemvParams& p, int row, int it, int lane) {
    if constexpr (!PACKED) {
        const uint16_t* src = p.w + size_t(row) * N + it * 512 + lane * 8;
        return *reinterpret_cast<const uint4*>(src);
    } else {
        const uint32_t entry = p.table[size_t(row) * (N / 128) + it * 4 + (lane >> 4)];
        const uint8_t* blk = reinterpret_cast<const uint8_t*>(p.w) + (entry & ~63u);
        const uint32_t tag = entry & 63u;
        const int sub = lane & 15;
        if (tag == 0) return *reinterpret_cast<const uint4*>(blk + sub * 16);
        const uint2 sm = *reinterpret_cast<const uint2*>(blk + sub * 8);
        const uint32_t nib = *reinterpret_cast<const uint32_t*>(blk + 128 + sub * 4);
        return p12_decode8(sm, nib, tag);
    }
}

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);  // Kernels.metal:716
}

// Sampler.select adjustments of one logit (Sampler.swift:11-24), FP32, no contraction.
__device__ __forceinline__ float sampled(float l, int32_t count, bool banned, const StepState* st) {
#pragma clang fp contract(off)
    if (count > 0) {
        if (st->penalty != 1.0f) l = l > 0.0f ? l / st->penalty : l * st->penalty;
        if (st->presence != 0.0f) l = l - st->presence;
        if (st->frequency != 0.0f) {
            const float f = st->frequency * float(count);
            l = l - f;
        }
    }
    return banned ? NEG_INF : l;
}

// ------------------------------------------------------------------------------- GEMV
template <int N, bool PACKED, int MAXR, int PRO, int EPI>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvParams p) {
    constexpr int IT = N / 512;
    constexpr int U = (EPI == EPI_SWIGLU) ? 4 : (N >= 6144 ? 2 : 4);
    __shared__ __align__(16) uint16_t xs[MAXR * N];
    __shared__ float red[MAXR * 4];
    __shared__ float cand_v[MAXR * 4];
    __shared__ uint32_t cand_i[MAXR * 4];
    __shared__ int s_last;

    const StepState* st = p.state;
    if (st && st->stopped) return;
    const int rows = st ? int(st->rows) : p.rows;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    stage_rows<N, MAXR, PRO>(p, rows, xs, red);
    __syncthreads();

    const int groups = (EPI == EPI_SWIGLU) ? p.m / 4 : p.m / U;
    float best_v[MAXR];
    uint32_t best_i[MAXR];
#pragma unroll
    for (int q = 0; q < MAXR; ++q) { best_v[q] = NEG_INF; best_i[q] = 0xffffffffu; }

    for (int g = blockIdx.x * 4 + wave; g < groups; g += gridDim.x * 4) {
        int wrow[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (EPI == EPI_SWIGLU) wrow[u] = (u < 2) ? 2 * g + u : INTER + 2 * g + (u - 2);
            else wrow[u] = g * U + u;
        }
        uint4 w[U][IT];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int it = 0; it < IT; ++it) w[u][it] = load_w<N, PACKED>(p, wrow[u], it, lane);
        float acc[U][MAXR];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int q = 0; q < MAXR; ++q) acc[u][q] = 0.f;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
#pragma unroll
            for (int q = 0; q < MAXR; ++q) {
                if (q < rows) {
                    const uint4 xv = *reinterpret_cast<const uint4*>(&xs[q * N + it * 512 + lane * 8]);
#pragma unroll
                    for (int u = 0; u < U; ++u) acc[u][q] = dot8(w[u][it], xv, acc[u][q]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int q = 0; q < MAXR; ++q) acc[u][q] = wave_sum(acc[u][q]);

        if constexpr (EPI == EPI_ROUND) {
            if (lane == 0)
#pragma unroll
                for (int q = 0; q < MAXR; ++q)
                    if (q < rows)
#pragma unroll
                        for (int u = 0; u < U; ++u) p.out[size_t(q) * p.m + wrow[u]] = roundbf(acc[u][q]);
        } else if constexpr (EPI == EPI_BF16) {
            if (lane == 0)
#pragma unroll
                for (int q = 0; q < MAXR; ++q)
                    if (q < rows)
#pragma unroll
                        for (int u = 0; u < U; ++u) p.out16[size_t(q) * p.m + wrow[u]] = uint16_t(bits(acc[u][q]));
        } else if constexpr (EPI == EPI_SWIGLU) {
            // gates = roundbf(g), ups = roundbf(u); y = roundbf(roundbf(g/(1+exp(-g))) * u)
            // (Kernels.metal:202-210)
            if (lane == 0)
#pragma unroll
                for (int q = 0; q < MAXR; ++q)
                    if (q < rows)
#pragma unroll
                        for (int k = 0; k < 2; ++k) {
                            const float gt = roundbf(acc[k][q]);
                            const float up = roundbf(acc[2 + k][q]);
                            p.out[size_t(q) * INTER + 2 * g + k] = roundbf(roundbf(gt / (1.0f + exp_det(-gt))) * up);
                        }
        } else {  // EPI_LOGITS
#pragma unroll
            for (int q = 0; q < MAXR; ++q) {
                if (q >= rows) continue;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t b = bits(acc[u][q]);
                    if (lane == 0) p.out16[size_t(q) * VOCAB + wrow[u]] = uint16_t(b);
                    float v = bf(b);
                    if (st && st->sampling) {
                        const uint32_t r = uint32_t(wrow[u]);
                        const int32_t c = p.bufs.counts[size_t(q) * VOCAB + r];
                        const bool ban = st->ngram > 1 &&
                                         ((p.bufs.banned[size_t(q) * (VOCAB / 32) + (r >> 5)] >> (r & 31)) & 1u);
                        v = sampled(v, c, ban, st);
                    }
                    if (better(v, uint32_t(wrow[u]), best_v[q], best_i[q])) { best_v[q] = v; best_i[q] = wrow[u]; }
                }
            }
        }
    }

    if constexpr (EPI == EPI_LOGITS) {
        // block partial -> ticket -> the last workgroup merges in block order
        if (lane == 0)
#pragma unroll
            for (int q = 0; q < MAXR; ++q) { cand_v[q * 4 + wave] = best_v[q]; cand_i[q * 4 + wave] = best_i[q]; }
        __syncthreads();
        if (tid < MAXR && tid < rows) {
            const int q = tid;
            float bv = cand_v[q * 4];
            uint32_t bi = cand_i[q * 4];
            for (int k = 1; k < 4; ++k)
                if (better(cand_v[q * 4 + k], cand_i[q * 4 + k], bv, bi)) { bv = cand_v[q * 4 + k]; bi = cand_i[q * 4 + k]; }
            p.bufs.head_v[q * HEAD_BLOCKS + blockIdx.x] = bv;
            p.bufs.head_i[q * HEAD_BLOCKS + blockIdx.x] = bi;
        }
        __threadfence();
        __syncthreads();
        if (tid == 0) {
            const uint32_t prev = atomicAdd(&p.bufs.tickets[0], 1u);
            s_last = prev == gridDim.x - 1;
        }
        __syncthreads();
        if (!s_last) return;
        __threadfence();
        if (tid < MAXR && tid < rows) {
            const int q = tid;
            float bv = NEG_INF;
            uint32_t bi = 0xffffffffu;
            for (int k = 0; k < int(gridDim.x); ++k) {
                const float v = __builtin_nontemporal_load(&p.bufs.head_v[q * HEAD_BLOCKS + k]);
                const uint32_t i = __builtin_nontemporal_load(&p.bufs.head_i[q * HEAD_BLOCKS + k]);
                if (better(v, i, bv, bi)) { bv = v; bi = i; }
            }
            StepState* sw = p.bufs.state;
            if (sw->sampling && bi == 0xffffffffu) bi = 0;  // Sampler.select default index (Sampler.swift:26)
            sw->next[q] = bi;
            if (sw->loop) {
                sw->token[q] = int32_t(bi);
                sw->pos[q] += 1;
            }
        }
        if (tid == 0) p.bufs.tickets[0] = 0;
    }
}

// ---------------------------------------------------------------------- decode attention
constexpr int KP = KEYS_PER_PART;
constexpr int KS = 129;  // padded LDS row of rotated keys

template <bool FULL>
__global__ __launch_bounds__(256) void attn_decode_kernel(const AttnParams p) {
#pragma clang fp contract(off)  // fixed rounding sequence, reproduced by the CPU oracle
    __shared__ float zs[17 * HEAD_DIM];
    __shared__ float qs[HEADS * HEAD_DIM];
    __shared__ float ks[KP * KS];
    __shared__ __align__(16) uint16_t vs[KP * HEAD_DIM];
    __shared__ float ps[HEADS * KP];
    __shared__ int s_last;

    const StepState* st = p.state;
    const int q = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Row geometry.  Visible keys are the absolute positions first..pos (window 2048 on the
    // local layers); key r sits at ring slot (first + r) % capacity.  Local keys rotate
    // with coordinate coff + r and the query with qcoord, both relative to the RoPE base
    // of the reference's 16-token chunk: base = max(0, chunk_start - 2047)
    // (Runtime.swift:389, Kernels.metal:251,283-284).  Decode is a chunk of one token.
    uint32_t pos, lanei, first, coff, qcoord;
    if (st) {
        if (st->stopped || q >= int(st->rows)) return;
        pos = st->pos[q];
        lanei = st->lane[q];
        first = FULL ? 0u : (pos > uint32_t(WINDOW - 1) ? pos - uint32_t(WINDOW - 1) : 0u);
        coff = 0;
        qcoord = FULL ? pos : pos - first;
    } else {
        pos = p.p0 + q;
        lanei = p.lane;
        const uint32_t chunk = p.p0 + (uint32_t(q) / CHUNK) * CHUNK;
        const uint32_t base = chunk > uint32_t(WINDOW - 1) ? chunk - uint32_t(WINDOW - 1) : 0u;
        first = FULL ? 0u : (pos > uint32_t(WINDOW - 1) ? pos - uint32_t(WINDOW - 1) : 0u);
        coff = first - base;
        qcoord = FULL ? pos : pos - base;
    }
    const uint32_t count = pos + 1 - first;
    const uint32_t k0 = blockIdx.x * KP;
    const uint32_t cap = p.capacity;
    const uint32_t start = first % cap;
    uint16_t* K = p.keys + size_t(lanei) * cap * HEAD_DIM;
    uint16_t* V = p.values + size_t(lanei) * cap * HEAD_DIM;
    const size_t pslot = size_t(q) * p.parts + blockIdx.x;

    if (k0 < count) {
        // q/k RMSNorm over 128 with +1 offset (Kernels.metal:236-246)
        const float* x = p.qkv + size_t(q) * QKV;
        for (int h = tid >> 4; h < 17; h += 16) {
            const int sub = tid & 15;
            float v[8];
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[j] = x[h * HEAD_DIM + sub * 8 + j];
                ss += v[j] * v[j];
            }
            ss = group16_sum(ss);
            const float r = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
            const uint16_t* g = h < HEADS ? p.q_norm : p.k_norm;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = sub * 8 + j;
                zs[h * HEAD_DIM + d] = roundbf(roundbf(v[j] * r) * roundbf(bf(g[d]) + 1.0f));
            }
        }
        __syncthreads();
        // RoPE of the queries: global at pos, local at pos-base (Kernels.metal:250-252)
        const float2* qrope = FULL ? p.global_rope + size_t(pos) * 64 : p.local_rope + size_t(qcoord) * 64;
        for (int e = tid; e < HEADS * 64; e += 256) {
            const int h = e >> 6, d = e & 63;
            float ra, rb;
            rope_pair(zs[h * HEAD_DIM + d], zs[h * HEAD_DIM + d + 64], qrope[d], ra, rb);
            qs[h * HEAD_DIM + d] = ra;
            qs[h * HEAD_DIM + d + 64] = rb;
        }
        // Keys and values of this partition.  The newest key (relative index count-1) is
        // produced here: stored normalised-unrotated (local) or rotated at pos (global),
        // written to slot pos % capacity (Kernels.metal:253-257).
        const uint32_t newest = st ? count - 1 : 0xffffffffu;  // prefill keys are already cached
        for (int e = tid; e < KP * 16; e += 256) {
            const int j = e >> 4, c8 = e & 15;
            const uint32_t r = k0 + j;
            uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
            if (r < count && r != newest) {
                uint32_t phys = start + r;
                phys = phys >= cap ? phys - cap : phys;  // visible keys (<= capacity) wrap at most once
                kv = *reinterpret_cast<const uint4*>(K + size_t(phys) * HEAD_DIM + c8 * 8);
                vv = *reinterpret_cast<const uint4*>(V + size_t(phys) * HEAD_DIM + c8 * 8);
            }
            float* kr = ks + j * KS + c8 * 8;
            kr[0] = lo(kv.x); kr[1] = hi(kv.x); kr[2] = lo(kv.y); kr[3] = hi(kv.y);
            kr[4] = lo(kv.z); kr[5] = hi(kv.z); kr[6] = lo(kv.w); kr[7] = hi(kv.w);
            *reinterpret_cast<uint4*>(vs + j * HEAD_DIM + c8 * 8) = vv;
        }
        __syncthreads();
        if (newest >= k0 && newest < k0 + KP) {
            const int j = int(newest - k0);
            const size_t slot = size_t(pos % cap) * HEAD_DIM;
            if (tid < 64) {
                const int d = tid;
                float a = zs[16 * HEAD_DIM + d], b = zs[16 * HEAD_DIM + d + 64];
                if (FULL) rope_pair(a, b, p.global_rope[size_t(pos) * 64 + d], a, b);
                const uint32_t ba = bits(a), bb = bits(b);
                K[slot + d] = uint16_t(ba);
                K[slot + d + 64] = uint16_t(bb);
                ks[j * KS + d] = bf(ba);
                ks[j * KS + d + 64] = bf(bb);
            } else if (tid < 192) {
                const int d = tid - 64;
                const uint32_t bv = bits(x[QKV - HEAD_DIM + d]);
                V[slot + d] = uint16_t(bv);
                vs[j * HEAD_DIM + d] = uint16_t(bv);
            }
            __syncthreads();
        }
        // Local keys are rotated with their chunk-relative coordinate r (Kernels.metal:283-284)
        if (!FULL) {
            for (int e = tid; e < KP * 64; e += 256) {
                const int j = e >> 6, d = e & 63;
                const uint32_t r = k0 + j;
                if (r < count) {
                    float ra, rb;
                    rope_pair(ks[j * KS + d], ks[j * KS + d + 64], p.local_rope[size_t(coff + r) * 64 + d], ra, rb);
                    ks[j * KS + d] = ra;
                    ks[j * KS + d + 64] = rb;
                }
            }
            __syncthreads();
        }
        // scores for 4 heads per wave, one key per lane
        {
            const int j = lane, hb = wave * 4;
            float s[4] = {0.f, 0.f, 0.f, 0.f};
            for (int d = 0; d < HEAD_DIM; ++d) {
                const float kd = ks[j * KS + d];
#pragma unroll
                for (int hh = 0; hh < 4; ++hh) s[hh] = fmaf(qs[(hb + hh) * HEAD_DIM + d], kd, s[hh]);
            }
            const bool valid = k0 + j < count;
#pragma unroll
            for (int hh = 0; hh < 4; ++hh) {
                const float sc = valid ? s[hh] * SCALE : NEG_INF;
                const float m = wave_max(sc);
                const float e = valid ? exp_det(sc - m) : 0.f;
                const float l = wave_sum(e);
                ps[(hb + hh) * KP + j] = e;
                if (lane == 0) {
                    p.part_m[pslot * HEADS + hb + hh] = m;
                    p.part_l[pslot * HEADS + hb + hh] = l;
                }
            }
        }
        __syncthreads();
        // unnormalised P.V for 8 heads x 1 dim per thread
        {
            const int d = tid & 127, hb = (tid >> 7) * 8;
            float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int j = 0; j < KP; ++j) {
                const float v = bf(vs[j * HEAD_DIM + d]);
#pragma unroll
                for (int hh = 0; hh < 8; ++hh) o[hh] = o[hh] + ps[(hb + hh) * KP + j] * v;
            }
#pragma unroll
            for (int hh = 0; hh < 8; ++hh) p.part_o[(pslot * HEADS + hb + hh) * HEAD_DIM + d] = o[hh];
        }
    }
    // ticket: the last workgroup of this row merges the partitions
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&p.tickets[q], 1u);
        s_last = prev == gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const uint32_t nparts = (count + KP - 1) / KP;
    const size_t row0 = size_t(q) * p.parts;
    for (int e = tid; e < HEADS * HEAD_DIM; e += 256) {
        const int h = e >> 7, d = e & 127;
        float M = NEG_INF;
        for (uint32_t k = 0; k < nparts; ++k) M = fmaxf(M, __builtin_nontemporal_load(&p.part_m[(row0 + k) * HEADS + h]));
        float num = 0.f, den = 0.f;
        for (uint32_t k = 0; k < nparts; ++k) {
            const float w = exp_det(__builtin_nontemporal_load(&p.part_m[(row0 + k) * HEADS + h]) - M);
            den += __builtin_nontemporal_load(&p.part_l[(row0 + k) * HEADS + h]) * w;
            num += __builtin_nontemporal_load(&p.part_o[((row0 + k) * HEADS + h) * HEAD_DIM + d]) * w;
        }
        const float o = roundbf(num / den);
        if (p.out16) p.out16[size_t(q) * ATTN + h * HEAD_DIM + d] = uint16_t(bits(o));
        else p.out[size_t(q) * ATTN + h * HEAD_DIM + d] = o;
    }
    if (tid == 0) p.tickets[q] = 0;
}

// ------------------------------------------------------------------------- step begin
// Device side of the token loop (Main.swift:278-287) and of the sampler history
// (Main.swift:237-244; Sampler.swift:11-24,54-70).
__global__ __launch_bounds__(256) void step_begin_kernel(DecodeBuffers b) {
    StepState* st = b.state;
    __shared__ int s_stop;
    if (st->stopped) return;
    const int tid = threadIdx.x;
    if (tid == 0) {
        s_stop = 0;
        if (st->loop) {
            const int32_t tok = st->token[0];
            if (st->stop_enabled && (tok == 1 || tok == 16)) {
                st->stopped = 1; st->reason = 1; s_stop = 1;
            } else if (tok < 0 || tok >= VOCAB) {
                st->stopped = 1; st->reason = 3; s_stop = 1;
            } else {
                b.out_ids[st->produced] = tok;
                st->produced += 1;
                if (st->sampling && st->hist_len[0] < b.hist_cap) {
                    b.history[st->hist_len[0]] = tok;
                    st->hist_len[0] += 1;
                }
                if (st->produced >= st->max_tokens) { st->stopped = 1; st->reason = 2; s_stop = 1; }
            }
        }
    }
    __syncthreads();
    if (s_stop || !st->sampling) return;
    for (uint32_t q = 0; q < st->rows; ++q) {
        const int32_t* hist = b.history + size_t(q) * b.hist_cap;
        const uint32_t len = st->hist_len[q];
        if (tid == 0) {
            for (uint32_t i = st->counted[q]; i < len; ++i) {
                const int32_t id = hist[i];
                if (id >= 0 && id < VOCAB) b.counts[size_t(q) * VOCAB + id] += 1;
            }
            st->counted[q] = len;
        }
        if (st->ngram > 1) {
            uint32_t* ban = b.banned + size_t(q) * (VOCAB / 32);
            for (int i = tid; i < VOCAB / 32; i += 256) ban[i] = 0;
            __syncthreads();
            const int n = st->ngram, span = n - 1;
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

__global__ void unpack_kernel(const uint8_t* payload, const uint32_t* table, uint16_t* out, int64_t count) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint32_t entry = table[i / 128];
    const uint8_t* blk = payload + (entry & ~63u);
    const uint32_t tag = entry & 63u, k = uint32_t(i % 128);
    if (tag == 0) { out[i] = uint16_t(blk[2 * k] | (blk[2 * k + 1] << 8)); return; }
    const uint32_t code = (blk[128 + k / 2] >> ((k % 2) * 4)) & 15u;
    out[i] = uint16_t(p12_word(blk[k], code, tag + 107u));
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, size_t n) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

template <int N, bool PACKED, int MAXR>
void gemv_dispatch_epi(Prologue pro, Epilogue epi, const GemvParams& p, int blocks, hipStream_t s) {
    const dim3 grid(blocks), block(256);
#define PLAMO_GEMV(PRO, EPI) hipLaunchKernelGGL((gemv_kernel<N, PACKED, MAXR, PRO, EPI>), grid, block, 0, s, p)
    if (pro == PRO_PLAIN) {
        if (epi == EPI_ROUND) PLAMO_GEMV(PRO_PLAIN, EPI_ROUND);
        else if (epi == EPI_BF16) PLAMO_GEMV(PRO_PLAIN, EPI_BF16);
        else throw Error(E_INVAL, "unsupported GEMV variant");
        return;
    }
    if constexpr (N == HIDDEN) {
        if (pro == PRO_EMBED && epi == EPI_ROUND) PLAMO_GEMV(PRO_EMBED, EPI_ROUND);
        else if (pro == PRO_RESID && epi == EPI_ROUND) PLAMO_GEMV(PRO_RESID, EPI_ROUND);
        else if (pro == PRO_RESID && epi == EPI_SWIGLU) PLAMO_GEMV(PRO_RESID, EPI_SWIGLU);
        else if (pro == PRO_RESID && epi == EPI_LOGITS) PLAMO_GEMV(PRO_RESID, EPI_LOGITS);
        else if (pro == PRO_PLAIN && epi == EPI_LOGITS) PLAMO_GEMV(PRO_PLAIN, EPI_LOGITS);
        else throw Error(E_INVAL, "unsupported GEMV variant");
    } else {
        throw Error(E_INVAL, "unsupported GEMV variant");
    }
#undef PLAMO_GEMV
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

void launch_gemv(int n, bool packed, int maxr, Prologue pro, Epilogue epi, const GemvParams& p, int blocks,
                 hipStream_t s) {
    if (n == HIDDEN) gemv_dispatch_n<HIDDEN>(packed, maxr, pro, epi, p, blocks, s);
    else if (n == ATTN) gemv_dispatch_n<ATTN>(packed, maxr, pro, epi, p, blocks, s);
    else if (n == INTER) gemv_dispatch_n<INTER>(packed, maxr, pro, epi, p, blocks, s);
    else throw Error(E_INVAL, "GEMV input width must be 1536, 2048 or 6144");
}

void launch_attention(bool full, const AttnParams& p, int rows, hipStream_t s) {
    const dim3 grid(p.parts, rows), block(256);
    if (full) hipLaunchKernelGGL(attn_decode_kernel<true>, grid, block, 0, s, p);
    else hipLaunchKernelGGL(attn_decode_kernel<false>, grid, block, 0, s, p);
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

void launch_unpack(const uint8_t* payload, const uint32_t* table, uint16_t* out, int64_t count, hipStream_t s) {
    if (count <= 0) return;
    hipLaunchKernelGGL(unpack_kernel, dim3(unsigned((count + 255) / 256)), dim3(256), 0, s, payload, table, out, count);
}

void launch_fill_u32(uint32_t* p, uint32_t value, size_t count, hipStream_t s) {
    if (!count) return;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(unsigned((count + 255) / 256)), dim3(256), 0, s, p, value, count);
}

}  // namespace plamo
