// Prefill kernels for gfx950: MFMA BF16 GEMM (plain or .p12 weights) with fused epilogues,
// row RMSNorm / residual kernels and the K/V cache writer.
//
//   gemm_kernel     Y[t][m] = sum_k X[t][k] W[m][k]; 128x128 tiles, BK 64, LDS-staged,
//                   v_mfma_f32_32x32x16_bf16.  Replaces `matrix` (Kernels.metal:149-200) for
//                   the projections and `swiglu` (Kernels.metal:202-210) as an epilogue.
//   rows_norm       `norm` (Kernels.metal:46-90) for T rows: embedding gather + norm, or
//                   post-norm + residual + next norm.
//   kv_write        the K/V half of `qkv` (Kernels.metal:236-257): k RMSNorm, RoPE for the
//                   global layers, cache slot pos % capacity.
#include <hip/hip_runtime.h>

#include "common.h"
#include "device.h"
#include "kernels.h"
#include "prefill.h"

namespace plamo {
using namespace dev;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64, LDS_STRIDE = BK + 8;  // +16 B per row against bank conflicts

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

template <bool PACKED, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmParams p) {
    __shared__ __align__(16) uint16_t As[BM * LDS_STRIDE];
    __shared__ __align__(16) uint16_t Bs[BN * LDS_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * (EPI == GEMM_SWIGLU ? BN / 2 : BN);
    const int K = p.k;

    floatx16 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;

    for (int k0 = 0; k0 < K; k0 += BK) {
        // A tile: 128 token rows x 64 (X is BF16 [tokens][K])
#pragma unroll
        for (int e = tid; e < BM * BK / 8; e += 256) {
            const int r = e >> 3, c8 = e & 7;
            const int t = t0 + r;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (t < p.tokens) v = *reinterpret_cast<const uint4*>(p.x + size_t(t) * K + k0 + c8 * 8);
            *reinterpret_cast<uint4*>(&As[r * LDS_STRIDE + c8 * 8]) = v;
        }
        // B tile: 128 weight rows x 64
#pragma unroll
        for (int e = tid; e < BN * BK / 8; e += 256) {
            const int r = e >> 3, c8 = e & 7;
            int row;
            if constexpr (EPI == GEMM_SWIGLU) row = r < BN / 2 ? n0 + r : INTER + n0 + (r - BN / 2);
            else row = n0 + r;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row < p.m) {
                const int kk = k0 + c8 * 8;
                if constexpr (!PACKED) {
                    v = *reinterpret_cast<const uint4*>(p.w + size_t(row) * K + kk);
                } else {
                    const uint32_t entry = p.table[size_t(row) * (K / 128) + kk / 128];
                    const uint8_t* blk = reinterpret_cast<const uint8_t*>(p.w) + (entry & ~63u);
                    const uint32_t tag = entry & 63u;
                    const int sub = (kk % 128) / 8;
                    if (tag == 0) v = *reinterpret_cast<const uint4*>(blk + sub * 16);
                    else
                        v = p12_decode8(*reinterpret_cast<const uint2*>(blk + sub * 8),
                                        *reinterpret_cast<const uint32_t*>(blk + 128 + sub * 4), tag);
                }
            }
            *reinterpret_cast<uint4*>(&Bs[r * LDS_STRIDE + c8 * 8]) = v;
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kc = ks * 16 + (lane >> 5) * 8;
            const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(&As[(wave * 32 + (lane & 31)) * LDS_STRIDE + kc]));
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const bf16x8 b = as_bf16x8(*reinterpret_cast<const uint4*>(&Bs[(c * 32 + (lane & 31)) * LDS_STRIDE + kc]));
                acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // C layout of the 32x32 tile: column j = lane%32, row i = (r/4)*8 + (lane/32)*4 + r%4
    const int j = lane & 31;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        const int t = t0 + wave * 32 + i;
        if (t >= p.tokens) continue;
        if constexpr (EPI == GEMM_SWIGLU) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int m = n0 + c * 32 + j;
                const float g = roundbf(acc[c][r]);
                const float u = roundbf(acc[c + 2][r]);
                p.y16[size_t(t) * INTER + m] = uint16_t(bits(roundbf(g / (1.0f + exp_det(-g))) * u));
            }
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int m = n0 + c * 32 + j;
                if (m >= p.m) continue;
                if constexpr (EPI == GEMM_F32) p.y[size_t(t) * p.m + m] = roundbf(acc[c][r]);
                else if constexpr (EPI == GEMM_RAW) p.y[size_t(t) * p.m + m] = acc[c][r];
                else p.y16[size_t(t) * p.m + m] = uint16_t(bits(acc[c][r]));
            }
        }
    }
}

// ------------------------------------------------------------------------------ norms
// One workgroup per token, 6 elements per thread (Kernels.metal:46-90).
__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(256) void rows_norm_kernel(const RowsNormParams p) {
    __shared__ float red[4];
    constexpr int E = HIDDEN / 256;
    const int t = blockIdx.x, tid = threadIdx.x;
    float xv[E];
    if (p.tokens_in) {
        int tok = p.tokens_in[t];
        tok = (tok < 0 || tok >= VOCAB) ? 0 : tok;
#pragma unroll
        for (int k = 0; k < E; ++k) xv[k] = bf(p.embed[size_t(tok) * HIDDEN + tid + 256 * k]);
    } else {
        float pv[E], ss = 0.f;
#pragma unroll
        for (int k = 0; k < E; ++k) {
            pv[k] = p.in[size_t(t) * HIDDEN + tid + 256 * k];
            ss += pv[k] * pv[k];
        }
        const float r = 1.0f / sqrtf(block_sum256(ss, red) / float(HIDDEN) + 1e-6f);
#pragma unroll
        for (int k = 0; k < E; ++k) {
            const int i = tid + 256 * k;
            const float z = roundbf(roundbf(pv[k] * r) * roundbf(bf(p.g_post[i]) + p.post_offset));
            xv[k] = roundbf(p.x[size_t(t) * HIDDEN + i] + z);
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < E; ++k) ss += xv[k] * xv[k];
    const float r = 1.0f / sqrtf(block_sum256(ss, red) / float(HIDDEN) + 1e-6f);
#pragma unroll
    for (int k = 0; k < E; ++k) {
        const int i = tid + 256 * k;
        p.x[size_t(t) * HIDDEN + i] = xv[k];
        if (p.xn) p.xn[size_t(t) * HIDDEN + i] = uint16_t(bits(roundbf(roundbf(xv[k] * r) * roundbf(bf(p.g_next[i]) + 1.0f))));
    }
}

// ---------------------------------------------------------------------------- kv write
// 16 lanes per token: k RMSNorm (+1), RoPE at the absolute position for global layers,
// then K/V to slot pos % capacity (Kernels.metal:236-257).
__global__ __launch_bounds__(256) void kv_write_kernel(const KvWriteParams p) {
    const int tl = threadIdx.x >> 4, sub = threadIdx.x & 15;
    const int t = blockIdx.x * 16 + tl;
    const bool valid = t < p.tokens;
    const uint32_t pos = p.p0 + (valid ? t : 0);
    const float* x = p.qkv + size_t(valid ? t : 0) * QKV;
    const float4 klo = *reinterpret_cast<const float4*>(x + ATTN + sub * 4);
    const float4 khi = *reinterpret_cast<const float4*>(x + ATTN + 64 + sub * 4);
    const uint2 gl = *reinterpret_cast<const uint2*>(p.k_norm + sub * 4);
    const uint2 gh = *reinterpret_cast<const uint2*>(p.k_norm + 64 + sub * 4);
    float z[8];
    head_norm8(klo, khi, gl, gh, z);
    if (!valid) return;
    if (p.full) {
        const uint4 gr = *reinterpret_cast<const uint4*>(p.global_rope + size_t(pos) * 64 + sub * 4);
        const uint32_t c4[4] = {gr.x, gr.y, gr.z, gr.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) rope_pair(z[j], z[4 + j], c4[j], z[j], z[4 + j]);
    }
    const size_t slot = size_t(pos % p.capacity) * HEAD_DIM;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        p.keys[slot + sub * 4 + j] = uint16_t(bits(z[j]));
        p.keys[slot + 64 + sub * 4 + j] = uint16_t(bits(z[4 + j]));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int d = sub * 8 + j;
        p.values[slot + d] = uint16_t(bits(x[ATTN + HEAD_DIM + d]));
    }
}

}  // namespace

void launch_gemm(bool packed, GemmEpilogue epi, const GemmParams& p, hipStream_t s) {
    const int cols = epi == GEMM_SWIGLU ? INTER / (BN / 2) : (p.m + BN - 1) / BN;
    const dim3 grid(cols, (p.tokens + BM - 1) / BM), block(256);
    if (p.k % BK != 0 || (epi == GEMM_SWIGLU && p.m != 2 * INTER)) throw Error(E_INVAL, "unsupported GEMM shape");
#define PLAMO_GEMM(PK, EP) hipLaunchKernelGGL((gemm_kernel<PK, EP>), grid, block, 0, s, p)
    if (packed) {
        if (epi == GEMM_F32) PLAMO_GEMM(true, GEMM_F32);
        else if (epi == GEMM_BF16) PLAMO_GEMM(true, GEMM_BF16);
        else if (epi == GEMM_RAW) PLAMO_GEMM(true, GEMM_RAW);
        else PLAMO_GEMM(true, GEMM_SWIGLU);
    } else {
        if (epi == GEMM_F32) PLAMO_GEMM(false, GEMM_F32);
        else if (epi == GEMM_BF16) PLAMO_GEMM(false, GEMM_BF16);
        else if (epi == GEMM_RAW) PLAMO_GEMM(false, GEMM_RAW);
        else PLAMO_GEMM(false, GEMM_SWIGLU);
    }
#undef PLAMO_GEMM
}

void launch_rows_norm(const RowsNormParams& p, int tokens, hipStream_t s) {
    hipLaunchKernelGGL(rows_norm_kernel, dim3(tokens), dim3(256), 0, s, p);
}

void launch_kv_write(const KvWriteParams& p, hipStream_t s) {
    hipLaunchKernelGGL(kv_write_kernel, dim3((p.tokens + 15) / 16), dim3(256), 0, s, p);
}

}  // namespace plamo
