// Parameter blocks of the prefill kernels (prefill.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace plamo {

enum GemmEpilogue { GEMM_F32 = 0, GEMM_BF16 = 1, GEMM_SWIGLU = 2, GEMM_RAW = 3 };

struct GemmParams {
    const uint16_t* w;      // plain BF16 [m][k] or .p12 payload
    const uint32_t* table;  // .p12 block table
    const uint16_t* x;      // BF16 [tokens][k]
    float* y;               // F32: [tokens][m]
    uint16_t* y16;          // BF16: [tokens][m]; SWIGLU: [tokens][6144]
    int m, k, tokens;
};

struct RowsNormParams {
    const int32_t* tokens_in;  // embedding mode when set
    const uint16_t* embed;
    const float* in;           // residual mode: projection output [T][1536]
    const uint16_t* g_post;
    float post_offset;
    float* x;                  // residual stream [T][1536] (updated in place)
    const uint16_t* g_next;
    uint16_t* xn;              // next-norm output BF16 [T][1536] (optional)
};

struct QkPrepParams {
    const float* qkv;          // [T][2304]
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    uint16_t* q16;             // out: [T][16][128] BF16, normalised and rotated queries
    uint16_t* keys;            // lane slice [capacity][128]
    uint16_t* values;
    uint32_t capacity, p0;
    int tokens;
    int full;
    const uint32_t* local_rope;   // [2064][64] BF16 (cos | sin << 16)
    const uint32_t* global_rope;  // [context][64]
};

struct FlashParams {
    const uint16_t* q;         // [T][16][128] BF16, normalised and rotated
    const uint16_t* keys;      // lane slice [capacity][128]
    const uint16_t* values;
    const uint32_t* local_rope;   // local layers: keys rotate with chunk-relative coordinates
    uint16_t* out;             // [T][2048] BF16
    uint32_t capacity, p0;
    int tokens;
    int full;
};

void launch_gemm(bool packed, GemmEpilogue epi, const GemmParams& p, hipStream_t s);
void launch_rows_norm(const RowsNormParams& p, int tokens, hipStream_t s);
void launch_qk_prep(const QkPrepParams& p, hipStream_t s);
void launch_flash_prefill(const FlashParams& p, hipStream_t s);

}  // namespace plamo
