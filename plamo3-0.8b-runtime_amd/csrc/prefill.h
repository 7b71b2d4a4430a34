// Parameter blocks of the prefill kernels (prefill.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

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
    const uint16_t* in;        // residual mode: projection output [T][1536] BF16
    const uint16_t* g_post;
    float post_offset;
    uint16_t* x;               // residual stream [T][1536] BF16 (updated in place; every value
                               // is BF16-rounded, so the BF16 copy is lossless)
    const uint16_t* g_next;
    uint16_t* xn;              // next-norm output BF16 [T][1536] (optional)
    int tokens;                // set by launch_rows_norm
};

struct QkPrepParams {
    const uint16_t* qkv;       // [T][2304] BF16
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    uint16_t* q16;             // out: [T][16][128] BF16, normalised and rotated queries
    uint16_t* keys;            // lane slice [capacity][128]
    uint16_t* values;
    uint16_t* keys_rot;        // local layers: lane slice [rot_rows][128] (null: none)
    uint32_t rot_rows;
    uint32_t capacity, p0;
    int tokens;
    int full;
    const uint32_t* local_rope;   // [2064][64] BF16 (cos | sin << 16)
    const uint32_t* global_rope;  // [context][64]
};

// Flash prefill splits the key tiles of a query block (8 tokens x 16 heads) over up to
// FLASH_PARTS workgroups; their partial results meet in a workspace.
constexpr int FLASH_PARTS = 3;
constexpr int FLASH_PART_TILES = 11;         // 64-key tiles a part aims at
__host__ __device__ inline int flash_blocks(int tokens) { return (tokens + 7) / 8; }
// workspace floats: per block and part, O^T [128 columns][128 dims] and (m, l) per column
// Key tiles (64 keys) that query block qb of a call attends to, and the parts they are split
// into (contiguous tile ranges, part q from q * tiles / parts).
__host__ __device__ inline int flash_block_tiles(int tokens, uint32_t p0, int full, int qb) {
    const int t0 = qb * 8, t1 = t0 + 8 < tokens ? t0 + 8 : tokens;
    const uint32_t plo = p0 + uint32_t(t0), khi = p0 + uint32_t(t1 - 1);
    const uint32_t klo = full ? 0u : (plo > uint32_t(WINDOW - 1) ? plo - uint32_t(WINDOW - 1) : 0u);
    return int((khi + 1 - klo + 63) / 64);
}
__host__ __device__ inline int flash_block_parts(int tiles) {
    const int parts = (tiles + FLASH_PART_TILES - 1) / FLASH_PART_TILES;
    return parts < FLASH_PARTS ? parts : FLASH_PARTS;
}
// The order in which workgroups take the (query block, part) items of a call: item w of the
// launch is item[w] (qb << 2 | part).  n = 0: workgroup w takes part w / blocks of block
// blocks - 1 - w % blocks (and returns if the block has fewer parts).
constexpr int FLASH_SCHEDULE_MAX = 768;  // the items of a 2048-token call, at most
struct FlashSchedule {
    uint32_t n;
    uint16_t item[FLASH_SCHEDULE_MAX];
};
inline size_t flash_part_o_floats(int tokens) { return size_t(flash_blocks(tokens)) * FLASH_PARTS * 128 * 128; }
inline size_t flash_part_ml_floats(int tokens) { return size_t(flash_blocks(tokens)) * FLASH_PARTS * 128 * 2; }

struct FlashParams {
    const uint16_t* q;         // [T][16][128] BF16, normalised and rotated
    const uint16_t* keys;      // lane slice [capacity][128]
    const uint16_t* values;
    const uint32_t* local_rope;   // local layers: keys rotate with chunk-relative coordinates
    const uint16_t* keys_rot;  // local layers: lane slice [rot_rows][128] of keys rotated at their
                               // own position (null: rotate every key)
    uint32_t rot_rows;
    uint16_t* out;             // [T][2048] BF16
    uint32_t capacity, p0;
    int tokens;
    int full;
    float* part_o;             // flash_part_o_floats(tokens)
    float* part_ml;            // flash_part_ml_floats(tokens)
    uint32_t* tickets;         // flash_blocks(tokens), zero between launches
    const uint32_t* qsa_mask;  // global layers with QSA: token t's selected blocks of four keys
                               // (bit b of word t * qsa_words + b / 32); null: every key
    uint32_t qsa_words;
};

void launch_gemm(bool packed, GemmEpilogue epi, const GemmParams& p, hipStream_t s);
void launch_rows_norm(const RowsNormParams& p, int tokens, hipStream_t s);
void launch_qk_prep(const QkPrepParams& p, hipStream_t s);
void launch_flash_prefill(const FlashParams& p, hipStream_t s);

}  // namespace plamo
