// Host-side definitions shared by the runtime: model geometry, errors, HIP checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace plamo {

// Geometry the reference's config loader insists on (Runtime.swift:181-188).
constexpr int HIDDEN = 1536;
constexpr int LAYERS = 16;
constexpr int HEADS = 16;
constexpr int HEAD_DIM = 128;
constexpr int ATTN = HEADS * HEAD_DIM;        // 2048
constexpr int QKV = ATTN + 2 * HEAD_DIM;      // 2304: q 0..2047, k 2048..2175, v 2176..2303
constexpr int INTER = 6144;
constexpr int VOCAB = 107520;
constexpr int WINDOW = 2048;
constexpr int MAX_CONTEXT = 32768;
constexpr int CHUNK = 16;                     // Runtime.chunk (Runtime.swift:129)
constexpr int MAX_ROWS = 4;                   // Batch lanes (Batch.swift:40)
constexpr int LOCAL_ROPE_ROWS = WINDOW + CHUNK;  // Runtime.swift:266
constexpr float POST_MIXER_OFFSET = 0.2f;     // Runtime.swift:446
constexpr float NEXT_OFFSET = 1.0f;           // Runtime.swift:377,455
// Trained adapters (Auxiliary.swift:87-111): the MTP head's rank and input width, the QSA
// indexer's projection width (4 query heads + 1 key of 128), rows one verification pass
// outputs (Runtime.verifyRows, Runtime.swift:130)
constexpr int MTP_RANK = 256;
constexpr int MTP_IN = 2 * HIDDEN;            // 3072: [hidden | embedding]
constexpr int QSA_PROJ = 5 * HEAD_DIM;        // 640
constexpr int VERIFY_ROWS = 2;

inline bool is_global_layer(int layer) { return layer % 8 == 7; }  // Runtime.swift:239

enum ErrorCode { E_INVAL = 1, E_IO = 2, E_FORMAT = 3, E_DEVICE = 4, E_STATE = 5 };

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define PLAMO_HIP(call)                                                                    \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess)                                                              \
            throw ::plamo::Error(::plamo::E_DEVICE, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

inline float host_bf(uint16_t h) {
    uint32_t u = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline uint16_t host_bits(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float post_mlp_offset();  // Float(1 / pow(5.0, 1.5)) (Runtime.swift:450)

// SHA-256 of a file (FIPS 180-4), hex digest.
std::string sha256_file(const std::string& path);

}  // namespace plamo
