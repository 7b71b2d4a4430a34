// Device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace plamo {
namespace dev {

constexpr float SCALE = 0.08838834764831845f;  // 1/sqrt(128) (Kernels.metal:372)
constexpr float NEG_INF = -__builtin_inff();

// BF16 <-> FP32 exactly as Kernels.metal:5-10: integer round-to-nearest-even on the FP32
// bit pattern with wrap-around and no NaN special case.
__device__ __forceinline__ float bf(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ uint32_t bits(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float roundbf(float x) { return bf(bits(x)); }
__device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float lo_bf(uint32_t w) { return lo(w); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return hi(w); }

// Value of lane (lane ^ O) on VALU-speed cross-lane paths instead of the LDS crossbar:
// O = 32 / 16 by the gfx950 permlane swaps, O = 8 / 4 by DPP row rotations, O = 2 / 1 by
// DPP quad permutes.  (Lane mappings verified on gfx950: permlane32_swap(v, v) yields
// {lanes 0-31 of v in both halves, lanes 32-63 in both halves}; permlane16_swap(v, v)
// {even rows, odd rows}; row_ror:n moves lane i to i + n within a row of 16.)
template <int O>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    const uint32_t lane = threadIdx.x & 63u;
    if constexpr (O == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32u) ? r[0] : r[1];
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16u) ? r[0] : r[1];
    } else if constexpr (O == 8) {
        return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x128, 0xf, 0xf, false));  // row_ror:8
    } else if constexpr (O == 4) {
        const uint32_t up = uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x12C, 0xf, 0xf, false));  // lane + 4
        const uint32_t dn = uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x124, 0xf, 0xf, false));  // lane - 4
        return (lane & 4u) ? dn : up;
    } else if constexpr (O == 2) {
        return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x4E, 0xf, 0xf, false));  // quad_perm 2,3,0,1
    } else {
        static_assert(O == 1, "xor offset");
        return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0xB1, 0xf, 0xf, false));  // quad_perm 1,0,3,2
    }
}
template <int O>
__device__ __forceinline__ float xor_lane(float v) {
    return __uint_as_float(xor_lane<O>(__float_as_uint(v)));
}

// One level of a reduce-scatter over K live values: lanes with bit O set keep the upper half,
// the others the lower half, each adding the partner lane's copy (own + partner, as the
// butterfly does).
template <int K, int O>
__device__ __forceinline__ void rs_level(float* v, uint32_t lane) {
    const bool upper = (lane & uint32_t(O)) != 0;
#pragma unroll
    for (int i = 0; i < K / 2; ++i) {
        const float keep = upper ? v[i + K / 2] : v[i];
        const float send = upper ? v[i] : v[i + K / 2];
        v[i] = keep + xor_lane<O>(send);
    }
}

// Sums of K values over the wavefront (K a power of two, at most 64) with exactly the
// pairwise additions of K butterflies, but one exchange per value and level only while the
// values last: afterwards every lane holds the total of value lane >> (6 - log2 K).
template <int K>
__device__ __forceinline__ float wave_sum_scatter(float (&v)[K]) {
    static_assert(K >= 1 && K <= 64 && (K & (K - 1)) == 0, "power of two up to 64");
    const uint32_t lane = threadIdx.x & 63u;
    if constexpr (K >= 2) rs_level<K, 32>(v, lane);
    if constexpr (K >= 4) rs_level<K / 2, 16>(v, lane);
    if constexpr (K >= 8) rs_level<K / 4, 8>(v, lane);
    if constexpr (K >= 16) rs_level<K / 8, 4>(v, lane);
    if constexpr (K >= 32) rs_level<K / 16, 2>(v, lane);
    if constexpr (K >= 64) rs_level<K / 32, 1>(v, lane);
    float t = v[0];
    if constexpr (K < 2) t += xor_lane<32>(t);
    if constexpr (K < 4) t += xor_lane<16>(t);
    if constexpr (K < 8) t += xor_lane<8>(t);
    if constexpr (K < 16) t += xor_lane<4>(t);
    if constexpr (K < 32) t += xor_lane<2>(t);
    if constexpr (K < 64) t += xor_lane<1>(t);
    return t;
}
constexpr int log2_pow2(int k) { return k <= 1 ? 0 : 1 + log2_pow2(k / 2); }

// Butterfly reductions over the 64-lane wavefront (XOR offsets 32, 16, 8, 4, 2, 1): lane i
// adds lane i ^ o at each level, so every lane ends with the same bits.
__device__ __forceinline__ float wave_sum(float v) {
    v += xor_lane<32>(v);
    v += xor_lane<16>(v);
    v += xor_lane<8>(v);
    v += xor_lane<4>(v);
    v += xor_lane<2>(v);
    v += xor_lane<1>(v);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, xor_lane<32>(v));
    v = fmaxf(v, xor_lane<16>(v));
    v = fmaxf(v, xor_lane<8>(v));
    v = fmaxf(v, xor_lane<4>(v));
    v = fmaxf(v, xor_lane<2>(v));
    v = fmaxf(v, xor_lane<1>(v));
    return v;
}
// Reduction over aligned groups of 16 lanes (offsets 8, 4, 2, 1).
__device__ __forceinline__ float group16_sum(float v) {
    v += xor_lane<8>(v);
    v += xor_lane<4>(v);
    v += xor_lane<2>(v);
    v += xor_lane<1>(v);
    return v;
}

// v_dot2_f32_bf16: acc + a.lo * b.lo + a.hi * b.hi on two BF16 pairs, the two exact
// products folded into the FP32 accumulator in one step (truncated at 24 bits below the
// larger product's exponent window, the sum floored 31 bits below its leading bit, then
// rounded to nearest even -- the MFMA accumulation with a group of two).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc,
                                           false);
}

// a.b over 8 BF16 pairs packed in two uint4: four dot2 steps in element-pair order.  One
// instruction per two weights and no unpacking of either operand.
__device__ __forceinline__ float dot8(const uint4 w, const uint4 x, float acc) {
    acc = dot2bf(w.x, x.x, acc);
    acc = dot2bf(w.y, x.y, acc);
    acc = dot2bf(w.z, x.z, acc);
    acc = dot2bf(w.w, x.w, acc);
    return acc;
}

// .p12 decode of the 8 weights a lane owns inside a 128-weight block
// (Kernels.metal:23-44): sm = 8 sign/mantissa bytes, nib = 8 exponent codes.
__device__ __forceinline__ uint32_t p12_word(uint32_t s, uint32_t code, uint32_t minimum) {
    const uint32_t e = code == 15u ? 0u : minimum + code;
    return (s & 127u) | ((s & 128u) << 8) | (e << 7);
}
// p12_word for all eight weights at once, byte-parallel (about 3 VALU operations per weight
// instead of 8): the exponent bytes are code + minimum (at most 184: no carry between
// bytes), cleared where the code is 15 by a v_perm_b32 mask (with all-ones sources a
// selector byte yields 0x00 only for selector 12 = 15 ^ 3, and 0xFF for 0..11 and 13..15);
// then each BF16 is assembled from its low byte (exponent bit 0 | 7 mantissa bits) and its
// high byte (sign | exponent bits 7..1), pairs interleaved by v_perm_b32.
__device__ __forceinline__ uint4 p12_decode8(uint2 sm, uint32_t nib, uint32_t tag) {
    const uint32_t mrep = tag * 0x01010101u + 0x6b6b6b6bu;  // (tag + 107) in every byte
    const uint32_t ce = nib & 0x0f0f0f0fu;                  // codes of weights 0, 2, 4, 6
    const uint32_t co = (nib >> 4) & 0x0f0f0f0fu;           // codes of weights 1, 3, 5, 7
    const uint32_t ee = (ce + mrep) & __builtin_amdgcn_perm(~0u, ~0u, ce ^ 0x03030303u);
    const uint32_t eo = (co + mrep) & __builtin_amdgcn_perm(~0u, ~0u, co ^ 0x03030303u);
    // exponents in weight order: ea = weights 0..3, eb = weights 4..7 (selector bytes 0..3
    // take the second operand's bytes, 4..7 the first's)
    const uint32_t ea = __builtin_amdgcn_perm(eo, ee, 0x05010400u);
    const uint32_t eb = __builtin_amdgcn_perm(eo, ee, 0x07030602u);
    const uint32_t la = (sm.x & 0x7f7f7f7fu) | ((ea << 7) & 0x80808080u);
    const uint32_t ha = (sm.x & 0x80808080u) | ((ea >> 1) & 0x7f7f7f7fu);
    const uint32_t lb = (sm.y & 0x7f7f7f7fu) | ((eb << 7) & 0x80808080u);
    const uint32_t hb = (sm.y & 0x80808080u) | ((eb >> 1) & 0x7f7f7f7fu);
    uint4 r;
    r.x = __builtin_amdgcn_perm(ha, la, 0x05010400u);  // (low, high) bytes of weights 0, 1
    r.y = __builtin_amdgcn_perm(ha, la, 0x07030602u);  // weights 2, 3
    r.z = __builtin_amdgcn_perm(hb, lb, 0x05010400u);
    r.w = __builtin_amdgcn_perm(hb, lb, 0x07030602u);
    return r;
}

// Raw buffer views (gfx9 resource word 3 = 0x00020000): base + 32-bit byte offset held in one
// VGPR; a read at or past `bytes` returns zero instead of touching memory.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_view(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
// Same, marked volatile: the compiler issues it where it stands and may not sink it towards
// its first use (software-pipelined prefetches rely on that).
__device__ __forceinline__ uint4 buffer_prefetch16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, int(0x80000000u));
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 buffer_load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
// Device-coherent exchange between workgroups without whole-cache fences: stores with the
// sc1 policy write through this XCD's L2, loads with sc1 read the coherent copy (the cache
// policy of agent-scope relaxed atomics).  A writer waits for its stores (vmcnt 0) before it
// publishes them with an atomic; a reader issues its loads after observing the atomic.
constexpr int SC1 = 16;
__device__ __forceinline__ void buffer_store16_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 v) {
    const u32x4_t w = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(w, r, off, 0, SC1);
}
__device__ __forceinline__ void buffer_store8_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off, uint2 v) {
    const u32x2_t w = {v.x, v.y};
    __builtin_amdgcn_raw_buffer_store_b64(w, r, off, 0, SC1);
}
__device__ __forceinline__ uint4 buffer_load16_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, SC1);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 buffer_load8_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, SC1);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ void buffer_store4_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, SC1);
}
__device__ __forceinline__ uint32_t buffer_load4_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, SC1);
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

// Stores at or past the view's size are dropped (OOB_OFFSET is past every view).
constexpr uint32_t OOB_OFFSET = 0x80000000u;
__device__ __forceinline__ void buffer_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
}
__device__ __forceinline__ void buffer_store2(__amdgpu_buffer_rsrc_t r, uint32_t off, uint16_t v) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, 0);
}

// 2^x for the softmax weights of flash attention (x <= 0 or -inf), with a fixed operation
// sequence the CPU oracle reproduces bit for bit: x = k + f with k = rint(x) and f = x - k
// exact (|f| <= 1/2), the degree-6 Taylor polynomial of 2^f = e^(f ln 2) in Horner form with
// fused multiply-adds, then an exact 2^k scale.  Arguments below -64 give 0 (a weight under
// 2^-64 of the running maximum's moves nothing), so every result is a normal number.
// Accuracy: about 3 ulp.  Branch-free: the polynomial runs on every argument and the result
// is selected afterwards (a per-element branch costs exec-mask writes and keeps the
// scheduler from interleaving the polynomial with other work; same bits).  What -inf, NaN
// or arguments below -64 produce on the way is discarded by the select.
__device__ __forceinline__ float exp2_det(float x) {
#pragma clang fp contract(off)
    const float k = rintf(x);
    const float f = x - k;
    float p = 1.54035304e-04f;                 // ln2^6 / 6!
    p = __builtin_fmaf(p, f, 1.33335581e-03f); // ln2^5 / 5!
    p = __builtin_fmaf(p, f, 9.61812911e-03f); // ln2^4 / 4!
    p = __builtin_fmaf(p, f, 5.55041087e-02f); // ln2^3 / 3!
    p = __builtin_fmaf(p, f, 2.40226507e-01f); // ln2^2 / 2!
    p = __builtin_fmaf(p, f, 6.93147182e-01f); // ln2
    p = __builtin_fmaf(p, f, 1.0f);
    const float r = ldexpf(p, int(k));
    return x >= -64.0f ? r : 0.0f;  // -inf and NaN give 0
}

// exp(x) with a fixed operation sequence the CPU oracle reproduces bit for bit:
// Cody-Waite reduction x = k*ln2 + r (ln2 split in a 16-bit head, so k*LN2_HI is exact for
// |k| <= 128), degree-7 Taylor polynomial of e^r in Horner form, then an exact 2^k scale.
// Every product and sum is rounded separately (no contraction).  Accuracy: about 2 ulp.
// Branch-free like exp2_det: the result is selected at the end.
__device__ __forceinline__ float exp_det(float x) {
#pragma clang fp contract(off)
    const float k = rintf(x * 1.44269502162933349609375f);
    const float r = (x - k * 0.693145751953125f) - k * 1.428606765330187e-06f;
    float p = 1.98412698e-04f;                 // 1/7!
    p = p * r + 1.38888889e-03f;               // 1/6!
    p = p * r + 8.33333377e-03f;               // 1/5!
    p = p * r + 4.16666679e-02f;               // 1/4!
    p = p * r + 1.66666672e-01f;               // 1/3!
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const float e = ldexpf(p, int(k));
    // above the FP32 range: inf; at or below -80 (no subnormal results), -inf, NaN: 0
    return x > 88.72283935546875f ? __builtin_inff() : x > -80.0f ? e : 0.0f;
}

// Rotate-half RoPE of the pair (a = x[d], b = x[d+64]) (Kernels.metal:261-274):
// out[d] = roundbf(roundbf(a*c) + roundbf(-b*s)), out[d+64] = roundbf(roundbf(b*c) + roundbf(a*s)).
// `cs` packs the BF16 table entry: cos in the low half, sin in the high half.
__device__ __forceinline__ void rope_pair(float a, float b, uint32_t cs, float& ra, float& rb) {
    const float c = lo(cs), s = hi(cs);
    const float na = roundbf(roundbf(a * c) + roundbf(-b * s));
    const float nb = roundbf(roundbf(b * c) + roundbf(a * s));
    ra = na;
    rb = nb;
}

// roundbf of two values with one packed conversion (same bits as two `roundbf` calls).
__device__ __forceinline__ void round_bf16x2(float x, float y, float& rx, float& ry);

// rope_pair on two BF16 pairs at once (a = packed x[d], x'[d]; b = packed x[d+64], x'[d+64];
// cs0 / cs1 their cos | sin << 16) with the hardware round-to-nearest-even packed conversion
// (v_cvt_pk_bf16_f32), which rounds every non-NaN FP32 value (denormals included, FP32
// denormals are not flushed) exactly as `bits` does: the results equal two rope_pair calls.
typedef __bf16 dev_bf16x2 __attribute__((ext_vector_type(2)));
typedef float dev_floatx2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float x, float y) {
    const dev_floatx2 v = {x, y};
    const dev_bf16x2 h = __builtin_convertvector(v, dev_bf16x2);
    uint32_t w;
    __builtin_memcpy(&w, &h, 4);
    return w;
}
__device__ __forceinline__ void rope_pair_x2(uint32_t a, uint32_t b, uint32_t cs0, uint32_t cs1, uint32_t& na, uint32_t& nb) {
    const float a0 = lo(a), a1 = hi(a), b0 = lo(b), b1 = hi(b);
    const float c0 = lo(cs0), s0 = hi(cs0), c1 = lo(cs1), s1 = hi(cs1);
    const uint32_t ac = pack_bf16(a0 * c0, a1 * c1), bs = pack_bf16(-b0 * s0, -b1 * s1);
    const uint32_t bc = pack_bf16(b0 * c0, b1 * c1), as = pack_bf16(a0 * s0, a1 * s1);
    na = pack_bf16(lo(ac) + lo(bs), hi(ac) + hi(bs));
    nb = pack_bf16(lo(bc) + lo(as), hi(bc) + hi(as));
}

__device__ __forceinline__ void round_bf16x2(float x, float y, float& rx, float& ry) {
    const uint32_t w = pack_bf16(x, y);
    rx = lo(w);
    ry = hi(w);
}

// Same on FP32 operands (BF16-valued), results as FP32: (a0, b0) with cs0 and (a1, b1) with cs1.
__device__ __forceinline__ void rope_pair_x2f(float& a0, float& b0, uint32_t cs0, float& a1, float& b1, uint32_t cs1) {
    const float c0 = lo(cs0), s0 = hi(cs0), c1 = lo(cs1), s1 = hi(cs1);
    const uint32_t ac = pack_bf16(a0 * c0, a1 * c1), bs = pack_bf16(-b0 * s0, -b1 * s1);
    const uint32_t bc = pack_bf16(b0 * c0, b1 * c1), as = pack_bf16(a0 * s0, a1 * s1);
    const uint32_t na = pack_bf16(lo(ac) + lo(bs), hi(ac) + hi(bs));
    const uint32_t nb = pack_bf16(lo(bc) + lo(as), hi(bc) + hi(as));
    a0 = lo(na); a1 = hi(na);
    b0 = lo(nb); b1 = hi(nb);
}

// q/k RMSNorm over 128 with +1 offset (Kernels.metal:236-246) for the 8 dims a lane of a
// 16-lane group owns: d = sub*4+j and d+64 (j = 0..3).  Squares are summed in that order,
// then over the 16 lanes by an XOR butterfly.
__device__ __forceinline__ void head_norm8(const float4 lo, const float4 hi, const uint2 glo, const uint2 ghi,
                                           float z[8]) {
    float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += v[j] * v[j];
    ss = group16_sum(ss);
    const float r = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
    const uint32_t g[4] = {glo.x, glo.y, ghi.x, ghi.y};
    // z = roundbf(roundbf(v r) roundbf(w + 1)), two elements per packed RNE conversion
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        float g0, g1, t0, t1;
        round_bf16x2(lo_bf(g[j >> 1]) + 1.0f, hi_bf(g[j >> 1]) + 1.0f, g0, g1);
        round_bf16x2(v[j] * r, v[j + 1] * r, t0, t1);
        round_bf16x2(t0 * g0, t1 * g1, z[j], z[j + 1]);
    }
}

}  // namespace dev
}  // namespace plamo
