// Prefill kernels for gfx950: MFMA BF16 GEMM (plain or .p12 weights) with fused epilogues,
// row RMSNorm / residual kernels and the K/V cache writer.
//
//   gemm_dma_kernel Y[t][m] = sum_k X[t][k] W[m][k] for plain BF16 weights: 256x128 or 128x128
//                   tiles, BK 64, operands loaded straight into three swizzled LDS stages,
//                   v_mfma_f32_32x32x16_bf16, XCD-grouped tiles.
//   gemm_kernel     the same product for .p12 weights, expanded in registers on the way to a
//                   double-buffered LDS tile.  Both replace `matrix` (Kernels.metal:149-200)
//                   for the projections and `swiglu` (Kernels.metal:202-210) as an epilogue.
//   rows_norm       `norm` (Kernels.metal:46-90) for T rows: embedding gather + norm, or
//                   post-norm + residual + next norm.
//   qk_prep         `qkv` (Kernels.metal:223-259) for a chunk: q/k RMSNorm, RoPE, K/V to
//                   cache slot pos % capacity, normalised rotated queries as BF16.
//   flash_prefill   prefill attention (Runtime.swift:389-444) as MFMA flash attention.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "device.h"
#include "kernels.h"
#include "prefill.h"

namespace plamo {
using namespace dev;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

constexpr int BK = 64, LDS_STRIDE = BK + 8;  // +16 B per row against bank conflicts

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// Weight row feeding LDS row r of a B tile.  SwiGLU tiles interleave 32 gate and 32 up rows
// (g0-31, u0-31, g32-63, u32-63, ...) so that each wave's column tiles pair gate with up.
template <int EPI>
__device__ __forceinline__ int b_row(int n0, int r) {
    if constexpr (EPI == GEMM_SWIGLU) return ((r >> 5) & 1 ? INTER : 0) + n0 + (r >> 6) * 32 + (r & 31);
    else return n0 + r;
}

// One K step of operands in registers: thread tid loads 16 bytes of rows tid/8 + 32*i.
template <int BT, int BW, int NT>
struct GemmStage {
    static constexpr int RP = NT / 8;  // rows covered by one pass of the workgroup
    uint4 a[BT / RP], b[BW / RP];
};

// Operand views of one GEMM: rows past `tokens` (activations) or `m` (plain weights) read as
// zero.  .p12 payload offsets come from the validated block table.
struct GemmViews {
    __amdgpu_buffer_rsrc_t x, w, table;
};

__device__ __forceinline__ GemmViews gemm_views(const GemmParams& p, bool packed) {
    GemmViews v;
    v.x = buffer_view(p.x, uint32_t(p.tokens) * uint32_t(p.k) * 2u);
    v.w = buffer_view(p.w, packed ? 0x7fffffffu : uint32_t(p.m) * uint32_t(p.k) * 2u);
    v.table = buffer_view(p.table, packed ? uint32_t(p.m) * uint32_t(p.k / 128) * 4u : 0u);
    return v;
}

// Loads K step k0 of both operands.  A step past the end (live == false) is still issued, with
// every offset outside its view: it reads zeros without touching memory, and the loads stay
// unconditional, so the wait before each LDS store counts only the loads of the step it stores.
template <bool PACKED, int EPI, int BT, int BW, int NT>
__device__ __forceinline__ void gemm_load(const GemmParams& p, const GemmViews& v, int t0, int n0, int k0, bool live,
                                          GemmStage<BT, BW, NT>& g) {
    constexpr int RP = GemmStage<BT, BW, NT>::RP;
    const int tid = threadIdx.x, c8 = tid & 7;
    const uint32_t K = uint32_t(p.k);
    const uint32_t kk = uint32_t(k0 + c8 * 8);
    const uint32_t kill = live ? 0u : OOB_OFFSET;
#pragma unroll
    for (int i = 0; i < BT / RP; ++i) {
        const uint32_t t = uint32_t(t0 + (tid >> 3) + RP * i);
        g.a[i] = buffer_prefetch16(v.x, ((t * K + kk) * 2u) | kill);
    }
#pragma unroll
    for (int i = 0; i < BW / RP; ++i) {
        const uint32_t row = uint32_t(b_row<EPI>(n0, (tid >> 3) + RP * i));
        if constexpr (!PACKED) {
            g.b[i] = buffer_prefetch16(v.w, ((row * K + kk) * 2u) | kill);
        } else {
            const uint32_t entry = buffer_load4(v.table, ((row * (K / 128) + kk / 128) * 4u) | kill);
            const uint32_t blk = (entry & ~63u) | kill, tag = entry & 63u;
            const uint32_t sub = (kk % 128) / 8;
            if (tag == 0) g.b[i] = buffer_load16(v.w, blk + sub * 16);
            else g.b[i] = p12_decode8(buffer_load8(v.w, blk + sub * 8), buffer_load4(v.w, blk + 128 + sub * 4), tag);
        }
    }
}

template <int BT, int BW, int NT>
__device__ __forceinline__ void gemm_store(const GemmStage<BT, BW, NT>& g, uint16_t* As, uint16_t* Bs) {
    constexpr int RP = GemmStage<BT, BW, NT>::RP;
    const int tid = threadIdx.x, c8 = tid & 7;
#pragma unroll
    for (int i = 0; i < BT / RP; ++i)
        *reinterpret_cast<uint4*>(&As[((tid >> 3) + RP * i) * LDS_STRIDE + c8 * 8]) = g.a[i];
#pragma unroll
    for (int i = 0; i < BW / RP; ++i)
        *reinterpret_cast<uint4*>(&Bs[((tid >> 3) + RP * i) * LDS_STRIDE + c8 * 8]) = g.b[i];
}

// Writes a wave's TT x TW accumulator tiles (tokens from tw0, LDS weight-row tiles of wave
// column ww) with the chosen epilogue.
template <int EPI, int TT, int TW>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p, const floatx16 (&acc)[TT][TW], int tw0, int n0, int ww,
                                              int lane) {
    // C layout of a 32x32 tile: column j = lane%32, row i = (r/4)*8 + (lane/32)*4 + r%4.
    // Stores go through views bounded by the output size, so rows past `tokens` are dropped
    // without branches (columns past m get an offset outside the view).
    const int jc = lane & 31;
    const uint32_t M = uint32_t(p.m);
    const __amdgpu_buffer_rsrc_t yv =
        EPI == GEMM_SWIGLU ? buffer_view(p.y16, uint32_t(p.tokens) * INTER * 2u)
                           : (EPI == GEMM_BF16 ? buffer_view(p.y16, uint32_t(p.tokens) * M * 2u)
                                               : buffer_view(p.y, uint32_t(p.tokens) * M * 4u));
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t t = uint32_t(tw0 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3));
            if constexpr (EPI == GEMM_SWIGLU) {
#pragma unroll
                for (int j = 0; j < TW; j += 2) {  // LDS rows of tile j are gate rows, of j + 1 the matching up rows
                    const uint32_t m = uint32_t(n0 + ((ww * TW + j) >> 1) * 32 + jc);
                    // g / (1 + exp(-g)) with IEEE division (Kernels.metal:202-210), the exp of
                    // the decode epilogue (`exp_det`): decode and prefill round alike
                    const float gt = roundbf(acc[i][j][r]);
                    const float up = roundbf(acc[i][j + 1][r]);
                    const float silu = gt / (1.0f + exp_det(-gt));
                    buffer_store2(yv, (t * INTER + m) * 2u, uint16_t(bits(roundbf(silu) * up)));
                }
            } else {
#pragma unroll
                for (int j = 0; j < TW; ++j) {
                    const uint32_t m = uint32_t(n0 + ww * TW * 32 + j * 32 + jc);
                    const uint32_t e = m < M ? t * M + m : OOB_OFFSET / 4;
                    if constexpr (EPI == GEMM_F32) buffer_store4(yv, e * 4u, __float_as_uint(roundbf(acc[i][j][r])));
                    else if constexpr (EPI == GEMM_RAW) buffer_store4(yv, e * 4u, __float_as_uint(acc[i][j][r]));
                    else buffer_store2(yv, e * 2u, uint16_t(bits(acc[i][j][r])));
                }
            }
        }
}

// Y[t][m] = sum_k X[t][k] W[m][k] on BT x BW tiles (tokens x weight rows): four waves in a
// WT x (4 / WT) grid, each owning (BT / WT) x (BW * WT / 4) outputs as 32x32 MFMA tiles.  The
// next two K steps are in flight in registers while the current one is multiplied from LDS
// (double-buffered, one barrier per step).  Tiles are dealt to workgroups so that each XCD
// (workgroup id % 8) owns a contiguous run of tiles sharing weight columns, which keeps the
// weight tiles in that XCD's L2.  Larger tiles read fewer operand bytes per FLOP from L2.
template <bool PACKED, int EPI, int BT, int BW, int WT, int NT>
__global__ __launch_bounds__(NT) void gemm_kernel(const GemmParams p, int col_tiles, int row_tiles) {
    constexpr int WW = NT / 64 / WT, TT = BT / WT / 32, TW = BW / WW / 32;
    static_assert(EPI != GEMM_SWIGLU || TW % 2 == 0, "SwiGLU pairs gate and up tiles inside a wave");
    __shared__ __align__(16) uint16_t As[2][BT * LDS_STRIDE];
    __shared__ __align__(16) uint16_t Bs[2][BW * LDS_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
    const int wt = wave / WW, ww = wave % WW;
    const int tiles = col_tiles * row_tiles;
    const int per = (tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (tile >= tiles) return;
    const int ct = tile / row_tiles, rt = tile % row_tiles;
    const int t0 = rt * BT;
    const int n0 = ct * (EPI == GEMM_SWIGLU ? BW / 2 : BW);
    const int nk = p.k / BK;

    floatx16 acc[TT][TW];
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Two K steps of operands are in flight in registers while one is multiplied from LDS:
    // step kt+1 was requested one iteration ago and goes to the other LDS buffer during this
    // step, step kt+2 is requested now.  Inside a step the operands of 16-deep K slice ks+1 are
    // read from LDS while slice ks is multiplied.
    auto read_ops = [&](const uint16_t* A, const uint16_t* B, int ks, bf16x8 (&a)[TT], bf16x8 (&b)[TW]) {
        const int kc = ks * 16 + (lane >> 5) * 8;
#pragma unroll
        for (int i = 0; i < TT; ++i)
            a[i] = as_bf16x8(*reinterpret_cast<const uint4*>(&A[(wt * TT * 32 + i * 32 + (lane & 31)) * LDS_STRIDE + kc]));
#pragma unroll
        for (int j = 0; j < TW; ++j)
            b[j] = as_bf16x8(*reinterpret_cast<const uint4*>(&B[(ww * TW * 32 + j * 32 + (lane & 31)) * LDS_STRIDE + kc]));
    };
    const GemmViews views = gemm_views(p, PACKED);
    GemmStage<BT, BW, NT> g[2];
    gemm_load<PACKED, EPI>(p, views, t0, n0, 0, true, g[0]);
    gemm_load<PACKED, EPI>(p, views, t0, n0, BK, nk > 1, g[1]);
    gemm_store(g[0], As[0], Bs[0]);
    __syncthreads();
    auto step = [&](int kt, GemmStage<BT, BW, NT>& next, GemmStage<BT, BW, NT>& later) {
        const int buf = kt & 1;
        const uint16_t* A = As[buf];
        const uint16_t* B = Bs[buf];
        bf16x8 a[2][TT], b[2][TW];
        read_ops(A, B, 0, a[0], b[0]);
        gemm_load<PACKED, EPI>(p, views, t0, n0, (kt + 2) * BK, kt + 2 < nk, later);
        // the other buffer was last read before the previous barrier; past the last step the
        // stored stage is zeros that nobody reads, so the store needs no branch
        gemm_store(next, As[buf ^ 1], Bs[buf ^ 1]);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            if (ks + 1 < BK / 16) read_ops(A, B, ks + 1, a[(ks + 1) & 1], b[(ks + 1) & 1]);
#pragma unroll
            for (int i = 0; i < TT; ++i)
#pragma unroll
                for (int j = 0; j < TW; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks & 1][i], b[ks & 1][j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    };
    // both halves of the loop body are unconditional, so each stage keeps its registers
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        step(kt, g[1], g[0]);
        step(kt + 1, g[0], g[1]);
    }
    if (kt < nk) step(kt, g[1], g[0]);

    gemm_epilogue<EPI, TT, TW>(p, acc, t0 + wt * TT * 32, n0, ww, lane);
}

// s_waitcnt on the vector-memory counter only (gfx9 encoding: expcnt and lgkmcnt at maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}
// The same, and every LDS operation of the wave done (lgkmcnt 0).
template <int N>
__device__ __forceinline__ void wait_vmcnt_lds() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);
}

// Calls f(std::integral_constant<int, I>) for I = B .. E-1.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;
__device__ __forceinline__ void load_to_lds(__amdgpu_buffer_rsrc_t v, void* lds, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(v, (lds_ptr_t)lds, 16, off, 0, 0, 0);
}

// Plain-weight GEMM whose operand tiles go from memory straight into LDS (buffer loads with
// the LDS destination): no staging registers and no LDS store instructions.  NS LDS stages of
// KD K values each, NS - 1 stages in flight.  A stage holds BT activation rows then BW weight
// rows of KD * 2 bytes; the 16-byte chunk c of row R sits in slot c ^ ((R >> SH) & (CPR - 1))
// (SH = 1 for 128-byte rows, 2 for 64-byte rows), which spreads both the loads' row segments
// and the operand reads' 16-row columns over all banks.  Each wave loads Q 1 KB blocks per
// stage.  Waves synchronise with a bare s_barrier after waiting for their own stage loads and
// LDS reads, so the later stages stay in flight across the barrier.
template <int EPI, int BT, int BW, int WT, int NT, int KD, int NS>
__global__ __launch_bounds__(NT) void gemm_dma_kernel(const GemmParams p, int col_tiles, int row_tiles) {
    constexpr int NW = NT / 64, WW = NW / WT, TT = BT / WT / 32, TW = BW / WW / 32;
    constexpr int ROWB = KD * 2, CPR = ROWB / 16, RPI = 1024 / ROWB, SH = ROWB == 128 ? 1 : 2;
    constexpr int ROWS = BT + BW, STAGE = ROWS * ROWB, Q = ROWS / RPI / NW;
    static_assert(KD == 64 || KD == 32, "stage depth");
    static_assert(ROWS % (RPI * NW) == 0 && BT % 16 == 0, "stage blocks per wave");
    static_assert(EPI != GEMM_SWIGLU || TW % 2 == 0, "SwiGLU pairs gate and up tiles inside a wave");
    static_assert(NS >= 3, "at least two stages in flight");
    // one array per stage: the compiler then tells the stages apart and waits for the loads
    // into a stage only before reading that stage (one shared array would make every read
    // wait for every load in flight)
    __shared__ __align__(1024) uint8_t S0[STAGE];
    __shared__ __align__(1024) uint8_t S1[STAGE];
    __shared__ __align__(1024) uint8_t S2[STAGE];
    __shared__ __align__(1024) uint8_t S3[NS > 3 ? STAGE : 16];
    __shared__ __align__(1024) uint8_t S4[NS > 4 ? STAGE : 16];
    __shared__ __align__(1024) uint8_t S5[NS > 5 ? STAGE : 16];
    static_assert(NS <= 6, "at most six stages");
    auto stage_of = [&](auto idx) -> uint8_t* {
        constexpr int i = decltype(idx)::value;
        if constexpr (i == 0) return S0;
        else if constexpr (i == 1) return S1;
        else if constexpr (i == 2) return S2;
        else if constexpr (i == 3) return S3;
        else if constexpr (i == 4) return S4;
        else return S5;
    };
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
    const int wt = wave / WW, ww = wave % WW;
    const int tiles = col_tiles * row_tiles;
    const int per = (tiles + 7) / 8;
    const int tile = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (tile >= tiles) return;
    const int ct = tile / row_tiles, rt = tile % row_tiles;
    const int t0 = rt * BT;
    const int n0 = ct * (EPI == GEMM_SWIGLU ? BW / 2 : BW);
    const int nk = p.k / KD;
    const uint32_t K = uint32_t(p.k);
    const GemmViews views = gemm_views(p, false);

    // this lane's source offset (K step 0) for each of the wave's Q blocks
    uint32_t goff[Q];
    bool from_x[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int R = (wave * Q + q) * RPI + lane / CPR;
        const uint32_t c = uint32_t((lane % CPR) ^ ((R >> SH) & (CPR - 1)));
        from_x[q] = (wave * Q + q) * RPI < BT;
        const uint32_t row = from_x[q] ? uint32_t(t0 + R) : uint32_t(b_row<EPI>(n0, R - BT));
        goff[q] = (row * K + c * 8) * 2u;
    }
    auto issue = [&](uint8_t* stage, int kt) {
        const uint32_t kill = kt < nk ? 0u : OOB_OFFSET;
        const uint32_t kb = uint32_t(kt) * KD * 2u;
#pragma unroll
        for (int q = 0; q < Q; ++q)
            load_to_lds(from_x[q] ? views.x : views.w, stage + (wave * Q + q) * 1024, (goff[q] + kb) | kill);
    };
    floatx16 acc[TT][TW];
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    auto compute = [&](const uint8_t* stage) {
#pragma unroll
        for (int ks = 0; ks < KD / 16; ++ks) {
            const int c = ks * 2 + (lane >> 5);
            bf16x8 a[TT], b[TW];
#pragma unroll
            for (int i = 0; i < TT; ++i) {
                const int R = wt * TT * 32 + i * 32 + (lane & 31);
                a[i] = as_bf16x8(*reinterpret_cast<const uint4*>(stage + R * ROWB + ((c ^ ((R >> SH) & (CPR - 1))) << 4)));
            }
#pragma unroll
            for (int j = 0; j < TW; ++j) {
                const int R = BT + ww * TW * 32 + j * 32 + (lane & 31);
                b[j] = as_bf16x8(*reinterpret_cast<const uint4*>(stage + R * ROWB + ((c ^ ((R >> SH) & (CPR - 1))) << 4)));
            }
#pragma unroll
            for (int i = 0; i < TT; ++i)
#pragma unroll
                for (int j = 0; j < TW; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };
    // step kt: this wave's loads of stage kt are done once at most the loads of the NS - 2
    // later stages are outstanding, and its reads of stage kt - 1 once no LDS operation is
    // (a read issued before the barrier may still be queued in the LDS, and a load into the
    // freed buffer can return before it runs: from L2, or at once when out of range); after
    // the barrier every wave's are, and the buffer of stage kt - 1 is free for stage kt + NS - 1
    auto step = [&](const uint8_t* cur, uint8_t* freed, int kt) {
        __asm__ volatile("" ::: "memory");  // no LDS access of the previous step moves below
        wait_vmcnt_lds<(NS - 2) * Q>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        issue(freed, kt + NS - 1);
        compute(cur);
    };
    static_for<0, NS - 1>([&](auto b) { issue(stage_of(b), decltype(b)::value); });
    int kt = 0;
    for (; kt + NS <= nk; kt += NS)
        static_for<0, NS>([&](auto b) {
            constexpr int i = decltype(b)::value;
            step(stage_of(b), stage_of(std::integral_constant<int, (i + NS - 1) % NS>{}), kt + i);
        });
    static_for<0, NS - 1>([&](auto b) {
        constexpr int i = decltype(b)::value;
        if (kt + i < nk) step(stage_of(b), stage_of(std::integral_constant<int, (i + NS - 1) % NS>{}), kt + i);
    });
    // The last steps issued loads for the stages past the end (out of range: they write zeros
    // into LDS, and keep the per-step load counts uniform).  No wave ends with a load into LDS
    // in flight: the workgroup's LDS may go to the next workgroup on this CU.
    wait_vmcnt<0>();
    gemm_epilogue<EPI, TT, TW>(p, acc, t0 + wt * TT * 32, n0, ww, lane);
}

// ------------------------------------------------------------------------------ norms
// Post-norm + residual + next norm of prefill rows (Kernels.metal:46-90).  One wave per
// token, four tokens per workgroup: lane l owns elements 512c + 8l .. +8 (c < 3), read and
// written as 16-byte rows; both sums of squares are wave reductions.
__global__ __launch_bounds__(256) void rows_norm_kernel(const RowsNormParams p) {
    constexpr int C = HIDDEN / 512;
    const int lane = threadIdx.x & 63;
    const int t = int(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    if (t >= p.tokens) return;
    auto unpack = [](const uint4 w, float (&f)[8]) {
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) { f[2 * k] = lo(u[k]); f[2 * k + 1] = hi(u[k]); }
    };
    float xv[C][8];
    const size_t row = size_t(t) * HIDDEN;
    // the next norm's gains are requested with the row's inputs (off the reductions' path)
    uint4 gnw[C];
#pragma unroll
    for (int c = 0; c < C; ++c)
        gnw[c] = p.xn ? *reinterpret_cast<const uint4*>(p.g_next + 512 * c + 8 * lane) : make_uint4(0, 0, 0, 0);
    if (p.tokens_in) {
        int tok = p.tokens_in[t];
        tok = (tok < 0 || tok >= VOCAB) ? 0 : tok;
#pragma unroll
        for (int c = 0; c < C; ++c)
            unpack(*reinterpret_cast<const uint4*>(p.embed + size_t(tok) * HIDDEN + 512 * c + 8 * lane), xv[c]);
    } else {
        float pv[C][8], rv[C][8], gp[C][8];
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int i = 512 * c + 8 * lane;
            unpack(*reinterpret_cast<const uint4*>(p.in + row + i), pv[c]);
            unpack(*reinterpret_cast<const uint4*>(p.x + row + i), rv[c]);
            unpack(*reinterpret_cast<const uint4*>(p.g_post + i), gp[c]);
        }
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 8; ++k) ss += pv[c][k] * pv[c][k];
        const float r = 1.0f / sqrtf(wave_sum(ss) / float(HIDDEN) + 1e-6f);
        // z = roundbf(roundbf(p r) roundbf(w + offset)), x = roundbf(x + z): the roundings two
        // at a time with the packed RNE conversion (same bits as `roundbf`)
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int k = 0; k < 8; k += 2) {
                float t0, t1, g0, g1, z0, z1;
                round_bf16x2(pv[c][k] * r, pv[c][k + 1] * r, t0, t1);
                round_bf16x2(gp[c][k] + p.post_offset, gp[c][k + 1] + p.post_offset, g0, g1);
                round_bf16x2(t0 * g0, t1 * g1, z0, z1);
                round_bf16x2(rv[c][k] + z0, rv[c][k + 1] + z1, xv[c][k], xv[c][k + 1]);
            }
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int k = 0; k < 8; ++k) ss += xv[c][k] * xv[c][k];
    const float r = 1.0f / sqrtf(wave_sum(ss) / float(HIDDEN) + 1e-6f);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int i = 512 * c + 8 * lane;
        uint32_t xw[4], nw[4];
        float gn[8];
        unpack(gnw[c], gn);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            xw[k] = pack_bf16(xv[c][2 * k], xv[c][2 * k + 1]);  // BF16 values: exact
            if (p.xn) {
                float t0, t1, g0, g1;
                round_bf16x2(xv[c][2 * k] * r, xv[c][2 * k + 1] * r, t0, t1);
                round_bf16x2(gn[2 * k] + 1.0f, gn[2 * k + 1] + 1.0f, g0, g1);
                nw[k] = pack_bf16(t0 * g0, t1 * g1);
            }
        }
        *reinterpret_cast<uint4*>(p.x + row + i) = make_uint4(xw[0], xw[1], xw[2], xw[3]);
        if (p.xn) *reinterpret_cast<uint4*>(p.xn + row + i) = make_uint4(nw[0], nw[1], nw[2], nw[3]);
    }
}

// ---------------------------------------------------------------------------- qk prep
// One workgroup per token (the `qkv` kernel, Kernels.metal:223-259, for a prefill chunk):
// thread (h, s) = (tid/16, tid%16) normalises and rotates RoPE pairs (d, d+64) for
// d = 4s..4s+3 of query head h -- global layers at the absolute position, local layers at
// pos - base with base = max(0, chunk_start - 2047) of the token's 16-token chunk
// (Runtime.swift:389, Kernels.metal:251,283-284).  Threads 0..15 do the same for the key
// (rotated only on global layers; local keys are cached unrotated) and write it to slot
// pos % capacity; threads 64..191 copy the value row.
__global__ __launch_bounds__(256) void qk_prep_kernel(const QkPrepParams p) {
    const int t = blockIdx.x, tid = threadIdx.x;
    const int hq = tid >> 4, sq = tid & 15;
    const uint32_t pos = p.p0 + uint32_t(t);
    const uint32_t chunk = p.p0 + (uint32_t(t) / CHUNK) * CHUNK;
    const uint32_t base = chunk > uint32_t(WINDOW - 1) ? chunk - uint32_t(WINDOW - 1) : 0u;
    const uint32_t qcoord = p.full ? pos : pos - base;
    const uint16_t* x = p.qkv + size_t(t) * QKV;
    // four BF16 values as FP32
    auto load4 = [](const uint16_t* s) {
        const uint2 w = *reinterpret_cast<const uint2*>(s);
        return make_float4(lo(w.x), hi(w.x), lo(w.y), hi(w.y));
    };
    // the key part's inputs (threads 0..15) are requested with the queries'
    const bool kthread = tid < 16;
    const bool krot = !p.full && p.keys_rot && pos < p.rot_rows;
    float4 klo = make_float4(0.f, 0.f, 0.f, 0.f), khi = klo;
    uint2 kgl = make_uint2(0, 0), kgh = kgl;
    uint4 kr4 = make_uint4(0, 0, 0, 0);
    if (kthread) {
        klo = load4(x + ATTN + tid * 4);
        khi = load4(x + ATTN + 64 + tid * 4);
        kgl = *reinterpret_cast<const uint2*>(p.k_norm + tid * 4);
        kgh = *reinterpret_cast<const uint2*>(p.k_norm + 64 + tid * 4);
        if (p.full || krot)
            kr4 = *reinterpret_cast<const uint4*>((p.full ? p.global_rope : p.local_rope) + size_t(pos) * 64 + tid * 4);
    }
    {
        const float4 qlo = load4(x + hq * HEAD_DIM + sq * 4);
        const float4 qhi = load4(x + hq * HEAD_DIM + 64 + sq * 4);
        const uint2 glo = *reinterpret_cast<const uint2*>(p.q_norm + sq * 4);
        const uint2 ghi = *reinterpret_cast<const uint2*>(p.q_norm + 64 + sq * 4);
        const uint4 qr = *reinterpret_cast<const uint4*>((p.full ? p.global_rope : p.local_rope) + size_t(qcoord) * 64 + sq * 4);
        float z[8];
        head_norm8(qlo, qhi, glo, ghi, z);
        const uint32_t c4[4] = {qr.x, qr.y, qr.z, qr.w};
        // rope_pair_x2f: two RoPE pairs per packed RNE conversion (same bits as rope_pair)
#pragma unroll
        for (int j = 0; j < 4; j += 2) rope_pair_x2f(z[j], z[4 + j], c4[j], z[j + 1], z[4 + j + 1], c4[j + 1]);
        uint16_t* qo = p.q16 + (size_t(t) * HEADS + hq) * HEAD_DIM;
        *reinterpret_cast<uint2*>(qo + sq * 4) = make_uint2(pack_bf16(z[0], z[1]), pack_bf16(z[2], z[3]));
        *reinterpret_cast<uint2*>(qo + 64 + sq * 4) = make_uint2(pack_bf16(z[4], z[5]), pack_bf16(z[6], z[7]));
    }
    const size_t slot = size_t(pos % p.capacity) * HEAD_DIM;
    if (kthread) {
        float z[8];
        head_norm8(klo, khi, kgl, kgh, z);
        const uint32_t c4[4] = {kr4.x, kr4.y, kr4.z, kr4.w};
        if (p.full) {
#pragma unroll
            for (int j = 0; j < 4; j += 2) rope_pair_x2f(z[j], z[4 + j], c4[j], z[j + 1], z[4 + j + 1], c4[j + 1]);
        } else if (krot) {
            // the copy rotated at the key's own position (decode inside the first window)
            float zr[8] = {z[0], z[1], z[2], z[3], z[4], z[5], z[6], z[7]};
#pragma unroll
            for (int j = 0; j < 4; j += 2) rope_pair_x2f(zr[j], zr[4 + j], c4[j], zr[j + 1], zr[4 + j + 1], c4[j + 1]);
            uint16_t* kr = p.keys_rot + size_t(pos) * HEAD_DIM;
            *reinterpret_cast<uint2*>(kr + tid * 4) = make_uint2(pack_bf16(zr[0], zr[1]), pack_bf16(zr[2], zr[3]));
            *reinterpret_cast<uint2*>(kr + 64 + tid * 4) = make_uint2(pack_bf16(zr[4], zr[5]), pack_bf16(zr[6], zr[7]));
        }
        auto word = [](float a, float b) { return (bits(a) & 0xffffu) | (bits(b) << 16); };
        *reinterpret_cast<uint2*>(p.keys + slot + tid * 4) = make_uint2(word(z[0], z[1]), word(z[2], z[3]));
        *reinterpret_cast<uint2*>(p.keys + slot + 64 + tid * 4) = make_uint2(word(z[4], z[5]), word(z[6], z[7]));
    }
    if (tid >= 64 && tid < 64 + HEAD_DIM) {
        const int d = tid - 64;
        p.values[slot + d] = x[ATTN + HEAD_DIM + d];
    }
}

// --------------------------------------------------------------------- flash attention
// Prefill attention (Runtime.swift:389-444: scores, scale 1/sqrt(128) before the max,
// softmax, roundbf(sum p v)) as MFMA flash attention over the cached keys.
//
// A workgroup takes 8 tokens x 16 heads = 128 query columns; wave w owns tokens 2w, 2w+1:
// lane column c = lane%32 is token 2w + c/16, head c%16 (MQA: every head reads the same
// keys, so one K/V tile serves all 128 columns).  With keys as rows,
//   S^T = K Q^T   and   O^T = V^T P^T,
// a query's 64 scores of a tile sit in one lane column (two halves of 32 lanes), so the
// online-softmax statistics need a single cross-half exchange, and the S^T accumulator is
// already the B operand layout of the P.V product.  P is split as hi + lo BF16 so the
// P.V product keeps ~16 significant bits of the FP32 probabilities.  The softmax weights come
// from `exp2_det` and nothing is contracted, so every output is a fixed function of the
// inputs that a CPU restatement reproduces bit for bit.
//
// Two kernels share that arithmetic: the staged one (K/V tiles through registers into K rows
// and V^T in LDS; the only one that can rotate keys while staging) and the direct one (K/V
// tiles loaded straight into LDS, V^T operands by transposing LDS reads), used when no block
// of a call rotates its keys: global layers, and local layers inside the rotated-key cache.
//
// Keys of local layers are rotated while staged, with coordinate key_pos - base of the
// workgroup's 16-token chunk (base = max(0, chunk_start - 2047)); where base is 0 and every
// key of the block lies in the rotated-key cache, that coordinate is the key's position and
// the cached rotations (written by qk_prep_kernel) are staged as they are.
constexpr int FT = 8;                 // tokens per query block (workgroup)
constexpr int FK = 64;                // keys per tile
static_assert(FT == 8 && FK == 64, "flash_block_tiles (prefill.h) assumes these sizes");
// Direct path row strides (BF16 elements): key rows of 272 bytes (17 16-byte chunks, the
// last one padding: consecutive rows start 4 banks apart), value rows of 320 bytes (20
// chunks: 16 banks apart)
constexpr int DK_ROW = 136, DV_ROW = 160;
constexpr int DK_CHUNKS = DK_ROW / 8, DV_CHUNKS = DV_ROW / 8;
constexpr int KST = HEAD_DIM + 8;     // K tile row stride (BF16), 16-byte aligned rows
constexpr int VST = FK + 4;           // V^T tile row stride (BF16): 34 dwords, so 16 lanes reading
                                      // 8 bytes from 16 consecutive rows hit 32 distinct banks
constexpr float SCALE_LOG2E = 0.08838834764831845f * 1.4426950408889634f;

struct KvStage {
    uint4 ka[2], kb[2], rr[4], v[4];
};
// Where a tile's keys come from: unrotated (rotate while staged), rotated (global layers, or
// the rotated-key cache of a local layer).
struct KvSource {
    const uint16_t* keys;
    bool rotate;
};

// Global loads of one tile: thread -> key tid/4 with RoPE pairs (d, d+64), d = 16*(tid%4)
// .. +16; and values of keys 4*(tid%16) .. +4 at dims 8*(tid/16) .. +8.  Keys past khi (the
// last tile's tail) load key khi instead: their scores are masked and their weights are
// exactly 0, so any finite row serves, every load stays on a written key, and no register
// has to be cleared or load predicated.
__device__ __forceinline__ void flash_load(const FlashParams& p, const KvSource& src, uint32_t k0, uint32_t khi,
                                           uint32_t base, KvStage& s) {
    const int tid = threadIdx.x;
    const int part = tid & 3;
    // ring slots: one modulo per tile, then at most one wrap per key when the ring holds a
    // whole tile (offsets are below 64); smaller rings wrap by repeated subtraction
    const uint32_t slot0 = k0 % p.capacity;
    const bool big_ring = p.capacity >= uint32_t(FK);
    auto ring = [&](uint32_t off) {
        uint32_t slot = slot0 + off;
        if (big_ring) return slot >= p.capacity ? slot - p.capacity : slot;
        while (slot >= p.capacity) slot -= p.capacity;
        return slot;
    };
    const uint32_t kp = min(k0 + uint32_t(tid >> 2), khi);
    // the rotated-key cache is indexed by position (kp < rot_rows), the ring by slot
    const uint16_t* row = src.keys + size_t(src.rotate || p.full ? ring(kp - k0) : kp) * HEAD_DIM;
    s.ka[0] = *reinterpret_cast<const uint4*>(row + part * 16);
    s.ka[1] = *reinterpret_cast<const uint4*>(row + part * 16 + 8);
    s.kb[0] = *reinterpret_cast<const uint4*>(row + 64 + part * 16);
    s.kb[1] = *reinterpret_cast<const uint4*>(row + 64 + part * 16 + 8);
    if (src.rotate) {
        const uint4* rr = reinterpret_cast<const uint4*>(p.local_rope + size_t(kp - base) * 64 + part * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) s.rr[i] = rr[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t kv = min(k0 + uint32_t(4 * (tid & 15) + i), khi);
        s.v[i] = *reinterpret_cast<const uint4*>(p.values + size_t(ring(kv - k0)) * HEAD_DIM + 8 * (tid >> 4));
    }
}

__device__ __forceinline__ uint32_t u16_of(const uint4& v, int k) {
    const uint32_t w = k < 2 ? v.x : k < 4 ? v.y : k < 6 ? v.z : v.w;
    return (k & 1) ? (w >> 16) : (w & 0xffffu);
}

__device__ __forceinline__ void flash_store(const KvSource& src, const KvStage& s, uint16_t* Ks, uint16_t* Vt) {
    const int tid = threadIdx.x;
    const int part = tid & 3, key = tid >> 2;
    uint16_t* krow = Ks + key * KST;
    if (!src.rotate) {
        *reinterpret_cast<uint4*>(krow + part * 16) = s.ka[0];
        *reinterpret_cast<uint4*>(krow + part * 16 + 8) = s.ka[1];
        *reinterpret_cast<uint4*>(krow + 64 + part * 16) = s.kb[0];
        *reinterpret_cast<uint4*>(krow + 64 + part * 16 + 8) = s.kb[1];
    } else {
        const uint32_t aw[8] = {s.ka[0].x, s.ka[0].y, s.ka[0].z, s.ka[0].w, s.ka[1].x, s.ka[1].y, s.ka[1].z, s.ka[1].w};
        const uint32_t bw[8] = {s.kb[0].x, s.kb[0].y, s.kb[0].z, s.kb[0].w, s.kb[1].x, s.kb[1].y, s.kb[1].z, s.kb[1].w};
        const uint32_t rw[16] = {s.rr[0].x, s.rr[0].y, s.rr[0].z, s.rr[0].w, s.rr[1].x, s.rr[1].y, s.rr[1].z, s.rr[1].w,
                                 s.rr[2].x, s.rr[2].y, s.rr[2].z, s.rr[2].w, s.rr[3].x, s.rr[3].y, s.rr[3].z, s.rr[3].w};
        uint32_t ao[8], bo[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) rope_pair_x2(aw[i], bw[i], rw[2 * i], rw[2 * i + 1], ao[i], bo[i]);
        *reinterpret_cast<uint4*>(krow + part * 16) = make_uint4(ao[0], ao[1], ao[2], ao[3]);
        *reinterpret_cast<uint4*>(krow + part * 16 + 8) = make_uint4(ao[4], ao[5], ao[6], ao[7]);
        *reinterpret_cast<uint4*>(krow + 64 + part * 16) = make_uint4(bo[0], bo[1], bo[2], bo[3]);
        *reinterpret_cast<uint4*>(krow + 64 + part * 16 + 8) = make_uint4(bo[4], bo[5], bo[6], bo[7]);
    }
    // V^T: 4 keys of one dim per 8-byte store
    const int kg = 4 * (tid & 15), d0 = 8 * (tid >> 4);  // consecutive lanes: consecutive key groups
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t w0 = u16_of(s.v[0], j) | (u16_of(s.v[1], j) << 16);
        const uint32_t w1 = u16_of(s.v[2], j) | (u16_of(s.v[3], j) << 16);
        *reinterpret_cast<uint2*>(Vt + (d0 + j) * VST + kg) = make_uint2(w0, w1);
    }
}

// Two FP32 values as BF16 pairs hi + lo (RNE, v_cvt_pk_bf16_f32): hi + lo carries ~16
// significant bits of each value.
__device__ __forceinline__ void split_bf16(float a, float b, uint32_t& hw, uint32_t& lw) {
    const floatx2 v = {a, b};
    const bf16x2 h = __builtin_convertvector(v, bf16x2);
    __builtin_memcpy(&hw, &h, 4);
    const floatx2 back = {__uint_as_float(hw << 16), __uint_as_float(hw & 0xffff0000u)};
    const bf16x2 l = __builtin_convertvector(v - back, bf16x2);
    __builtin_memcpy(&lw, &l, 4);
}

// Part `part` of query block qb.  QSA: global layers with a selection bitmap (a separate
// instance, so the dense kernel's edge tiles carry no bitmap test).
template <bool QSA, bool DIRECT>
__device__ __forceinline__ void flash_prefill(const FlashParams& p, const int qb, const int part) {
#pragma clang fp contract(off)  // fixed rounding sequence, reproduced by the CPU oracle
    // four distinct arrays (the compiler then tells the buffers apart and waits for the loads
    // into one of them only before reading that one): K and V^T tiles of the staged path, or K
    // and V tiles of the direct path, double-buffered
    static_assert(FK * KST == FK * DK_ROW && HEAD_DIM * VST <= FK * DV_ROW, "tile buffers");
    __shared__ __align__(1024) uint16_t L0[FK * DK_ROW];
    __shared__ __align__(1024) uint16_t L1[FK * DK_ROW];
    __shared__ __align__(1024) uint16_t L2[FK * DV_ROW];
    __shared__ __align__(1024) uint16_t L3[FK * DV_ROW];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int t0 = qb * FT;
    const int t1 = min(t0 + FT, p.tokens);
    const int tq = t0 + wave * 2 + (col >> 4);
    const int head = col & 15;
    const bool qvalid = tq < p.tokens;
    const int tqc = qvalid ? tq : t1 - 1;
    const uint32_t qpos = p.p0 + uint32_t(tqc);
    const uint32_t chunk = p.p0 + (uint32_t(t0) / CHUNK) * CHUNK;
    const uint32_t base = p.full ? 0u : (chunk > uint32_t(WINDOW - 1) ? chunk - uint32_t(WINDOW - 1) : 0u);
    const uint32_t plo = p.p0 + uint32_t(t0), khi = p.p0 + uint32_t(t1 - 1);
    const uint32_t klo = p.full ? 0u : (plo > uint32_t(WINDOW - 1) ? plo - uint32_t(WINDOW - 1) : 0u);
    // The block's key tiles are split over up to FLASH_PARTS workgroups of about
    // FLASH_PART_TILES tiles each, so long (late) query blocks do not set the kernel's length.
    const int ntiles = flash_block_tiles(p.tokens, p.p0, p.full, qb);
    const int parts = flash_block_parts(ntiles);
    if (part >= parts) return;
    const int j0 = part * ntiles / parts, j1 = (part + 1) * ntiles / parts;

    // Q^T fragments (B operand of S^T): k-step s covers dims 16s + 8*half .. +8
    bf16x8 qf[8];
    {
        const uint16_t* qrow = p.q + (size_t(tqc) * HEADS + head) * HEAD_DIM;
#pragma unroll
        for (int s = 0; s < 8; ++s) qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(qrow + 16 * s + 8 * half));
    }
    floatx16 oacc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
    float m = NEG_INF, ls = 0.f;

    // QSA: the query's blocks of four keys complete at its position are seen only when
    // selected (bit b of its bitmap word b / 32); its unfinished block always is
    const uint32_t* qmask = QSA ? p.qsa_mask + size_t(tqc) * p.qsa_words : nullptr;
    const uint32_t qcomplete = (qpos + 1) / 4;
    const bool cached = !p.full && p.keys_rot != nullptr && base == 0 && khi < p.rot_rows;
    const KvSource src{cached ? p.keys_rot : p.keys, !p.full && !cached};

    // Online softmax of tile j in the base-2 domain: x = score * scale * log2(e),
    // p = 2^(x - max).  Element i of tile r is key k0 + 32r + 8(i/4) + 4*half + i%4.  Only
    // tiles that cross a query's causal edge or window start need the mask.  QSA: every tile
    // is masked by the query's selected blocks (its unfinished block is always seen).  Leaves
    // the probabilities in sacc and rescales oacc.
    // Online softmax of tile j in the base-2 domain: x = score * scale * log2(e),
    // p = 2^(x - max).  Element i of tile r is key k0 + 32r + 8(i/4) + 4*half + i%4.  Only
    // tiles that cross a query's causal edge or window start need the mask.  QSA: every tile
    // is masked by the query's selected blocks (its unfinished block is always seen).  Leaves
    // the probabilities in sacc and rescales oacc.
    auto softmax = [&](int j, floatx16 (&sacc)[2]) {
        const uint32_t k0 = klo + uint32_t(j * FK);
        const bool edge = QSA || !(k0 + uint32_t(FK - 1) <= plo && (p.full || k0 + uint32_t(WINDOW - 1) >= khi));
        float mt = NEG_INF;
        if (edge) {
            // QSA (global layers: k0 is a multiple of 64): the tile's 16 blocks b0 .. b0 + 15
            // are bits 0..15 of one bitmap word shifted by b0 % 32, read once per tile; blocks
            // at or past qcomplete are not tested
            uint32_t qbits = 0u;
            const uint32_t b0 = k0 >> 2;
            if (QSA && b0 < qcomplete) qbits = qmask[b0 >> 5] >> (b0 & 31);
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t kp = k0 + uint32_t(32 * r + 8 * (i >> 2) + 4 * half + (i & 3));
                    bool vis = kp <= qpos && (p.full || kp + uint32_t(WINDOW - 1) >= qpos);
                    if (QSA) {
                        const uint32_t b = kp >> 2;
                        vis = vis && (b >= qcomplete || ((qbits >> (b - b0)) & 1u));
                    }
                    const float x = vis ? sacc[r][i] * SCALE_LOG2E : NEG_INF;
                    sacc[r][i] = x;
                    mt = fmaxf(mt, x);
                }
        } else {
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float x = sacc[r][i] * SCALE_LOG2E;
                    sacc[r][i] = x;
                    mt = fmaxf(mt, x);
                }
        }
        mt = fmaxf(mt, xor_lane<32>(mt));
        const float mn = fmaxf(m, mt);
        const float ms = mn == NEG_INF ? 0.0f : mn;  // nothing visible yet: every p is 0
        const float alpha = exp2_det(m - ms);
        ls *= alpha;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float e = exp2_det(sacc[r][i] - ms);
                sacc[r][i] = e;
                ls += e;
            }
        m = mn;
        // alpha is exactly 1 where the running maximum did not move: the wave skips the
        // rescale when that holds in every lane (multiplying by 1 changes nothing)
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
        }
    };
    // O^T += V^T P^T; k-step s takes keys 16s + 4*half + {0..3} and 16s + 8 + 4*half + {0..3};
    // vt(dt, s) returns the V^T operand of d-tile dt at k-step s
    auto pv = [&](const floatx16 (&sacc)[2], auto vt) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int r = s >> 1, i0 = (s & 1) * 8;
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) split_bf16(sacc[r][i0 + 2 * k], sacc[r][i0 + 2 * k + 1], hw[k], lw[k]);
            const bf16x8 ph = as_bf16x8(make_uint4(hw[0], hw[1], hw[2], hw[3]));
            const bf16x8 pl = as_bf16x8(make_uint4(lw[0], lw[1], lw[2], lw[3]));
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const bf16x8 a = vt(dt, s);
                oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, ph, oacc[dt], 0, 0, 0);
                oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pl, oacc[dt], 0, 0, 0);
            }
        }
    };
    // S^T = K Q^T for 64 keys (two 32-row tiles); kop(r, s) returns the K operand of row tile
    // r at k-step s
    auto qk = [&](floatx16 (&sacc)[2], auto kop) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 16; ++i) sacc[r][i] = 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
#pragma unroll
            for (int r = 0; r < 2; ++r) sacc[r] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop(r, s), qf[s], sacc[r], 0, 0, 0);
        }
    };

    if constexpr (!DIRECT) {
        // staged through registers (keys rotated on the way where the block needs it): K rows
        // and V^T in LDS
        KvStage st;
        flash_load(p, src, klo + uint32_t(j0 * FK), khi, base, st);
        flash_store(src, st, L0, L2);
        __syncthreads();
        for (int j = j0; j < j1; ++j) {
            const bool odd = ((j - j0) & 1) != 0;
            const uint16_t* Kc = odd ? L1 : L0;
            const uint16_t* Vc = odd ? L3 : L2;
            if (j + 1 < j1) flash_load(p, src, klo + uint32_t((j + 1) * FK), khi, base, st);
            floatx16 sacc[2];
            qk(sacc, [&](int r, int s) {
                return as_bf16x8(*reinterpret_cast<const uint4*>(&Kc[(r * 32 + col) * KST + 16 * s + 8 * half]));
            });
            softmax(j, sacc);
            pv(sacc, [&](int dt, int s) {
                const uint16_t* vrow = &Vc[(dt * 32 + col) * VST + 16 * s + 4 * half];
                const uint2 x0 = *reinterpret_cast<const uint2*>(vrow);
                const uint2 x1 = *reinterpret_cast<const uint2*>(vrow + 8);
                return as_bf16x8(make_uint4(x0.x, x0.y, x1.x, x1.y));
            });
            if (j + 1 < j1) flash_store(src, st, odd ? L0 : L1, odd ? L2 : L3);
            __syncthreads();
        }
    } else {
        // (DIRECT: the launch holds only blocks whose keys need no rotation)
        // Keys (already rotated) and values loaded straight into LDS (buffer loads with the
        // LDS destination, no staging registers), in padded rows: key row R at R * 272 bytes
        // (the S^T operand reads of 16 consecutive rows hit every bank), value row R at
        // R * 320 bytes (the transposing V^T operand reads, ds_read_b64_tr_b16, of four rows x
        // 64 bytes per half wave hit every bank).  Every operand read is one base address plus
        // an immediate offset.  Tile j's keys and values go to buffer (j - j0) % 2 (L0/L1
        // keys, L2/L3 values) and are requested at the start of tile j - 1.  Same arithmetic
        // as the staged path.
        // A tile is loaded as 16-byte chunks: chunk L of the tile (row L / chunks per row,
        // piece L % chunks per row, pieces past 15 being padding) is lane L % 64 of load L / 64;
        // wave w issues loads w, w + 4, ...  Its lanes' offsets within the tile are fixed: a
        // tile whose 64 keys are consecutive ring slots without a wrap adds the first slot as
        // a scalar offset; the last tile of a block (keys past khi load key khi) and tiles
        // across the ring's end take per-lane slots.
        constexpr int KLOADS = FK * DK_CHUNKS / 64, VLOADS = FK * DV_CHUNKS / 64;  // 17, 20
        constexpr int KPER = (KLOADS + 3) / 4, VPER = VLOADS / 4;                 // 5, 5
        static_assert(VLOADS % 4 == 0 && FK * DK_CHUNKS % 64 == 0, "tile loads");
        const uint32_t krows = cached ? p.rot_rows : p.capacity;
        const __amdgpu_buffer_rsrc_t kview = buffer_view(src.keys, krows * uint32_t(HEAD_DIM * 2));
        const __amdgpu_buffer_rsrc_t vview = buffer_view(p.values, p.capacity * uint32_t(HEAD_DIM * 2));
        // per load t of this wave: row (bits 0..7) and piece (bits 8..15) of this lane's chunk
        uint32_t kpiece[KPER], vpiece[VPER];
#pragma unroll
        for (int t = 0; t < KPER; ++t) {
            const int L = 64 * (wave + 4 * t) + lane;
            kpiece[t] = uint32_t(L / DK_CHUNKS) | (uint32_t(L % DK_CHUNKS) << 8);
        }
#pragma unroll
        for (int t = 0; t < VPER; ++t) {
            const int L = 64 * (wave + 4 * t) + lane;
            vpiece[t] = uint32_t(L / DV_CHUNKS) | (uint32_t(L % DV_CHUNKS) << 8);
        }
        auto tile_load = [&](const __amdgpu_buffer_rsrc_t view, uint16_t* dst, const uint32_t* piece, auto nloads,
                             auto row_elems, int j, bool by_position) {
            constexpr int N = decltype(nloads)::value, RE = decltype(row_elems)::value;
            const uint32_t k0 = klo + uint32_t(j * FK);
            const uint32_t slot0 = by_position ? k0 : k0 % p.capacity;
            const bool plain = k0 + uint32_t(FK - 1) <= khi && (by_position || slot0 + uint32_t(FK - 1) < p.capacity);
#pragma unroll
            for (int t = 0; t < N; ++t) {
                const int li = wave + 4 * t;
                if (li * 64 >= FK * (RE / 8)) break;
                const uint32_t row = piece[t] & 255u, pc = piece[t] >> 8;
                uint32_t off;
                if (plain) {
                    off = row * uint32_t(HEAD_DIM * 2) + pc * 16u;
                } else {
                    const uint32_t kp = min(k0 + row, khi);
                    uint32_t slot = by_position ? kp : slot0 + (kp - k0);
                    slot = slot >= p.capacity && !by_position ? slot - p.capacity : slot;
                    off = slot * uint32_t(HEAD_DIM * 2) + pc * 16u;
                }
                off = pc < 16u ? off : OOB_OFFSET;  // padding: nothing to load
                __builtin_amdgcn_raw_ptr_buffer_load_lds(view, (lds_ptr_t)(dst + li * 512), 16, off,
                                                         plain ? int(slot0 * uint32_t(HEAD_DIM * 2)) : 0, 0, 0);
            }
        };
        using KN = std::integral_constant<int, KPER>;
        using VN = std::integral_constant<int, VPER>;
        using KR = std::integral_constant<int, DK_ROW>;
        using VR = std::integral_constant<int, DV_ROW>;
        auto dma_k = [&](uint16_t* dst, int j) { tile_load(kview, dst, kpiece, KN{}, KR{}, j, cached || p.full); };
        auto dma_v = [&](uint16_t* dst, int j) { tile_load(vview, dst, vpiece, VN{}, VR{}, j, false); };
        // S^T operand of row tile r, k-step s: key row 32r + col, dims 16s + 8 half .. + 8
        auto kop_of = [&](const uint16_t* Kb) {
            const uint16_t* base = Kb + col * DK_ROW + 8 * half;
            return [=](int r, int s) {
                return as_bf16x8(*reinterpret_cast<const uint4*>(base + 32 * r * DK_ROW + 16 * s));
            };
        };
        // V^T operand of d-tile dt, k-step s: source lane sl = lane % 16 of 16-lane group g =
        // lane / 16 addresses keys 16s + 4(g / 2) + sl / 4 (and + 8), dims 32dt + 16(g % 2) +
        // 4(sl % 4) .. + 3; the transposing read hands lane j of the group element j % 4 of
        // source lane 4t + j / 4 as its element t: dim 32dt + 16(g % 2) + j of keys 16s + 4(g / 2)
        // + t (and + 8 + t), the rows of the P^T operand's k-step s
        typedef short short4_t __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) short4_t* tr_ptr_t;
        const int sl = lane & 15, grp = lane >> 4;
        const int vlane = (4 * (grp >> 1) + (sl >> 2)) * DV_ROW + 16 * (grp & 1) + 4 * (sl & 3);
        auto vop_of = [&](const uint16_t* Vb) {
            const uint16_t* base = Vb + vlane;
            return [=](int dt, int s) {
                const short4_t x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((tr_ptr_t)(base + 16 * s * DV_ROW + 32 * dt));
                const short4_t x1 =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((tr_ptr_t)(base + (16 * s + 8) * DV_ROW + 32 * dt));
                bf16x8 a;
                __builtin_memcpy(&a, &x0, 8);
                __builtin_memcpy(reinterpret_cast<char*>(&a) + 8, &x1, 8);
                return a;
            };
        };
        // tile j: its keys and values are in Kc / Vc; the next tile's go to Kn / Vn (free:
        // read by tile j - 1 before this tile's barrier)
        auto tile = [&](int j, const uint16_t* Kc, uint16_t* Kn, const uint16_t* Vc, uint16_t* Vn) {
            // tile j is in (each wave waits for its own loads into LDS: the barrier's fence
            // covers LDS operations, not loads into LDS, and every wave reads rows that other
            // waves loaded); tile j - 1 is done with Kn and Vn
            wait_vmcnt<0>();
            __syncthreads();
            if (j + 1 < j1) {
                dma_k(Kn, j + 1);
                dma_v(Vn, j + 1);
            }
            floatx16 sacc[2];
            qk(sacc, kop_of(Kc));
            softmax(j, sacc);
            pv(sacc, vop_of(Vc));
        };
        dma_k(L0, j0);
        dma_v(L2, j0);
        for (int j = j0; j < j1; j += 2) {
            tile(j, L0, L1, L2, L3);
            if (j + 1 < j1) tile(j + 1, L1, L0, L3, L2);
        }
    }
    // O = O^T / l; element i of d-tile dt is dim 32dt + 8(i/4) + 4*half + i%4
    float lt = ls + xor_lane<32>(ls);
    if (parts > 1) {
        // Partial (m, l, unnormalised O^T) of this part; the last part to finish merges all
        // parts of the block in part order: M = max m_q, w_q = 2^(m_q - M),
        // O = sum O_q w_q / sum l_q w_q.
        const int colg = wave * 32 + col;
        const uint32_t nslots = uint32_t(flash_blocks(p.tokens)) * FLASH_PARTS;
        const __amdgpu_buffer_rsrc_t ov = buffer_view(p.part_o, nslots * (FT * HEADS) * HEAD_DIM * 4u);
        const __amdgpu_buffer_rsrc_t mv = buffer_view(p.part_ml, nslots * (FT * HEADS) * 8u);
        auto o_off = [&](int q) { return uint32_t(((size_t(qb) * FLASH_PARTS + q) * (FT * HEADS) + colg) * HEAD_DIM * 4); };
        auto ml_off = [&](int q) { return uint32_t(((size_t(qb) * FLASH_PARTS + q) * (FT * HEADS) + colg) * 8); };
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                buffer_store16_sc1(ov, o_off(part) + (32 * dt + 8 * g + 4 * half) * 4,
                                   make_uint4(__float_as_uint(oacc[dt][4 * g]), __float_as_uint(oacc[dt][4 * g + 1]),
                                              __float_as_uint(oacc[dt][4 * g + 2]), __float_as_uint(oacc[dt][4 * g + 3])));
        if (half == 0) buffer_store8_sc1(mv, ml_off(part), make_uint2(__float_as_uint(m), __float_as_uint(lt)));
        wait_stores();
        __syncthreads();
        if (tid == 0) s_last = atomicAdd(p.tickets + qb, 1u) == uint32_t(parts - 1);
        __syncthreads();
        if (!s_last) return;
        float mq[FLASH_PARTS], lq[FLASH_PARTS];
        float M = NEG_INF;
#pragma unroll
        for (int q = 0; q < FLASH_PARTS; ++q) {
            if (q < parts) {
                const uint2 v = buffer_load8_sc1(mv, ml_off(q));
                mq[q] = __uint_as_float(v.x);
                lq[q] = __uint_as_float(v.y);
                M = fmaxf(M, mq[q]);
            }
        }
        lt = 0.f;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
#pragma unroll
        for (int q = 0; q < FLASH_PARTS; ++q) {
            if (q < parts) {
                const float w = exp2_det(mq[q] - M);
                lt += lq[q] * w;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const uint4 v = buffer_load16_sc1(ov, o_off(q) + (32 * dt + 8 * g + 4 * half) * 4);
                        oacc[dt][4 * g] += __uint_as_float(v.x) * w;
                        oacc[dt][4 * g + 1] += __uint_as_float(v.y) * w;
                        oacc[dt][4 * g + 2] += __uint_as_float(v.z) * w;
                        oacc[dt][4 * g + 3] += __uint_as_float(v.w) * w;
                    }
            }
        }
        if (tid == 0) atomicExch(p.tickets + qb, 0u);  // ready for the next launch
    }
    if (!qvalid) return;
    uint16_t* orow = p.out + size_t(tq) * ATTN + head * HEAD_DIM;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint32_t w[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t a = bits(roundbf(oacc[dt][4 * g + 2 * k] / lt));
                const uint32_t b = bits(roundbf(oacc[dt][4 * g + 2 * k + 1] / lt));
                w[k] = (a & 0xffffu) | (b << 16);
            }
            *reinterpret_cast<uint2*>(orow + 32 * dt + 8 * g + 4 * half) = make_uint2(w[0], w[1]);
        }
}

// Workgroup w takes part w / blocks of query block blocks - 1 - w % blocks (consecutive
// workgroups, dealt round-robin to the XCDs, take different blocks; a block's parts share an
// XCD) and returns if the block has fewer parts.
template <bool QSA, bool DIRECT>
__global__ __launch_bounds__(256, 2) void flash_prefill_kernel(const FlashParams p) {
    const int nqb = flash_blocks(p.tokens);
    flash_prefill<QSA, DIRECT>(p, nqb - 1 - int(blockIdx.x) % nqb, int(blockIdx.x) / nqb);
}

// Workgroup w takes the item the host's schedule ranks for it (qb << 2 | part).
template <bool QSA, bool DIRECT>
__global__ __launch_bounds__(256, 2) void flash_prefill_ranked_kernel(const FlashParams p, const FlashSchedule sched) {
    const uint32_t item = sched.item[blockIdx.x];
    flash_prefill<QSA, DIRECT>(p, int(item >> 2), int(item & 3u));
}

template <int BT, int BW, int WT, int NT, int KD, int NS>
void launch_gemm_dma(GemmEpilogue epi, const GemmParams& p, hipStream_t s) {
    const int cols = epi == GEMM_SWIGLU ? INTER / (BW / 2) : (p.m + BW - 1) / BW;
    const int rows = (p.tokens + BT - 1) / BT;
    const int per = (cols * rows + 7) / 8;
    const dim3 grid(8 * per), block(NT);
#define PLAMO_GEMM(EP) hipLaunchKernelGGL((gemm_dma_kernel<EP, BT, BW, WT, NT, KD, NS>), grid, block, 0, s, p, cols, rows)
    constexpr int TW = BW / (NT / 64 / WT) / 32;  // 32-column blocks per wave
    if (epi == GEMM_F32) PLAMO_GEMM(GEMM_F32);
    else if (epi == GEMM_BF16) PLAMO_GEMM(GEMM_BF16);
    else if (epi == GEMM_RAW) PLAMO_GEMM(GEMM_RAW);
    else if constexpr (TW % 2 == 0) PLAMO_GEMM(GEMM_SWIGLU);  // gate and up blocks pair inside a wave
    else throw Error(E_INVAL, "SwiGLU GEMM needs an even number of column blocks per wave");
#undef PLAMO_GEMM
}

template <int BT, int BW, int WT, int NT>
void launch_gemm_packed(GemmEpilogue epi, const GemmParams& p, hipStream_t s) {
    const int cols = epi == GEMM_SWIGLU ? INTER / (BW / 2) : (p.m + BW - 1) / BW;
    const int rows = (p.tokens + BT - 1) / BT;
    const int per = (cols * rows + 7) / 8;
    const dim3 grid(8 * per), block(NT);
#define PLAMO_GEMM(PK, EP) hipLaunchKernelGGL((gemm_kernel<PK, EP, BT, BW, WT, NT>), grid, block, 0, s, p, cols, rows)
    if (epi == GEMM_F32) PLAMO_GEMM(true, GEMM_F32);
    else if (epi == GEMM_BF16) PLAMO_GEMM(true, GEMM_BF16);
    else if (epi == GEMM_RAW) PLAMO_GEMM(true, GEMM_RAW);
    else PLAMO_GEMM(true, GEMM_SWIGLU);
#undef PLAMO_GEMM
}

}  // namespace

void launch_gemm(bool packed, GemmEpilogue epi, const GemmParams& p, hipStream_t s) {
    if (p.k % BK != 0 || p.tokens < 1 || p.m < 1 || (epi == GEMM_SWIGLU && p.m != 2 * INTER))
        throw Error(E_INVAL, "unsupported GEMM shape");
    // operand and output views take 32-bit byte offsets (rows of the last tile included)
    const uint64_t t_pad = uint64_t(p.tokens) + 256;
    if (t_pad * uint64_t(p.k) * 2 >= (1ull << 31) || uint64_t(p.m) * uint64_t(p.k) * 2 >= (1ull << 31) ||
        t_pad * uint64_t(p.m) * 4 >= (1ull << 31))
        throw Error(E_INVAL, "GEMM operands exceed 2 GiB");
    // Tile choice (measured on the prefill shapes, 2048 tokens): 256 x 128 tiles for the wide
    // projections (gate_up, qkv), smaller ones for the 1536-row ones (o, down), where larger
    // tiles leave CUs idle; plain weights go straight to LDS, .p12 weights are expanded in
    // registers on the way.
    const bool wide = p.tokens > 128 && (epi == GEMM_SWIGLU || p.m > 2048);
    if (packed) {
        if (wide) launch_gemm_packed<256, 128, 4, 512>(epi, p, s);
        else launch_gemm_packed<128, 128, 2, 256>(epi, p, s);
    } else {
        // gate_up: 256 x 128 tiles on eight waves, three 64-deep stages (48 KB each): twice the
        // MFMAs per barrier of 32-deep stages (gate_up 100 -> 72-77 us); 2048 tokens make 768
        // tiles, three per CU
        // qkv (2304 rows): 128 x 192 tiles on eight waves (192 tiles; 256 x 128 makes 144 and
        // leaves 112 CUs idle): 22.3 -> 19.7-20.2 us at 2048 tokens
        // 128 x 128 fallback (SwiGLU below 129 tokens): six 32-deep stages, five in flight
        // 1536-row projections (o, down): 128 x 96 tiles with four waves, 64-deep stages, so
        // 2048 tokens make exactly 256 tiles (128 x 128 left a quarter of the CUs idle)
        if (wide && epi == GEMM_SWIGLU) launch_gemm_dma<256, 128, 4, 512, 64, 3>(epi, p, s);
        else if (wide && p.m % 192 == 0) launch_gemm_dma<128, 192, 4, 512, 64, 3>(epi, p, s);
        else if (wide) launch_gemm_dma<256, 128, 4, 512, 64, 3>(epi, p, s);
        else if (epi != GEMM_SWIGLU && p.m % 96 == 0) launch_gemm_dma<128, 96, 4, 256, 64, 4>(epi, p, s);
        else launch_gemm_dma<128, 128, 4, 512, 32, 6>(epi, p, s);
    }
}

void launch_rows_norm(const RowsNormParams& p, int tokens, hipStream_t s) {
    RowsNormParams q = p;
    q.tokens = tokens;
    hipLaunchKernelGGL(rows_norm_kernel, dim3((tokens + 3) / 4), dim3(256), 0, s, q);
}

void launch_qk_prep(const QkPrepParams& p, hipStream_t s) {
    if (p.tokens < 1) return;
    hipLaunchKernelGGL(qk_prep_kernel, dim3(p.tokens), dim3(256), 0, s, p);
}

namespace {

// Workgroup order of a flash call whose items all fit on the GPU at once (its arithmetic does
// not depend on the order).  The items (query block, part) are ranked by their tile count,
// largest first (ties: later block, then lower part).  Two workgroups of this kernel fit on a
// CU, and workgroups w and w + CUs of a launch whose workgroups all start together share a
// CU, so workgroups CUs .. take the ranks from CUs on in reverse: the largest items share a CU
// with the smallest.  Measured on a 2048-token call from position 0 (504 items): the most
// tiles on one CU 23 -> 18, flash 66 -> 62 us.  Calls with more items than two per CU keep
// the default order (all parts of a block on one XCD): the ranked order measured 3 % slower
// on the later chunks of a 30,720-token prompt.
void flash_schedule(const FlashParams& p, FlashSchedule& sched) {
    // the last schedule of local and of global layers, per host thread
    thread_local struct {
        int device = -1, cus = 0, tokens = -1;
        uint32_t p0 = 0;
        FlashSchedule sched{};
    } cache[2];
    int device = 0;
    PLAMO_HIP(hipGetDevice(&device));
    auto& c = cache[p.full ? 1 : 0];
    if (c.device != device) {
        PLAMO_HIP(hipDeviceGetAttribute(&c.cus, hipDeviceAttributeMultiprocessorCount, device));
        c.device = device;
        c.tokens = -1;
    }
    if (c.tokens != p.tokens || c.p0 != p.p0) {
        struct Item {
            int tiles, qb, part;
        };
        Item items[FLASH_SCHEDULE_MAX];
        int n = 0;
        for (int qb = 0; qb < flash_blocks(p.tokens); ++qb) {
            const int tiles = flash_block_tiles(p.tokens, p.p0, p.full, qb), parts = flash_block_parts(tiles);
            for (int q = 0; q < parts; ++q) items[n++] = {(q + 1) * tiles / parts - q * tiles / parts, qb, q};
        }
        const int C = std::max(c.cus, 1);
        c.sched.n = 0;
        if (n <= 2 * C) {
            std::sort(items, items + n, [](const Item& a, const Item& b) {
                if (a.tiles != b.tiles) return a.tiles > b.tiles;
                if (a.qb != b.qb) return a.qb > b.qb;
                return a.part < b.part;
            });
            for (int w = 0; w < n; ++w) {
                const int rank = w < C ? w : C + (n - 1 - w);
                c.sched.item[w] = uint16_t((items[rank].qb << 2) | items[rank].part);
            }
            c.sched.n = uint32_t(n);
        }
        c.tokens = p.tokens;
        c.p0 = p.p0;
    }
    sched = c.sched;
}

}  // namespace

void launch_flash_prefill(const FlashParams& p, hipStream_t s) {
    if (p.tokens < 1) return;
    if (p.tokens > 65536 / FLASH_PARTS * 8) throw Error(E_INVAL, "flash prefill: too many tokens in one call");
    const bool qsa = p.full && p.qsa_mask;
    FlashSchedule sched;
    sched.n = 0;
    if (flash_blocks(p.tokens) * FLASH_PARTS <= FLASH_SCHEDULE_MAX) flash_schedule(p, sched);
    // keys straight into LDS when no block of the call rotates its keys: global layers, and
    // local layers whose keys all sit in the rotated-key cache (window base 0)
    const uint32_t last = p.p0 + uint32_t(p.tokens) - 1;
    const bool direct = p.capacity >= uint32_t(FK) &&
                        (p.full || (p.keys_rot != nullptr && last < p.rot_rows && last < uint32_t(WINDOW)));
    const dim3 block(256);
    if (sched.n) {
        // the schedule travels in the kernel arguments (1.5 KB): only the launches that use it
        const dim3 grid(sched.n);
#define PLAMO_FLASH(Q, D) hipLaunchKernelGGL((flash_prefill_ranked_kernel<Q, D>), grid, block, 0, s, p, sched)
        if (qsa) PLAMO_FLASH(true, true);
        else if (direct) PLAMO_FLASH(false, true);
        else PLAMO_FLASH(false, false);
#undef PLAMO_FLASH
    } else {
        const dim3 grid(uint32_t(flash_blocks(p.tokens) * FLASH_PARTS));
#define PLAMO_FLASH(Q, D) hipLaunchKernelGGL((flash_prefill_kernel<Q, D>), grid, block, 0, s, p)
        if (qsa) PLAMO_FLASH(true, true);
        else if (direct) PLAMO_FLASH(false, true);
        else PLAMO_FLASH(false, false);
#undef PLAMO_FLASH
    }
}

}  // namespace plamo
