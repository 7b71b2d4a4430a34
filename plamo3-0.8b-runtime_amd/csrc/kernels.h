// Kernel parameter blocks and host-side launchers (defined in the .hip files).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace plamo {

constexpr int ROWS = 4;       // activation rows of one decode step (Batch lanes)
constexpr int KEYS_PER_PART = 64;  // keys per split-K decode attention partition
constexpr int HEAD_BLOCKS = 1024;  // workgroups of the LM-head GEMV (argmax partials)

// Per-step state kept in device memory so one captured graph replays every step.
struct StepState {
    uint32_t rows;            // active rows (1..4)
    uint32_t stopped;         // device loop finished: every kernel returns at once
    uint32_t loop;            // device-driven loop: feed `next` back as `token`, advance pos
    uint32_t stop_enabled;    // loop stops on token 1 or 16 (Main.swift:279)
    uint32_t max_tokens;      // loop: emitted-token limit
    uint32_t produced;        // loop: tokens emitted so far
    uint32_t reason;          // loop: 1 stop, 2 length, 3 invalid token
    uint32_t sampling;        // Sampler.select controls active
    float penalty, frequency, presence;
    int32_t ngram;
    uint32_t lane[ROWS];      // KV slice of each row
    uint32_t pos[ROWS];       // absolute position of each row's input token
    int32_t token[ROWS];      // input token of each row
    uint32_t next[ROWS];      // selected next token of each row
    uint32_t hist_len[ROWS];  // generated-history length (sampler)
    uint32_t counted[ROWS];   // history entries already folded into the counts
    // Device-driven batch loop (decodeBatch, BatchDecode.swift:8-37): lane bookkeeping
    // before each step packs the running lanes into rows; the head feeds predictions back.
    uint32_t quad;            // batch loop active
    uint32_t lanes;           // lanes in the batch (1..4)
    uint32_t last;            // last lane still served (stopOnTruncation lowers it)
    uint32_t trunc_stop;      // stopOnTruncation
    uint32_t out_stride;      // out_ids entries per lane
    uint32_t lpos[ROWS];      // position of each lane's next input token
    int32_t lnext[ROWS];      // each lane's latest prediction
    uint32_t lcount[ROWS];    // tokens emitted per lane
    uint32_t llimit[ROWS];    // per-lane token limit
    uint32_t lreason[ROWS];   // 0 running, 1 stop token, 2 length
    // Verification rows (Runtime.forward(all: sequential:) with two rows): every row reads and
    // writes KV slice 0 at its own position; `lane` then only names its output slot.
    uint32_t kv_shared;
};
static_assert(sizeof(StepState) <= 256, "the kernel-level attention workspace keeps 256 B for the state");

// Buffers the decode kernels share.
struct DecodeBuffers {
    StepState* state;
    int32_t* out_ids;         // loop: emitted tokens
    int32_t* history;         // [ROWS][hist_cap]
    uint32_t hist_cap;
    int32_t* counts;          // [ROWS][VOCAB]
    uint32_t* banned;         // [ROWS][VOCAB/32]
    float* head_v;            // [ROWS][HEAD_BLOCKS] argmax partials
    uint32_t* head_i;
    uint32_t* tickets;        // [1] spare ticket, zero between launches
};

// PRO_MERGE: the one-row o projection whose prologue merges the attention partitions of a
// row with 2..MERGE_IN_O of them (the attention kernel then skips its own merge), else reads
// the attention output as PRO_PLAIN16 does.
enum Prologue { PRO_PLAIN = 0, PRO_EMBED = 1, PRO_RESID = 2, PRO_PLAIN16 = 3, PRO_RESID16 = 4, PRO_MERGE = 5 };
constexpr uint32_t MERGE_IN_O = 6;  // partitions (64 keys each) the o prologue merges
enum Epilogue { EPI_ROUND = 0, EPI_SWIGLU = 1, EPI_LOGITS = 2, EPI_BF16 = 3, EPI_RAW = 4 };  // RAW: FP32 sums, unrounded

struct GemvParams {
    const uint16_t* w;        // plain BF16 [m][n] or .p12 payload
    const uint32_t* table;    // .p12 block table (packed only)
    int m;                    // weight rows
    int rows;                 // rows the input buffers hold (the active rows when no
                              // StepState is given; the state's rows never exceed it)
    const StepState* state;   // may be null (kernel-level entry points)
    uint32_t lane_mask;       // always 0: makes the state read a per-lane (vector) load
    // prologue
    const float* in;          // PLAIN: [rows][n]; RESID: projection output [rows][1536]
    const uint16_t* in16;     // PLAIN16: BF16 [rows][n] (half the bytes every workgroup stages);
                              // RESID16: BF16 projection output [rows][1536]
    const float* resid_in;    // RESID: residual stream x
    float* resid_out;         // RESID: updated residual (written by block 0)
    const uint16_t* resid16_in;  // RESID16: residual stream x as BF16 (every value is BF16-exact)
    uint16_t* resid16_out;    // EMBED/RESID16: updated residual as BF16 (written by block 0)
    const uint16_t* g_post;   // RESID: post norm weight
    float post_offset;
    const uint16_t* g_next;   // EMBED/RESID: following norm weight (+1.0)
    const uint16_t* embed;    // EMBED: embedding table [VOCAB][1536]
    float* hidden;            // optional: normalised rows (final hidden)
    // epilogue
    float* out;               // ROUND: FP32 [rows][m]
    uint16_t* out16;          // LOGITS/BF16: [rows][m]; SWIGLU: BF16 [rows][m/2]
    DecodeBuffers bufs;       // LOGITS: sampler + argmax partials + state update
    uint32_t tag;             // step-timeline slot of this launch (timeline builds only)
    // MERGE: the attention partition buffers of the layer and its geometry
    const float* part_m;
    const float* part_l;
    const float* part_o;
    uint32_t parts;           // partitions per row in the buffers
    uint32_t merge_full;      // global layer (all keys visible), else the 2048-key window
};

struct AttnParams {
    const StepState* state;   // rows, positions and KV slices of the step
    uint32_t row0;            // the launch covers rows row0 .. row0 + gridDim.z - 1
    const float* qkv;         // [rows][2304] (BF16-valued FP32)
    const uint16_t* q_norm;   // [128]
    const uint16_t* k_norm;
    uint16_t* keys;           // [lanes][capacity][128]
    uint16_t* values;
    uint16_t* keys_rot;       // local layers: [lanes][rot_rows][128] keys rotated at their own
                              // position, for rows whose window starts at 0 (null: rotate)
    uint32_t rot_rows;
    uint32_t capacity;
    const uint32_t* local_rope;  // [2064][64] BF16 (cos | sin << 16)
    const uint32_t* global_rope; // [context][64]
    float* part_m;            // [ROWS][parts][16]
    float* part_l;
    float* part_o;            // [ROWS][parts][16][128]
    uint32_t parts;           // grid.x
    uint32_t* tickets;        // [rows][head groups], zero between launches
    uint16_t* out16;          // BF16 [rows][2048]
    uint32_t defer;           // rows with more partitions than this (0: none) are merged by
                              // attn_merge_kernel instead of the attention kernel's last workgroup
    uint32_t tag;             // step-timeline slot (the merge kernel uses tag + 1)
    uint32_t window;          // local layers: WINDOW (the keys a row sees), global layers: 0 (all)
    uint32_t merge_in_o;      // rows with 2..MERGE_IN_O partitions are merged by the next
                              // kernel (the o GEMV's PRO_MERGE prologue): no ticket, no merge
    const uint32_t* qsa_mask; // global layers with QSA: row q's selected blocks of four keys
                              // (bit b of word q * qsa_words + b / 32); keys of the unfinished
                              // block are always seen; null: every key
    uint32_t qsa_words;
};

// QSA block indexer of a global layer for `tokens` rows (qsa.hip).
struct QsaParams {
    const StepState* state;   // decode: one row at state->pos[0]; null: rows at p0 + t
    uint32_t p0;
    int tokens;
    const uint16_t* proj;     // [tokens][640] BF16 indexer projection of the normed rows
    const uint16_t* q_norm;   // [128]
    const uint16_t* k_norm;
    const uint32_t* global_rope;  // [context][64]
    uint16_t* queries;        // [tokens][512] BF16 rotated indexer queries
    uint16_t* raw;            // [context][128] raw keys by position
    uint16_t* pooled;         // [context / 4][128] block keys
    float* scores;            // [tokens][blocks]
    uint32_t* mask;           // [tokens][words] selected blocks
    uint32_t blocks, words;   // context / 4, its 32-bit words
    int budget;               // keys a query may select (multiple of four)
};
// qsa_prep, qsa_pool, qsa_scores (max_blocks: blocks the widest row may score), qsa_select.
void launch_qsa(const QsaParams& p, int max_blocks, hipStream_t s);
// The selection alone, on scores the caller supplies (p.scores, p.blocks, p.mask, p.words).
void launch_qsa_select(const QsaParams& p, hipStream_t s);
// Partitions a row may have before its merge moves to attn_merge_kernel: past 8 partitions
// (positions from 512 on) its 64 workgroups per row merge faster than the last workgroup of
// each head group (long-context decode 1515 -> 1554 tok/s, batch 4 5848 -> 6077 tok/s).
constexpr uint32_t ATTN_MERGE_INLINE = 8;
// attn_merge_kernel sums partitions in blocks of this many, one wave per block (block sums
// in partition order, then added in block order): 480 partitions at 30,720 keys run as
// four chains of 128 and one of 4 instead of one chain of 480 (8.5 us of the kernel's 13.6
// us at that size); rows of up to 128 partitions (8,192 keys) keep the single chain
constexpr uint32_t MERGE_BLOCK = 128;
// Four-row batches whose graph launches attn_merge_kernel anyway (contexts past 8
// partitions) send it every row past 2 partitions as well (batch 4 6074 -> 6126 tok/s; past
// 1 partition: the same).
constexpr uint32_t ATTN_MERGE_INLINE_BATCH = 2;

// Step timeline (builds with -DPLAMO_TIMELINE): per-workgroup start/end stamps of the
// decode-step kernels in a [TIMELINE_TAGS][TIMELINE_BLOCKS][2] table of s_memrealtime
// ticks (100 MHz), rewritten by every launch with the same tag.  Tags: layer * 8 + 0 qkv,
// 1 attention, 2 attention merge, 3 o, 4 gate_up, 5 down; 200 LM head, 250 head merge,
// 251 step begin.
constexpr int TIMELINE_TAGS = 256, TIMELINE_BLOCKS = 1024;
constexpr uint32_t TL_HEAD = 200, TL_HEAD_MERGE = 250, TL_STEP_BEGIN = 251;
// Copies the table out (`out` non-null, `words` = TIMELINE_TAGS * TIMELINE_BLOCKS * 2) and/or
// clears it; throws E_INVAL in builds without the timeline.
void timeline_copy(uint64_t* out, size_t words, bool clear);

// decode.hip
int gemv_group_rows(int n, int maxr, Epilogue epi, bool packed);     // weight rows per wave group
int gemv_blocks(int n, int maxr, Epilogue epi, int m, bool packed);  // workgroups for one group per wave
// LM-head workgroups (argmax partials, at most HEAD_BLOCKS): four waves each for one row;
// for four rows one eight-wave workgroup per CU.
inline int head_blocks(int maxr) { return maxr == 1 ? HEAD_BLOCKS : HEAD_BLOCKS / 4; }
void launch_gemv(int n, bool packed, int maxr, Prologue pro, Epilogue epi, const GemvParams& p, int blocks,
                 hipStream_t s);
// Rows p.row0 .. p.row0 + rows - 1 of the step (one launch per row for verification rows).
void launch_attention(bool full, const AttnParams& p, int rows, hipStream_t s);
void launch_attention_merge(const AttnParams& p, int rows, hipStream_t s);  // rows past the inline merge
void launch_step_begin(const DecodeBuffers& b, hipStream_t s);
// begin_next: device loops run the next step's bookkeeping (step_begin) in the same kernel
void launch_head_merge(const DecodeBuffers& b, int blocks, bool begin_next, hipStream_t s);
void launch_argmax(const void* x, uint32_t* out, int n, int rows, bool bf16, hipStream_t s);
void launch_select(float* logits, int n, const int32_t* history, int hist, float penalty, int ngram, float frequency,
                   float presence, int32_t* out, hipStream_t s);
void launch_unpack(const uint8_t* payload, const uint32_t* table, uint16_t* out, int64_t count, hipStream_t s);
// MTP adapter (Runtime.swift:485-520): input row [hidden | embed(token)], and the
// activation + down projection + residual after the up projection (a 3072-wide GEMV).
void launch_mtp_input(const float* hidden, const uint16_t* embed, int token, float* out, hipStream_t s);
void launch_mtp_down(const float* up, const float* x, const uint16_t* w, float* out, hipStream_t s);
void launch_fill_u32(uint32_t* p, uint32_t value, size_t count, hipStream_t s);
// Device workspace of a kernel-level decode attention call, 256-byte aligned: the step state
// (256 B), the attention tickets [ROWS][4 head groups] (256 B), then the partition
// statistics m, l [ROWS][parts][16] and outputs [ROWS][parts][16][128] (FP32), the layout the
// runtime's engine uses.
constexpr size_t attn_workspace_bytes(uint32_t parts) {
    return 512 + size_t(ROWS) * parts * 16 * (2 + 128) * 4;
}
// Partitions (64 keys each) the allocation-free entry point's static scratch holds: 8192 keys.
constexpr uint32_t STATIC_ATTN_PARTS = 128;
// Device address of this device's static scratch (attn_workspace_bytes(STATIC_ATTN_PARTS)
// bytes), looked up once per device; every call on a device shares it.
void* static_attn_scratch();

// Step state of a kernel-level decode attention call: `rows` rows at `pos` (row q reads and
// writes KV slice q), every other field zero; clears the rows' attention tickets.  Written by
// a kernel from its arguments, so the call needs no host copy.
void launch_attn_state(StepState* st, uint32_t* tickets, const int32_t* pos, int rows, hipStream_t s);

// prefill.hip
struct PrefillParams;
}  // namespace plamo
