/*
 * plamo_hip.h -- C ABI of the MI355X (gfx950) PLaMo-3 0.8B token loop.
 *
 * This is the drop-in boundary for the hot path of mikuteto-dev/plamo3-0.8b-runtime:
 * the Swift `Runtime` / `Batch` / `Sampler` / `decodeBatch` surface
 * (Sources/Plamo/Runtime.swift, Batch.swift, Sampler.swift, BatchDecode.swift) whose
 * Metal dispatches (Kernels.metal, Batch.metal) are replaced by hand-written HIP
 * kernels.  Plain pointers and sizes only; no C++ or torch types cross it.
 *
 * Conventions
 *   - Every function that can fail returns PLAMO_OK (0) or a PLAMO_E* code and, when
 *     `err` is non-NULL, writes a NUL-terminated message of at most `errlen` bytes.
 *     Message substrings the reference's callers match are kept verbatim.
 *   - Validation happens before any state changes (Runtime.swift:328-330): a failed
 *     call leaves position, logits and KV exactly as they were.
 *   - A handle is not re-entrant: one HIP stream per handle, every call returns after
 *     its GPU work completed (the reference commits and waits per call).
 *   - Token IDs are int32.  The greedy argmax of an all-NaN logits row is 0xffffffff in
 *     the reference (Kernels.metal:713-728); it is returned as the int32 -1.
 */
#ifndef PLAMO_HIP_H
#define PLAMO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PLAMO_OK 0
#define PLAMO_EINVAL 1  /* invalid argument, token, length or context exhausted */
#define PLAMO_EIO 2     /* file missing or unreadable */
#define PLAMO_EFORMAT 3 /* malformed safetensors / .p12 / config */
#define PLAMO_EDEVICE 4 /* HIP runtime or kernel failure */
#define PLAMO_ESTATE 5  /* call not valid in the current state */

typedef struct plamo_runtime plamo_runtime;
typedef struct plamo_batch plamo_batch;

typedef struct plamo_stats {
    int64_t position;         /* Runtime.position (Runtime.swift:154) */
    double gpu_seconds;       /* Runtime.gpuSeconds (Runtime.swift:155,463) */
    int64_t device_bytes;     /* all device memory held by the handle */
    int64_t weight_bytes;     /* Weights.gpuBytes (Runtime.swift:25) */
    int64_t linear_bytes;     /* bytes of the 16x4 projections + LM head read per decode step */
    int32_t context;          /* Runtime.context (Runtime.swift:147) */
    int32_t packed;           /* 1 when the .p12 archive is used (Runtime.swift:148) */
    int32_t last_output_rows; /* Runtime.lastOutputRows (Runtime.swift:153) */
    int32_t local_capacity;   /* ring slots of a sliding-window layer */
    /* wall seconds of the last plamo_generate's two phases, timed as Main.swift:245-247,287
     * times them for prefill_seconds / decode_seconds (0 before the first call) */
    double last_prefill_seconds;
    double last_decode_seconds;
    /* trained adapters in device memory (auxiliary_weight_bytes, Main.swift:342) and the QSA
     * counters Runtime.sparseQueries / sparseKeys / denseKeys (Runtime.swift:160-162,409-414) */
    int64_t auxiliary_bytes;
    int64_t sparse_queries;
    int64_t sparse_keys;
    int64_t dense_keys;
} plamo_stats;

/* ---- Runtime (Runtime.swift:128-553) ------------------------------------------- */

/* Runtime.init(directory:context:packed:) (Runtime.swift:164-286): validates
 * config.json (Runtime.swift:180-190), model.safetensors (Runtime.swift:33-101) or
 * model.p12 (Packed.swift:12-91), config-mlx.json RoPE frequencies (Runtime.swift:268-274),
 * uploads the weights to HBM and allocates the ring/global KV.  `source_sha256` is the
 * value the .p12 header must carry (Packed.swift:35); NULL selects the reference's
 * pinned checksum of the original model. */
int plamo_open(const char* directory, int32_t context, int32_t packed, const char* source_sha256,
               plamo_runtime** out, char* err, size_t errlen);
/* Runtime.init(directory:context:packed:qsaBudget:mtp:) (Runtime.swift:164-176,248): as
 * plamo_open, plus the trained adapters of auxiliary.safetensors (Auxiliary.swift:14-62,
 * format plamo-aux-v1, whose teacher_sha256 must equal `source_sha256`, NULL = the pinned
 * checksum).  `qsa_budget` 0 = dense attention, else a multiple of four in 4..2048 ("QSA budget
 * must be a multiple of four in 4...2048"): the global layers' block indexers select
 * qsa_budget / 4 blocks of four keys plus the unfinished block for each query once a row sees
 * more than the budget (Kernels.metal:564-702).  `mtp` loads the MTP head (plamo_draft,
 * plamo_forward_ex with all/sequential, plamo_rewind). */
int plamo_open_aux(const char* directory, int32_t context, int32_t packed, const char* source_sha256,
                   int32_t qsa_budget, int32_t mtp, plamo_runtime** out, char* err, size_t errlen);
/* Releases the runtime.  Batches opened on it share its stream and weights: while any is
 * open the release is deferred to the last plamo_batch_close (the handle must not be used
 * after plamo_close either way). */
void plamo_close(plamo_runtime* rt);

/* Runtime.reset() (Runtime.swift:319); also clears the sampler history. */
void plamo_reset(plamo_runtime* rt);

/* Runtime.forward(_:output:) (Runtime.swift:321-467): 1..min(context,16) tokens at the
 * current position.  With output, `*next` receives the selected next token: the greedy
 * argmax, or Sampler.select when sampling controls are set (plamo_set_sampling).
 * Error "Invalid tokens or context exhausted" (Runtime.swift:330). */
int plamo_forward(plamo_runtime* rt, const int32_t* tokens, int32_t count, int32_t output,
                  int32_t* next, char* err, size_t errlen);

/* Runtime.forward(_:output:all:sequential:) (Runtime.swift:322-467).  `all`: every row's
 * logits (slots 0 .. count-1 of plamo_logits) and prediction (plamo_predictions);
 * `sequential`: each row takes the local RoPE coordinates of a scalar decode step
 * (Kernels.metal:288-298), so its outputs equal count single-token forwards; with `all`,
 * two rows and no sampling controls or QSA they run as one pass over the weights (the
 * reference's linear_pair pass, Runtime.swift:370-371).  Both need an MTP runtime and
 * count <= 2 (Runtime.verifyRows), else "Invalid tokens or context exhausted". */
int plamo_forward_ex(plamo_runtime* rt, const int32_t* tokens, int32_t count, int32_t output, int32_t all,
                     int32_t sequential, int32_t* next, char* err, size_t errlen);

/* Runtime.draft(_:) (Runtime.swift:485-520): the MTP head's one-token draft after `first`,
 * from the first output row's normalised hidden state and first's embedding.  Leaves the
 * position and the logits slots alone; the draft replaces the first prediction.  Error "MTP
 * requires a prefetched context and trained adapters". */
int plamo_draft(plamo_runtime* rt, int32_t first, int32_t* draft, char* err, size_t errlen);

/* Runtime.rewind(_:hiddenIndex:) (Runtime.swift:527-538): keeps output row `hidden_index` of
 * the last forward (logits, hidden state, prediction) and moves the position to
 * `new_position`, which must be position - rows + hidden_index + 1 ("Invalid verification
 * rollback"). */
int plamo_rewind(plamo_runtime* rt, int64_t new_position, int32_t hidden_index, char* err, size_t errlen);

/* Runtime.prefill(_:) (Runtime.swift:469-483): any prompt length up to the context.
 * Processed in large MFMA chunks with the reference's 16-token chunk RoPE coordinates.
 * Error "Input exceeds context" (Runtime.swift:474). */
int plamo_prefill(plamo_runtime* rt, const int32_t* tokens, int32_t count, int32_t* next,
                  char* err, size_t errlen);

/* Runtime.logits(into:slot:) (Runtime.swift:547-552): BF16 logits widened to 107520
 * floats.  `bf16` variant copies the raw bits (Runtime.logitValues bit patterns). */
int plamo_logits(plamo_runtime* rt, int32_t slot, float* values, char* err, size_t errlen);
int plamo_logits_bf16(plamo_runtime* rt, int32_t slot, uint16_t* bits, char* err, size_t errlen);

/* Final normalised hidden state of the last output row (Runtime.normalized, used by the
 * batch equivalence test BatchMapTests.swift:22-24). 1536 floats. */
int plamo_hidden(plamo_runtime* rt, float* values, char* err, size_t errlen);

/* Runtime.predictions() (Runtime.swift:522-525). */
int plamo_predictions(plamo_runtime* rt, int32_t* out, int32_t capacity, int32_t* count);

int plamo_get_stats(plamo_runtime* rt, plamo_stats* out);

/* Copies the ring/global KV of `layer` (BF16 bits, [capacity][128] each) to host memory.
 * Mirrors the layer.keys / layer.values buffers the reference tests read
 * (BatchMapTests.swift:25-29).  `capacity` receives the slot count. */
int plamo_kv(plamo_runtime* rt, int32_t layer, uint16_t* keys, uint16_t* values, int32_t* capacity,
             char* err, size_t errlen);

/* ---- On-GPU sampling controls (Sampler.swift:9-70, Main.swift:235-244) ------------- */

/* Enables Sampler.select semantics for every subsequent output: FP32 repetition penalty
 * (divide if positive else multiply), presence, frequency x count, no-repeat-n-gram ban,
 * then the first strict maximum with default 0.  All run on the GPU over the full
 * vocabulary.  penalty 1, presence 0, frequency 0, ngram <= 1 restores pure greedy. */
int plamo_set_sampling(plamo_runtime* rt, float repetition_penalty, float frequency_penalty,
                       float presence_penalty, int32_t no_repeat_ngram);
/* `generated.append(id)` of Main.swift:280: adds to the history the controls see
 * (generated tokens only, Main.swift:237-238).  Cleared by plamo_reset. */
int plamo_sampler_observe(plamo_runtime* rt, int32_t id);

/* The token loop of Main.swift:235-288 driven on the device: prefill `prompt`, then up to
 * `max_tokens` emitted tokens, stopping on token 1 or 16 (Main.swift:279).  Each decode
 * step is one replay of a captured hipGraph; the next token is fed back on the device.
 * `out_ids` (capacity max_tokens) receives the emitted tokens, `*stop_reason` 1 for
 * "stop", 0 for the length limit. */
int plamo_generate(plamo_runtime* rt, const int32_t* prompt, int32_t count, int32_t max_tokens,
                   int32_t* out_ids, int32_t* out_count, int32_t* stop_reason, char* err,
                   size_t errlen);

/* Device-timed decode microbenchmark: replays the captured decode step `steps` times
 * back to back (token fed back on the device) from the current state, returning the
 * average GPU milliseconds per step measured with HIP events on the handle's stream.
 * Leaves the runtime advanced by `steps` positions. */
int plamo_bench_decode(plamo_runtime* rt, int32_t steps, double* ms_per_step, char* err,
                       size_t errlen);

/* ---- Batch of up to four sequences (Batch.swift:4-187) ------------------------------ */

/* Batch(_ scalar:) (Batch.swift:33-78): shares the runtime's weights, owns 4 KV slices.
 * Requires context below 8192 ("Batch requires dense greedy inference with context below
 * 8192"). */
int plamo_batch_open(plamo_runtime* rt, plamo_batch** out, char* err, size_t errlen);
void plamo_batch_close(plamo_batch* b);

/* Batch.prefill (Batch.swift:80-107): `count` prompts (1..4) laid out back to back in
 * `tokens` with `lengths[i]` tokens each; `next[i]` receives each lane's prediction. */
int plamo_batch_prefill(plamo_batch* b, const int32_t* tokens, const int32_t* lengths, int32_t count,
                        int32_t* next, char* err, size_t errlen);

/* Batch.step (Batch.swift:109-180): tokens[i] < 0 marks an inactive lane (Swift nil).
 * All active lanes run in one decode step that reads every weight once.  `next` receives
 * predictions for every lane (Batch.predictions). */
int plamo_batch_step(plamo_batch* b, const int32_t* tokens, int32_t count, int32_t* next, char* err,
                     size_t errlen);
void plamo_batch_reset(plamo_batch* b);

/* Lane state read-back for the batch == scalar invariant (BatchMapTests.swift:21-31). */
int plamo_batch_logits_bf16(plamo_batch* b, int32_t lane, uint16_t* bits, char* err, size_t errlen);
int plamo_batch_hidden(plamo_batch* b, int32_t lane, float* values, char* err, size_t errlen);
int plamo_batch_kv(plamo_batch* b, int32_t lane, int32_t layer, uint16_t* keys, uint16_t* values,
                   int32_t* capacity, char* err, size_t errlen);
int plamo_batch_positions(plamo_batch* b, int32_t* out, int32_t capacity, int32_t* count);
/* Fills every lane's K and V of every layer with the BF16 pattern `bits`.  No API
 * counterpart: the reference's test writes its Metal buffers directly
 * (BatchMapTests.swift:15-18 fills them with 0xff bytes, NaN) to show unused KV is never read. */
int plamo_batch_fill_kv(plamo_batch* b, uint16_t bits);

/* Step timeline, for profiling the replayed decode graph (no counterpart in the reference,
 * whose ProfileTests.swift times kernels one dispatch at a time).  Libraries built with
 * `make timeline` (lib/libplamo_hip_timeline.so) record every decode-step kernel's
 * per-workgroup start and end in s_memrealtime ticks (100 MHz): `out` receives
 * PLAMO_TIMELINE_WORDS words, [tag][block][start, end], tag = layer * 8 + (0 qkv,
 * 1 attention, 2 attention merge, 3 o, 4 gate_up, 5 down), 200 LM head, 250 head merge,
 * 251 step begin, block < 1024; each launch rewrites its tag's slots, zero = not run.
 * `clear` zeroes the table after the copy.  The normal library returns PLAMO_EINVAL. */
#define PLAMO_TIMELINE_WORDS (256 * 1024 * 2)
int plamo_timeline(uint64_t* out, size_t words, int32_t clear, char* err, size_t errlen);

/* ---- Lane scheduler (BatchDecode.swift:8-47) --------------------------------------- */

/* step: receives `count` tokens (<0 = nil) and writes `count` predictions; returns 0 to
 * continue, non-zero to abort.  emit(lane, id), finish(lane, ids, n, reason) likewise. */
typedef int (*plamo_step_fn)(void* user, const int32_t* tokens, int32_t count, int32_t* next);
typedef int (*plamo_emit_fn)(void* user, int32_t lane, int32_t id);
typedef int (*plamo_finish_fn)(void* user, int32_t lane, const int32_t* ids, int32_t n, int32_t reason);

#define PLAMO_REASON_STOP 1
#define PLAMO_REASON_LENGTH 2

/* decodeBatch(_:limits:step:emit:finish:stopOnTruncation:) (BatchDecode.swift:8-37).
 * Pure host logic.  Outputs: `ids` is [count][ids_stride], `lengths[count]`,
 * `reasons[count]`; `*lanes` receives the number of lanes reported (last+1). */
int plamo_decode_batch(const int32_t* initial, const int32_t* limits, int32_t count, plamo_step_fn step,
                       plamo_emit_fn emit, plamo_finish_fn finish, void* user, int32_t stop_on_truncation,
                       int32_t* ids, int32_t ids_stride, int32_t* lengths, int32_t* reasons, int32_t* lanes,
                       char* err, size_t errlen);

/* Batch.generate (BatchDecode.swift:40-47): prefill + decodeBatch over the GPU batch. */
int plamo_batch_generate(plamo_batch* b, const int32_t* tokens, const int32_t* lengths, const int32_t* limits,
                         int32_t count, int32_t stop_on_truncation, int32_t* ids, int32_t ids_stride,
                         int32_t* out_lengths, int32_t* reasons, int32_t* lanes, char* err, size_t errlen);

/* decodeBatch(initial:limits:step: Batch.step, stopOnTruncation:) (BatchDecode.swift:8-37,
 * as Batch.generate calls it at BatchDecode.swift:44-46) after plamo_batch_prefill: the lane
 * pass and the token feedback run on the device, 16 steps per host synchronisation.
 * `initial[count]` are the lanes' first predictions (count = the prefilled lanes).  Outputs
 * as plamo_decode_batch; lane positions and predictions advance as with plamo_batch_step. */
int plamo_batch_decode(plamo_batch* b, const int32_t* initial, const int32_t* limits, int32_t count,
                       int32_t stop_on_truncation, int32_t* ids, int32_t ids_stride, int32_t* lengths,
                       int32_t* reasons, int32_t* lanes, char* err, size_t errlen);

/* ---- Weight formats (Runtime.swift:23-111, Packed.swift, scripts/pack_weights.py) ---- */

typedef struct plamo_pack_report {
    int64_t original_linear_bytes; /* pack_weights.py:140 */
    int64_t packed_linear_bytes;
    int64_t archive_bytes;
    int64_t compressed_blocks;
    int64_t blocks;
} plamo_pack_report;

/* scripts/pack_weights.py main (pack_weights.py:89-142): writes `output` (.p12) from a
 * BF16 safetensors file, skipping the input embedding; every block is verified to
 * round-trip bit-exactly.  Written atomically (.part + rename). */
int plamo_pack(const char* safetensors, const char* output, const char* source_sha256,
               plamo_pack_report* report, char* err, size_t errlen);

/* pack_weights.py pack()/tag() (pack_weights.py:19-50,71-74) on one in-memory BF16 tensor of
 * `count` values (count % 128 == 0): writes the payload (capacity `payload_cap` bytes; at most
 * count*2) and count/128 tagged table entries; `*payload_bytes` receives the payload size. */
int plamo_pack_tensor(const uint16_t* values, int64_t count, uint8_t* payload, int64_t payload_cap,
                      uint32_t* table, int64_t* payload_bytes, char* err, size_t errlen);

/* Auxiliary.init + tensor checks (Auxiliary.swift:14-62) on auxiliary.safetensors without a
 * device: the archive, then the MTP head (`mtp`) and the global layers' QSA indexers (`qsa`);
 * the reference's messages ("Trained adapters missing; ...", "Invalid adapter size", "Invalid
 * adapter header", "Incompatible trained adapters", "Invalid adapter tensor: NAME"). */
int plamo_check_aux(const char* path, const char* teacher_sha256, int32_t mtp, int32_t qsa, char* err,
                    size_t errlen);
/* Weights(path:).tensor(name, shape) validation (Runtime.swift:33-101) without a device. */
int plamo_check_weights(const char* path, const char* name, const int64_t* shape, int32_t ndim, char* err,
                        size_t errlen);

/* Packed(path:).tensor(name, shape) validation (Packed.swift:12-91) without a device;
 * `*is_packed` = 1 for a 2-D block-table tensor. */
int plamo_check_packed(const char* path, const char* source_sha256, const char* name, const int64_t* shape,
                       int32_t ndim, int32_t* is_packed, char* err, size_t errlen);

/* ---- Kernel-level entry points (Metal kernel dispatch ABI, Kernels.metal) ----------
 * Device pointers are passed as plain addresses; `stream` is a hipStream_t (NULL =
 * default stream).  Used by the kernel parity tests and the GEMV microbenchmark. */

/* `linear` (Kernels.metal:92-114) / `project{2,3,4}` (Batch.metal:171-221): y = W.x for
 * `rows` activation rows.  `table` != 0 selects the .p12 decode (`w` = payload).  mode 0:
 * y FP32 roundbf; mode 1: y the FP32 sums unrounded; mode 2: y BF16 bits (LM head).
 * n in {1536, 2048, 6144}. */
int plamo_kernel_linear(uint64_t w, uint64_t table, uint64_t x, uint64_t y, int32_t n, int32_t m, int32_t rows,
                        int32_t mode, uint64_t stream);

/* `packed_bits` decode of `count` consecutive weights (Kernels.metal:23-44) into BF16 bits
 * (PackedDecodeTests.swift:34-42). */
int plamo_kernel_unpack(uint64_t payload, uint64_t table, uint64_t out, int64_t count, uint64_t stream);

/* `argmax` (Kernels.metal:704-729): rows x n logits, FP32 (bf16 == 0) or BF16 bits. */
int plamo_kernel_argmax(uint64_t x, uint64_t out, int32_t n, int32_t rows, int32_t bf16, uint64_t stream);

/* `Sampler.select` on the GPU over FP32 logits (modified in place, like the Swift API):
 * history of `hist` int32 ids; result written to `out` (device int32). */
int plamo_kernel_select(uint64_t logits, int32_t n, uint64_t history, int32_t hist, float penalty,
                        int32_t ngram, float frequency, float presence, uint64_t out, uint64_t stream);

/* `qsa_select` (Kernels.metal:618-682, QSATests.swift:6-46): for query rows t = 0 .. tokens-1 at
 * positions start + t, the min(complete, budget / 4) blocks of largest max(score, 0) among the
 * complete = (start + t + 1) / 4 blocks, ties to the lower index (every block when the budget
 * covers them).  scores: FP32 [tokens][blocks]; out: uint32 [tokens][(blocks + 31) / 32], bit
 * b of word b / 32 set for a chosen block (the reference lists the chosen keys instead; the
 * keys of the unfinished block are always attended).  blocks <= 8192. */
int plamo_kernel_qsa_select(uint64_t scores, int32_t blocks, int32_t tokens, int32_t start, int32_t budget,
                            uint64_t out, uint64_t stream);

/* MFMA BF16 GEMM of the prefill path: Y[t][m] = sum_k X[t][k] W[m][k] with X BF16
 * [tokens][n] and W plain BF16 or .p12 ([m][n]).  out_mode 0: Y FP32 BF16-rounded
 * (`matrix` full == 0); 1: Y BF16 bits (full == 2); 2: Y raw FP32 (full == 1,
 * Kernels.metal:196-197); 3: the gate_up projection (m = 12288, n = 1536) followed by
 * `swiglu` (Kernels.metal:202-210), Y BF16 bits [tokens][6144]. */
int plamo_kernel_gemm(uint64_t w, uint64_t table, uint64_t x, uint64_t y, int32_t n, int32_t m, int32_t tokens,
                      int32_t out_mode, uint64_t stream);

/* Prefill attention of `tokens` queries at positions p0.. (Runtime.swift:389-444 with the
 * `matrix_rotary`/`softmax`/`attend` dispatches, Kernels.metal:276-437) as MFMA flash
 * attention.  q16: BF16 [tokens][16][128] normalised, rotated queries; keys/values: BF16
 * [capacity][128] with position p in slot p % capacity (keys of global layers rotated at
 * their position, local keys unrotated); full != 0: causal over all keys, else the
 * 2048-key window with keys rotated at key_pos - base of each 16-token chunk
 * (local_rope: [2064][64] uint32 = BF16 cos | sin << 16).  out16: BF16 [tokens][2048]. */
int plamo_kernel_attention_prefill(uint64_t q16, uint64_t keys, uint64_t values, int32_t capacity, int32_t p0,
                                   int32_t tokens, int32_t full, uint64_t local_rope, uint64_t out16,
                                   uint64_t stream);

/* Decode attention of `rows` (1..4) one-token rows: the `qkv` (Kernels.metal:223-259) and
 * attention dispatches of Runtime.swift:389-444 for a one-token chunk, i.e. q/k RMSNorm (+1
 * gains `q_norm`, `k_norm`: BF16 [128]), RoPE, the new key and value written to slot
 * pos % capacity, then split-K attention over the visible keys (`matrix_rotary`, `softmax`,
 * `attend`, or `attention` + `attention_merge`, Kernels.metal:301-562) with the partitions
 * merged on the device.  qkv: FP32 [rows][2304] (BF16-valued); keys/values: BF16
 * [rows][capacity][128], row q using slice q, position p in slot p % capacity (global keys
 * stored rotated, local keys normalised and unrotated); positions: host int32 [rows];
 * full != 0: keys 0..pos (global layer, pos < capacity, global_rope holds capacity rows of
 * [64] uint32 BF16 cos | sin << 16), else the 2048-key window ending at pos, keys rotated
 * with coordinate key_pos - max(0, pos - 2047) (local_rope: [2064][64]); out16: BF16
 * [rows][2048].  Uses a per-device workspace the library grows on demand. */
int plamo_kernel_attention_decode(uint64_t qkv, uint64_t q_norm, uint64_t k_norm, uint64_t keys, uint64_t values,
                                  int32_t capacity, const int32_t* positions, int32_t rows, int32_t full,
                                  uint64_t local_rope, uint64_t global_rope, uint64_t out16, uint64_t stream);

/* plamo_kernel_attention_decode without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same kernels and results;
 * the step state, tickets and partition buffers live in a static device array of
 * 4,260,352 bytes per GPU (held until the process ends), which limits every row to 8192
 * visible keys (global layers: pos < 8192): larger calls fail with PLAMO_EINVAL.  All calls
 * on one GPU share that array and every call rewrites the state and clears the tickets it
 * uses, so calls that overlap on one GPU (several streams or threads) race: serialise them.
 * The caller passes every input and output, as for plamo_kernel_attention_decode. */
int plamo_kernel_attention_decode_static(uint64_t qkv, uint64_t q_norm, uint64_t k_norm, uint64_t keys,
                                         uint64_t values, int32_t capacity, const int32_t* positions, int32_t rows,
                                         int32_t full, uint64_t local_rope, uint64_t global_rope, uint64_t out16,
                                         uint64_t stream, char* err, size_t errlen);

/* The host RoPE table builder the runtime uploads (`init_rope`, Kernels.metal:212-219; global
 * factors of `rotated`, Kernels.metal:264-267): `rows` x 64 entries of BF16 cos | sin << 16
 * from 64 inverse frequencies (config-mlx.json plamo_rope_inv_freq, Runtime.swift:268-274).
 * Host only; exposed so the tables can be compared with the CPU restatement bit for bit. */
int plamo_rope_table(const double* freqs, int32_t rows, int32_t global, uint32_t* out, char* err, size_t errlen);

/* Library build identification (gfx arch, HIP version). */
const char* plamo_version(void);

/* ---- Text side: the PLaMo tokenizer (Tokenizer.swift:11-282) -------------------- */
/* Host-only (no GPU work).  Byte outputs are raw UTF-8: when `cap` is too small the call
 * fails with PLAMO_EINVAL and `*n_out` holds the size needed. */
typedef struct plamo_tokenizer plamo_tokenizer;
typedef struct plamo_token_stream plamo_token_stream;

/* Tokenizer.init(path:) reading tokenizer.jsonl (Tokenizer.swift:59-131): lines
 * [piece, score, kind]; BYTE pieces "<0xNN>"; scores scaled by 1e4 and rounded half to
 * even.  Errors "Invalid byte token", "Invalid tokenizer score", "Expected the PLaMo 3
 * Translate 0.8B vocabulary" (Tokenizer.swift:90-118).  The reference's .trie cache
 * (Tokenizer.swift:45-57) is pinned to the original vocabulary's SHA-256 and is not read. */
int plamo_tokenizer_open(const char* path, plamo_tokenizer** out, char* err, size_t errlen);
void plamo_tokenizer_close(plamo_tokenizer* t);

/* Tokenizer.encode(_:bos:) (Tokenizer.swift:144-190): `text` is UTF-8 (invalid UTF-8 is
 * PLAMO_EINVAL "Invalid UTF-8 text"). */
int plamo_tokenizer_encode(const plamo_tokenizer* t, const char* text, size_t len, int32_t bos, int32_t* ids,
                           size_t cap, size_t* n_out, char* err, size_t errlen);

/* Tokenizer.decode(_:) as bytes (Tokenizer.swift:203-232); error "Token ID out of range". */
int plamo_tokenizer_decode(const plamo_tokenizer* t, const int32_t* ids, size_t count, char* out, size_t cap,
                           size_t* n_out, char* err, size_t errlen);

/* Tokenizer.Stream (Tokenizer.swift:236-269): push returns the complete UTF-8 prefix of
 * everything pushed so far, holding back an unfinished trailing sequence; finish returns
 * the rest.  The stream keeps a pointer to its tokenizer, which must outlive it. */
int plamo_token_stream_open(const plamo_tokenizer* t, plamo_token_stream** out, char* err, size_t errlen);
int plamo_token_stream_push(plamo_token_stream* s, int32_t id, char* out, size_t cap, size_t* n_out, char* err,
                            size_t errlen);
int plamo_token_stream_finish(plamo_token_stream* s, char* out, size_t cap, size_t* n_out, char* err, size_t errlen);
void plamo_token_stream_close(plamo_token_stream* s);

/* OrderedOutput (OrderedOutput.swift:24-67): up to four documents' tokens, emitted in
 * document order through `emit` (repaired UTF-8 chunks; a nonzero return cancels: the
 * calling append/finish fails with PLAMO_ESTATE "Cancelled").  The first prefix is emitted by
 * open.  Errors "Expected one to four output prefixes", "Output after document finish",
 * "Invalid document finish"; `reason` is "stop" or "length" (BatchDecode.swift:3-6). */
typedef struct plamo_ordered plamo_ordered;
typedef int (*plamo_text_fn)(void* user, const char* text, size_t len);
int plamo_ordered_open(const plamo_tokenizer* t, const char* const* prefixes, const size_t* prefix_lens,
                       int32_t count, const char* tail, size_t tail_len, plamo_text_fn emit, void* user,
                       plamo_ordered** out, char* err, size_t errlen);
int plamo_ordered_append(plamo_ordered* o, int32_t lane, int32_t id, char* err, size_t errlen);
int plamo_ordered_finish(plamo_ordered* o, int32_t lane, const char* reason, char* err, size_t errlen);
void plamo_ordered_close(plamo_ordered* o);

/* DocumentPlan (OrderedOutput.swift:3-21) of `count` segments (Segments.swift:4-7): segment i
 * is `texts[i]` (`text_lens[i]` UTF-8 bytes) with `tokens[i]` (`token_counts[i]` prompt ids;
 * none: a whitespace run kept verbatim).  Document d has input tokens and a prefix (the
 * whitespace since the previous document, or "\n" between adjacent documents); prefix index
 * `documents` is the tail.  Error "No documents to translate". */
typedef struct plamo_plan plamo_plan;
int plamo_document_plan(const char* const* texts, const size_t* text_lens, const int32_t* const* tokens,
                        const int32_t* token_counts, int32_t count, plamo_plan** out, char* err, size_t errlen);
int32_t plamo_plan_documents(const plamo_plan* p);
int plamo_plan_input(const plamo_plan* p, int32_t document, const int32_t** tokens, int32_t* count);
int plamo_plan_prefix(const plamo_plan* p, int32_t document, const char** text, size_t* len);
void plamo_plan_close(plamo_plan* p);

/* DocumentOutput (OrderedOutput.swift:69-76). */
typedef struct plamo_document_output {
    int32_t sequences;               /* documents reported in ids / lengths / reasons */
    double gpu_seconds;              /* Batch.gpuSeconds summed over the groups */
    int64_t discarded_tokens;        /* emitted by lanes past a truncation, not reported */
    int64_t prefilled_input_tokens;
    double prefill_seconds, decode_seconds;
} plamo_document_output;

/* Batch.translateOrdered (OrderedOutput.swift:79-115): the DocumentPlan of the segments,
 * then groups of up to four documents: Batch.prefill, decodeBatch with Batch.step and
 * stopOnTruncation, every token streamed through an OrderedOutput in document order
 * (`emit` as for plamo_ordered_open; the last group also emits the tail); a group whose
 * last reported lane did not stop ends the document.  Errors "No documents to translate",
 * "Invalid document tokens or context budget" (limit 0..8191, every input + limit within
 * the context, ids below 107520); on any error the batch is reset.  Outputs: `ids`
 * [documents][ids_stride], `lengths`, `reasons` (PLAMO_REASON_*) of the reported documents. */
int plamo_batch_translate_ordered(plamo_batch* b, const plamo_tokenizer* t, const char* const* texts,
                                  const size_t* text_lens, const int32_t* const* tokens, const int32_t* token_counts,
                                  int32_t count, int32_t limit, plamo_text_fn emit, void* user, int32_t* ids,
                                  int32_t ids_stride, int32_t* lengths, int32_t* reasons, plamo_document_output* out,
                                  char* err, size_t errlen);

/* Tokenizer.prompt(_:target:) (Tokenizer.swift:272-281): errors "Unsupported target
 * language", "Source must be nonempty and contain no reserved PLaMo delimiters". */
int plamo_translation_prompt(const char* text, size_t len, const char* target, char* out, size_t cap,
                             size_t* n_out, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif
