// Host runtime: the MI355X counterparts of Runtime, Batch and Weights
// (Sources/Plamo/Runtime.swift:128-553, Batch.swift:4-187).
#pragma once

#include <hip/hip_runtime.h>

#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "formats.h"
#include "kernels.h"
#include "prefill.h"

namespace plamo {

// Device memory owned by one object; freed together.
class DeviceArena {
  public:
    ~DeviceArena();
    void* alloc(size_t bytes);
    template <class T>
    T* alloc_n(size_t n) { return static_cast<T*>(alloc(n * sizeof(T))); }
    size_t bytes() const { return bytes_; }

  private:
    std::vector<void*> ptrs_;
    size_t bytes_ = 0;
};

struct Linear {
    const uint16_t* w = nullptr;    // plain BF16 rows or .p12 payload
    const uint32_t* table = nullptr;
    int64_t bytes = 0;              // bytes a full GEMV pass reads (payload + table)
};

struct LayerWeights {
    Linear qkv, o, up, down;
    const uint16_t *pre = nullptr, *post = nullptr, *pre_mlp = nullptr, *post_mlp = nullptr;
    const uint16_t *q_norm = nullptr, *k_norm = nullptr;
};

// Weights in HBM plus the RoPE tables; shared by a Runtime and its Batch.
struct Model {
    bool packed = false;
    LayerWeights layers[LAYERS];
    Linear head;
    const uint16_t* final_norm = nullptr;
    const uint16_t* embed = nullptr;
    uint32_t* local_rope = nullptr;   // [2064][64] BF16 cos | sin << 16
    uint32_t* global_rope = nullptr;  // [context][64]
    int64_t weight_bytes = 0, linear_bytes = 0;
    DeviceArena arena;
};

// Trained adapters in HBM (Auxiliary.swift:5-111): the MTP head (Predictor) and, on the
// global layers, the QSA block indexers (Indexer), plus the draft and verification scratch.
struct Aux {
    const uint16_t* mtp_up = nullptr;    // [256][3072]
    const uint16_t* mtp_down = nullptr;  // [1536][256]
    const uint16_t* qsa_proj[LAYERS] = {};    // [640][1536] (global layers)
    const uint16_t* qsa_q_norm[LAYERS] = {};  // [128]
    const uint16_t* qsa_k_norm[LAYERS] = {};
    int64_t bytes = 0;                   // adapter bytes in HBM (auxiliary_weight_bytes)
    // draft: input [hidden | embedding], up projection, adapter output, its logits
    float *mtp_in = nullptr, *mtp_up_out = nullptr, *mtp_hidden = nullptr;
    uint16_t* mtp_logits = nullptr;
    // rows of the last verification pass (forward with all): logits, hidden, prediction
    uint16_t* slot_logits = nullptr;     // [VERIFY_ROWS][VOCAB]
    float* slot_hidden = nullptr;        // [VERIFY_ROWS][HIDDEN]
    int32_t* slot_next = nullptr;        // [VERIFY_ROWS]
    DeviceArena arena;
};

// Predictor/Indexer tensors of a validated archive (Runtime.swift:174-176,248) in HBM: `mtp`
// the MTP head, `qsa` the indexers of the global layers.
std::unique_ptr<Aux> load_aux(const AuxArchive& archive, bool mtp, bool qsa);
// Names and shapes the runtime reads from auxiliary.safetensors (Auxiliary.swift:72-111).
void check_aux_tensors(const AuxArchive& archive, bool mtp, bool qsa);

// KV, scratch, step state and the captured decode graph for `lanes` sequences.
class Engine {
  public:
    Engine(std::shared_ptr<Model> model, int context, int lanes, hipStream_t stream);
    ~Engine();

    std::shared_ptr<Model> model;
    int context, lanes, chunk, local_capacity;
    hipStream_t stream;
    DeviceArena arena;
    uint16_t *keys[LAYERS], *values[LAYERS];
    // Local layers: every lane's keys rotated at their own position for positions below
    // rot_rows[l] = min(capacity, 2048), where a row's window starts at 0 and the rotation
    // coordinate of a key is its position; decode attention reads them instead of rotating.
    uint16_t* keys_rot[LAYERS];
    int rot_rows[LAYERS];
    int capacity[LAYERS];
    // decode scratch (ROWS rows)
    float *qkv, *hidden;
    uint16_t* resid_scratch;
    uint16_t *proj, *x0, *x1;  // BF16 projection output and residual stream (BF16-exact values)
    uint16_t *att, *act;  // BF16 attention output and SwiGLU activations
    uint16_t* logits;
    StepState* state;        // device
    StepState* host_state;   // pinned mirror
    DecodeBuffers bufs;
    float *part_m, *part_l, *part_o;
    uint32_t* attn_tickets;
    uint32_t decode_parts_local, decode_parts_global;
    // prefill scratch (chunk rows)
    uint16_t *p_x, *p_qkv, *p_proj;  // BF16: every value is BF16-rounded
    uint16_t *p_xn, *p_att, *p_act, *p_q16;
    float *p_flash_o, *p_flash_ml;  // split flash prefill workspace
    uint32_t* p_flash_tickets;
    // .p12 models: one projection's weights expanded to BF16 rows for the prefill GEMMs
    // (the largest, gate_up: 37.7 MB), rewritten before each GEMM of a chunk
    uint16_t* p_wexp = nullptr;
    int32_t* p_tokens;
    size_t part_rows_cap;    // rows x parts the partial buffers hold
    // graph
    hipGraphExec_t graph = nullptr;       // one host step (bookkeeping kernel first)
    hipGraphExec_t graph_loop = nullptr;  // one device-loop step (bookkeeping in its head merge)
    hipGraphExec_t graph16 = nullptr;     // LOOP_GRAPH_STEPS consecutive device-loop steps
    hipGraphExec_t graph_verify = nullptr;  // the two-row verification step
    bool use_graph = true;

    hipEvent_t ev0, ev1;

    // QSA block indexers of the global layers (Runtime.swift:380-418); null: dense attention
    const Aux* qsa_aux = nullptr;
    int qsa_budget = 0;
    uint16_t *qsa_proj = nullptr, *qsa_q = nullptr;  // [chunk][640], [chunk][512] BF16
    uint16_t* qsa_raw[LAYERS] = {};                   // global layers: [context][128] raw keys
    uint16_t* qsa_pooled[LAYERS] = {};                // global layers: [context / 4][128] block keys
    float* qsa_scores = nullptr;                      // [chunk][context / 4]
    uint32_t* qsa_mask = nullptr;                     // [chunk][words] selected blocks
    uint32_t qsa_blocks = 0, qsa_words = 0;
    void enable_qsa(const Aux* aux, int budget);
    QsaParams qsa_params(int layer, int tokens, const StepState* st, uint32_t p0) const;

    // one decode step for state->rows rows; `loop`: a device-loop step (no bookkeeping kernel,
    // the head merge prepares the next step)
    // verify: the two verification rows of one sequence (StepState::kv_shared) through the
    // multi-row kernels, each row's attention launched after the previous row's
    void enqueue_step(bool head = true, bool loop = false, bool verify = false);
    void run_step();
    void run_verify();  // enqueue_step(true, false, true), replayed from a captured graph                        // host step: graph replay (or direct launches)
    // Device loops: begin_loop once (the first step's bookkeeping), then n steps as replays of
    // a LOOP_GRAPH_STEPS-step graph and single-step graphs (one launch per 16 steps)
    static constexpr int LOOP_GRAPH_STEPS = 16;
    void begin_loop();
    void run_steps(int n);
    void prepare_loop_graph();
    // prefill of `n` tokens of one lane at position p0 (n > 1); head on the last token.
    void prefill(const int32_t* tokens, int n, int p0, int lane, bool output);
    // after a prefill without output: the head of each of its first n rows, row i's logits,
    // final hidden row and prediction copied to slot i (the engine keeps row n - 1's)
    void prefill_heads(int n, uint16_t* slot_logits, float* slot_hidden, int32_t* slot_next);
    void zero_sampler();

  private:
    void enqueue_prefill_chunk(int n, int p0, int lane, bool last_chunk, bool output);
    void enqueue_head(const uint16_t* in, const uint16_t* resid_in, int in_rows);  // prefill rows
    void enqueue_head16(bool loop, int maxr);                                 // decode: BF16 stream
    void capture_loop(int steps, hipGraphExec_t* out);
};

// RoPE table of `rows` positions, one uint32 per (position, pair): BF16 cos | sin << 16.
std::vector<uint32_t> rope_table(const std::vector<double>& freqs, int rows, bool global);

std::shared_ptr<Model> load_model(const std::string& dir, int context, bool packed, const std::string& sha,
                                  hipStream_t stream);

struct RuntimeImpl {
    std::shared_ptr<Model> model;
    std::unique_ptr<Engine> eng;
    hipStream_t stream = nullptr;
    int context = 0;
    int64_t position = 0;
    int last_output_rows = 0;
    double gpu_seconds = 0;
    double last_prefill_seconds = 0, last_decode_seconds = 0;  // phases of the last generate
    std::vector<int32_t> predictions;
    // sampler
    bool sampling = false;
    float penalty = 1, frequency = 0, presence = 0;
    int ngram = 0;
    std::vector<int32_t> history;   // generated ids (Main.swift:236-238)
    size_t uploaded = 0;            // history entries already on the device
    bool counts_dirty = true;

    // trained adapters (Runtime.swift:170-176): MTP draft, QSA budget (0: dense attention)
    std::unique_ptr<Aux> aux;
    bool mtp = false;
    int qsa_budget = 0;
    int64_t sparse_queries = 0, sparse_keys = 0, dense_keys = 0;  // Runtime.swift:160-162
    // the QSA counters of one reference forward of n tokens at p0 (Runtime.swift:405-414)
    void count_qsa(int64_t p0, int n);

    ~RuntimeImpl();
    void reset();
    int forward(const int32_t* tokens, int n, bool output);
    // Runtime.forward(_:output:all:sequential:) (Runtime.swift:322-467): `all` outputs every
    // row (at most VERIFY_ROWS, MTP only); `sequential` gives each row the local RoPE
    // coordinates of a scalar decode step (rotate_steps, Kernels.metal:288-298)
    int forward_ex(const int32_t* tokens, int n, bool output, bool all, bool sequential);
    int draft(int first);                                   // Runtime.draft (Runtime.swift:485-520)
    void rewind(int64_t new_position, int hidden_index);    // Runtime.rewind (Runtime.swift:527-538)
    const uint16_t* logits_row(int slot) const;             // device logits of output row `slot`
    const float* hidden_row() const;                        // device final hidden of the last row
    int prefill(const int32_t* tokens, int n);
    void begin_timing();
    void end_timing();
    void sync_sampler(Engine& e, int row);
    std::vector<int32_t> generate(const int32_t* prompt, int n, int max_tokens, int* reason);
    double bench_decode(int steps);
};

struct BatchImpl {
    RuntimeImpl* rt;
    std::unique_ptr<Engine> eng;
    std::vector<int64_t> positions;
    bool ready = false;
    double gpu_seconds = 0;
    uint16_t* lane_logits;   // [4][VOCAB] (the engine's head output, indexed by lane)
    float* lane_hidden;      // [4][1536]
    int32_t lane_next[ROWS];

    explicit BatchImpl(RuntimeImpl* rt);
    ~BatchImpl();
    std::vector<int32_t> prefill(const std::vector<std::vector<int32_t>>& prompts);
    std::vector<int32_t> step(const std::vector<int32_t>& tokens);
    struct Decoded {
        std::vector<std::vector<int32_t>> ids;  // emitted tokens of lanes 0..last
        std::vector<int> reasons;               // 1 stop token, 2 length
    };
    Decoded decode(const std::vector<int32_t>& first, const std::vector<int32_t>& limits, bool stop_on_truncation);
    void reset();
};

}  // namespace plamo
