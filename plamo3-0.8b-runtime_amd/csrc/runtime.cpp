// Host runtime: model upload, KV management, decode step graph, prefill, batch lanes.
#include "runtime.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <fstream>
#include <sstream>

#include "formats.h"
#include "json.h"

namespace plamo {

// ------------------------------------------------------------------------------ arena
DeviceArena::~DeviceArena() {
    for (void* p : ptrs_) (void)hipFree(p);
}

void* DeviceArena::alloc(size_t bytes) {
    void* p = nullptr;
    const size_t n = std::max<size_t>(256, (bytes + 255) / 256 * 256);
    PLAMO_HIP(hipMalloc(&p, n));
    ptrs_.push_back(p);
    bytes_ += n;
    return p;
}

// ------------------------------------------------------------------------- model load
namespace {
std::string read_text(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error(E_IO, "Cannot read " + path);
    std::stringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

// Runtime.swift:180-190
void validate_config(const std::string& dir) {
    const std::string msg = "Only the original BF16 PLaMo 3 Translate 0.8B configuration is supported";
    json::Value c;
    try {
        c = json::parse(read_text(dir + "/config.json"));
    } catch (const Error&) {
        throw;
    } catch (const std::exception&) {
        throw Error(E_FORMAT, msg);
    }
    const std::pair<const char*, int64_t> ints[] = {
        {"hidden_size", 1536}, {"num_hidden_layers", 16}, {"num_attention_heads", 16}, {"num_key_value_heads", 1},
        {"head_dim", 128}, {"intermediate_size", 6144}, {"vocab_size", 107520}, {"window_size", 2048},
        {"sliding_window_pattern", 8}};
    for (auto& kv : ints) {
        const json::Value* v = c.get(kv.first);
        if (!v || v->kind != json::Value::Number || v->num != double(kv.second)) throw Error(E_FORMAT, msg);
    }
    auto is_false = [&](const char* k) {
        const json::Value* v = c.get(k);
        return v && v->kind == json::Value::Bool && !v->b;
    };
    auto is_str = [&](const char* k, const char* s) {
        const json::Value* v = c.get(k);
        return v && v->kind == json::Value::String && v->str == s;
    };
    auto is_num = [&](const char* k, double d) {
        const json::Value* v = c.get(k);
        return v && v->kind == json::Value::Number && v->num == d;
    };
    if (!is_false("tie_word_embeddings") || !is_false("scale_embedding") || !is_str("model_type", "plamo3") ||
        !is_str("dtype", "bfloat16") || !is_num("rope_theta", 1000000.0) || !is_num("rope_local_theta", 10000.0) ||
        !is_num("rope_scaling_factor", 256.0) || !is_num("rms_norm_eps", 1e-6))
        throw Error(E_FORMAT, msg);
}

// config-mlx.json plamo_rope_inv_freq (Runtime.swift:268-274)
void read_frequencies(const std::string& dir, std::vector<double>& local, std::vector<double>& full) {
    const std::string msg = "Missing source-exact RoPE frequencies in config-mlx.json";
    json::Value c;
    try {
        c = json::parse(read_text(dir + "/config-mlx.json"));
    } catch (const std::exception&) {
        throw Error(E_FORMAT, msg);
    }
    const json::Value* f = c.get("plamo_rope_inv_freq");
    const json::Value* l = f ? f->get("local") : nullptr;
    const json::Value* g = f ? f->get("full") : nullptr;
    if (!l || !g || l->kind != json::Value::Array || g->kind != json::Value::Array || l->arr.size() != 64 ||
        g->arr.size() != 64)
        throw Error(E_FORMAT, msg);
    for (int i = 0; i < 64; ++i) {
        if (l->arr[i].kind != json::Value::Number || g->arr[i].kind != json::Value::Number) throw Error(E_FORMAT, msg);
        const double a = l->arr[i].num, b = g->arr[i].num;
        if (!std::isfinite(a) || !std::isfinite(b) || a <= 0 || b <= 0) throw Error(E_FORMAT, msg);
        local.push_back(a);
        full.push_back(b);
    }
}

}  // namespace

// Local table: (bits(cos), bits(sin)) of float(pos)*f (Kernels.metal:212-219).  Global
// factors: roundbf(roundbf(cos(angle))*1.5545177444479562f) (Kernels.metal:264-267).  cos
// and sin of the FP32 angle are evaluated in double precision and rounded to FP32.
std::vector<uint32_t> rope_table(const std::vector<double>& freqs, int rows, bool global) {
    std::vector<uint32_t> t(size_t(rows) * 64);
    const float mscale = 1.5545177444479562f;
    for (int p = 0; p < rows; ++p)
        for (int d = 0; d < 64; ++d) {
            const float angle = float(p) * float(freqs[d]);
            float c = host_bf(host_bits(float(std::cos(double(angle)))));
            float s = host_bf(host_bits(float(std::sin(double(angle)))));
            if (global) {
                c = host_bf(host_bits(c * mscale));
                s = host_bf(host_bits(s * mscale));
            }
            t[size_t(p) * 64 + d] = uint32_t(host_bits(c)) | (uint32_t(host_bits(s)) << 16);
        }
    return t;
}

namespace {
template <class T>
T* upload(DeviceArena& a, const void* src, size_t bytes) {
    T* p = static_cast<T*>(a.alloc(bytes));
    PLAMO_HIP(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice));
    return p;
}
}  // namespace

std::shared_ptr<Model> load_model(const std::string& dir, int context, bool packed, const std::string& sha,
                                  hipStream_t) {
    validate_config(dir);
    SafeTensors st(dir + "/model.safetensors");
    std::unique_ptr<PackedArchive> pk;
    if (packed) pk = std::make_unique<PackedArchive>(dir + "/model.p12", sha);
    std::vector<double> flocal, ffull;
    // Tensor validation in the order of Runtime.swift:233-250 before any device work.
    struct Req { std::string name; std::vector<int64_t> shape; };
    std::vector<Req> reqs = {{"lm_head.weight", {VOCAB, HIDDEN}}, {"model.norm.weight", {HIDDEN}}};
    for (int i = 0; i < LAYERS; ++i) {
        const std::string p = "model.layers.layers." + std::to_string(i) + ".";
        reqs.push_back({p + "pre_mixer_norm.weight", {HIDDEN}});
        reqs.push_back({p + "post_mixer_norm.weight", {HIDDEN}});
        reqs.push_back({p + "pre_mlp_norm.weight", {HIDDEN}});
        reqs.push_back({p + "post_mlp_norm.weight", {HIDDEN}});
        reqs.push_back({p + "mixer.qkv_proj.weight", {QKV, HIDDEN}});
        reqs.push_back({p + "mixer.o_proj.weight", {HIDDEN, ATTN}});
        reqs.push_back({p + "mixer.q_norm.weight", {HEAD_DIM}});
        reqs.push_back({p + "mixer.k_norm.weight", {HEAD_DIM}});
        reqs.push_back({p + "mlp.gate_up_proj.weight", {2 * INTER, HIDDEN}});
        reqs.push_back({p + "mlp.down_proj.weight", {HIDDEN, INTER}});
    }
    std::vector<TensorView> views;
    std::vector<PackedTensor> ptens;
    for (auto& r : reqs) {
        views.push_back(st.tensor(r.name, r.shape));
        if (pk) ptens.push_back(pk->tensor(r.name, r.shape));
    }
    read_frequencies(dir, flocal, ffull);

    auto m = std::make_shared<Model>();
    m->packed = packed;
    DeviceArena& a = m->arena;
    const uint8_t* payload = nullptr;
    if (pk) payload = upload<uint8_t>(a, pk->payload(), pk->payload_bytes());
    size_t idx = 0;
    auto linear = [&](int64_t rows, int64_t cols) {
        Linear L;
        if (pk) {
            const PackedTensor& t = ptens[idx];
            L.w = reinterpret_cast<const uint16_t*>(payload + t.data_offset);
            L.table = reinterpret_cast<const uint32_t*>(payload + t.table_offset);
            L.bytes = int64_t(t.data_bytes + t.blocks * 4);
        } else {
            L.w = upload<uint16_t>(a, views[idx].data, views[idx].bytes);
            L.bytes = rows * cols * 2;
        }
        ++idx;
        m->linear_bytes += L.bytes;
        return L;
    };
    auto vec = [&]() {
        const uint16_t* p;
        if (pk) p = reinterpret_cast<const uint16_t*>(payload + ptens[idx].data_offset);
        else p = upload<uint16_t>(a, views[idx].data, views[idx].bytes);
        ++idx;
        return p;
    };
    m->head = linear(VOCAB, HIDDEN);
    m->final_norm = vec();
    for (int i = 0; i < LAYERS; ++i) {
        LayerWeights& L = m->layers[i];
        L.pre = vec();
        L.post = vec();
        L.pre_mlp = vec();
        L.post_mlp = vec();
        L.qkv = linear(QKV, HIDDEN);
        L.o = linear(HIDDEN, ATTN);
        L.q_norm = vec();
        L.k_norm = vec();
        L.up = linear(2 * INTER, HIDDEN);
        L.down = linear(HIDDEN, INTER);
    }
    // The input embedding moves to HBM so the gather runs inside the decode graph.
    m->embed = upload<uint16_t>(a, st.embedding().data, st.embedding().bytes);
    auto lt = rope_table(flocal, LOCAL_ROPE_ROWS, false);
    auto gt = rope_table(ffull, context, true);
    m->local_rope = upload<uint32_t>(a, lt.data(), lt.size() * sizeof(uint32_t));
    m->global_rope = upload<uint32_t>(a, gt.data(), gt.size() * sizeof(uint32_t));
    m->weight_bytes = int64_t(a.bytes());
    return m;
}

// ----------------------------------------------------------------------------- engine
Engine::Engine(std::shared_ptr<Model> mdl, int ctx, int nl, hipStream_t s)
    : model(std::move(mdl)), context(ctx), lanes(nl), stream(s) {
    const char* ng = std::getenv("PLAMO_NO_GRAPH");
    use_graph = !(ng && ng[0] == '1');
    const int parts_max = (context + KEYS_PER_PART - 1) / KEYS_PER_PART;
    // Prefill chunk: up to 2048 tokens (a multiple of the reference's 16-token chunk, so
    // the RoPE bases of its chunks are unchanged).
    chunk = std::min(2048, (context + CHUNK - 1) / CHUNK * CHUNK);
    // Ring = window + one prefill chunk (the reference's rule with its 16-token chunk,
    // Runtime.swift:240): the chunk's keys and the 2047 before it are resident at once.
    local_capacity = std::min(context, WINDOW + chunk);
    for (int l = 0; l < LAYERS; ++l) {
        capacity[l] = is_global_layer(l) ? context : local_capacity;
        const size_t n = size_t(lanes) * capacity[l] * HEAD_DIM;
        keys[l] = arena.alloc_n<uint16_t>(n);
        values[l] = arena.alloc_n<uint16_t>(n);
        PLAMO_HIP(hipMemsetAsync(keys[l], 0, n * 2, stream));
        PLAMO_HIP(hipMemsetAsync(values[l], 0, n * 2, stream));
        rot_rows[l] = is_global_layer(l) ? 0 : std::min(capacity[l], WINDOW);
        keys_rot[l] = nullptr;
        if (rot_rows[l]) {
            const size_t nr = size_t(lanes) * rot_rows[l] * HEAD_DIM;
            keys_rot[l] = arena.alloc_n<uint16_t>(nr);
            PLAMO_HIP(hipMemsetAsync(keys_rot[l], 0, nr * 2, stream));
        }
    }
    qkv = arena.alloc_n<float>(ROWS * QKV);
    att = arena.alloc_n<uint16_t>(ROWS * ATTN);
    proj = arena.alloc_n<uint16_t>(ROWS * HIDDEN);
    x0 = arena.alloc_n<uint16_t>(ROWS * HIDDEN);
    x1 = arena.alloc_n<uint16_t>(ROWS * HIDDEN);
    act = arena.alloc_n<uint16_t>(ROWS * INTER);
    hidden = arena.alloc_n<float>(ROWS * HIDDEN);
    resid_scratch = arena.alloc_n<uint16_t>(ROWS * HIDDEN);
    logits = arena.alloc_n<uint16_t>(size_t(ROWS) * VOCAB);
    state = arena.alloc_n<StepState>(1);
    PLAMO_HIP(hipHostMalloc(reinterpret_cast<void**>(&host_state), sizeof(StepState), hipHostMallocDefault));
    std::memset(host_state, 0, sizeof(StepState));
    host_state->penalty = 1.0f;
    PLAMO_HIP(hipMemsetAsync(state, 0, sizeof(StepState), stream));
    bufs.state = state;
    bufs.out_ids = arena.alloc_n<int32_t>(size_t(ROWS) * (size_t(context) + 1));  // [lane][context + 1]
    bufs.hist_cap = uint32_t(context);
    bufs.history = arena.alloc_n<int32_t>(size_t(ROWS) * context);
    bufs.counts = arena.alloc_n<int32_t>(size_t(ROWS) * VOCAB);
    bufs.banned = arena.alloc_n<uint32_t>(size_t(ROWS) * (VOCAB / 32));
    bufs.head_v = arena.alloc_n<float>(size_t(ROWS) * HEAD_BLOCKS);
    bufs.head_i = arena.alloc_n<uint32_t>(size_t(ROWS) * HEAD_BLOCKS);
    bufs.tickets = arena.alloc_n<uint32_t>(1);

    PLAMO_HIP(hipMemsetAsync(bufs.tickets, 0, 4, stream));
    PLAMO_HIP(hipMemsetAsync(bufs.counts, 0, size_t(ROWS) * VOCAB * 4, stream));
    PLAMO_HIP(hipMemsetAsync(bufs.banned, 0, size_t(ROWS) * (VOCAB / 32) * 4, stream));
    decode_parts_local = uint32_t((std::min(context, WINDOW) + KEYS_PER_PART - 1) / KEYS_PER_PART);
    decode_parts_global = uint32_t(parts_max);
    part_rows_cap = size_t(ROWS) * parts_max;
    part_m = arena.alloc_n<float>(part_rows_cap * HEADS);
    part_l = arena.alloc_n<float>(part_rows_cap * HEADS);
    part_o = arena.alloc_n<float>(part_rows_cap * HEADS * HEAD_DIM);
    attn_tickets = arena.alloc_n<uint32_t>(size_t(ROWS) * HEADS);  // [row][head group]
    PLAMO_HIP(hipMemsetAsync(attn_tickets, 0, size_t(ROWS) * HEADS * 4, stream));
    p_x = arena.alloc_n<uint16_t>(size_t(chunk) * HIDDEN);
    p_qkv = arena.alloc_n<uint16_t>(size_t(chunk) * QKV);
    p_proj = arena.alloc_n<uint16_t>(size_t(chunk) * HIDDEN);
    p_xn = arena.alloc_n<uint16_t>(size_t(chunk) * HIDDEN);
    p_att = arena.alloc_n<uint16_t>(size_t(chunk) * ATTN);
    p_q16 = arena.alloc_n<uint16_t>(size_t(chunk) * ATTN);
    p_flash_o = arena.alloc_n<float>(flash_part_o_floats(chunk));
    p_flash_ml = arena.alloc_n<float>(flash_part_ml_floats(chunk));
    p_flash_tickets = arena.alloc_n<uint32_t>(size_t(flash_blocks(chunk)));
    if (model->packed) p_wexp = arena.alloc_n<uint16_t>(size_t(2 * INTER) * HIDDEN);
    PLAMO_HIP(hipMemsetAsync(p_flash_tickets, 0, size_t(flash_blocks(chunk)) * 4, stream));
    p_act = arena.alloc_n<uint16_t>(size_t(chunk) * INTER);
    p_tokens = arena.alloc_n<int32_t>(size_t(chunk));
    PLAMO_HIP(hipEventCreate(&ev0));
    PLAMO_HIP(hipEventCreate(&ev1));
    PLAMO_HIP(hipStreamSynchronize(stream));
}

Engine::~Engine() {
    if (graph) (void)hipGraphExecDestroy(graph);
    if (graph_loop) (void)hipGraphExecDestroy(graph_loop);
    if (graph16) (void)hipGraphExecDestroy(graph16);
    if (graph_verify) (void)hipGraphExecDestroy(graph_verify);

    (void)hipEventDestroy(ev0);
    (void)hipEventDestroy(ev1);
    if (host_state) (void)hipHostFree(host_state);
}

void Engine::zero_sampler() {
    PLAMO_HIP(hipMemsetAsync(bufs.counts, 0, size_t(ROWS) * VOCAB * 4, stream));
}

void Engine::enable_qsa(const Aux* aux, int budget) {
    qsa_aux = aux;
    qsa_budget = budget;
    qsa_blocks = uint32_t(context / 4);
    qsa_words = (qsa_blocks + 31) / 32;
    qsa_proj = arena.alloc_n<uint16_t>(size_t(chunk) * QSA_PROJ);
    qsa_q = arena.alloc_n<uint16_t>(size_t(chunk) * 4 * HEAD_DIM);
    for (int l = 0; l < LAYERS; ++l) {
        if (!is_global_layer(l)) continue;
        qsa_raw[l] = arena.alloc_n<uint16_t>(size_t(context) * HEAD_DIM);
        qsa_pooled[l] = arena.alloc_n<uint16_t>(size_t(std::max<uint32_t>(qsa_blocks, 1)) * HEAD_DIM);
    }
    qsa_scores = arena.alloc_n<float>(size_t(chunk) * std::max<uint32_t>(qsa_blocks, 1));
    qsa_mask = arena.alloc_n<uint32_t>(size_t(chunk) * std::max<uint32_t>(qsa_words, 1));
}

QsaParams Engine::qsa_params(int layer, int tokens, const StepState* st, uint32_t p0) const {
    QsaParams q{};
    q.state = st;
    q.p0 = p0;
    q.tokens = tokens;
    q.proj = qsa_proj;
    q.q_norm = qsa_aux->qsa_q_norm[layer];
    q.k_norm = qsa_aux->qsa_k_norm[layer];
    q.global_rope = model->global_rope;
    q.queries = qsa_q;
    q.raw = qsa_raw[layer];
    q.pooled = qsa_pooled[layer];
    q.scores = qsa_scores;
    q.mask = qsa_mask;
    q.blocks = qsa_blocks;
    q.words = qsa_words;
    q.budget = qsa_budget;
    return q;
}

void Engine::enqueue_head(const uint16_t* in, const uint16_t* resid_in, int in_rows) {
    const Model& m = *model;
    const int maxr = lanes == 1 ? 1 : ROWS;
    GemvParams g{};
    g.state = state;
    g.rows = in_rows;
    g.m = VOCAB;
    g.w = m.head.w;
    g.table = m.head.table;
    g.tag = TL_HEAD;
    g.in16 = in;
    g.resid16_in = resid_in;
    g.resid16_out = resid_scratch;
    g.g_post = m.layers[LAYERS - 1].post_mlp;
    g.post_offset = post_mlp_offset();
    g.g_next = m.final_norm;
    g.hidden = hidden;
    g.out16 = logits;
    g.bufs = bufs;
    launch_gemv(HIDDEN, m.packed, maxr, PRO_RESID16, EPI_LOGITS, g, head_blocks(maxr), stream);
    launch_head_merge(bufs, head_blocks(maxr), false, stream);
}

void Engine::enqueue_head16(bool loop, int maxr) {
    const Model& m = *model;
    GemvParams g{};
    g.state = state;
    g.rows = ROWS;
    g.m = VOCAB;
    g.w = m.head.w;
    g.table = m.head.table;
    g.tag = TL_HEAD;
    g.in16 = proj;
    g.resid16_in = x1;
    g.resid16_out = x0;  // final residual, not read again
    g.g_post = m.layers[LAYERS - 1].post_mlp;
    g.post_offset = post_mlp_offset();
    g.g_next = m.final_norm;
    g.hidden = hidden;
    g.out16 = logits;
    g.bufs = bufs;
    launch_gemv(HIDDEN, m.packed, maxr, PRO_RESID16, EPI_LOGITS, g, head_blocks(maxr), stream);
    launch_head_merge(bufs, head_blocks(maxr), loop, stream);
}

// One decode step (Runtime.swift:376-458 for one token per row; Batch.swift:147-165).  A host
// step starts with the bookkeeping kernel; a device-loop step finds its bookkeeping done by the
// previous step's head merge (or by begin_loop before the first replay).
void Engine::enqueue_step(bool head, bool loop, bool verify) {
    const Model& m = *model;
    const bool pk = m.packed;
    const int maxr = lanes == 1 && !verify ? 1 : ROWS;
    if (!loop) launch_step_begin(bufs, stream);
    for (int l = 0; l < LAYERS; ++l) {
        const LayerWeights& L = m.layers[l];
        const bool full = is_global_layer(l);
        GemvParams g{};
        g.state = state;
        g.rows = ROWS;
        // QKV with the (embedding or post-MLP residual) + pre-attention norm prologue
        g.m = QKV;
        g.w = L.qkv.w;
        g.table = L.qkv.table;
        g.tag = uint32_t(l) * 8;
        g.resid16_out = x0;
        g.g_next = L.pre;
        g.out = qkv;
        if (l == 0) {
            g.embed = m.embed;
            launch_gemv(HIDDEN, pk, maxr, PRO_EMBED, EPI_ROUND, g, gemv_blocks(HIDDEN, maxr, EPI_ROUND, QKV, pk), stream);
        } else {
            g.in16 = proj;
            g.resid16_in = x1;
            g.g_post = m.layers[l - 1].post_mlp;
            g.post_offset = post_mlp_offset();
            launch_gemv(HIDDEN, pk, maxr, PRO_RESID16, EPI_ROUND, g, gemv_blocks(HIDDEN, maxr, EPI_ROUND, QKV, pk), stream);
        }
        const bool qsa = full && qsa_aux && lanes == 1 && !verify;
        if (qsa) {
            // the indexer projection of the same normed row (same prologue, Runtime.swift:381),
            // then queries, raw key, block key, scores and the selection (Runtime.swift:382-403)
            GemvParams x = g;
            x.m = QSA_PROJ;
            x.w = qsa_aux->qsa_proj[l];
            x.table = nullptr;
            x.out = nullptr;
            x.out16 = qsa_proj;
            x.resid16_out = resid_scratch;
            x.tag = uint32_t(TIMELINE_TAGS);
            launch_gemv(HIDDEN, false, 1, PRO_RESID16, EPI_BF16, x, gemv_blocks(HIDDEN, 1, EPI_BF16, QSA_PROJ, false),
                        stream);
            launch_qsa(qsa_params(l, 1, state, 0), int(qsa_blocks), stream);
        }
        AttnParams a{};
        a.state = state;
        a.qkv = qkv;
        a.q_norm = L.q_norm;
        a.k_norm = L.k_norm;
        a.keys = keys[l];
        a.values = values[l];
        a.keys_rot = keys_rot[l];
        a.rot_rows = uint32_t(rot_rows[l]);
        a.capacity = uint32_t(capacity[l]);
        a.local_rope = m.local_rope;
        a.global_rope = m.global_rope;
        a.part_m = part_m;
        a.part_l = part_l;
        a.part_o = part_o;
        a.parts = full ? decode_parts_global : decode_parts_local;
        a.tickets = attn_tickets;
        a.out16 = att;
        a.tag = uint32_t(l) * 8 + 1;
        // batch 1: rows of 2..MERGE_IN_O partitions are merged by the o projection's prologue
        a.merge_in_o = maxr == 1 ? 1u : 0u;
        // rows past ATTN_MERGE_INLINE partitions merge in their own kernel (past
        // ATTN_MERGE_INLINE_BATCH in four-row batches, once that kernel is launched)
        a.defer = a.parts > ATTN_MERGE_INLINE ? (maxr > 1 ? ATTN_MERGE_INLINE_BATCH : ATTN_MERGE_INLINE) : 0u;
        a.window = full ? 0u : uint32_t(WINDOW);
        a.qsa_mask = qsa ? qsa_mask : nullptr;
        a.qsa_words = qsa_words;
        if (verify) {
            // row 1 reads the key and value row 0 writes at its position: one launch per row
            for (uint32_t r = 0; r < VERIFY_ROWS; ++r) {
                a.row0 = r;
                launch_attention(full, a, 1, stream);
            }
            a.row0 = 0;
        } else {
            launch_attention(full, a, ROWS, stream);
        }
        if (a.defer) launch_attention_merge(a, ROWS, stream);
        GemvParams o{};
        o.state = state;
        o.rows = ROWS;
        o.m = HIDDEN;
        o.w = L.o.w;
        o.table = L.o.table;
        o.tag = uint32_t(l) * 8 + 3;
        o.in16 = att;
        o.out16 = proj;
        o.part_m = part_m;
        o.part_l = part_l;
        o.part_o = part_o;
        o.parts = a.parts;
        o.merge_full = full ? 1u : 0u;
        launch_gemv(ATTN, pk, maxr, maxr == 1 ? PRO_MERGE : PRO_PLAIN16, EPI_BF16, o,
                    gemv_blocks(ATTN, maxr, EPI_BF16, HIDDEN, pk), stream);
        GemvParams u{};
        u.state = state;
        u.rows = ROWS;
        u.m = 2 * INTER;
        u.w = L.up.w;
        u.table = L.up.table;
        u.tag = uint32_t(l) * 8 + 4;
        u.in16 = proj;
        u.resid16_in = x0;
        u.resid16_out = x1;
        u.g_post = L.post;
        u.post_offset = POST_MIXER_OFFSET;
        u.g_next = L.pre_mlp;
        u.out16 = act;
        launch_gemv(HIDDEN, pk, maxr, PRO_RESID16, EPI_SWIGLU, u, gemv_blocks(HIDDEN, maxr, EPI_SWIGLU, 2 * INTER, pk), stream);
        GemvParams d{};
        d.state = state;
        d.rows = ROWS;
        d.m = HIDDEN;
        d.w = L.down.w;
        d.table = L.down.table;
        d.tag = uint32_t(l) * 8 + 5;
        d.in16 = act;
        d.out16 = proj;
        launch_gemv(INTER, pk, maxr, PRO_PLAIN16, EPI_BF16, d, gemv_blocks(INTER, maxr, EPI_BF16, HIDDEN, pk), stream);
    }
    if (head) enqueue_head16(loop, maxr);
}

namespace {
// Captures (without running) what `enqueue` puts on `stream` into `out`.
template <typename F>
void capture_graph(hipStream_t stream, hipGraphExec_t* out, F enqueue) {
    hipGraph_t g = nullptr;
    PLAMO_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    try {
        enqueue();
    } catch (...) {
        (void)hipStreamEndCapture(stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    PLAMO_HIP(hipStreamEndCapture(stream, &g));
    PLAMO_HIP(hipGraphInstantiate(out, g, nullptr, nullptr, 0));
    PLAMO_HIP(hipGraphDestroy(g));
}
}  // namespace

void Engine::run_step() {
    if (!use_graph) {
        enqueue_step();
        return;
    }
    if (!graph) capture_graph(stream, &graph, [&] { enqueue_step(); });
    PLAMO_HIP(hipGraphLaunch(graph, stream));
}

void Engine::run_verify() {
    if (!use_graph) {
        enqueue_step(true, false, true);
        return;
    }
    if (!graph_verify) capture_graph(stream, &graph_verify, [&] { enqueue_step(true, false, true); });
    PLAMO_HIP(hipGraphLaunch(graph_verify, stream));
}

// Captures (without running) `steps` consecutive device-loop steps into `out`.
void Engine::capture_loop(int steps, hipGraphExec_t* out) {
    capture_graph(stream, out, [&] {
        for (int k = 0; k < steps; ++k) enqueue_step(true, true);
    });
}

void Engine::prepare_loop_graph() {
    if (!use_graph) return;
    if (!graph_loop) capture_loop(1, &graph_loop);
    if (!graph16) capture_loop(LOOP_GRAPH_STEPS, &graph16);
}

void Engine::begin_loop() { launch_step_begin(bufs, stream); }

void Engine::run_steps(int n) {
    if (!use_graph) {
        for (; n > 0; --n) enqueue_step(true, true);
        return;
    }
    prepare_loop_graph();
    for (; n >= LOOP_GRAPH_STEPS; n -= LOOP_GRAPH_STEPS) PLAMO_HIP(hipGraphLaunch(graph16, stream));
    for (; n > 0; --n) PLAMO_HIP(hipGraphLaunch(graph_loop, stream));
}

void check_aux_tensors(const AuxArchive& ar, bool mtp, bool qsa) {
    if (mtp) {  // Predictor (Auxiliary.swift:101-102)
        ar.tensor("mtp.heads.0.up.weight", {MTP_RANK, MTP_IN});
        ar.tensor("mtp.heads.0.down.weight", {HIDDEN, MTP_RANK});
    }
    if (qsa)  // Indexer of each global layer (Auxiliary.swift:75-77)
        for (int l = 0; l < LAYERS; ++l) {
            if (!is_global_layer(l)) continue;
            const std::string p = "qsa." + std::to_string(l) + ".";
            ar.tensor(p + "proj.weight", {QSA_PROJ, HIDDEN});
            ar.tensor(p + "q_norm.weight", {HEAD_DIM});
            ar.tensor(p + "k_norm.weight", {HEAD_DIM});
        }
}

std::unique_ptr<Aux> load_aux(const AuxArchive& ar, bool mtp, bool qsa) {
    check_aux_tensors(ar, mtp, qsa);
    auto x = std::make_unique<Aux>();
    DeviceArena& a = x->arena;
    auto put = [&](const std::string& name, std::vector<int64_t> shape) {
        const TensorView t = ar.tensor(name, shape);
        x->bytes += int64_t(t.bytes);
        return upload<uint16_t>(a, t.data, t.bytes);
    };
    if (mtp) {
        x->mtp_up = put("mtp.heads.0.up.weight", {MTP_RANK, MTP_IN});
        x->mtp_down = put("mtp.heads.0.down.weight", {HIDDEN, MTP_RANK});
        x->mtp_in = a.alloc_n<float>(MTP_IN);
        x->mtp_up_out = a.alloc_n<float>(MTP_RANK);
        x->mtp_hidden = a.alloc_n<float>(HIDDEN);
        x->mtp_logits = a.alloc_n<uint16_t>(VOCAB);
        x->slot_logits = a.alloc_n<uint16_t>(size_t(VERIFY_ROWS) * VOCAB);
        x->slot_hidden = a.alloc_n<float>(size_t(VERIFY_ROWS) * HIDDEN);
        x->slot_next = a.alloc_n<int32_t>(VERIFY_ROWS);
    }
    if (qsa) {
        for (int l = 0; l < LAYERS; ++l) {
            if (!is_global_layer(l)) continue;
            const std::string p = "qsa." + std::to_string(l) + ".";
            x->qsa_proj[l] = put(p + "proj.weight", {QSA_PROJ, HIDDEN});
            x->qsa_q_norm[l] = put(p + "q_norm.weight", {HEAD_DIM});
            x->qsa_k_norm[l] = put(p + "k_norm.weight", {HEAD_DIM});
        }
    }
    return x;
}

// A prefill chunk of n tokens at p0 for one lane: every layer as MFMA GEMMs, K/V written
// for the chunk, then MFMA flash attention of the chunk's queries over their visible keys.
void Engine::enqueue_prefill_chunk(int n, int p0, int lane, bool last_chunk, bool output) {
    const Model& m = *model;
    const bool pk = m.packed;
    RowsNormParams rn{};
    rn.tokens_in = p_tokens;
    rn.embed = m.embed;
    rn.x = p_x;
    rn.g_next = m.layers[0].pre;
    rn.xn = p_xn;
    launch_rows_norm(rn, n, stream);
    // .p12 weights are expanded to BF16 rows (bit-identical to the plain tensor) right before
    // their GEMM, which then loads them straight into LDS like plain weights: expanding each
    // block in the GEMM's registers was up to seven times slower at short prompts
    auto gemm = [&](const Linear& W, GemmEpilogue epi, GemmParams g) {
        if (pk) {
            launch_unpack(reinterpret_cast<const uint8_t*>(W.w), W.table, p_wexp, int64_t(g.m) * g.k, stream);
            g.w = p_wexp;
        } else {
            g.w = W.w;
        }
        g.table = nullptr;
        launch_gemm(false, epi, g, stream);
    };
    for (int l = 0; l < LAYERS; ++l) {
        const LayerWeights& L = m.layers[l];
        const bool full = is_global_layer(l);
        GemmParams q{};
        q.x = p_xn; q.y16 = p_qkv; q.m = QKV; q.k = HIDDEN; q.tokens = n;
        gemm(L.qkv, GEMM_BF16, q);
        QkPrepParams qp{};
        qp.qkv = p_qkv;
        qp.q_norm = L.q_norm;
        qp.k_norm = L.k_norm;
        qp.q16 = p_q16;
        qp.keys = keys[l] + size_t(lane) * capacity[l] * HEAD_DIM;
        qp.values = values[l] + size_t(lane) * capacity[l] * HEAD_DIM;
        qp.keys_rot = keys_rot[l] ? keys_rot[l] + size_t(lane) * rot_rows[l] * HEAD_DIM : nullptr;
        qp.rot_rows = uint32_t(rot_rows[l]);
        qp.capacity = uint32_t(capacity[l]);
        qp.p0 = uint32_t(p0);
        qp.tokens = n;
        qp.full = full;
        qp.local_rope = m.local_rope;
        qp.global_rope = m.global_rope;
        launch_qk_prep(qp, stream);
        const bool qsa = full && qsa_aux && lanes == 1;
        if (qsa) {
            // the indexer on the chunk's normed rows: every token selects its own blocks
            GemmParams xg{};
            xg.w = qsa_aux->qsa_proj[l];
            xg.x = p_xn;
            xg.y16 = qsa_proj;
            xg.m = QSA_PROJ;
            xg.k = HIDDEN;
            xg.tokens = n;
            launch_gemm(false, GEMM_BF16, xg, stream);
            launch_qsa(qsa_params(l, n, nullptr, uint32_t(p0)), std::min<int>(int(qsa_blocks), (p0 + n) / 4 + 1),
                       stream);
        }
        FlashParams fa{};
        fa.q = p_q16;
        fa.keys = qp.keys;
        fa.values = qp.values;
        fa.local_rope = m.local_rope;
        fa.keys_rot = qp.keys_rot;
        fa.rot_rows = qp.rot_rows;
        fa.out = p_att;
        fa.capacity = qp.capacity;
        fa.p0 = uint32_t(p0);
        fa.tokens = n;
        fa.full = full;
        fa.part_o = p_flash_o;
        fa.part_ml = p_flash_ml;
        fa.tickets = p_flash_tickets;
        fa.qsa_mask = qsa ? qsa_mask : nullptr;
        fa.qsa_words = qsa_words;
        launch_flash_prefill(fa, stream);
        GemmParams o{};
        o.x = p_att; o.y16 = p_proj; o.m = HIDDEN; o.k = ATTN; o.tokens = n;
        gemm(L.o, GEMM_BF16, o);
        RowsNormParams r1{};
        r1.in = p_proj; r1.g_post = L.post; r1.post_offset = POST_MIXER_OFFSET; r1.x = p_x; r1.g_next = L.pre_mlp;
        r1.xn = p_xn;
        launch_rows_norm(r1, n, stream);
        GemmParams u{};
        u.x = p_xn; u.y16 = p_act; u.m = 2 * INTER; u.k = HIDDEN; u.tokens = n;
        gemm(L.up, GEMM_SWIGLU, u);
        GemmParams d{};
        d.x = p_act; d.y16 = p_proj; d.m = HIDDEN; d.k = INTER; d.tokens = n;
        gemm(L.down, GEMM_BF16, d);
        if (l + 1 < LAYERS) {
            RowsNormParams r2{};
            r2.in = p_proj; r2.g_post = L.post_mlp; r2.post_offset = post_mlp_offset(); r2.x = p_x;
            r2.g_next = m.layers[l + 1].pre; r2.xn = p_xn;
            launch_rows_norm(r2, n, stream);
        }
    }
    if (last_chunk && output) {
        launch_step_begin(bufs, stream);
        enqueue_head(p_proj + size_t(n - 1) * HIDDEN, p_x + size_t(n - 1) * HIDDEN, 1);
    }
}

void Engine::prefill(const int32_t* tokens, int n, int p0, int lane, bool output) {
    for (int c0 = 0; c0 < n; c0 += chunk) {
        const int cn = std::min(chunk, n - c0);
        PLAMO_HIP(hipMemcpyAsync(p_tokens, tokens + c0, size_t(cn) * 4, hipMemcpyHostToDevice, stream));
        enqueue_prefill_chunk(cn, p0 + c0, lane, c0 + cn == n, output);
    }
}

void Engine::prefill_heads(int n, uint16_t* slot_logits, float* slot_hidden, int32_t* slot_next) {
    for (int i = 0; i < n; ++i) {
        launch_step_begin(bufs, stream);
        enqueue_head(p_proj + size_t(i) * HIDDEN, p_x + size_t(i) * HIDDEN, 1);
        PLAMO_HIP(hipMemcpyAsync(slot_logits + size_t(i) * VOCAB, logits, size_t(VOCAB) * 2, hipMemcpyDeviceToDevice,
                                 stream));
        PLAMO_HIP(hipMemcpyAsync(slot_hidden + size_t(i) * HIDDEN, hidden, size_t(HIDDEN) * 4, hipMemcpyDeviceToDevice,
                                 stream));
        PLAMO_HIP(hipMemcpyAsync(slot_next + i, &state->next[0], 4, hipMemcpyDeviceToDevice, stream));
    }
}

// ---------------------------------------------------------------------------- runtime
RuntimeImpl::~RuntimeImpl() {
    eng.reset();
    model.reset();
    if (stream) (void)hipStreamDestroy(stream);
}

void RuntimeImpl::reset() {
    position = 0;
    gpu_seconds = 0;
    last_output_rows = 0;
    sparse_queries = sparse_keys = dense_keys = 0;
    history.clear();
    uploaded = 0;
    counts_dirty = true;
}

void RuntimeImpl::begin_timing() { PLAMO_HIP(hipEventRecord(eng->ev0, stream)); }

void RuntimeImpl::end_timing() {
    PLAMO_HIP(hipEventRecord(eng->ev1, stream));
    PLAMO_HIP(hipEventSynchronize(eng->ev1));
    float ms = 0;
    PLAMO_HIP(hipEventElapsedTime(&ms, eng->ev0, eng->ev1));
    gpu_seconds += ms / 1000.0;
}

// Uploads the generated history not yet on the device and the sampler settings.
void RuntimeImpl::sync_sampler(Engine& e, int row) {
    StepState& hs = *e.host_state;
    hs.sampling = sampling ? 1 : 0;
    hs.penalty = penalty;
    hs.frequency = frequency;
    hs.presence = presence;
    hs.ngram = ngram;
    if (counts_dirty) {
        e.zero_sampler();
        hs.counted[row] = 0;
        counts_dirty = false;
    }
    if (!sampling) {
        hs.hist_len[row] = uint32_t(std::min<size_t>(history.size(), e.bufs.hist_cap));
        return;
    }
    const size_t n = std::min<size_t>(history.size(), e.bufs.hist_cap);
    if (uploaded < n) {
        PLAMO_HIP(hipMemcpyAsync(e.bufs.history + size_t(row) * e.bufs.hist_cap + uploaded, history.data() + uploaded,
                                 (n - uploaded) * 4, hipMemcpyHostToDevice, stream));
        uploaded = n;
    }
    hs.hist_len[row] = uint32_t(n);
}

int RuntimeImpl::forward(const int32_t* tokens, int n, bool output) {
    // Runtime.swift:328-330: validate before touching any state.
    const int limit = std::min(context, CHUNK);
    bool ok = n > 0 && n <= limit && position + n <= context;
    for (int i = 0; ok && i < n; ++i) ok = tokens[i] >= 0 && tokens[i] < VOCAB;
    if (!ok) throw Error(E_INVAL, "Invalid tokens or context exhausted");
    Engine& e = *eng;
    StepState& hs = *e.host_state;
    hs.rows = 1;
    hs.lane[0] = 0;
    hs.pos[0] = uint32_t(position);
    hs.token[0] = tokens[0];
    hs.loop = 0;
    hs.stopped = 0;
    sync_sampler(e, 0);
    PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, stream));
    begin_timing();
    if (n == 1 && output) {
        e.run_step();
    } else if (n == 1) {
        // no head: the reference leaves logits untouched without output (Runtime.swift:453-458)
        e.enqueue_step(false);
    } else {
        e.prefill(tokens, n, int(position), 0, output);
    }
    end_timing();
    PLAMO_HIP(hipMemcpyAsync(&hs, e.state, sizeof(StepState), hipMemcpyDeviceToHost, stream));
    PLAMO_HIP(hipStreamSynchronize(stream));
    PLAMO_HIP(hipGetLastError());
    count_qsa(position, n);
    position += n;
    last_output_rows = output ? 1 : 0;
    if (!output) return -1;
    const int next = int32_t(hs.next[0]);
    predictions.assign(1, next);
    return next;
}

int RuntimeImpl::prefill(const int32_t* tokens, int n) {
    // Runtime.swift:474
    bool ok = n > 0 && position + n <= context;
    for (int i = 0; ok && i < n; ++i) ok = tokens[i] >= 0 && tokens[i] < VOCAB;
    if (!ok) throw Error(E_INVAL, "Input exceeds context");
    if (n == 1) return forward(tokens, 1, true);
    Engine& e = *eng;
    StepState& hs = *e.host_state;
    hs.rows = 1;
    hs.lane[0] = 0;
    hs.pos[0] = uint32_t(position);
    hs.loop = 0;
    hs.stopped = 0;
    sync_sampler(e, 0);
    PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, stream));
    begin_timing();
    e.prefill(tokens, n, int(position), 0, true);
    end_timing();
    PLAMO_HIP(hipMemcpyAsync(&hs, e.state, sizeof(StepState), hipMemcpyDeviceToHost, stream));
    PLAMO_HIP(hipStreamSynchronize(stream));
    PLAMO_HIP(hipGetLastError());
    for (int s0 = 0; s0 < n; s0 += std::min(context, CHUNK))  // Runtime.fill's forwards (Runtime.swift:476)
        count_qsa(position + s0, std::min(std::min(context, CHUNK), n - s0));
    position += n;
    last_output_rows = 1;
    const int next = int32_t(hs.next[0]);
    predictions.assign(1, next);
    return next;
}

int RuntimeImpl::forward_ex(const int32_t* tokens, int n, bool output, bool all, bool sequential) {
    // Runtime.swift:328-330: validate before touching any state
    const int limit = std::min(context, CHUNK);
    bool ok = n > 0 && n <= limit && position + n <= context;
    for (int i = 0; ok && i < n; ++i) ok = tokens[i] >= 0 && tokens[i] < VOCAB;
    if (all && !(mtp && n <= VERIFY_ROWS)) ok = false;
    if (sequential && !(mtp && n <= VERIFY_ROWS)) ok = false;
    if (!ok) throw Error(E_INVAL, "Invalid tokens or context exhausted");
    if (!all && !sequential) return forward(tokens, n, output);
    Engine& e = *eng;
    StepState& hs = *e.host_state;
    const int rows = output ? (all ? n : 1) : 0;  // Runtime.swift:453
    begin_timing();
    if (sequential && n == VERIFY_ROWS && output && all && !sampling && !e.qsa_aux) {
        // Both rows in one pass over the weights (the linear_pair pass of Runtime.swift:370-371):
        // the multi-row kernels with each row at its own position in KV slice 0 and its outputs
        // in slot i; row 1's attention runs after row 0's, whose key and value it reads.  Per
        // row these are the operations of a scalar step, so the bits are those of
        // forward([tokens[0]]) then forward([tokens[1]]).
        hs.rows = VERIFY_ROWS;
        for (int i = 0; i < VERIFY_ROWS; ++i) {
            hs.lane[i] = uint32_t(i);
            hs.pos[i] = uint32_t(position + i);
            hs.token[i] = tokens[i];
            sync_sampler(e, i);
        }
        hs.kv_shared = 1;
        hs.loop = 0;
        hs.stopped = 0;
        PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, stream));
        e.run_verify();
        PLAMO_HIP(hipMemcpyAsync(aux->slot_logits, e.logits, size_t(VERIFY_ROWS) * VOCAB * 2, hipMemcpyDeviceToDevice,
                                 stream));
        PLAMO_HIP(hipMemcpyAsync(aux->slot_hidden, e.hidden, size_t(VERIFY_ROWS) * HIDDEN * 4,
                                 hipMemcpyDeviceToDevice, stream));
        PLAMO_HIP(hipMemcpyAsync(aux->slot_next, &e.state->next[0], size_t(VERIFY_ROWS) * 4, hipMemcpyDeviceToDevice,
                                 stream));
        // slot 0 then holds the last row, as after two scalar steps (rewind to the last row)
        PLAMO_HIP(hipMemcpyAsync(e.logits, aux->slot_logits + size_t(VERIFY_ROWS - 1) * VOCAB, size_t(VOCAB) * 2,
                                 hipMemcpyDeviceToDevice, stream));
        PLAMO_HIP(hipMemcpyAsync(e.hidden, aux->slot_hidden + size_t(VERIFY_ROWS - 1) * HIDDEN, size_t(HIDDEN) * 4,
                                 hipMemcpyDeviceToDevice, stream));
    } else if (sequential || n == 1) {
        // Each row as a scalar decode step at its own position: its local keys and query take
        // the coordinates of that step (rotate_steps, Kernels.metal:288-298), so row i's
        // outputs are those of forward([tokens[i]]) after rows 0 .. i - 1.
        for (int i = 0; i < n; ++i) {
            hs.rows = 1;
            hs.lane[0] = 0;
            hs.pos[0] = uint32_t(position + i);
            hs.token[0] = tokens[i];
            hs.loop = 0;
            hs.stopped = 0;
            sync_sampler(e, 0);
            PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, stream));
            const bool head = output && (all || i == n - 1);
            if (head) e.run_step();
            else e.enqueue_step(false);
            if (head && all) {
                PLAMO_HIP(hipMemcpyAsync(aux->slot_logits + size_t(i) * VOCAB, e.logits, size_t(VOCAB) * 2,
                                         hipMemcpyDeviceToDevice, stream));
                PLAMO_HIP(hipMemcpyAsync(aux->slot_hidden + size_t(i) * HIDDEN, e.hidden, size_t(HIDDEN) * 4,
                                         hipMemcpyDeviceToDevice, stream));
                PLAMO_HIP(hipMemcpyAsync(aux->slot_next + i, &e.state->next[0], 4, hipMemcpyDeviceToDevice, stream));
            }
        }
    } else {
        // one chunk of n rows (chunk-relative local coordinates, Runtime.swift:389), then a
        // head per row
        hs.rows = 1;
        hs.lane[0] = 0;
        hs.pos[0] = uint32_t(position);
        hs.loop = 0;
        hs.stopped = 0;
        sync_sampler(e, 0);
        PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, stream));
        e.prefill(tokens, n, int(position), 0, false);
        if (output) e.prefill_heads(n, aux->slot_logits, aux->slot_hidden, aux->slot_next);
    }
    end_timing();
    int32_t next[VERIFY_ROWS] = {-1, -1};
    if (rows > 1) PLAMO_HIP(hipMemcpyAsync(next, aux->slot_next, size_t(rows) * 4, hipMemcpyDeviceToHost, stream));
    PLAMO_HIP(hipMemcpyAsync(&hs, e.state, sizeof(StepState), hipMemcpyDeviceToHost, stream));
    PLAMO_HIP(hipStreamSynchronize(stream));
    PLAMO_HIP(hipGetLastError());
    hs.kv_shared = 0;  // later uploads run single rows again
    count_qsa(position, n);
    position += n;
    last_output_rows = rows;
    if (!output) return -1;
    if (rows > 1) predictions.assign(next, next + rows);
    else predictions.assign(1, int32_t(hs.next[0]));
    return predictions.back();
}

void RuntimeImpl::count_qsa(int64_t p0, int n) {
    if (!eng->qsa_aux || p0 + n <= qsa_budget) return;  // selected = position + batch > budget
    for (int l = 0; l < LAYERS; ++l) {
        if (!is_global_layer(l)) continue;
        sparse_queries += n;
        for (int t = 0; t < n; ++t) {
            const int64_t visible = p0 + t + 1;
            dense_keys += visible;
            sparse_keys += std::min<int64_t>(visible / 4, qsa_budget / 4) * 4 + visible % 4;
        }
    }
}

const uint16_t* RuntimeImpl::logits_row(int slot) const {
    return last_output_rows > 1 ? aux->slot_logits + size_t(slot) * VOCAB : eng->logits;
}

const float* RuntimeImpl::hidden_row() const { return eng->hidden; }

int RuntimeImpl::draft(int first) {
    // Runtime.swift:489-491
    if (!mtp || !aux || position <= 0 || first < 0 || first >= VOCAB || first == 1 || first == 16)
        throw Error(E_STATE, "MTP requires a prefetched context and trained adapters");
    Engine& e = *eng;
    const Model& m = *model;
    StepState& hs = *e.host_state;
    begin_timing();
    // the first row's normalised hidden state (Runtime.swift:493), then the token's embedding
    const float* h = last_output_rows > 1 ? aux->slot_hidden : e.hidden;
    launch_mtp_input(h, m.embed, first, aux->mtp_in, stream);
    GemvParams u{};
    u.rows = 1;
    u.m = MTP_RANK;
    u.w = aux->mtp_up;
    u.in = aux->mtp_in;
    u.out = aux->mtp_up_out;
    u.tag = uint32_t(TIMELINE_TAGS);
    launch_gemv(MTP_IN, false, 1, PRO_PLAIN, EPI_ROUND, u, gemv_blocks(MTP_IN, 1, EPI_ROUND, MTP_RANK, false), stream);
    launch_mtp_down(aux->mtp_up_out, aux->mtp_in, aux->mtp_down, aux->mtp_hidden, stream);
    // the LM head and argmax (Runtime.swift:502-503), greedy whatever the sampler settings
    hs.rows = 1;
    hs.lane[0] = 0;
    hs.loop = 0;
    hs.stopped = 0;
    hs.sampling = 0;
    PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, stream));
    GemvParams g{};
    g.state = e.state;
    g.rows = 1;
    g.m = VOCAB;
    g.w = m.head.w;
    g.table = m.head.table;
    g.tag = uint32_t(TIMELINE_TAGS);
    g.in = aux->mtp_hidden;
    g.out16 = aux->mtp_logits;
    g.bufs = e.bufs;
    launch_gemv(HIDDEN, m.packed, 1, PRO_PLAIN, EPI_LOGITS, g, head_blocks(1), stream);
    launch_head_merge(e.bufs, head_blocks(1), false, stream);
    end_timing();
    PLAMO_HIP(hipMemcpyAsync(&hs, e.state, sizeof(StepState), hipMemcpyDeviceToHost, stream));
    PLAMO_HIP(hipStreamSynchronize(stream));
    PLAMO_HIP(hipGetLastError());
    const int32_t d = int32_t(hs.next[0]);
    // the draft lands in the first prediction slot (Runtime.swift:503-507)
    if (!predictions.empty()) predictions[0] = d;
    return d;
}

void RuntimeImpl::rewind(int64_t new_position, int hidden_index) {
    // Runtime.swift:528-531
    if (hidden_index < 0 || hidden_index >= last_output_rows ||
        new_position != position - last_output_rows + hidden_index + 1)
        throw Error(E_STATE, "Invalid verification rollback");
    Engine& e = *eng;
    if (last_output_rows > 1 && hidden_index != last_output_rows - 1) {
        PLAMO_HIP(hipMemcpyAsync(e.logits, aux->slot_logits + size_t(hidden_index) * VOCAB, size_t(VOCAB) * 2,
                                 hipMemcpyDeviceToDevice, stream));
        PLAMO_HIP(hipMemcpyAsync(e.hidden, aux->slot_hidden + size_t(hidden_index) * HIDDEN, size_t(HIDDEN) * 4,
                                 hipMemcpyDeviceToDevice, stream));
        PLAMO_HIP(hipStreamSynchronize(stream));
    }
    predictions.assign(1, predictions[size_t(hidden_index)]);
    position = new_position;
    last_output_rows = 1;
}

// ------------------------------------------------------------------------------ batch
BatchImpl::BatchImpl(RuntimeImpl* r) : rt(r) {
    if (rt->qsa_budget > 0 || rt->mtp)
        throw Error(E_INVAL, "Batch requires dense greedy inference with context below 8192");  // Batch.swift:34-36
    if (rt->context < 1 || rt->context >= 8192)
        throw Error(E_INVAL, "Batch requires dense greedy inference with context below 8192");  // Batch.swift:34-36
    eng = std::make_unique<Engine>(rt->model, rt->context, ROWS, rt->stream);
    // The LM head writes each row's logits and final hidden state into its lane's slot.
    lane_logits = eng->logits;
    lane_hidden = eng->hidden;
    for (auto& v : lane_next) v = 0;
}

BatchImpl::~BatchImpl() { eng.reset(); }

void BatchImpl::reset() {
    ready = false;
    positions.clear();
    gpu_seconds = 0;
}

std::vector<int32_t> BatchImpl::prefill(const std::vector<std::vector<int32_t>>& prompts) {
    // Batch.swift:81-83
    bool ok = prompts.size() >= 1 && prompts.size() <= 4;
    for (auto& p : prompts) {
        ok = ok && !p.empty() && int(p.size()) <= rt->context;
        for (int32_t t : p) ok = ok && t >= 0 && t < VOCAB;
    }
    if (!ok) throw Error(E_INVAL, "Expected one to four valid prompts");
    ready = false;
    gpu_seconds = 0;
    Engine& e = *eng;
    hipStream_t s = e.stream;
    StepState& hs = *e.host_state;
    for (size_t lane = 0; lane < prompts.size(); ++lane) {
        const auto& p = prompts[lane];
        std::memset(&hs, 0, sizeof(StepState));
        hs.rows = 1;
        hs.lane[0] = uint32_t(lane);
        hs.pos[0] = 0;
        hs.token[0] = p[0];
        hs.penalty = 1.0f;
        PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, s));
        PLAMO_HIP(hipEventRecord(e.ev0, s));
        if (p.size() == 1) e.run_step();
        else e.prefill(p.data(), int(p.size()), 0, int(lane), true);
        PLAMO_HIP(hipEventRecord(e.ev1, s));
        PLAMO_HIP(hipMemcpyAsync(&hs, e.state, sizeof(StepState), hipMemcpyDeviceToHost, s));
        PLAMO_HIP(hipStreamSynchronize(s));
        PLAMO_HIP(hipGetLastError());
        float ms = 0;
        PLAMO_HIP(hipEventElapsedTime(&ms, e.ev0, e.ev1));
        gpu_seconds += ms / 1000.0;
        lane_next[lane] = int32_t(hs.next[0]);
    }
    positions.assign(prompts.size(), 0);
    for (size_t i = 0; i < prompts.size(); ++i) positions[i] = int64_t(prompts[i].size());
    ready = true;
    return std::vector<int32_t>(lane_next, lane_next + prompts.size());
}

std::vector<int32_t> BatchImpl::step(const std::vector<int32_t>& tokens) {
    // Batch.swift:110-112
    bool ok = ready && tokens.size() == positions.size();
    bool any = false;
    for (size_t i = 0; ok && i < tokens.size(); ++i) {
        if (tokens[i] < 0) continue;
        any = true;
        ok = tokens[i] < VOCAB && positions[i] < rt->context;
    }
    if (!ok || !any) throw Error(E_INVAL, "Invalid quad step or context exhausted");
    Engine& e = *eng;
    hipStream_t s = e.stream;
    StepState& hs = *e.host_state;
    std::memset(&hs, 0, sizeof(StepState));
    hs.penalty = 1.0f;
    std::vector<int> active;
    for (size_t i = 0; i < tokens.size(); ++i)
        if (tokens[i] >= 0) {
            const int q = int(active.size());
            hs.lane[q] = uint32_t(i);
            hs.pos[q] = uint32_t(positions[i]);
            hs.token[q] = tokens[i];
            active.push_back(int(i));
        }
    hs.rows = uint32_t(active.size());
    PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, s));
    PLAMO_HIP(hipEventRecord(e.ev0, s));
    e.run_step();
    PLAMO_HIP(hipEventRecord(e.ev1, s));
    // Packed query rows are temporary; the head writes logits and hidden state at each row's
    // lane, so persistent outputs stay indexed by lane (Batch.swift:167-173).
    PLAMO_HIP(hipMemcpyAsync(&hs, e.state, sizeof(StepState), hipMemcpyDeviceToHost, s));
    const hipError_t sync = hipStreamSynchronize(s);
    if (sync != hipSuccess) {
        ready = false;
        throw Error(E_DEVICE, std::string("Quad execution failed: ") + hipGetErrorString(sync));
    }
    float ms = 0;
    PLAMO_HIP(hipEventElapsedTime(&ms, e.ev0, e.ev1));
    gpu_seconds += ms / 1000.0;
    for (size_t q = 0; q < active.size(); ++q) {
        lane_next[active[q]] = int32_t(hs.next[q]);
        positions[active[q]] += 1;
    }
    return std::vector<int32_t>(lane_next, lane_next + positions.size());
}

// decodeBatch (BatchDecode.swift:8-37) after a prefill, with the lane bookkeeping and the
// token feedback on the device: 16 graph replays per host synchronisation.
BatchImpl::Decoded BatchImpl::decode(const std::vector<int32_t>& first, const std::vector<int32_t>& limits,
                                     bool stop_on_truncation) {
    const int count = int(first.size());
    bool ok = ready && count >= 1 && count <= ROWS && int(limits.size()) == count && count == int(positions.size());
    for (int i = 0; ok && i < count; ++i)
        ok = first[i] >= 0 && first[i] < VOCAB && limits[i] >= 0 && limits[i] <= 8191 &&
             positions[i] + limits[i] <= rt->context;
    if (!ok) throw Error(E_INVAL, "Invalid quad decode inputs");
    Engine& e = *eng;
    hipStream_t s = e.stream;
    StepState& hs = *e.host_state;
    std::memset(&hs, 0, sizeof(StepState));
    hs.penalty = 1.0f;
    hs.quad = 1;
    hs.lanes = uint32_t(count);
    hs.last = uint32_t(count - 1);
    hs.trunc_stop = stop_on_truncation ? 1u : 0u;
    hs.out_stride = uint32_t(rt->context) + 1;
    int max_steps = 0;
    for (int i = 0; i < count; ++i) {
        hs.lpos[i] = uint32_t(positions[i]);
        hs.lnext[i] = first[i];
        hs.llimit[i] = uint32_t(limits[i]);
        max_steps = std::max(max_steps, limits[i]);
    }
    PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, s));
    PLAMO_HIP(hipEventRecord(e.ev0, s));
    // every step with running lanes emits a token on each of them, so the lane pass stops
    // the loop after at most max(limit) + 1 steps
    int launched = 0;
    e.begin_loop();
    while (true) {
        e.run_steps(16);
        launched += 16;
        PLAMO_HIP(hipMemcpyAsync(&hs, e.state, sizeof(StepState), hipMemcpyDeviceToHost, s));
        const hipError_t sync = hipStreamSynchronize(s);
        if (sync != hipSuccess) {
            ready = false;
            throw Error(E_DEVICE, std::string("Quad execution failed: ") + hipGetErrorString(sync));
        }
        if (hs.stopped) break;
        if (launched > max_steps + 16) {
            ready = false;
            throw Error(E_DEVICE, "Quad device loop did not stop");
        }
    }
    PLAMO_HIP(hipEventRecord(e.ev1, s));
    PLAMO_HIP(hipEventSynchronize(e.ev1));
    float ms = 0;
    PLAMO_HIP(hipEventElapsedTime(&ms, e.ev0, e.ev1));
    gpu_seconds += ms / 1000.0;
    for (int i = 0; i < count; ++i) {
        positions[i] = int64_t(hs.lpos[i]);
        lane_next[i] = hs.lnext[i];
    }
    if (hs.reason == 3) throw Error(E_INVAL, "Invalid quad predictions");
    Decoded out;
    const int lanes_out = int(hs.last) + 1;
    out.ids.resize(size_t(lanes_out));
    out.reasons.resize(size_t(lanes_out));
    for (int i = 0; i < lanes_out; ++i) {
        out.reasons[i] = int(hs.lreason[i]);
        out.ids[i].resize(hs.lcount[i]);
        if (hs.lcount[i])
            PLAMO_HIP(hipMemcpy(out.ids[i].data(), e.bufs.out_ids + size_t(i) * hs.out_stride, size_t(hs.lcount[i]) * 4,
                                hipMemcpyDeviceToHost));
    }
    return out;
}

}  // namespace plamo

namespace plamo {

// The token loop of Main.swift:235-288 with the next token fed back on the device.
std::vector<int32_t> RuntimeImpl::generate(const int32_t* prompt, int n, int max_tokens, int* reason) {
    if (n <= 0 || max_tokens < 0 || int64_t(n) + max_tokens > context)
        throw Error(E_INVAL, "Input plus output limit exceeds context");  // Main.swift:168-169
    for (int i = 0; i < n; ++i)
        if (prompt[i] < 0 || prompt[i] >= VOCAB) throw Error(E_INVAL, "Input exceeds context");
    reset();
    const auto t0 = std::chrono::steady_clock::now();
    const int first = prefill(prompt, n);  // returns after the stream synchronised
    const auto t1 = std::chrono::steady_clock::now();
    last_prefill_seconds = std::chrono::duration<double>(t1 - t0).count();
    last_decode_seconds = 0;
    *reason = 0;
    if (max_tokens == 0) return {};
    Engine& e = *eng;
    StepState& hs = *e.host_state;
    hs.rows = 1;
    hs.lane[0] = 0;
    hs.pos[0] = uint32_t(position);
    hs.token[0] = first;
    hs.loop = 1;
    hs.stop_enabled = 1;
    hs.max_tokens = uint32_t(max_tokens);
    hs.produced = 0;
    hs.reason = 0;
    hs.stopped = 0;
    sync_sampler(e, 0);
    PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, stream));
    begin_timing();
    e.begin_loop();
    int launched = 0;
    while (launched < max_tokens) {
        const int batch = std::min(16, max_tokens - launched);
        e.run_steps(batch);
        launched += batch;
        PLAMO_HIP(hipMemcpyAsync(&hs, e.state, sizeof(StepState), hipMemcpyDeviceToHost, stream));
        PLAMO_HIP(hipStreamSynchronize(stream));
        if (hs.stopped) break;
    }
    end_timing();
    last_decode_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
    PLAMO_HIP(hipGetLastError());
    std::vector<int32_t> out(hs.produced);
    if (hs.produced)
        PLAMO_HIP(hipMemcpy(out.data(), e.bufs.out_ids, size_t(hs.produced) * 4, hipMemcpyDeviceToHost));
    for (int64_t p = position; p < int64_t(hs.pos[0]); ++p) count_qsa(p, 1);
    position = hs.pos[0];
    *reason = int(hs.reason);
    hs.loop = 0;
    if (sampling) {
        history.insert(history.end(), out.begin(), out.end());
        uploaded = history.size();
    }
    last_output_rows = 1;
    predictions.assign(1, int32_t(hs.next[0]));
    return out;
}

// Back-to-back replays of the decode graph, timed with HIP events on the handle's stream.
double RuntimeImpl::bench_decode(int steps) {
    if (steps <= 0 || position + steps > context) throw Error(E_INVAL, "Invalid tokens or context exhausted");
    Engine& e = *eng;
    StepState& hs = *e.host_state;
    hs.rows = 1;
    hs.lane[0] = 0;
    hs.pos[0] = uint32_t(position);
    hs.token[0] = predictions.empty() || predictions[0] < 0 || predictions[0] >= VOCAB ? 1000 : predictions[0];
    hs.loop = 1;
    hs.stop_enabled = 0;
    hs.max_tokens = uint32_t(steps + 1);
    hs.produced = 0;
    hs.reason = 0;
    hs.stopped = 0;
    sync_sampler(e, 0);
    PLAMO_HIP(hipMemcpyAsync(e.state, &hs, sizeof(StepState), hipMemcpyHostToDevice, stream));
    e.prepare_loop_graph();  // captured outside the timed region (not run)
    e.begin_loop();
    e.run_steps(1);
    PLAMO_HIP(hipStreamSynchronize(stream));
    PLAMO_HIP(hipEventRecord(e.ev0, stream));
    e.run_steps(steps - 1);
    PLAMO_HIP(hipEventRecord(e.ev1, stream));
    PLAMO_HIP(hipEventSynchronize(e.ev1));
    float ms = 0;
    PLAMO_HIP(hipEventElapsedTime(&ms, e.ev0, e.ev1));
    PLAMO_HIP(hipMemcpyAsync(&hs, e.state, sizeof(StepState), hipMemcpyDeviceToHost, stream));
    PLAMO_HIP(hipStreamSynchronize(stream));
    PLAMO_HIP(hipGetLastError());
    position = hs.pos[0];
    hs.loop = 0;
    last_output_rows = 1;
    predictions.assign(1, int32_t(hs.next[0]));
    return steps > 1 ? double(ms) / (steps - 1) : 0.0;
}

}  // namespace plamo
