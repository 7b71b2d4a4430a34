// extern "C" boundary (include/plamo_hip.h).  No C++ exception crosses it.
#include <chrono>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <functional>

#include "../../include/plamo_hip.h"
#include "formats.h"
#include "runtime.h"
#include "tokenizer.h"

struct plamo_runtime {
    plamo::RuntimeImpl impl;
    // Batches share the runtime's stream and weights: closing the runtime while batches
    // are open defers its destruction to the last plamo_batch_close.
    int open_batches = 0;
    bool close_requested = false;
};
struct plamo_batch {
    std::unique_ptr<plamo::BatchImpl> impl;
    plamo_runtime* rt;
};

namespace {
void set_err(char* err, size_t len, const std::string& m) {
    if (err && len) {
        std::snprintf(err, len, "%s", m.c_str());
    }
}

int guard(char* err, size_t len, const std::function<void()>& f) {
    try {
        f();
        return PLAMO_OK;
    } catch (const plamo::Error& e) {
        set_err(err, len, e.what());
        return e.code;
    } catch (const std::bad_alloc&) {
        set_err(err, len, "out of host memory");
        return PLAMO_EDEVICE;
    } catch (const std::exception& e) {
        set_err(err, len, e.what());
        return PLAMO_EFORMAT;
    }
}

std::vector<std::vector<int32_t>> split_prompts(const int32_t* tokens, const int32_t* lengths, int32_t count) {
    if (count < 1 || count > 4 || !tokens || !lengths) throw plamo::Error(plamo::E_INVAL, "Expected one to four valid prompts");
    std::vector<std::vector<int32_t>> p;
    size_t off = 0;
    for (int i = 0; i < count; ++i) {
        if (lengths[i] < 0) throw plamo::Error(plamo::E_INVAL, "Expected one to four valid prompts");
        p.emplace_back(tokens + off, tokens + off + lengths[i]);
        off += size_t(lengths[i]);
    }
    return p;
}

// decodeBatch (BatchDecode.swift:8-37)
struct LaneOutput {
    std::vector<int32_t> ids;
    int reason = 0;
};

std::vector<LaneOutput> decode_batch(const std::vector<int32_t>& initial, const std::vector<int32_t>& limits,
                                     const std::function<std::vector<int32_t>(const std::vector<int32_t>&)>& step,
                                     const std::function<void(int, int)>& emit,
                                     const std::function<void(int, const LaneOutput&)>& finish, bool stop_on_truncation) {
    const int count = int(initial.size());
    bool ok = count >= 1 && count <= 4 && int(limits.size()) == count;
    for (int i = 0; ok && i < count; ++i) ok = initial[i] >= 0 && initial[i] < plamo::VOCAB && limits[i] >= 0 && limits[i] <= 8191;
    if (!ok) throw plamo::Error(plamo::E_INVAL, "Invalid quad decode inputs");
    std::vector<int32_t> next = initial;
    std::vector<LaneOutput> out(count);
    int last = count - 1;
    auto pending = [&]() {
        for (int i = 0; i <= last; ++i)
            if (!out[i].reason) return true;
        return false;
    };
    while (pending()) {
        std::vector<int32_t> tokens(count, -1);
        for (int lane = 0; lane < count; ++lane) {
            if (lane > last) break;
            if (out[lane].reason) continue;
            if (int(out[lane].ids.size()) == limits[lane]) out[lane].reason = PLAMO_REASON_LENGTH;
            else if (next[lane] == 1 || next[lane] == 16) out[lane].reason = PLAMO_REASON_STOP;
            else {
                out[lane].ids.push_back(next[lane]);
                emit(lane, next[lane]);
                if (int(out[lane].ids.size()) == limits[lane]) out[lane].reason = PLAMO_REASON_LENGTH;
                else tokens[lane] = next[lane];
            }
            if (out[lane].reason) {
                if (stop_on_truncation && out[lane].reason == PLAMO_REASON_LENGTH) last = std::min(last, lane);
                finish(lane, out[lane]);
            }
        }
        bool any = false;
        for (int32_t t : tokens) any |= t >= 0;
        if (!any) break;
        next = step(tokens);
        bool valid = int(next.size()) == count;
        for (int i = 0; valid && i < count; ++i) valid = next[i] >= 0 && next[i] < plamo::VOCAB;
        if (!valid) throw plamo::Error(plamo::E_INVAL, "Invalid quad predictions");
    }
    out.resize(size_t(last) + 1);
    return out;
}

struct CallbackAbort {};

void write_outputs(const std::vector<LaneOutput>& res, int32_t* ids, int32_t stride, int32_t* lengths, int32_t* reasons,
                   int32_t* lanes) {
    for (size_t i = 0; i < res.size(); ++i) {
        const int n = int(res[i].ids.size());
        if (n > stride) throw plamo::Error(plamo::E_INVAL, "output buffer too small");
        if (ids && n > 0) std::memcpy(ids + i * size_t(stride), res[i].ids.data(), size_t(n) * 4);
        if (lengths) lengths[i] = n;
        if (reasons) reasons[i] = res[i].reason;
    }
    if (lanes) *lanes = int32_t(res.size());
}
}  // namespace

extern "C" {

const char* plamo_version(void) {
    static char text[96];
    std::snprintf(text, sizeof(text), "plamo_hip 0.1 gfx950 HIP %d.%d.%d", HIP_VERSION_MAJOR, HIP_VERSION_MINOR,
                  HIP_VERSION_PATCH);
    return text;
}

int plamo_open(const char* directory, int32_t context, int32_t packed, const char* sha, plamo_runtime** out, char* err,
               size_t errlen) {
    return guard(err, errlen, [&] {
        if (!out || !directory) throw plamo::Error(plamo::E_INVAL, "null argument");
        *out = nullptr;
        if (context < 1 || context > plamo::MAX_CONTEXT) throw plamo::Error(plamo::E_INVAL, "Context must be 1...32768");
        auto rt = std::make_unique<plamo_runtime>();
        auto& r = rt->impl;
        r.context = context;
        int dev = 0;
        if (hipGetDeviceCount(&dev) != hipSuccess || dev < 1)
            throw plamo::Error(plamo::E_DEVICE, "An MI355X (gfx950) HIP device is required");
        PLAMO_HIP(hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking));
        r.model = plamo::load_model(directory, context, packed != 0, sha ? sha : "", r.stream);
        r.eng = std::make_unique<plamo::Engine>(r.model, context, 1, r.stream);
        *out = rt.release();
    });
}

int plamo_open_aux(const char* directory, int32_t context, int32_t packed, const char* sha, int32_t qsa_budget,
                   int32_t mtp, plamo_runtime** out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!out || !directory) throw plamo::Error(plamo::E_INVAL, "null argument");
        *out = nullptr;
        // Runtime.swift:165,171-175: context, budget, then the adapters before the model
        if (context < 1 || context > plamo::MAX_CONTEXT) throw plamo::Error(plamo::E_INVAL, "Context must be 1...32768");
        if (qsa_budget != 0 && (qsa_budget < 4 || qsa_budget > 2048 || qsa_budget % 4 != 0))
            throw plamo::Error(plamo::E_INVAL, "QSA budget must be a multiple of four in 4...2048");
        const bool indexers = qsa_budget > 0 && context > qsa_budget;  // Runtime.swift:248
        std::unique_ptr<plamo::AuxArchive> ar;
        if (qsa_budget > 0 || mtp) {
            ar = std::make_unique<plamo::AuxArchive>(std::string(directory) + "/auxiliary.safetensors", sha ? sha : "");
            plamo::check_aux_tensors(*ar, mtp != 0, false);  // the Predictor before the model
        }
        auto rt = std::make_unique<plamo_runtime>();
        auto& r = rt->impl;
        r.context = context;
        int dev = 0;
        if (hipGetDeviceCount(&dev) != hipSuccess || dev < 1)
            throw plamo::Error(plamo::E_DEVICE, "An MI355X (gfx950) HIP device is required");
        PLAMO_HIP(hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking));
        r.model = plamo::load_model(directory, context, packed != 0, sha ? sha : "", r.stream);
        r.eng = std::make_unique<plamo::Engine>(r.model, context, 1, r.stream);
        if (ar) r.aux = plamo::load_aux(*ar, mtp != 0, indexers);  // indexers after the layers
        if (indexers) r.eng->enable_qsa(r.aux.get(), qsa_budget);
        r.mtp = mtp != 0;
        r.qsa_budget = qsa_budget;
        *out = rt.release();
    });
}

void plamo_close(plamo_runtime* rt) {
    if (!rt) return;
    if (rt->open_batches > 0) {
        rt->close_requested = true;
        return;
    }
    delete rt;
}

void plamo_reset(plamo_runtime* rt) {
    if (rt) rt->impl.reset();
}

int plamo_forward(plamo_runtime* rt, const int32_t* tokens, int32_t count, int32_t output, int32_t* next, char* err,
                  size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt || (!tokens && count)) throw plamo::Error(plamo::E_INVAL, "Invalid tokens or context exhausted");
        const int n = rt->impl.forward(tokens, count, output != 0);
        if (next) *next = n;
    });
}

int plamo_forward_ex(plamo_runtime* rt, const int32_t* tokens, int32_t count, int32_t output, int32_t all,
                     int32_t sequential, int32_t* next, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt || (!tokens && count)) throw plamo::Error(plamo::E_INVAL, "Invalid tokens or context exhausted");
        const int n = rt->impl.forward_ex(tokens, count, output != 0, all != 0, sequential != 0);
        if (next) *next = n;
    });
}

int plamo_draft(plamo_runtime* rt, int32_t first, int32_t* draft, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt) throw plamo::Error(plamo::E_INVAL, "null argument");
        const int d = rt->impl.draft(first);
        if (draft) *draft = d;
    });
}

int plamo_rewind(plamo_runtime* rt, int64_t new_position, int32_t hidden_index, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt) throw plamo::Error(plamo::E_INVAL, "null argument");
        rt->impl.rewind(new_position, hidden_index);
    });
}

int plamo_prefill(plamo_runtime* rt, const int32_t* tokens, int32_t count, int32_t* next, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt || (!tokens && count)) throw plamo::Error(plamo::E_INVAL, "Input exceeds context");
        const int n = rt->impl.prefill(tokens, count);
        if (next) *next = n;
    });
}

int plamo_logits_bf16(plamo_runtime* rt, int32_t slot, uint16_t* bits, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt || !bits || slot < 0 || slot >= std::max(1, rt->impl.last_output_rows))
            throw plamo::Error(plamo::E_INVAL, "Invalid logits slot");
        PLAMO_HIP(hipMemcpy(bits, rt->impl.logits_row(slot), plamo::VOCAB * 2, hipMemcpyDeviceToHost));
    });
}

int plamo_logits(plamo_runtime* rt, int32_t slot, float* values, char* err, size_t errlen) {
    std::vector<uint16_t> b(plamo::VOCAB);
    int rc = plamo_logits_bf16(rt, slot, b.data(), err, errlen);
    if (rc) return rc;
    if (!values) return PLAMO_EINVAL;
    for (int i = 0; i < plamo::VOCAB; ++i) values[i] = plamo::host_bf(b[i]);
    return PLAMO_OK;
}

int plamo_hidden(plamo_runtime* rt, float* values, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt || !values) throw plamo::Error(plamo::E_INVAL, "null argument");
        PLAMO_HIP(hipMemcpy(values, rt->impl.hidden_row(), plamo::HIDDEN * 4, hipMemcpyDeviceToHost));
    });
}

int plamo_predictions(plamo_runtime* rt, int32_t* out, int32_t capacity, int32_t* count) {
    if (!rt) return PLAMO_EINVAL;
    const int n = rt->impl.last_output_rows ? int(rt->impl.predictions.size()) : 0;
    for (int i = 0; i < n && i < capacity; ++i) out[i] = rt->impl.predictions[i];
    if (count) *count = n;
    return PLAMO_OK;
}

int plamo_get_stats(plamo_runtime* rt, plamo_stats* s) {
    if (!rt || !s) return PLAMO_EINVAL;
    auto& r = rt->impl;
    s->position = r.position;
    s->gpu_seconds = r.gpu_seconds;
    s->device_bytes = int64_t(r.model->arena.bytes() + r.eng->arena.bytes());
    s->weight_bytes = r.model->weight_bytes;
    s->linear_bytes = r.model->linear_bytes;
    s->context = r.context;
    s->packed = r.model->packed ? 1 : 0;
    s->last_output_rows = r.last_output_rows;
    s->local_capacity = r.eng->local_capacity;
    s->last_prefill_seconds = r.last_prefill_seconds;
    s->last_decode_seconds = r.last_decode_seconds;
    s->auxiliary_bytes = r.aux ? r.aux->bytes : 0;
    s->sparse_queries = r.sparse_queries;
    s->sparse_keys = r.sparse_keys;
    s->dense_keys = r.dense_keys;
    s->device_bytes += r.aux ? int64_t(r.aux->arena.bytes()) : 0;
    return PLAMO_OK;
}

int plamo_kv(plamo_runtime* rt, int32_t layer, uint16_t* keys, uint16_t* values, int32_t* capacity, char* err,
             size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt || layer < 0 || layer >= plamo::LAYERS) throw plamo::Error(plamo::E_INVAL, "Invalid layer");
        auto& e = *rt->impl.eng;
        const size_t n = size_t(e.capacity[layer]) * plamo::HEAD_DIM * 2;
        if (keys) PLAMO_HIP(hipMemcpy(keys, e.keys[layer], n, hipMemcpyDeviceToHost));
        if (values) PLAMO_HIP(hipMemcpy(values, e.values[layer], n, hipMemcpyDeviceToHost));
        if (capacity) *capacity = e.capacity[layer];
    });
}

int plamo_set_sampling(plamo_runtime* rt, float penalty, float frequency, float presence, int32_t ngram) {
    if (!rt) return PLAMO_EINVAL;
    auto& r = rt->impl;
    r.penalty = penalty;
    r.frequency = frequency;
    r.presence = presence;
    r.ngram = ngram;
    r.sampling = penalty != 1.0f || frequency != 0.0f || presence != 0.0f || ngram > 1;
    return PLAMO_OK;
}

int plamo_sampler_observe(plamo_runtime* rt, int32_t id) {
    if (!rt) return PLAMO_EINVAL;
    rt->impl.history.push_back(id);
    return PLAMO_OK;
}

int plamo_generate(plamo_runtime* rt, const int32_t* prompt, int32_t count, int32_t max_tokens, int32_t* out_ids,
                   int32_t* out_count, int32_t* stop_reason, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt || !prompt) throw plamo::Error(plamo::E_INVAL, "null argument");
        int reason = 0;
        auto ids = rt->impl.generate(prompt, count, max_tokens, &reason);
        if (out_ids && !ids.empty()) std::memcpy(out_ids, ids.data(), ids.size() * 4);
        if (out_count) *out_count = int32_t(ids.size());
        if (stop_reason) *stop_reason = reason == 1 ? 1 : 0;
        if (reason == 3) throw plamo::Error(plamo::E_INVAL, "Invalid tokens or context exhausted");
    });
}

int plamo_bench_decode(plamo_runtime* rt, int32_t steps, double* ms, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt) throw plamo::Error(plamo::E_INVAL, "null argument");
        const double v = rt->impl.bench_decode(steps);
        if (ms) *ms = v;
    });
}

// ---------------------------------------------------------------------------- batch
int plamo_batch_open(plamo_runtime* rt, plamo_batch** out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!rt || !out) throw plamo::Error(plamo::E_INVAL, "null argument");
        auto b = std::make_unique<plamo_batch>();
        b->rt = rt;
        b->impl = std::make_unique<plamo::BatchImpl>(&rt->impl);
        rt->open_batches += 1;
        *out = b.release();
    });
}

void plamo_batch_close(plamo_batch* b) {
    if (!b) return;
    plamo_runtime* rt = b->rt;
    delete b;
    if (rt && --rt->open_batches == 0 && rt->close_requested) delete rt;
}

int plamo_batch_prefill(plamo_batch* b, const int32_t* tokens, const int32_t* lengths, int32_t count, int32_t* next,
                        char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!b) throw plamo::Error(plamo::E_INVAL, "null argument");
        auto res = b->impl->prefill(split_prompts(tokens, lengths, count));
        if (next && !res.empty()) std::memcpy(next, res.data(), res.size() * 4);
    });
}

int plamo_batch_step(plamo_batch* b, const int32_t* tokens, int32_t count, int32_t* next, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!b || !tokens || count < 0) throw plamo::Error(plamo::E_INVAL, "Invalid quad step or context exhausted");
        auto res = b->impl->step(std::vector<int32_t>(tokens, tokens + count));
        if (next && !res.empty()) std::memcpy(next, res.data(), res.size() * 4);
    });
}

void plamo_batch_reset(plamo_batch* b) {
    if (b) b->impl->reset();
}

int plamo_batch_logits_bf16(plamo_batch* b, int32_t lane, uint16_t* bits, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!b || !bits || lane < 0 || lane >= plamo::ROWS) throw plamo::Error(plamo::E_INVAL, "Invalid lane");
        PLAMO_HIP(hipMemcpy(bits, b->impl->lane_logits + size_t(lane) * plamo::VOCAB, plamo::VOCAB * 2,
                            hipMemcpyDeviceToHost));
    });
}

int plamo_batch_hidden(plamo_batch* b, int32_t lane, float* values, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!b || !values || lane < 0 || lane >= plamo::ROWS) throw plamo::Error(plamo::E_INVAL, "Invalid lane");
        PLAMO_HIP(hipMemcpy(values, b->impl->lane_hidden + size_t(lane) * plamo::HIDDEN, plamo::HIDDEN * 4,
                            hipMemcpyDeviceToHost));
    });
}

int plamo_batch_kv(plamo_batch* b, int32_t lane, int32_t layer, uint16_t* keys, uint16_t* values, int32_t* capacity,
                   char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!b || lane < 0 || lane >= plamo::ROWS || layer < 0 || layer >= plamo::LAYERS)
            throw plamo::Error(plamo::E_INVAL, "Invalid lane or layer");
        auto& e = *b->impl->eng;
        const size_t n = size_t(e.capacity[layer]) * plamo::HEAD_DIM;
        if (keys) PLAMO_HIP(hipMemcpy(keys, e.keys[layer] + size_t(lane) * n, n * 2, hipMemcpyDeviceToHost));
        if (values) PLAMO_HIP(hipMemcpy(values, e.values[layer] + size_t(lane) * n, n * 2, hipMemcpyDeviceToHost));
        if (capacity) *capacity = e.capacity[layer];
    });
}

int plamo_batch_fill_kv(plamo_batch* b, uint16_t bits) {
    return guard(nullptr, 0, [&] {
        if (!b) throw plamo::Error(plamo::E_INVAL, "Invalid batch");
        auto& e = *b->impl->eng;
        for (int l = 0; l < plamo::LAYERS; ++l) {
            const size_t n = size_t(e.lanes) * size_t(e.capacity[l]) * plamo::HEAD_DIM;
            PLAMO_HIP(hipMemsetD16Async(e.keys[l], bits, n, e.stream));
            PLAMO_HIP(hipMemsetD16Async(e.values[l], bits, n, e.stream));
            if (e.keys_rot[l])
                PLAMO_HIP(hipMemsetD16Async(e.keys_rot[l], bits, size_t(e.lanes) * e.rot_rows[l] * plamo::HEAD_DIM, e.stream));
        }
        PLAMO_HIP(hipStreamSynchronize(e.stream));
    });
}

int plamo_batch_positions(plamo_batch* b, int32_t* out, int32_t capacity, int32_t* count) {
    if (!b) return PLAMO_EINVAL;
    const auto& p = b->impl->positions;
    for (size_t i = 0; i < p.size() && int32_t(i) < capacity; ++i) out[i] = int32_t(p[i]);
    if (count) *count = int32_t(p.size());
    return PLAMO_OK;
}

int plamo_decode_batch(const int32_t* initial, const int32_t* limits, int32_t count, plamo_step_fn step,
                       plamo_emit_fn emit, plamo_finish_fn finish, void* user, int32_t stop_on_truncation, int32_t* ids,
                       int32_t ids_stride, int32_t* lengths, int32_t* reasons, int32_t* lanes, char* err,
                       size_t errlen) {
    return guard(err, errlen, [&] {
        if (!initial || !limits || !step || count < 1 || count > 4)
            throw plamo::Error(plamo::E_INVAL, "Invalid quad decode inputs");
        auto res = decode_batch(
            std::vector<int32_t>(initial, initial + count), std::vector<int32_t>(limits, limits + count),
            [&](const std::vector<int32_t>& t) {
                std::vector<int32_t> next(size_t(count), -1);
                if (step(user, t.data(), count, next.data()) != 0)
                    throw plamo::Error(plamo::E_STATE, "step callback aborted");
                return next;
            },
            [&](int lane, int id) {
                if (emit && emit(user, lane, id) != 0) throw plamo::Error(plamo::E_STATE, "emit callback aborted");
            },
            [&](int lane, const LaneOutput& o) {
                if (finish && finish(user, lane, o.ids.data(), int32_t(o.ids.size()), o.reason) != 0)
                    throw plamo::Error(plamo::E_STATE, "finish callback aborted");
            },
            stop_on_truncation != 0);
        write_outputs(res, ids, ids_stride, lengths, reasons, lanes);
    });
}

int plamo_batch_generate(plamo_batch* b, const int32_t* tokens, const int32_t* lengths, const int32_t* limits,
                         int32_t count, int32_t stop_on_truncation, int32_t* ids, int32_t ids_stride,
                         int32_t* out_lengths, int32_t* reasons, int32_t* lanes, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!b || !limits) throw plamo::Error(plamo::E_INVAL, "Quad output budget exceeds context");
        auto prompts = split_prompts(tokens, lengths, count);
        // Batch.generate (BatchDecode.swift:40-47)
        for (int i = 0; i < count; ++i)
            if (limits[i] < 0 || limits[i] > 8191 || int64_t(prompts[i].size()) + limits[i] > b->rt->impl.context)
                throw plamo::Error(plamo::E_INVAL, "Quad output budget exceeds context");
        try {
            auto first = b->impl->prefill(prompts);
            // decodeBatch with no callbacks runs as the device loop: same lane pass, no host
            // round trip per step
            auto dec = b->impl->decode(first, std::vector<int32_t>(limits, limits + count), stop_on_truncation != 0);
            std::vector<LaneOutput> res(dec.ids.size());
            for (size_t i = 0; i < res.size(); ++i) {
                res[i].ids = std::move(dec.ids[i]);
                res[i].reason = dec.reasons[i];
            }
            write_outputs(res, ids, ids_stride, out_lengths, reasons, lanes);
        } catch (...) {
            b->impl->reset();
            throw;
        }
    });
}

int plamo_batch_decode(plamo_batch* b, const int32_t* initial, const int32_t* limits, int32_t count,
                       int32_t stop_on_truncation, int32_t* ids, int32_t ids_stride, int32_t* lengths,
                       int32_t* reasons, int32_t* lanes, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!b || !initial || !limits || count < 1 || count > plamo::ROWS)
            throw plamo::Error(plamo::E_INVAL, "Invalid quad decode inputs");
        auto dec = b->impl->decode(std::vector<int32_t>(initial, initial + count),
                                   std::vector<int32_t>(limits, limits + count), stop_on_truncation != 0);
        std::vector<LaneOutput> res(dec.ids.size());
        for (size_t i = 0; i < res.size(); ++i) {
            res[i].ids = std::move(dec.ids[i]);
            res[i].reason = dec.reasons[i];
        }
        write_outputs(res, ids, ids_stride, lengths, reasons, lanes);
    });
}

// ------------------------------------------------------------------- weight formats
int plamo_pack(const char* src, const char* out, const char* sha, plamo_pack_report* report, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!src || !out) throw plamo::Error(plamo::E_INVAL, "null argument");
        auto r = plamo::pack_archive(src, out, sha ? sha : "");
        if (report) {
            report->original_linear_bytes = r.original_linear_bytes;
            report->packed_linear_bytes = r.packed_linear_bytes;
            report->archive_bytes = r.archive_bytes;
            report->compressed_blocks = r.compressed_blocks;
            report->blocks = r.blocks;
        }
    });
}

int plamo_pack_tensor(const uint16_t* values, int64_t count, uint8_t* payload, int64_t payload_cap, uint32_t* table,
                      int64_t* payload_bytes, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!values || !payload || !table || count <= 0 || count % 128 != 0)
            throw plamo::Error(plamo::E_INVAL, "pack_tensor expects a multiple of 128 values");
        std::vector<uint32_t> entries;
        auto data = plamo::pack_blocks(values, size_t(count), entries, nullptr);
        if (int64_t(data.size()) > payload_cap) throw plamo::Error(plamo::E_INVAL, "payload buffer too small");
        std::memcpy(payload, data.data(), data.size());
        std::memcpy(table, entries.data(), entries.size() * 4);
        if (payload_bytes) *payload_bytes = int64_t(data.size());
    });
}

int plamo_check_aux(const char* path, const char* teacher_sha256, int32_t mtp, int32_t qsa, char* err,
                    size_t errlen) {
    return guard(err, errlen, [&] {
        if (!path) throw plamo::Error(plamo::E_INVAL, "null argument");
        plamo::AuxArchive ar(path, teacher_sha256 ? teacher_sha256 : "");
        plamo::check_aux_tensors(ar, mtp != 0, qsa != 0);
    });
}

int plamo_check_weights(const char* path, const char* name, const int64_t* shape, int32_t ndim, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        plamo::SafeTensors st(path ? path : "");
        if (name) st.tensor(name, std::vector<int64_t>(shape, shape + ndim));
    });
}

int plamo_check_packed(const char* path, const char* sha, const char* name, const int64_t* shape, int32_t ndim,
                       int32_t* is_packed, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        plamo::PackedArchive pk(path ? path : "", sha ? sha : "");
        if (name) {
            auto t = pk.tensor(name, std::vector<int64_t>(shape, shape + ndim));
            if (is_packed) *is_packed = t.blocked ? 1 : 0;
        }
    });
}

// ------------------------------------------------------------------- kernel entries
int plamo_kernel_linear(uint64_t w, uint64_t table, uint64_t x, uint64_t y, int32_t n, int32_t m, int32_t rows,
                        int32_t mode, uint64_t stream) {
    return guard(nullptr, 0, [&] {
        if (rows < 1 || rows > plamo::ROWS || m < 4 || (n != 1536 && n != 2048 && n != 6144) ||
            m % (n >= 6144 ? 2 : 4) != 0 || mode < 0 || mode > 2)
            throw plamo::Error(plamo::E_INVAL, "unsupported linear shape");
        plamo::GemvParams g{};
        g.w = reinterpret_cast<const uint16_t*>(w);
        g.table = reinterpret_cast<const uint32_t*>(table);
        g.m = m;
        g.rows = rows;
        g.in = reinterpret_cast<const float*>(x);
        g.out = reinterpret_cast<float*>(y);
        g.out16 = reinterpret_cast<uint16_t*>(y);
        const int maxr = rows == 1 ? 1 : plamo::ROWS;
        const plamo::Epilogue epi = mode == 2 ? plamo::EPI_BF16 : mode == 1 ? plamo::EPI_RAW : plamo::EPI_ROUND;
        if (m % plamo::gemv_group_rows(n, maxr, epi, table != 0) != 0)
            throw plamo::Error(plamo::E_INVAL, "GEMV rows must be a multiple of the rows per wave group");
        const int blocks = std::max(1, std::min(4096, plamo::gemv_blocks(n, maxr, epi, m, table != 0)));
        plamo::launch_gemv(n, table != 0, maxr, plamo::PRO_PLAIN, epi, g, blocks, reinterpret_cast<hipStream_t>(stream));
        PLAMO_HIP(hipGetLastError());
    });
}

int plamo_kernel_unpack(uint64_t payload, uint64_t table, uint64_t out, int64_t count, uint64_t stream) {
    return guard(nullptr, 0, [&] {
        plamo::launch_unpack(reinterpret_cast<const uint8_t*>(payload), reinterpret_cast<const uint32_t*>(table),
                             reinterpret_cast<uint16_t*>(out), count, reinterpret_cast<hipStream_t>(stream));
        PLAMO_HIP(hipGetLastError());
    });
}

int plamo_kernel_argmax(uint64_t x, uint64_t out, int32_t n, int32_t rows, int32_t bf16, uint64_t stream) {
    return guard(nullptr, 0, [&] {
        if (n < 1 || rows < 1) throw plamo::Error(plamo::E_INVAL, "bad argmax shape");
        plamo::launch_argmax(reinterpret_cast<const void*>(x), reinterpret_cast<uint32_t*>(out), n, rows, bf16 != 0,
                             reinterpret_cast<hipStream_t>(stream));
        PLAMO_HIP(hipGetLastError());
    });
}

int plamo_kernel_select(uint64_t logits, int32_t n, uint64_t history, int32_t hist, float penalty, int32_t ngram,
                        float frequency, float presence, uint64_t out, uint64_t stream) {
    return guard(nullptr, 0, [&] {
        if (n < 1 || hist < 0) throw plamo::Error(plamo::E_INVAL, "bad select shape");
        plamo::launch_select(reinterpret_cast<float*>(logits), n, reinterpret_cast<const int32_t*>(history), hist,
                             penalty, ngram, frequency, presence, reinterpret_cast<int32_t*>(out),
                             reinterpret_cast<hipStream_t>(stream));
        PLAMO_HIP(hipGetLastError());
    });
}

int plamo_kernel_qsa_select(uint64_t scores, int32_t blocks, int32_t tokens, int32_t start, int32_t budget,
                            uint64_t out, uint64_t stream) {
    return guard(nullptr, 0, [&] {
        if (blocks < 1 || blocks > plamo::MAX_CONTEXT / 4 || tokens < 1 || start < 0 || budget < 0)
            throw plamo::Error(plamo::E_INVAL, "bad QSA select shape");
        // every row's complete blocks must lie inside its score row
        if (int64_t(start) + tokens > 4 * int64_t(blocks) + 3)
            throw plamo::Error(plamo::E_INVAL, "QSA select: positions past the score rows");
        if (!scores || !out) throw plamo::Error(plamo::E_INVAL, "null QSA select operand");
        plamo::QsaParams p{};
        p.p0 = uint32_t(start);
        p.tokens = tokens;
        p.scores = reinterpret_cast<float*>(scores);
        p.mask = reinterpret_cast<uint32_t*>(out);
        p.blocks = uint32_t(blocks);
        p.words = uint32_t((blocks + 31) / 32);
        p.budget = budget;
        plamo::launch_qsa_select(p, reinterpret_cast<hipStream_t>(stream));
        PLAMO_HIP(hipGetLastError());
    });
}

int plamo_kernel_gemm(uint64_t w, uint64_t table, uint64_t x, uint64_t y, int32_t n, int32_t m, int32_t tokens,
                      int32_t out_bf16, uint64_t stream) {
    return guard(nullptr, 0, [&] {
        if (n % 128 != 0 || m < 1 || tokens < 1) throw plamo::Error(plamo::E_INVAL, "bad GEMM shape");
        if (!w || !x || !y) throw plamo::Error(plamo::E_INVAL, "null GEMM operand");
        plamo::GemmParams g{};
        g.w = reinterpret_cast<const uint16_t*>(w);
        g.table = reinterpret_cast<const uint32_t*>(table);
        g.x = reinterpret_cast<const uint16_t*>(x);
        g.y = reinterpret_cast<float*>(y);
        g.y16 = reinterpret_cast<uint16_t*>(y);
        g.m = m;
        g.k = n;
        g.tokens = tokens;
        if (out_bf16 < 0 || out_bf16 > 3) throw plamo::Error(plamo::E_INVAL, "bad GEMM output mode");
        if (out_bf16 == 3 && (m != 2 * plamo::INTER || n != plamo::HIDDEN))
            throw plamo::Error(plamo::E_INVAL, "SwiGLU GEMM needs the 12288 x 1536 gate_up weight");
        const plamo::GemmEpilogue epi = out_bf16 == 1   ? plamo::GEMM_BF16
                                        : out_bf16 == 2 ? plamo::GEMM_RAW
                                        : out_bf16 == 3 ? plamo::GEMM_SWIGLU
                                                        : plamo::GEMM_F32;
        plamo::launch_gemm(table != 0, epi, g,
                           reinterpret_cast<hipStream_t>(stream));
        PLAMO_HIP(hipGetLastError());
    });
}

}  // extern "C" (the helper below is C++ only)

namespace {
// Workspace of the split flash prefill for the kernel-level entry, per device, grown on demand
// (the runtime keeps its own).  Growing synchronises the device before freeing the old one.
struct FlashWorkspace {
    float* o = nullptr;
    float* ml = nullptr;
    uint32_t* tickets = nullptr;
    int tokens = 0;
};
std::mutex g_flash_ws_mu;
std::map<int, FlashWorkspace> g_flash_ws;

FlashWorkspace flash_workspace(int tokens) {
    std::lock_guard<std::mutex> lk(g_flash_ws_mu);
    int dev = 0;
    PLAMO_HIP(hipGetDevice(&dev));
    FlashWorkspace& w = g_flash_ws[dev];
    if (w.tokens < tokens) {
        if (w.o) {
            PLAMO_HIP(hipDeviceSynchronize());
            (void)hipFree(w.o);
            (void)hipFree(w.ml);
            (void)hipFree(w.tickets);
            w = FlashWorkspace{};
        }
        PLAMO_HIP(hipMalloc(&w.o, plamo::flash_part_o_floats(tokens) * 4));
        PLAMO_HIP(hipMalloc(&w.ml, plamo::flash_part_ml_floats(tokens) * 4));
        PLAMO_HIP(hipMalloc(&w.tickets, size_t(plamo::flash_blocks(tokens)) * 4));
        PLAMO_HIP(hipMemset(w.tickets, 0, size_t(plamo::flash_blocks(tokens)) * 4));
        w.tokens = tokens;
    }
    return w;
}

// Workspace of the kernel-level decode attention, per device, grown on demand: the step
// state, the attention tickets [ROWS][4 head groups] and the partition statistics and
// outputs [ROWS][parts][16] (x128 for the outputs), the layout the runtime's engine uses.
struct AttnWorkspace {
    void* base = nullptr;
    uint32_t parts = 0;
};
std::mutex g_attn_ws_mu;
std::map<int, AttnWorkspace> g_attn_ws;


// Carves a workspace at `base` (256-byte aligned) into the attention parameter pointers.
void attn_workspace_bind(void* base, uint32_t parts, plamo::AttnParams& a, plamo::StepState*& st) {
    uint8_t* b = static_cast<uint8_t*>(base);
    const size_t stats = size_t(plamo::ROWS) * parts * plamo::HEADS;
    st = reinterpret_cast<plamo::StepState*>(b);
    a.tickets = reinterpret_cast<uint32_t*>(b + 256);
    a.part_m = reinterpret_cast<float*>(b + 512);
    a.part_l = a.part_m + stats;
    a.part_o = a.part_l + stats;
}

void* attn_workspace(uint32_t parts) {
    std::lock_guard<std::mutex> lk(g_attn_ws_mu);
    int dev = 0;
    PLAMO_HIP(hipGetDevice(&dev));
    AttnWorkspace& w = g_attn_ws[dev];
    if (w.parts < parts) {
        if (w.base) {
            PLAMO_HIP(hipDeviceSynchronize());
            (void)hipFree(w.base);
            w = AttnWorkspace{};
        }
        PLAMO_HIP(hipMalloc(&w.base, plamo::attn_workspace_bytes(parts)));
        w.parts = parts;
    }
    return w.base;
}


// Validates a kernel-level decode attention call and fills every parameter except the
// workspace pointers; returns the partition count (grid width).
uint32_t attn_decode_params(uint64_t qkv, uint64_t q_norm, uint64_t k_norm, uint64_t keys, uint64_t values,
                            int32_t capacity, const int32_t* positions, int32_t rows, int32_t full,
                            uint64_t local_rope, uint64_t global_rope, uint64_t out16, plamo::AttnParams& a) {
    if (rows < 1 || rows > plamo::ROWS || !positions || !qkv || !q_norm || !k_norm || !keys || !values || !out16 ||
        !local_rope || (full && !global_rope) || capacity < 1 || capacity > plamo::MAX_CONTEXT)
        throw plamo::Error(plamo::E_INVAL, "bad attention arguments");
    int64_t most = 1;
    for (int32_t q = 0; q < rows; ++q) {
        const int64_t pos = positions[q];
        if (pos < 0 || pos >= plamo::MAX_CONTEXT) throw plamo::Error(plamo::E_INVAL, "bad attention position");
        // visible keys: 0..pos (global), the 2048-key window ending at pos (local); all of
        // them must be resident in the lane's cache at once
        const int64_t count = full ? pos + 1 : std::min<int64_t>(pos + 1, plamo::WINDOW);
        if (full ? pos >= capacity : count > capacity)
            throw plamo::Error(plamo::E_INVAL, "attention keys exceed the cache capacity");
        most = std::max(most, count);
    }
    a.qkv = reinterpret_cast<const float*>(qkv);
    a.q_norm = reinterpret_cast<const uint16_t*>(q_norm);
    a.k_norm = reinterpret_cast<const uint16_t*>(k_norm);
    a.keys = reinterpret_cast<uint16_t*>(keys);
    a.values = reinterpret_cast<uint16_t*>(values);
    a.capacity = uint32_t(capacity);
    a.local_rope = reinterpret_cast<const uint32_t*>(local_rope);
    a.global_rope = reinterpret_cast<const uint32_t*>(global_rope);
    a.out16 = reinterpret_cast<uint16_t*>(out16);
    a.parts = uint32_t((most + plamo::KEYS_PER_PART - 1) / plamo::KEYS_PER_PART);
    a.defer = full && a.parts > plamo::ATTN_MERGE_INLINE ? plamo::ATTN_MERGE_INLINE : 0;
    return a.parts;
}

void attn_decode_launch(plamo::AttnParams& a, plamo::StepState* st, const int32_t* positions, int32_t rows,
                        bool full, hipStream_t s) {
    a.state = st;
    plamo::launch_attn_state(st, a.tickets, positions, rows, s);
    plamo::launch_attention(full, a, rows, s);
    if (a.defer) plamo::launch_attention_merge(a, rows, s);
}
}  // namespace

extern "C" {

int plamo_kernel_attention_decode(uint64_t qkv, uint64_t q_norm, uint64_t k_norm, uint64_t keys, uint64_t values,
                                  int32_t capacity, const int32_t* positions, int32_t rows, int32_t full,
                                  uint64_t local_rope, uint64_t global_rope, uint64_t out16, uint64_t stream) {
    return guard(nullptr, 0, [&] {
        plamo::AttnParams a{};
        const uint32_t parts = attn_decode_params(qkv, q_norm, k_norm, keys, values, capacity, positions, rows, full,
                                                  local_rope, global_rope, out16, a);
        plamo::StepState* st = nullptr;
        attn_workspace_bind(attn_workspace(parts), parts, a, st);
        attn_decode_launch(a, st, positions, rows, full != 0, reinterpret_cast<hipStream_t>(stream));
        PLAMO_HIP(hipGetLastError());
    });
}

int plamo_kernel_attention_decode_static(uint64_t qkv, uint64_t q_norm, uint64_t k_norm, uint64_t keys,
                                         uint64_t values, int32_t capacity, const int32_t* positions, int32_t rows,
                                         int32_t full, uint64_t local_rope, uint64_t global_rope, uint64_t out16,
                                         uint64_t stream, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        plamo::AttnParams a{};
        const uint32_t parts = attn_decode_params(qkv, q_norm, k_norm, keys, values, capacity, positions, rows, full,
                                                  local_rope, global_rope, out16, a);
        if (parts > plamo::STATIC_ATTN_PARTS)
            throw plamo::Error(plamo::E_INVAL, "attention exceeds the static scratch: at most " +
                                                   std::to_string(plamo::STATIC_ATTN_PARTS * plamo::KEYS_PER_PART) +
                                                   " visible keys per row");
        plamo::StepState* st = nullptr;
        attn_workspace_bind(plamo::static_attn_scratch(), parts, a, st);
        attn_decode_launch(a, st, positions, rows, full != 0, reinterpret_cast<hipStream_t>(stream));
        PLAMO_HIP(hipGetLastError());
    });
}

int plamo_rope_table(const double* freqs, int32_t rows, int32_t global, uint32_t* out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!freqs || !out || rows <= 0 || rows > plamo::MAX_CONTEXT)
            throw plamo::Error(plamo::E_INVAL, "bad RoPE table arguments");
        const std::vector<uint32_t> t = plamo::rope_table(std::vector<double>(freqs, freqs + 64), rows, global != 0);
        std::memcpy(out, t.data(), t.size() * 4);
    });
}

int plamo_kernel_attention_prefill(uint64_t q16, uint64_t keys, uint64_t values, int32_t capacity, int32_t p0,
                                   int32_t tokens, int32_t full, uint64_t local_rope, uint64_t out16,
                                   uint64_t stream) {
    return guard(nullptr, 0, [&] {
        if (tokens < 1 || p0 < 0 || capacity < 1 || !q16 || !keys || !values || !out16 || (!full && !local_rope))
            throw plamo::Error(plamo::E_INVAL, "bad attention arguments");
        // every visible key of every query must be resident in the ring
        const int64_t span = full ? int64_t(p0) + tokens
                                  : std::min<int64_t>(int64_t(p0) + tokens, int64_t(plamo::WINDOW) - 1 + tokens);
        if (span > capacity) throw plamo::Error(plamo::E_INVAL, "attention keys exceed the cache capacity");
        plamo::FlashParams f{};
        f.q = reinterpret_cast<const uint16_t*>(q16);
        f.keys = reinterpret_cast<const uint16_t*>(keys);
        f.values = reinterpret_cast<const uint16_t*>(values);
        f.local_rope = reinterpret_cast<const uint32_t*>(local_rope);
        f.out = reinterpret_cast<uint16_t*>(out16);
        f.capacity = uint32_t(capacity);
        f.p0 = uint32_t(p0);
        f.tokens = tokens;
        f.full = full ? 1 : 0;
        const FlashWorkspace ws = flash_workspace(tokens);
        f.part_o = ws.o;
        f.part_ml = ws.ml;
        f.tickets = ws.tickets;
        plamo::launch_flash_prefill(f, reinterpret_cast<hipStream_t>(stream));
        PLAMO_HIP(hipGetLastError());
    });
}


// ---- tokenizer (host only)
struct plamo_tokenizer {
    plamo::Tokenizer tok;
    explicit plamo_tokenizer(const std::string& path) : tok(path) {}
};
struct plamo_token_stream {
    plamo::TokenStream stream;
    explicit plamo_token_stream(const plamo::Tokenizer& t) : stream(t) {}
};

static void put_bytes(const std::string& s, char* out, size_t cap, size_t* n_out) {
    if (n_out) *n_out = s.size();
    if (s.size() > cap || (!out && !s.empty())) throw plamo::Error(plamo::E_INVAL, "output buffer too small");
    if (!s.empty()) std::memcpy(out, s.data(), s.size());
}

int plamo_tokenizer_open(const char* path, plamo_tokenizer** out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!path || !out) throw plamo::Error(plamo::E_INVAL, "bad tokenizer arguments");
        *out = nullptr;
        *out = new plamo_tokenizer(path);
    });
}

void plamo_tokenizer_close(plamo_tokenizer* t) { delete t; }

int plamo_tokenizer_encode(const plamo_tokenizer* t, const char* text, size_t len, int32_t bos, int32_t* ids,
                           size_t cap, size_t* n_out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!t || (!text && len)) throw plamo::Error(plamo::E_INVAL, "bad tokenizer arguments");
        const std::vector<int32_t> v = t->tok.encode(std::string(text ? text : "", len), bos != 0);
        if (n_out) *n_out = v.size();
        if (v.size() > cap || (!ids && !v.empty())) throw plamo::Error(plamo::E_INVAL, "output buffer too small");
        if (!v.empty()) std::memcpy(ids, v.data(), v.size() * sizeof(int32_t));
    });
}

int plamo_tokenizer_decode(const plamo_tokenizer* t, const int32_t* ids, size_t count, char* out, size_t cap,
                           size_t* n_out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!t || (!ids && count)) throw plamo::Error(plamo::E_INVAL, "bad tokenizer arguments");
        std::string s;
        for (size_t i = 0; i < count; ++i) t->tok.append_bytes(ids[i], s);
        put_bytes(s, out, cap, n_out);
    });
}

int plamo_token_stream_open(const plamo_tokenizer* t, plamo_token_stream** out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!t || !out) throw plamo::Error(plamo::E_INVAL, "bad tokenizer arguments");
        *out = nullptr;
        *out = new plamo_token_stream(t->tok);
    });
}

int plamo_token_stream_push(plamo_token_stream* s, int32_t id, char* out, size_t cap, size_t* n_out, char* err,
                            size_t errlen) {
    return guard(err, errlen, [&] {
        if (!s) throw plamo::Error(plamo::E_INVAL, "bad tokenizer arguments");
        // size first: a buffer that is too small fails the call with the stream unchanged,
        // so the caller retries the same id with a larger buffer
        const size_t need = s->stream.push_size(id);
        if (n_out) *n_out = need;
        if (need > cap || (!out && need)) throw plamo::Error(plamo::E_INVAL, "output buffer too small");
        put_bytes(s->stream.push(id), out, cap, n_out);
    });
}

int plamo_token_stream_finish(plamo_token_stream* s, char* out, size_t cap, size_t* n_out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!s) throw plamo::Error(plamo::E_INVAL, "bad tokenizer arguments");
        const size_t need = s->stream.finish_size();
        if (n_out) *n_out = need;
        if (need > cap || (!out && need)) throw plamo::Error(plamo::E_INVAL, "output buffer too small");
        put_bytes(s->stream.finish(), out, cap, n_out);
    });
}

void plamo_token_stream_close(plamo_token_stream* s) { delete s; }

struct plamo_ordered {
    std::unique_ptr<plamo::OrderedOutput> out;
};

static plamo::OrderedOutput::Emit text_emitter(plamo_text_fn emit, void* user) {
    return [emit, user](const std::string& s) {
        if (emit && emit(user, s.data(), s.size()) != 0) throw plamo::Error(plamo::E_STATE, "Cancelled");
    };
}

int plamo_ordered_open(const plamo_tokenizer* t, const char* const* prefixes, const size_t* prefix_lens,
                       int32_t count, const char* tail, size_t tail_len, plamo_text_fn emit, void* user,
                       plamo_ordered** out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!t || !out || count < 0 || (count > 0 && (!prefixes || !prefix_lens)) || (!tail && tail_len))
            throw plamo::Error(plamo::E_INVAL, "bad output arguments");
        *out = nullptr;
        std::vector<std::string> p;
        for (int32_t i = 0; i < count; ++i) p.emplace_back(prefixes[i] ? prefixes[i] : "", prefixes[i] ? prefix_lens[i] : 0);
        auto h = std::make_unique<plamo_ordered>();
        h->out = std::make_unique<plamo::OrderedOutput>(t->tok, std::move(p), std::string(tail ? tail : "", tail_len),
                                                         text_emitter(emit, user));
        *out = h.release();
    });
}

int plamo_ordered_append(plamo_ordered* o, int32_t lane, int32_t id, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!o) throw plamo::Error(plamo::E_INVAL, "bad output arguments");
        o->out->append(lane, id);
    });
}

int plamo_ordered_finish(plamo_ordered* o, int32_t lane, const char* reason, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!o || !reason) throw plamo::Error(plamo::E_INVAL, "bad output arguments");
        o->out->finish(lane, reason);
    });
}

void plamo_ordered_close(plamo_ordered* o) { delete o; }

int plamo_timeline(uint64_t* out, size_t words, int32_t clear, char* err, size_t errlen) {
    return guard(err, errlen, [&] { plamo::timeline_copy(out, words, clear != 0); });
}

int plamo_translation_prompt(const char* text, size_t len, const char* target, char* out, size_t cap,
                             size_t* n_out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if ((!text && len) || !target) throw plamo::Error(plamo::E_INVAL, "bad prompt arguments");
        put_bytes(plamo::translation_prompt(std::string(text ? text : "", len), target), out, cap, n_out);
    });
}

struct plamo_plan {
    plamo::DocumentPlan plan;
};

static std::vector<plamo::Segment> segments_of(const char* const* texts, const size_t* text_lens,
                                               const int32_t* const* tokens, const int32_t* token_counts, int32_t count) {
    if (count < 0 || (count > 0 && (!texts || !text_lens || !tokens || !token_counts)))
        throw plamo::Error(plamo::E_INVAL, "bad segment arguments");
    std::vector<plamo::Segment> parts(static_cast<size_t>(count));
    for (int32_t i = 0; i < count; ++i) {
        if ((!texts[i] && text_lens[i]) || token_counts[i] < 0 || (!tokens[i] && token_counts[i]))
            throw plamo::Error(plamo::E_INVAL, "bad segment arguments");
        if (text_lens[i]) parts[size_t(i)].text.assign(texts[i], text_lens[i]);
        if (token_counts[i]) parts[size_t(i)].tokens.assign(tokens[i], tokens[i] + token_counts[i]);
    }
    return parts;
}

int plamo_document_plan(const char* const* texts, const size_t* text_lens, const int32_t* const* tokens,
                        const int32_t* token_counts, int32_t count, plamo_plan** out, char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!out) throw plamo::Error(plamo::E_INVAL, "bad segment arguments");
        *out = nullptr;
        *out = new plamo_plan{plamo::DocumentPlan(segments_of(texts, text_lens, tokens, token_counts, count))};
    });
}

int32_t plamo_plan_documents(const plamo_plan* p) { return p ? int32_t(p->plan.inputs.size()) : 0; }

int plamo_plan_input(const plamo_plan* p, int32_t document, const int32_t** tokens, int32_t* count) {
    if (!p || document < 0 || size_t(document) >= p->plan.inputs.size() || !tokens || !count) return PLAMO_EINVAL;
    *tokens = p->plan.inputs[size_t(document)].data();
    *count = int32_t(p->plan.inputs[size_t(document)].size());
    return PLAMO_OK;
}

int plamo_plan_prefix(const plamo_plan* p, int32_t document, const char** text, size_t* len) {
    if (!p || document < 0 || size_t(document) > p->plan.prefixes.size() || !text || !len) return PLAMO_EINVAL;
    const std::string& s = size_t(document) == p->plan.prefixes.size() ? p->plan.tail : p->plan.prefixes[size_t(document)];
    *text = s.data();
    *len = s.size();
    return PLAMO_OK;
}

void plamo_plan_close(plamo_plan* p) { delete p; }

int plamo_batch_translate_ordered(plamo_batch* b, const plamo_tokenizer* t, const char* const* texts,
                                  const size_t* text_lens, const int32_t* const* tokens, const int32_t* token_counts,
                                  int32_t count, int32_t limit, plamo_text_fn emit, void* user, int32_t* ids,
                                  int32_t ids_stride, int32_t* lengths, int32_t* reasons, plamo_document_output* out,
                                  char* err, size_t errlen) {
    return guard(err, errlen, [&] {
        if (!b || !t) throw plamo::Error(plamo::E_INVAL, "bad segment arguments");
        const plamo::DocumentPlan plan(segments_of(texts, text_lens, tokens, token_counts, count));
        bool ok = limit >= 0 && limit <= 8191;
        for (const auto& in : plan.inputs) {
            ok = ok && int64_t(in.size()) + limit <= int64_t(b->rt->impl.context);
            for (int32_t id : in) ok = ok && id >= 0 && id < plamo::VOCAB;
        }
        if (!ok) throw plamo::Error(plamo::E_INVAL, "Invalid document tokens or context budget");
        using clock = std::chrono::steady_clock;
        std::vector<LaneOutput> outputs;
        double gpu = 0, prefill_s = 0, decode_s = 0;
        int64_t discarded = 0, prefilled = 0;
        const size_t n = plan.inputs.size();
        try {
            for (size_t start = 0; start < n; start += plamo::ROWS) {
                const size_t end = std::min(start + plamo::ROWS, n);
                plamo::OrderedOutput sink(t->tok, std::vector<std::string>(plan.prefixes.begin() + long(start),
                                                                           plan.prefixes.begin() + long(end)),
                                          end == n ? plan.tail : std::string(), text_emitter(emit, user));
                int64_t generated = 0;
                const std::vector<std::vector<int32_t>> inputs(plan.inputs.begin() + long(start), plan.inputs.begin() + long(end));
                const auto t0 = clock::now();
                const std::vector<int32_t> next = b->impl->prefill(inputs);
                const auto t1 = clock::now();
                auto batch = decode_batch(
                    next, std::vector<int32_t>(end - start, limit),
                    [&](const std::vector<int32_t>& tk) { return b->impl->step(tk); },
                    [&](int lane, int id) {
                        ++generated;
                        sink.append(lane, id);
                    },
                    [&](int lane, const LaneOutput& o) { sink.finish(lane, o.reason == PLAMO_REASON_STOP ? "stop" : "length"); },
                    true);
                prefill_s += std::chrono::duration<double>(t1 - t0).count();
                decode_s += std::chrono::duration<double>(clock::now() - t1).count();
                for (const auto& in : inputs) prefilled += int64_t(in.size());
                gpu += b->impl->gpu_seconds;
                int64_t reported = 0;
                for (const auto& o : batch) reported += int64_t(o.ids.size());
                discarded += generated - reported;
                const bool stopped = batch.back().reason == PLAMO_REASON_STOP;
                for (auto& o : batch) outputs.push_back(std::move(o));
                if (!stopped) break;
            }
        } catch (...) {
            b->impl->reset();
            throw;
        }
        write_outputs(outputs, ids, ids_stride, lengths, reasons, nullptr);
        if (out) {
            out->sequences = int32_t(outputs.size());
            out->gpu_seconds = gpu;
            out->discarded_tokens = discarded;
            out->prefilled_input_tokens = prefilled;
            out->prefill_seconds = prefill_s;
            out->decode_seconds = decode_s;
        }
    });
}

}  // extern "C"
