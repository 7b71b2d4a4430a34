// Weight formats: safetensors and the lossless .p12 archive (reader, validator, writer).
#include "formats.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <functional>
#include <sstream>
#include <thread>

#include "common.h"

namespace plamo {

const char* const REFERENCE_SOURCE_SHA = "7c9f0066d166c075bdbe83ada3d444e08bd7a6ee3f345f47a1f3c442aa6898c5";

float post_mlp_offset() { return float(1.0 / std::pow(5.0, 1.5)); }

// ---------------------------------------------------------------------------------- SHA-256
namespace {
struct Sha256 {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    uint8_t buf[64];
    size_t fill = 0;
    uint64_t total = 0;
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void block(const uint8_t* p) {
        static const uint32_t k[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = uint32_t(p[4 * i]) << 24 | uint32_t(p[4 * i + 1]) << 16 | uint32_t(p[4 * i + 2]) << 8 | p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; ++i) {
            uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
            uint32_t ch = (e & f) ^ (~e & g);
            uint32_t t1 = hh + S1 + ch + k[i] + w[i];
            uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
            uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
            uint32_t t2 = S0 + mj;
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    void update(const uint8_t* p, size_t n) {
        total += n;
        if (fill) {
            size_t take = std::min(n, 64 - fill);
            std::memcpy(buf + fill, p, take);
            fill += take; p += take; n -= take;
            if (fill == 64) { block(buf); fill = 0; }
        }
        while (n >= 64) { block(p); p += 64; n -= 64; }
        if (n) { std::memcpy(buf, p, n); fill = n; }
    }
    std::string hex() {
        uint64_t bitlen = total * 8;
        uint8_t pad = 0x80;
        update(&pad, 1);
        uint8_t zero = 0;
        while (fill != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = uint8_t(bitlen >> (56 - 8 * i));
        update(len, 8);
        char out[65];
        for (int i = 0; i < 8; ++i) std::snprintf(out + 8 * i, 9, "%08x", h[i]);
        return std::string(out, 64);
    }
};
}  // namespace

std::string sha256_file(const std::string& path) {
    MappedFile f(path, "Cannot open file");
    Sha256 s;
    s.update(f.data(), f.size());
    return s.hex();
}

// ------------------------------------------------------------------------------ MappedFile
MappedFile::MappedFile(const std::string& path, const char* open_error) {
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw Error(E_IO, std::string(open_error));
    struct stat st;
    if (fstat(fd, &st) != 0) { ::close(fd); throw Error(E_IO, std::string(open_error)); }
    size_ = size_t(st.st_size);
    if (size_ > 0) {
        void* p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) { ::close(fd); throw Error(E_IO, "Cannot map " + path); }
        data_ = static_cast<uint8_t*>(p);
        mapped_ = size_;
    }
    ::close(fd);
}

MappedFile::~MappedFile() {
    if (data_) munmap(data_, mapped_);
}

namespace {
uint64_t load_u64(const uint8_t* p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}

bool shape_is(const json::Value* v, const std::vector<int64_t>& shape) {
    if (!v || v->kind != json::Value::Array || v->arr.size() != shape.size()) return false;
    for (size_t i = 0; i < shape.size(); ++i)
        if (!v->arr[i].is_int() || v->arr[i].i != shape[i]) return false;
    return true;
}

bool int_pair(const json::Value* v, int64_t& a, int64_t& b) {
    if (!v || v->kind != json::Value::Array || v->arr.size() != 2 || !v->arr[0].is_int() || !v->arr[1].is_int())
        return false;
    a = v->arr[0].i;
    b = v->arr[1].i;
    return true;
}

bool is_integer(const json::Value* v, int64_t want) {
    return v && v->kind == json::Value::Number && std::floor(v->num) == v->num && v->num == double(want);
}
}  // namespace

// ----------------------------------------------------------------------------- SafeTensors
SafeTensors::SafeTensors(const std::string& path) {
    // Runtime.swift:34-35
    file_ = std::make_unique<MappedFile>(path, ("Cannot open weights: " + path).c_str());
    const size_t size = file_->size();
    if (size <= 8 || size > 2000000000ull) throw Error(E_FORMAT, "Invalid weights file");  // :38
    const uint64_t header_size = load_u64(file_->data());
    if (header_size > 1048576 || header_size >= size - 8) throw Error(E_FORMAT, "Invalid safetensors header size");
    data_start_ = 8 + header_size;
    if (data_start_ % 8 != 0) throw Error(E_FORMAT, "Unaligned safetensors header");  // :52-54
    try {
        header_ = json::parse(reinterpret_cast<const char*>(file_->data() + 8), header_size);
    } catch (const std::exception&) {
        throw Error(E_FORMAT, "Invalid safetensors header");
    }
    if (header_.kind != json::Value::Object) throw Error(E_FORMAT, "Invalid safetensors header");
    // Runtime.swift:59-65
    const json::Value* e = header_.get("model.embed_tokens.weight");
    int64_t a = 0, b = 0;
    const json::Value* dt = e ? e->get("dtype") : nullptr;
    if (!e || !dt || dt->kind != json::Value::String || dt->str != "BF16" || !shape_is(e->get("shape"), {VOCAB, HIDDEN}) ||
        !int_pair(e->get("data_offsets"), a, b) || a < 0 || a % 2 != 0 || b < a || b - a != 330301440 ||
        b > int64_t(size - data_start_))
        throw Error(E_FORMAT, "Invalid input embedding");
    embedding_.data = file_->data() + data_start_ + a;
    embedding_.bytes = size_t(b - a);
}

TensorView SafeTensors::tensor(const std::string& name, const std::vector<int64_t>& shape) const {
    // Runtime.swift:87-93
    const json::Value* t = header_.get(name);
    int64_t a = 0, b = 0, numel = 2;
    for (auto s : shape) numel *= s;
    const json::Value* dt = t ? t->get("dtype") : nullptr;
    if (!t || !dt || dt->kind != json::Value::String || dt->str != "BF16" || !shape_is(t->get("shape"), shape) ||
        !int_pair(t->get("data_offsets"), a, b) || a < 0 || a % 4 != 0 || b < a || b - a != numel ||
        b > int64_t(file_->size() - data_start_))
        throw Error(E_FORMAT, "Missing or incompatible BF16 tensor: " + name);
    return TensorView{file_->data() + data_start_ + a, size_t(b - a)};
}

// ------------------------------------------------------------------------------ AuxArchive
namespace {
// Swift's Int(String): optional sign, then decimal digits only
bool swift_int(const std::string& s, int64_t& out) {
    size_t i = (!s.empty() && (s[0] == '+' || s[0] == '-')) ? 1 : 0;
    if (i >= s.size() || s.size() - i > 18) return false;
    int64_t v = 0;
    for (size_t k = i; k < s.size(); ++k) {
        if (s[k] < '0' || s[k] > '9') return false;
        v = v * 10 + (s[k] - '0');
    }
    out = s[0] == '-' ? -v : v;
    return true;
}
}  // namespace

AuxArchive::AuxArchive(const std::string& path, const std::string& teacher_sha256) {
    // Auxiliary.swift:16-17
    file_ = std::make_unique<MappedFile>(path, "Trained adapters missing; run scripts/train_auxiliary.py --collect");
    const size_t size = file_->size();
    if (size <= 8 || size >= 268435456ull) throw Error(E_FORMAT, "Invalid adapter size");  // :20-22
    const uint64_t count = load_u64(file_->data());
    if (count > 1048576 || count >= size - 8 || (count + 8) % 8 != 0) throw Error(E_FORMAT, "Invalid adapter header");
    data_start_ = count + 8;
    const std::string incompatible = "Incompatible trained adapters";
    try {
        header_ = json::parse(reinterpret_cast<const char*>(file_->data() + 8), count);
    } catch (const std::exception&) {
        throw Error(E_FORMAT, incompatible);
    }
    // Auxiliary.swift:33-40: the metadata strings
    const std::string want = teacher_sha256.empty() ? REFERENCE_SOURCE_SHA : teacher_sha256;
    const json::Value* meta = header_.kind == json::Value::Object ? header_.get("__metadata__") : nullptr;
    auto text = [&](const char* key) -> const std::string* {
        const json::Value* v = meta ? meta->get(key) : nullptr;
        return v && v->kind == json::Value::String ? &v->str : nullptr;
    };
    int64_t qsa_steps = 0, mtp_steps = 0;
    const std::string *fmt = text("format"), *teacher = text("teacher_sha256"), *rank = text("rank");
    const std::string *qs = text("qsa_steps"), *ms = text("mtp_steps");
    if (!meta || meta->kind != json::Value::Object || !fmt || *fmt != "plamo-aux-v1" || !teacher || *teacher != want ||
        !rank || *rank != "256" || !qs || !swift_int(*qs, qsa_steps) || qsa_steps <= 0 || !ms ||
        !swift_int(*ms, mtp_steps) || mtp_steps <= 0)
        throw Error(E_FORMAT, incompatible);
}

TensorView AuxArchive::tensor(const std::string& name, const std::vector<int64_t>& shape) const {
    // Auxiliary.swift:44-49
    const json::Value* t = header_.get(name);
    int64_t a = 0, b = 0, numel = 2;
    for (auto s : shape) numel *= s;
    const json::Value* dt = t ? t->get("dtype") : nullptr;
    if (!t || t->kind != json::Value::Object || !dt || dt->kind != json::Value::String || dt->str != "BF16" ||
        !shape_is(t->get("shape"), shape) || !int_pair(t->get("data_offsets"), a, b) || a < 0 || a % 4 != 0 ||
        b < a || b - a != numel || b > int64_t(file_->size() - data_start_))
        throw Error(E_FORMAT, "Invalid adapter tensor: " + name);
    return TensorView{file_->data() + data_start_ + a, size_t(b - a)};
}

// --------------------------------------------------------------------------- PackedArchive
PackedArchive::PackedArchive(const std::string& path, const std::string& source_sha256) {
    file_ = std::make_unique<MappedFile>(path, "Packed weights missing; run scripts/pack_weights.py first");  // :14
    const size_t size = file_->size();
    if (size <= 8 || size > 2000000000ull) throw Error(E_FORMAT, "Invalid packed file size");  // :17-19
    const uint64_t count = load_u64(file_->data());
    if (count > 1048576 || count >= size - 8 || (count + 8) % 64 != 0) throw Error(E_FORMAT, "Invalid packed header");
    data_start_ = count + 8;
    const std::string incompatible = "Incompatible packed archive; run scripts/pack_weights.py to regenerate";
    try {
        header_ = json::parse(reinterpret_cast<const char*>(file_->data() + 8), count);
    } catch (const std::exception&) {
        throw Error(E_FORMAT, incompatible);
    }
    const std::string want = source_sha256.empty() ? REFERENCE_SOURCE_SHA : source_sha256;
    const json::Value* fmt = header_.get("format");
    const json::Value* sha = header_.get("source_sha256");
    const json::Value* pb = header_.get("payload_bytes");
    const json::Value* tensors = header_.get("tensors");
    // Packed.swift:33-39
    if (!fmt || fmt->kind != json::Value::String || fmt->str != "plamo-bf16-pack-v2" ||
        !is_integer(header_.get("block"), 128) || !is_integer(header_.get("minimum_base"), 107) || !sha ||
        sha->kind != json::Value::String || sha->str != want || !pb || !pb->is_int() ||
        pb->i != int64_t(size - data_start_) || !tensors || tensors->kind != json::Value::Object)
        throw Error(E_FORMAT, incompatible);
    payload_ = size_t(pb->i);
}

PackedTensor PackedArchive::tensor(const std::string& name, const std::vector<int64_t>& shape) const {
    const json::Value* record = header_.get("tensors")->get(name);
    if (!record || !shape_is(record->get("shape"), shape))
        throw Error(E_FORMAT, "Packed tensor shape mismatch: " + name);  // Packed.swift:50-52
    auto region = [&](const char* key) {  // Packed.swift:53-57
        int64_t a = 0, b = 0;
        if (!int_pair(record->get(key), a, b) || a < 0 || a % 64 != 0 || b < a || b > int64_t(payload_))
            throw Error(E_FORMAT, "Invalid packed region: " + name + "." + key);
        return std::pair<size_t, size_t>(size_t(a), size_t(b - a));
    };
    PackedTensor t;
    if (shape.size() == 1) {  // Packed.swift:58-62
        auto raw = region("raw");
        if (raw.second != size_t(shape[0]) * 2) throw Error(E_FORMAT, "Invalid packed norm");
        t.data = payload() + raw.first;
        t.data_bytes = raw.second;
        t.data_offset = raw.first;
        return t;
    }
    int64_t numel = 1;
    for (auto s : shape) numel *= s;
    const size_t count = size_t(numel / 128);
    auto offsets = region("offsets");
    auto data = region("data");
    if (offsets.second != count * 4) throw Error(E_FORMAT, "Invalid packed block table");  // :65
    // Packed.swift:66-89: every entry's aligned offset equals the running end; 256 B for a
    // raw block (tag 0) else 192 B; the chain ends exactly at the data region size.
    const uint8_t* table = payload() + offsets.first;
    size_t end = 0;
    for (size_t j = 0; j < count; ++j) {
        uint32_t entry;
        std::memcpy(&entry, table + 4 * j, 4);
        const size_t offset = entry & ~63u;
        const size_t bytes = (entry & 63u) == 0 ? 256 : 192;
        if (offset != end || offset + bytes > data.second) throw Error(E_FORMAT, "Packed block out of range: " + name);
        end = offset + bytes;
    }
    if (end != data.second) throw Error(E_FORMAT, "Packed payload size mismatch");
    t.blocked = true;
    t.data = payload() + data.first;
    t.data_bytes = data.second;
    t.data_offset = data.first;
    t.table = table;
    t.table_offset = offsets.first;
    t.blocks = count;
    return t;
}

// ------------------------------------------------------------------------------- packing
// pack_weights.py:19-50 per block: eligible when the nonzero exponents lie in
// [low, low+14] with 108 <= low <= 170 and no exponent 255.
static inline int block_minimum(const uint16_t* v) {
    int low = 255, high = 0;
    for (int i = 0; i < 128; ++i) {
        const int e = (v[i] >> 7) & 255;
        if (v[i] & 0x7fff) {
            low = std::min(low, e);
            high = std::max(high, e);
        }
    }
    const bool eligible = low >= 108 && low <= 170 && high < 255 && high - low < 15;
    return eligible ? low : 0;
}

static inline void encode_block(const uint16_t* v, int minimum, uint8_t* out) {
    if (!minimum) {
        std::memcpy(out, v, 256);
        return;
    }
    std::memset(out + 128, 0, 64);
    for (int i = 0; i < 128; ++i) {
        const uint16_t x = v[i];
        const int code = (x & 0x7fff) == 0 ? 15 : ((x >> 7) & 255) - minimum;
        out[i] = uint8_t((x & 127) | ((x >> 8) & 128));
        out[128 + i / 2] |= uint8_t(code << ((i % 2) * 4));
    }
}

static inline uint16_t decode_word(const uint8_t* block, int minimum, int i) {
    if (!minimum) return uint16_t(block[2 * i] | (block[2 * i + 1] << 8));
    const uint32_t sm = block[i], code = (block[128 + i / 2] >> ((i % 2) * 4)) & 15;
    const uint32_t exponent = code == 15 ? 0 : minimum + code;
    return uint16_t((sm & 127) | ((sm & 128) << 8) | (exponent << 7));
}

std::vector<uint8_t> pack_blocks(const uint16_t* values, size_t count, std::vector<uint32_t>& entries,
                                 int64_t* compressed) {
    const size_t blocks = count / 128;
    std::vector<uint8_t> minima(blocks);
    entries.assign(blocks, 0);
    const unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    auto parallel = [&](const std::function<void(size_t, size_t)>& f) {
        std::vector<std::thread> pool;
        const size_t per = (blocks + threads - 1) / threads;
        for (unsigned t = 0; t < threads; ++t) {
            const size_t a = t * per, b = std::min(blocks, a + per);
            if (a < b) pool.emplace_back(f, a, b);
        }
        for (auto& th : pool) th.join();
    };
    parallel([&](size_t a, size_t b) {
        for (size_t j = a; j < b; ++j) minima[j] = uint8_t(block_minimum(values + 128 * j));
    });
    size_t end = 0;
    int64_t packed = 0;
    for (size_t j = 0; j < blocks; ++j) {
        entries[j] = uint32_t(end) | (minima[j] ? uint32_t(minima[j] - 107) : 0u);  // tag(), :71-74
        end += minima[j] ? 192 : 256;
        packed += minima[j] != 0;
    }
    if (end > 0xffffffc0ull) throw Error(E_FORMAT, "Packed tensor too large");
    std::vector<uint8_t> data(end);
    bool ok = true;
    parallel([&](size_t a, size_t b) {
        bool good = true;
        for (size_t j = a; j < b; ++j) {
            uint8_t* out = data.data() + (entries[j] & ~63u);
            encode_block(values + 128 * j, minima[j], out);
            for (int i = 0; i < 128; ++i) good &= decode_word(out, minima[j], i) == values[128 * j + i];
        }
        if (!good) ok = false;
    });
    if (!ok) throw Error(E_FORMAT, "Packing changed BF16 bits");  // pack_weights.py:47-49
    if (compressed) *compressed = packed;
    return data;
}

void pack_self_test() {
    // pack_weights.py:77-86: every BF16 pattern, zero blocks, -0 blocks, {0,-0,1,-1} tiles.
    std::vector<std::vector<uint16_t>> cases(4);
    for (int i = 0; i < 65536; ++i) cases[0].push_back(uint16_t(i));
    cases[1].assign(256, 0);
    cases[2].assign(128, 0x8000);
    const uint16_t tile[4] = {0, 0x8000, 0x3f80, 0xbf80};
    for (int i = 0; i < 256; ++i) cases[3].push_back(tile[i % 4]);
    for (auto& v : cases) {
        std::vector<uint32_t> entries;
        auto data = pack_blocks(v.data(), v.size(), entries, nullptr);
        for (size_t j = 0; j < entries.size(); ++j) {
            const uint32_t tagv = entries[j] & 63;
            const int minimum = tagv ? int(tagv) + 107 : 0;
            for (int i = 0; i < 128; ++i)
                if (decode_word(data.data() + (entries[j] & ~63u), minimum, i) != v[128 * j + i])
                    throw Error(E_FORMAT, "Packer self-test failed");
        }
    }
}

PackReport pack_archive(const std::string& source, const std::string& output, const std::string& source_sha256) {
    pack_self_test();
    const std::string want = source_sha256.empty() ? REFERENCE_SOURCE_SHA : source_sha256;
    if (sha256_file(source) != want) throw Error(E_FORMAT, "Original weight checksum mismatch");  // :93-94
    SafeTensors st(source);
    const size_t HEADER = 65536;
    const std::string part = output + ".part";
    FILE* f = std::fopen(part.c_str(), "w+b");
    if (!f) throw Error(E_IO, "Cannot write " + part);
    PackReport report;
    std::ostringstream tensors;
    bool first = true;
    size_t pos = HEADER;
    try {
        std::vector<uint8_t> zeros(HEADER, 0);
        if (std::fwrite(zeros.data(), 1, HEADER, f) != HEADER) throw Error(E_IO, "write failed");
        auto append = [&](const void* p, size_t n) {  // pack_weights.py:105-110
            const size_t padding = (64 - pos % 64) % 64;
            if (padding && std::fwrite(zeros.data(), 1, padding, f) != padding) throw Error(E_IO, "write failed");
            pos += padding;
            const size_t begin = pos - HEADER;
            if (n && std::fwrite(p, 1, n, f) != n) throw Error(E_IO, "write failed");
            pos += n;
            return std::pair<size_t, size_t>(begin, pos - HEADER);
        };
        const json::Value& h = st.header();
        for (const std::string& name : h.keys) {
            if (name == "__metadata__" || name == "model.embed_tokens.weight") continue;
            const json::Value& t = h.obj.at(name);
            const json::Value* dt = t.get("dtype");
            if (!dt || dt->str != "BF16") throw Error(E_FORMAT, "Packer expects BF16 tensors: " + name);
            std::vector<int64_t> shape;
            for (auto& s : t.get("shape")->arr) shape.push_back(s.i);
            TensorView view = st.tensor(name, shape);
            std::ostringstream rec;
            rec << "\"" << name << "\":{\"shape\":[";
            for (size_t i = 0; i < shape.size(); ++i) rec << (i ? "," : "") << shape[i];
            rec << "]";
            if (shape.size() == 1) {
                auto r = append(view.data, view.bytes);
                rec << ",\"raw\":[" << r.first << "," << r.second << "]}";
            } else {
                const size_t count = view.bytes / 2;
                if (count % 128) throw Error(E_FORMAT, "Tensor size is not a multiple of 128: " + name);
                std::vector<uint16_t> values(count);
                if (count) std::memcpy(values.data(), view.data, view.bytes);
                std::vector<uint32_t> entries;
                int64_t compressed = 0;
                auto data = pack_blocks(values.data(), count, entries, &compressed);
                auto ro = append(entries.data(), entries.size() * 4);
                auto rd = append(data.data(), data.size());
                rec << ",\"offsets\":[" << ro.first << "," << ro.second << "],\"data\":[" << rd.first << ","
                    << rd.second << "]}";
                report.compressed_blocks += compressed;
                report.blocks += int64_t(entries.size());
                report.packed_linear_bytes += int64_t(data.size() + entries.size() * 4);
                report.original_linear_bytes += int64_t(view.bytes);
            }
            tensors << (first ? "" : ",") << rec.str();
            first = false;
        }
        std::ostringstream meta;
        meta << "{\"format\":\"plamo-bf16-pack-v2\",\"block\":128,\"minimum_base\":107,\"source_sha256\":\"" << want
             << "\",\"tensors\":{" << tensors.str() << "},\"payload_bytes\":" << (pos - HEADER) << "}";
        const std::string m = meta.str();
        if (m.size() > HEADER - 8) throw Error(E_FORMAT, "Packed header overflow");
        std::fseek(f, 0, SEEK_SET);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = uint8_t(uint64_t(HEADER - 8) >> (8 * i));
        std::string padded = m + std::string(HEADER - 8 - m.size(), ' ');
        if (std::fwrite(len, 1, 8, f) != 8 || std::fwrite(padded.data(), 1, padded.size(), f) != padded.size())
            throw Error(E_IO, "write failed");
        if (std::fclose(f) != 0) { f = nullptr; throw Error(E_IO, "write failed"); }
        f = nullptr;
        if (std::rename(part.c_str(), output.c_str()) != 0) throw Error(E_IO, "Cannot rename " + part);
    } catch (...) {
        if (f) std::fclose(f);
        std::remove(part.c_str());
        throw;
    }
    report.archive_bytes = int64_t(pos);
    return report;
}

}  // namespace plamo
