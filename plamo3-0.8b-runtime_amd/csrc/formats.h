// Weight formats: safetensors (Weights, Runtime.swift:23-111), the .p12 archive
// (Packed, Packed.swift:5-91) and its writer (scripts/pack_weights.py).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "json.h"

namespace plamo {

// Read-only mapping of a whole file.
class MappedFile {
  public:
    explicit MappedFile(const std::string& path, const char* open_error);
    ~MappedFile();
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
    const uint8_t* data() const { return data_; }
    size_t size() const { return size_; }

  private:
    uint8_t* data_ = nullptr;
    size_t size_ = 0;
    size_t mapped_ = 0;
};

struct TensorView {
    const uint8_t* data = nullptr;  // host pointer into the mapping
    size_t bytes = 0;
};

// model.safetensors with the reference's validation (Runtime.swift:33-101).
class SafeTensors {
  public:
    explicit SafeTensors(const std::string& path);
    // Weights.tensor(name, shape) (Runtime.swift:87-101).
    TensorView tensor(const std::string& name, const std::vector<int64_t>& shape) const;
    TensorView embedding() const { return embedding_; }
    const json::Value& header() const { return header_; }
    const MappedFile& file() const { return *file_; }
    size_t data_start() const { return data_start_; }

  private:
    std::unique_ptr<MappedFile> file_;
    json::Value header_;
    size_t data_start_ = 0;
    TensorView embedding_;
};

// One tensor of a .p12 archive (Packed.tensor, Packed.swift:49-91).
struct PackedTensor {
    bool blocked = false;              // 2-D block-table tensor
    const uint8_t* data = nullptr;     // payload (raw bytes for 1-D tensors)
    size_t data_bytes = 0;
    const uint8_t* table = nullptr;    // u32 block entries (offset | minimum-107)
    size_t blocks = 0;
    size_t data_offset = 0;            // offsets of the regions from the payload start
    size_t table_offset = 0;
};

class PackedArchive {
  public:
    // Packed.init (Packed.swift:12-47); `source_sha256` empty = the reference's pinned value.
    PackedArchive(const std::string& path, const std::string& source_sha256);
    PackedTensor tensor(const std::string& name, const std::vector<int64_t>& shape) const;
    const uint8_t* payload() const { return file_->data() + data_start_; }
    size_t payload_bytes() const { return payload_; }

  private:
    std::unique_ptr<MappedFile> file_;
    json::Value header_;
    size_t data_start_ = 0;
    size_t payload_ = 0;
};

// auxiliary.safetensors: the trained QSA indexers and MTP adapter (Auxiliary.swift:5-62).
class AuxArchive {
  public:
    // Auxiliary.init (Auxiliary.swift:14-41); `teacher_sha256` empty = the reference's pinned
    // checksum of the model the adapters were trained against.
    AuxArchive(const std::string& path, const std::string& teacher_sha256);
    // Auxiliary.tensor(name, shape) (Auxiliary.swift:43-62): BF16, exact shape, 4-byte aligned.
    TensorView tensor(const std::string& name, const std::vector<int64_t>& shape) const;

  private:
    std::unique_ptr<MappedFile> file_;
    json::Value header_;
    size_t data_start_ = 0;
};

extern const char* const REFERENCE_SOURCE_SHA;

struct PackReport {
    int64_t original_linear_bytes = 0, packed_linear_bytes = 0, archive_bytes = 0;
    int64_t compressed_blocks = 0, blocks = 0;
};

// pack_weights.py pack(): encodes `count` BF16 values (count % 128 == 0).
// Returns payload bytes; `entries` receives the tagged table (tag()).
std::vector<uint8_t> pack_blocks(const uint16_t* values, size_t count, std::vector<uint32_t>& entries,
                                 int64_t* compressed);
// pack_weights.py main(): writes the archive atomically.
PackReport pack_archive(const std::string& source, const std::string& output, const std::string& source_sha256);
// pack_weights.py self_test() on the packer above.
void pack_self_test();

}  // namespace plamo
