// GGUF model files: the document reader, the Llama shape rules and the
// metadata JSON of tvara_model_metadata, restating core/include/tvara/gguf.hpp
// and core/include/tvara/gguf_model.hpp (accepted files, limits and error
// messages are the reference's; the parser is a single pass over a read-only
// mapping).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

namespace tvara_amd::gguf {

// tvara::gguf::Error (gguf.hpp:16-19): a runtime_error
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// storage types the model path reads (gguf.hpp:171-177)
enum TensorType : uint32_t { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ8_0 = 8, kQ4_K = 12 };

struct Value {
    using Array = std::vector<Value>;
    // unsigned integers, signed integers, floats (f32 widened), bool, string, array
    std::variant<uint64_t, int64_t, double, bool, std::string, Array> data;
};

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;  // dims[0] varies fastest
    uint32_t type = 0;
    uint64_t offset = 0;         // from the start of the data section
};

struct Document {
    uint32_t version = 0;
    std::map<std::string, Value> metadata;
    std::map<std::string, TensorInfo> tensors;
    size_t alignment = 32;
    size_t data_offset = 0;
};

// read-only mapping of a file (mapped_file.hpp)
class Mapping {
public:
    explicit Mapping(const std::string& path);
    ~Mapping();
    Mapping(const Mapping&) = delete;
    Mapping& operator=(const Mapping&) = delete;
    const uint8_t* data() const { return data_; }
    size_t size() const { return size_; }

private:
    const uint8_t* data_ = nullptr;
    size_t size_ = 0;
};

// bytes of a tensor's payload (gguf.hpp:170-186)
size_t tensor_bytes(const TensorInfo& t);

// parse and check a whole document (gguf.hpp:187-209)
Document read_document(const uint8_t* bytes, size_t size);

class ModelFile {
public:
    explicit ModelFile(const std::string& path);
    const Document& document() const { return doc_; }
    const TensorInfo& tensor(const std::string& name) const;
    const uint8_t* payload(const TensorInfo& t) const { return map_->data() + doc_.data_offset + t.offset; }

private:
    std::shared_ptr<Mapping> map_;
    Document doc_;
};

// llama_shape / validate_llama_tensors (gguf_model.hpp:46-108)
struct LlamaShape {
    uint64_t vocab = 0, hidden = 0, intermediate = 0, layers = 0, heads = 0, kv_heads = 0, context = 0;
    double rms_epsilon = 1e-6, rope_theta = 10000;
    bool interleaved_rope = true;  // tvara.rope.layout (model.hpp:151-155)
};
LlamaShape llama_shape(const Document& doc);
void validate_llama_tensors(const Document& doc, const LlamaShape& s);

// {"key":value,...} in key order (c_api.cpp:19-33,40-41)
std::string metadata_json(const Document& doc);

}  // namespace tvara_amd::gguf
