// GGUF reader, Llama shape rules and metadata JSON (see gguf.hpp).
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>

namespace tvara_amd::gguf {
namespace {

constexpr uint64_t kCountLimit = 1000000;
constexpr uint64_t kStringLimit = 16u << 20;

// Little-endian cursor over the mapped bytes; every read is bounds-checked
// (gguf.hpp:20-41).
class Cursor {
public:
    Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
    size_t pos() const { return pos_; }
    size_t left() const { return n_ - pos_; }
    const uint8_t* take(size_t count) {
        if (count > left()) throw Error("truncated GGUF data");
        const uint8_t* r = p_ + pos_;
        pos_ += count;
        return r;
    }
    uint64_t le(size_t width) {
        const uint8_t* b = take(width);
        uint64_t v = 0;
        for (size_t i = 0; i < width; ++i) v |= static_cast<uint64_t>(b[i]) << (8 * i);
        return v;
    }
    std::string str() {
        const uint64_t count = le(8);
        if (count > kStringLimit || count > left()) throw Error("GGUF string length exceeds limits");
        const uint8_t* b = take(static_cast<size_t>(count));
        return std::string(reinterpret_cast<const char*>(b), static_cast<size_t>(count));
    }

private:
    const uint8_t* p_;
    size_t n_;
    size_t pos_ = 0;
};

template <class T, class U>
T bits_as(U u) {
    T t;
    std::memcpy(&t, &u, sizeof(T));
    return t;
}

// metadata value of GGUF type `type` (gguf.hpp:48-86)
Value read_value(Cursor& c, uint32_t type) {
    switch (type) {
        case 0: return {c.le(1)};
        case 1: return {static_cast<int64_t>(bits_as<int8_t>(static_cast<uint8_t>(c.le(1))))};
        case 2: return {c.le(2)};
        case 3: return {static_cast<int64_t>(bits_as<int16_t>(static_cast<uint16_t>(c.le(2))))};
        case 4: return {c.le(4)};
        case 5: return {static_cast<int64_t>(bits_as<int32_t>(static_cast<uint32_t>(c.le(4))))};
        case 6: return {static_cast<double>(bits_as<float>(static_cast<uint32_t>(c.le(4))))};
        case 7: {
            const uint64_t b = c.le(1);
            if (b > 1) throw Error("invalid boolean metadata");
            return {b != 0};
        }
        case 8: return {c.str()};
        case 9: {
            const auto element = static_cast<uint32_t>(c.le(4));
            const uint64_t count = c.le(8);
            if (element == 9 || element > 12 || count > kCountLimit || count > c.left())
                throw Error("invalid or oversized metadata array");
            Value::Array items;
            items.reserve(static_cast<size_t>(count));
            for (uint64_t i = 0; i < count; ++i) items.push_back(read_value(c, element));
            return {std::move(items)};
        }
        case 10: return {c.le(8)};
        case 11: return {bits_as<int64_t>(c.le(8))};
        case 12: return {bits_as<double>(c.le(8))};
        default: throw Error("unsupported scalar metadata type");
    }
}

size_t align_up(size_t position, size_t alignment) {
    if (alignment == 0 || alignment > 65536 || (alignment & (alignment - 1)) != 0)
        throw Error("GGUF alignment must be a bounded power of two");
    if (position > std::numeric_limits<size_t>::max() - (alignment - 1)) throw Error("GGUF alignment overflow");
    return (position + alignment - 1) & ~(alignment - 1);
}

void quote(std::string& out, const std::string& s) {
    out += '"';
    char buf[8];
    for (unsigned char ch : s) {
        if (ch == '"' || ch == '\\') {
            out += '\\';
            out += static_cast<char>(ch);
        } else if (ch < 32) {
            std::snprintf(buf, sizeof buf, "\\u%04x", static_cast<unsigned>(ch));
            out += buf;
        } else {
            out += static_cast<char>(ch);
        }
    }
    out += '"';
}

void json(std::string& out, const Value& v) {
    if (auto s = std::get_if<std::string>(&v.data)) {
        quote(out, *s);
    } else if (auto b = std::get_if<bool>(&v.data)) {
        out += *b ? "true" : "false";
    } else if (auto u = std::get_if<uint64_t>(&v.data)) {
        out += std::to_string(*u);
    } else if (auto i = std::get_if<int64_t>(&v.data)) {
        out += std::to_string(*i);
    } else if (auto d = std::get_if<double>(&v.data)) {
        if (!std::isfinite(*d)) throw std::runtime_error("nonfinite metadata");
        char buf[40];
        std::snprintf(buf, sizeof buf, "%.17g", *d);  // std::setprecision(17) in the default float format
        out += buf;
    } else {
        const auto& items = std::get<Value::Array>(v.data);
        out += '[';
        for (size_t k = 0; k < items.size(); ++k) {
            if (k) out += ',';
            json(out, items[k]);
        }
        out += ']';
    }
}

}  // namespace

Mapping::Mapping(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw Error("cannot open model file");
    struct stat st {};
    if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        throw Error("invalid model file size");
    }
    size_ = static_cast<size_t>(st.st_size);
    void* p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) throw Error("cannot map model file");
    data_ = static_cast<const uint8_t*>(p);
}

Mapping::~Mapping() {
    if (data_) ::munmap(const_cast<uint8_t*>(data_), size_);
}

size_t tensor_bytes(const TensorInfo& t) {
    size_t block = 1, width = 0;
    switch (t.type) {
        case kF32: width = 4; break;
        case kF16: width = 2; break;
        case kQ4_0: block = 32; width = 18; break;
        case kQ8_0: block = 32; width = 34; break;
        case kQ4_K: block = 256; width = 144; break;
        default: throw Error("unsupported GGUF tensor storage type");
    }
    if (t.dims.empty() || t.dims[0] % block) throw Error("invalid quantized row width");
    size_t elements = 1;
    for (uint64_t d : t.dims) {
        if (!d || d > std::numeric_limits<size_t>::max() / elements) throw Error("tensor shape overflow");
        elements *= static_cast<size_t>(d);
    }
    if (elements / block > std::numeric_limits<size_t>::max() / width) throw Error("tensor size overflow");
    return elements / block * width;
}

Document read_document(const uint8_t* bytes, size_t size) {
    Cursor c(bytes, size);
    Document doc;
    if (c.le(4) != 0x46554747u) throw Error("invalid GGUF magic or unsupported byte order");
    doc.version = static_cast<uint32_t>(c.le(4));
    if (doc.version != 2 && doc.version != 3) throw Error("unsupported GGUF version");
    const uint64_t ntensors = c.le(8), nmeta = c.le(8);
    if (ntensors > kCountLimit || nmeta > kCountLimit) throw Error("GGUF count limit exceeded");
    if (ntensors > c.left() / 24 || nmeta > c.left() / 13) throw Error("GGUF counts exceed available bytes");
    for (uint64_t i = 0; i < nmeta; ++i) {
        std::string key = c.str();
        Value v = read_value(c, static_cast<uint32_t>(c.le(4)));
        if (key.empty() || !doc.metadata.emplace(std::move(key), std::move(v)).second)
            throw Error("empty or duplicate GGUF metadata key");
    }
    for (uint64_t i = 0; i < ntensors; ++i) {
        TensorInfo t;
        t.name = c.str();
        const uint64_t rank = c.le(4);
        if (t.name.empty() || rank == 0 || rank > 4) throw Error("invalid GGUF tensor name or rank");
        for (uint64_t r = 0; r < rank; ++r) {
            const uint64_t d = c.le(8);
            if (d == 0) throw Error("zero GGUF tensor dimension");
            t.dims.push_back(d);
        }
        t.type = static_cast<uint32_t>(c.le(4));
        t.offset = c.le(8);
        std::string name = t.name;
        if (!doc.tensors.emplace(std::move(name), std::move(t)).second) throw Error("duplicate GGUF tensor name");
    }
    if (auto it = doc.metadata.find("general.alignment"); it != doc.metadata.end()) {
        auto a = std::get_if<uint64_t>(&it->second.data);
        if (!a || *a > 65536) throw Error("invalid general.alignment metadata");
        doc.alignment = static_cast<size_t>(*a);
    }
    doc.data_offset = align_up(c.pos(), doc.alignment);
    if (doc.data_offset > size) throw Error("truncated GGUF alignment padding");
    for (const auto& [name, t] : doc.tensors)
        if (t.offset % doc.alignment) throw Error("unaligned GGUF tensor offset");
    const uint64_t room = size - doc.data_offset;
    std::map<uint64_t, uint64_t> spans;  // start -> end of every payload
    for (const auto& [name, t] : doc.tensors) {
        const uint64_t n = tensor_bytes(t);
        if (t.offset > room || n > room - t.offset) throw Error("tensor payload exceeds GGUF file");
        const uint64_t end = t.offset + n;
        auto next = spans.lower_bound(t.offset);
        if ((next != spans.end() && next->first < end) || (next != spans.begin() && std::prev(next)->second > t.offset))
            throw Error("overlapping GGUF tensor payloads");
        spans.emplace(t.offset, end);
    }
    return doc;
}

ModelFile::ModelFile(const std::string& path) : map_(std::make_shared<Mapping>(path)) {
    doc_ = read_document(map_->data(), map_->size());
}

const TensorInfo& ModelFile::tensor(const std::string& name) const {
    auto it = doc_.tensors.find(name);
    if (it == doc_.tensors.end()) throw Error("missing GGUF tensor: " + name);
    return it->second;
}

LlamaShape llama_shape(const Document& doc) {
    auto find = [&](const std::string& key) -> const Value& {
        auto it = doc.metadata.find(key);
        if (it == doc.metadata.end()) throw Error("missing metadata: " + key);
        return it->second;
    };
    auto text = [&](const std::string& key) -> const std::string& {
        auto s = std::get_if<std::string>(&find(key).data);
        if (!s) throw Error("metadata must be a string: " + key);
        return *s;
    };
    auto number = [&](const std::string& key) -> uint64_t {
        auto u = std::get_if<uint64_t>(&find(key).data);
        if (!u || !*u || *u > 1000000) throw Error("invalid model dimension: " + key);
        return *u;
    };
    auto floating = [&](const std::string& key, double fallback) {
        auto it = doc.metadata.find(key);
        if (it == doc.metadata.end()) return fallback;
        auto d = std::get_if<double>(&it->second.data);
        if (!d || !std::isfinite(*d) || *d <= 0) throw Error("invalid floating metadata: " + key);
        return *d;
    };
    if (text("general.architecture") != "llama") throw Error("unsupported model architecture");
    auto tok = doc.metadata.find("tokenizer.ggml.tokens");
    if (tok == doc.metadata.end()) throw Error("missing tokenizer vocabulary");
    auto vocab = std::get_if<Value::Array>(&tok->second.data);
    if (!vocab || vocab->empty()) throw Error("invalid tokenizer vocabulary");
    LlamaShape s;
    s.vocab = vocab->size();
    s.hidden = number("llama.embedding_length");
    s.intermediate = number("llama.feed_forward_length");
    s.layers = number("llama.block_count");
    s.heads = number("llama.attention.head_count");
    s.kv_heads = number("llama.attention.head_count_kv");
    s.context = number("llama.context_length");
    s.rms_epsilon = floating("llama.attention.layer_norm_rms_epsilon", 1e-6);
    s.rope_theta = floating("llama.rope.freq_base", 10000);
    if (s.hidden % s.heads || s.heads % s.kv_heads || (s.hidden / s.heads) % 2) throw Error("invalid Llama head layout");
    if (auto it = doc.metadata.find("llama.rope.scaling.type"); it != doc.metadata.end()) {
        auto v = std::get_if<std::string>(&it->second.data);
        if (!v || *v != "none") throw Error("scaled RoPE requires a separate implementation");
    }
    return s;
}

void validate_llama_tensors(const Document& doc, const LlamaShape& s) {
    if (!s.vocab || !s.hidden || !s.intermediate || !s.layers || !s.heads || !s.kv_heads || s.hidden % s.heads ||
        s.heads % s.kv_heads)
        throw Error("invalid Llama dimensions");
    const uint64_t kv = s.hidden / s.heads * s.kv_heads;
    auto require = [&](const std::string& name, std::vector<uint64_t> dims) {
        auto it = doc.tensors.find(name);
        if (it == doc.tensors.end() || it->second.dims != dims) throw Error("missing or malformed Llama tensor: " + name);
    };
    require("token_embd.weight", {s.hidden, s.vocab});
    require("output_norm.weight", {s.hidden});
    if (doc.tensors.count("output.weight")) require("output.weight", {s.hidden, s.vocab});
    for (uint64_t i = 0; i < s.layers; ++i) {
        const std::string p = "blk." + std::to_string(i) + ".";
        require(p + "attn_norm.weight", {s.hidden});
        require(p + "ffn_norm.weight", {s.hidden});
        require(p + "attn_q.weight", {s.hidden, s.hidden});
        require(p + "attn_k.weight", {s.hidden, kv});
        require(p + "attn_v.weight", {s.hidden, kv});
        require(p + "attn_output.weight", {s.hidden, s.hidden});
        require(p + "ffn_gate.weight", {s.hidden, s.intermediate});
        require(p + "ffn_up.weight", {s.hidden, s.intermediate});
        require(p + "ffn_down.weight", {s.intermediate, s.hidden});
    }
}

std::string metadata_json(const Document& doc) {
    std::string out = "{";
    bool first = true;
    for (const auto& [key, value] : doc.metadata) {
        if (!first) out += ',';
        first = false;
        quote(out, key);
        out += ':';
        json(out, value);
    }
    out += '}';
    return out;
}

}  // namespace tvara_amd::gguf
