// Llama decode executor on the GPU (see model.hpp).
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <stdexcept>

#include "gguf.hpp"

namespace tvara_amd {

void ModelConfig::validate() const {
    // ModelConfig::validate (model.hpp:12-18)
    if (!vocab || !hidden || !intermediate || !layers || !heads || !kv_heads || !context || hidden % heads ||
        heads % kv_heads || (hidden / heads) % 2 || !std::isfinite(rms_epsilon) || rms_epsilon <= 0 ||
        !std::isfinite(rope_theta) || rope_theta <= 0)
        throw std::invalid_argument("invalid native model configuration");
}

namespace {

size_t elements(const gguf::TensorInfo& t) {
    size_t n = 1;
    for (uint64_t d : t.dims) n *= static_cast<size_t>(d);
    return n;
}

float* at(DeviceBuffer& b, size_t offset_floats) { return static_cast<float*>(b.ptr) + offset_floats; }

}  // namespace

DeviceModel::DeviceModel(const std::string& path, size_t max_blocks, size_t block_tokens) {
    gguf::ModelFile file(path);
    const gguf::Document& doc = file.document();
    const gguf::LlamaShape shape = gguf::llama_shape(doc);
    gguf::validate_llama_tensors(doc, shape);
    cfg_.vocab = shape.vocab;
    cfg_.hidden = shape.hidden;
    cfg_.intermediate = shape.intermediate;
    cfg_.layers = shape.layers;
    cfg_.heads = shape.heads;
    cfg_.kv_heads = shape.kv_heads;
    cfg_.context = shape.context;
    cfg_.rms_epsilon = static_cast<float>(shape.rms_epsilon);
    cfg_.rope_theta = static_cast<float>(shape.rope_theta);
    if (auto it = doc.metadata.find("tvara.rope.layout"); it != doc.metadata.end()) {
        auto layout = std::get_if<std::string>(&it->second.data);
        if (!layout || (*layout != "split" && *layout != "interleaved")) throw std::invalid_argument("invalid RoPE layout");
        cfg_.interleaved_rope = *layout == "interleaved";
    }
    cfg_.validate();
    const ModelConfig& c = cfg_;
    const size_t H = c.hidden, I = c.intermediate, KV = c.kv_width();

    // weights: norms and every matrix not in Q8_0 dequantised to f32 in HBM,
    // as load_weights does on the host (model.hpp:119-134,156-169); Q8_0
    // matrices stay quantised (tiled, see Weight) and dequantise inside the
    // products to the same floats.  Fused row blocks Wq|Wk|Wv and
    // Wgate|Wup feed one product each; a block is Q8_0 only when all its
    // parts are.
    DeviceBuffer staging;
    bad_.ensure(sizeof(int));
    TVARA_HIP(hipMemset(bad_.ptr, 0, sizeof(int)));
    int* bad_flag = static_cast<int*>(bad_.ptr);
    auto load = [&](const std::string& name, float* dst) {
        const gguf::TensorInfo& t = file.tensor(name);
        const size_t n = elements(t), bytes = gguf::tensor_bytes(t);
        const uint8_t* src = file.payload(t);
        if (t.type == gguf::kF32) {
            TVARA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
            launch_dequant(t.type, nullptr, n, dst, bad_flag, nullptr);
        } else {
            void* raw = staging.ensure(bytes);
            TVARA_HIP(hipMemcpy(raw, src, bytes, hipMemcpyHostToDevice));
            launch_dequant(t.type, static_cast<const uint8_t*>(raw), n, dst, bad_flag, nullptr);
        }
        TVARA_HIP(hipDeviceSynchronize());
    };
    // parts: (tensor name, rows); every part has `cols` columns.  With
    // `interleave` (two parts of equal rows, kept as Q8_0), row i of part k
    // becomes row 2i + k.
    auto load_weight = [&](const std::vector<std::pair<std::string, size_t>>& parts, size_t cols, Weight& w,
                           bool interleave = false) {
        size_t rows = 0;
        bool q8 = true;
        for (const auto& [name, r] : parts) {
            rows += r;
            q8 = q8 && file.tensor(name).type == gguf::kQ8_0;
        }
        if (rows > static_cast<size_t>(std::numeric_limits<int>::max()) || cols > (1u << 30))
            throw std::invalid_argument("invalid native model configuration");
        w.rows = static_cast<int>(rows);
        w.cols = static_cast<int>(cols);
        w.q8 = q8;
        if (!q8) {
            w.f32.ensure(rows * cols * sizeof(float));
            size_t offset = 0;
            for (const auto& [name, r] : parts) {
                load(name, at(w.f32, offset));
                offset += r * cols;
            }
            return;
        }
        const size_t tiles = static_cast<size_t>(w.tiles()), pairs = static_cast<size_t>(w.pairs());
        const size_t qbytes = tiles * pairs * 64 * 16, dbytes = tiles * pairs * 16 * 2 * sizeof(uint16_t);
        w.q.ensure(qbytes);
        w.d.ensure(dbytes);
        TVARA_HIP(hipMemset(w.q.ptr, 0, qbytes));
        TVARA_HIP(hipMemset(w.d.ptr, 0, dbytes));
        w.interleaved = interleave;
        int row0 = 0;
        for (const auto& [name, r] : parts) {
            const gguf::TensorInfo& t = file.tensor(name);
            const size_t bytes = gguf::tensor_bytes(t);
            void* raw = staging.ensure(bytes);
            TVARA_HIP(hipMemcpy(raw, file.payload(t), bytes, hipMemcpyHostToDevice));
            launch_q8_repack(static_cast<const uint8_t*>(raw), static_cast<int>(r), w.cols, row0, interleave ? 2 : 1, w,
                             bad_flag, nullptr);
            TVARA_HIP(hipDeviceSynchronize());
            row0 += interleave ? 1 : static_cast<int>(r);
        }
    };
    load_weight({{"token_embd.weight", c.vocab}}, H, embedding_);
    final_norm_.ensure(H * sizeof(float));
    load("output_norm.weight", at(final_norm_, 0));
    if (doc.tensors.count("output.weight")) {
        has_output_ = true;
        load_weight({{"output.weight", c.vocab}}, H, output_);
    }
    layers_.resize(c.layers);
    for (size_t i = 0; i < c.layers; ++i) {
        const std::string p = "blk." + std::to_string(i) + ".";
        Layer& L = layers_[i];
        L.attn_norm.ensure(H * sizeof(float));
        load(p + "attn_norm.weight", at(L.attn_norm, 0));
        L.ffn_norm.ensure(H * sizeof(float));
        load(p + "ffn_norm.weight", at(L.ffn_norm, 0));
        load_weight({{p + "attn_q.weight", H}, {p + "attn_k.weight", KV}, {p + "attn_v.weight", KV}}, H, L.qkv);
        load_weight({{p + "attn_output.weight", H}}, H, L.out);
        load_weight({{p + "ffn_gate.weight", I}, {p + "ffn_up.weight", I}}, H, L.gate_up, true);
        load_weight({{p + "ffn_down.weight", H}}, I, L.down);
    }
    int bad = 0;
    TVARA_HIP(hipMemcpy(&bad, bad_.ptr, sizeof(int), hipMemcpyDeviceToHost));
    if (bad) throw std::invalid_argument("nonfinite model weight");

    // the executor's cache (paged_model.hpp:8-9)
    Geometry g;
    g.layers = c.layers;
    g.kv_heads = c.kv_heads;
    g.head_dim = c.head_dim();
    g.tokens_per_block = block_tokens;
    g.max_blocks = max_blocks;
    cache_ = std::make_unique<DeviceCache>(g, kF32);

    x_.ensure(H * sizeof(float));
    norm_.ensure(H * sizeof(float));
    q_.ensure(H * sizeof(float));
    kall_.ensure(c.layers * KV * sizeof(float));
    vall_.ensure(c.layers * KV * sizeof(float));
    attn_.ensure(H * sizeof(float));
    gate_.ensure(I * sizeof(float));
    up_.ensure(I * sizeof(float));
    logits_.ensure(c.vocab * sizeof(float));
    rope_.ensure(c.head_dim() * sizeof(float));
    metadata_ = gguf::metadata_json(doc);
}

void DeviceModel::decode(uint64_t sequence, size_t token, float* logits_host) {
    const ModelConfig& c = cfg_;
    const size_t position = cache_->sequence(sequence).length;
    if (token >= c.vocab || position >= c.context)
        throw std::invalid_argument("paged decode exceeds token/context limits");
    hipStream_t s = cache_->stream();
    const int H = static_cast<int>(c.hidden), I = static_cast<int>(c.intermediate);
    const int KV = static_cast<int>(c.kv_width()), D = static_cast<int>(c.head_dim());
    float* x = at(x_, 0);
    float* q = at(q_, 0);
    float* attn = at(attn_, 0);
    float* gate = at(gate_, 0);
    float* up = at(up_, 0);

    if (embedding_.q8)
        launch_gather_embedding_q8(embedding_, nullptr, static_cast<uint32_t>(token), 1, x, s);
    else
        TVARA_HIP(hipMemcpyAsync(x, at(embedding_.f32, token * c.hidden), c.hidden * sizeof(float),
                                 hipMemcpyDeviceToDevice, s));
    // (cos, sin) of this position, computed as rotary() does (model.hpp:66-68)
    auto* cs = static_cast<float*>(rope_host_.acquire(c.head_dim() * sizeof(float)));
    for (int i = 0; i < D / 2; ++i) {
        const float angle =
            static_cast<float>(position) / std::pow(c.rope_theta, static_cast<float>(2 * i) / static_cast<float>(D));
        cs[2 * i] = std::cos(angle);
        cs[2 * i + 1] = std::sin(angle);
    }
    TVARA_HIP(hipMemcpyAsync(rope_.ptr, cs, c.head_dim() * sizeof(float), hipMemcpyHostToDevice, s));
    rope_host_.release(s);

    // attention rows: the cached tokens plus this token as the tail
    // (paged_model.hpp:22; attention.hpp:80)
    AttnPlan& plan = step_plan_;
    plan.build(cache_.get(), {sequence}, {position}, {1}, static_cast<int>(c.heads), 0);
    step_events_.ensure();

    for (size_t l = 0; l < c.layers; ++l) {
        Layer& L = layers_[l];
        float* kl = at(kall_, l * c.kv_width());
        float* vl = at(vall_, l * c.kv_width());
        const MatvecSegment qkv[3] = {{q, H, nullptr}, {kl, KV, nullptr}, {vl, KV, nullptr}};
        if (L.qkv.q8 && c.interleaved_rope) {  // RoPE in the product's epilogue
            launch_matvec_q8(L.qkv, x, qkv, 3, s, at(L.attn_norm, 0), c.rms_epsilon, at(rope_, 0), D, H + KV);
        } else {
            matvec(L.qkv, x, qkv, 3, s, at(L.attn_norm, 0));
            launch_rope(q, static_cast<int>(c.heads), kl, static_cast<int>(c.kv_heads), D, at(rope_, 0),
                        c.interleaved_rope, s);
        }
        plan.launch(static_cast<int>(l), q, kl, vl, attn, s);
        if (l + 1 == c.layers) TVARA_HIP(hipEventRecord(step_events_.attn, s));
        const MatvecSegment o[1] = {{x, H, x}};
        matvec(L.out, attn, o, 1, s);
        if (L.gate_up.interleaved) {  // SwiGLU in the product's epilogue, into gate
            const MatvecSegment gu[1] = {{gate, 2 * I, nullptr}};
            matvec(L.gate_up, x, gu, 1, s, at(L.ffn_norm, 0));
        } else {
            const MatvecSegment gu[2] = {{gate, I, nullptr}, {up, I, nullptr}};
            matvec(L.gate_up, x, gu, 2, s, at(L.ffn_norm, 0));
            launch_swiglu(gate, up, I, s);
        }
        const MatvecSegment d[1] = {{x, H, x}};
        matvec(L.down, gate, d, 1, s);
    }
    const MatvecSegment lg[1] = {{at(logits_, 0), static_cast<int>(c.vocab), nullptr}};
    matvec(has_output_ ? output_ : embedding_, x, lg, 1, s, at(final_norm_, 0));
    // a non-finite score fails the token before anything is appended; the
    // check waits for the last layer's attention only, so the append is
    // planned while the GPU finishes the layer and the logits
    plan.check_after(step_events_.attn);
    // the token's K/V for every layer, appended after all layers succeeded
    // (paged_model.hpp:27)
    cache_->append_batch(&sequence, 1, at(kall_, 0), at(vall_, 0), true);
    copier_.from_device(logits_host, logits_.ptr, c.vocab * sizeof(float), s);
}

void DeviceModel::matvec(const Weight& w, const float* v, const MatvecSegment* seg, int nseg, hipStream_t s,
                         const float* norm_w) {
    if (w.q8) {
        launch_matvec_q8(w, v, seg, nseg, s, norm_w, cfg_.rms_epsilon);
        return;
    }
    if (norm_w) {  // the f32 product reads a normalised copy
        launch_rmsnorm(v, norm_w, at(norm_, 0), w.cols, cfg_.rms_epsilon, s);
        v = at(norm_, 0);
    }
    launch_matvec(static_cast<const float*>(w.f32.ptr), w.rows, w.cols, v, seg, nseg, s);
}

void DeviceModel::ensure_batch(size_t n) {
    if (n <= batch_cap_) return;
    const ModelConfig& c = cfg_;
    const size_t H = c.hidden, I = c.intermediate, KV = c.kv_width(), L = c.layers, F = sizeof(float);
    if (!part_rows_) {
        auto note = [&](const Weight& w) { part_rows_ = std::max(part_rows_, static_cast<size_t>(batch_splits_max(w)) * w.rows); };
        for (const Layer& l : layers_) {
            note(l.qkv);
            note(l.out);
            note(l.gate_up);
            note(l.down);
        }
        note(has_output_ ? output_ : embedding_);
    }
    bx_.ensure(n * H * F);
    bnorm_.ensure(n * H * F);
    bq_.ensure(n * H * F);
    bk_.ensure(L * n * KV * F);
    bv_.ensure(L * n * KV * F);
    bkapp_.ensure(n * L * KV * F);
    bvapp_.ensure(n * L * KV * F);
    battn_.ensure(n * H * F);
    bgate_.ensure(n * I * F);
    blogits_.ensure(n * c.vocab * F);
    brope_.ensure(n * c.head_dim() * F);
    btok_.ensure(n * sizeof(uint32_t));
    bpart_.ensure(n * part_rows_ * F);
    bhalves_.ensure((n + 15) / 16 * 16 * std::max(H, I) * 2 * sizeof(_Float16));
    bunscale_.ensure(n * F);
    batch_cap_ = n;
}

void DeviceModel::StepEvents::ensure() {
    if (!copy) TVARA_HIP(hipStreamCreateWithFlags(&copy, hipStreamNonBlocking));
    if (!attn) TVARA_HIP(hipEventCreateWithFlags(&attn, hipEventDisableTiming));
    for (hipEvent_t& e : band)
        if (!e) TVARA_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
}

DeviceModel::StepEvents::~StepEvents() {
    for (hipEvent_t e : band)
        if (e) (void)hipEventDestroy(e);
    if (attn) (void)hipEventDestroy(attn);
    if (copy) (void)hipStreamDestroy(copy);
}

void DeviceModel::decode_many(const uint64_t* sequences, const uint32_t* tokens, size_t n, float* logits_host) {
    if (!n) return;
    const ModelConfig& c = cfg_;
    std::vector<uint64_t> seqs(sequences, sequences + n);
    std::vector<size_t> positions(n);
    {
        std::vector<uint64_t> sorted = seqs;
        std::sort(sorted.begin(), sorted.end());
        if (std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end())
            throw std::invalid_argument("duplicate sequence in decode batch");
    }
    for (size_t i = 0; i < n; ++i) {
        positions[i] = cache_->sequence(seqs[i]).length;
        if (tokens[i] >= c.vocab || positions[i] >= c.context)
            throw std::invalid_argument("paged decode exceeds token/context limits");
    }
    if (n > static_cast<size_t>(std::numeric_limits<int>::max() / std::max<size_t>(c.vocab, c.hidden)))
        throw std::invalid_argument("decode batch too large");
    if (!batched_widths()) {
        size_t done = 0;
        try {
            for (; done < n; ++done) decode(seqs[done], tokens[done], logits_host + done * c.vocab);
        } catch (...) {
            for (size_t i = 0; i < done; ++i) cache_->truncate(seqs[i], positions[i]);
            throw;
        }
        return;
    }
    ensure_batch(n);
    hipStream_t s = cache_->stream();
    const int N = static_cast<int>(n), KV = static_cast<int>(c.kv_width());
    stage_rows(tokens, positions.data(), n);
    // each row reads its sequence's cached tokens, then its own token as the tail
    AttnPlan& plan = batch_plan_;
    plan.build(cache_.get(), seqs, positions, std::vector<uint8_t>(n, 1), static_cast<int>(c.heads), 0);
    layer_stack(n, [&](int l, const float* q, float* kl, float* vl, float* attn) {
        plan.launch(l, q, kl, vl, attn, s);
    });
    const LogitsBands bands = launch_logits(n, 0);
    plan.check_after(step_events_.attn);
    launch_interleave_layers(at(bk_, 0), at(bkapp_, 0), static_cast<int>(c.layers), N, KV, s);
    launch_interleave_layers(at(bv_, 0), at(bvapp_, 0), static_cast<int>(c.layers), N, KV, s);
    size_t applied = 0;
    try {
        cache_->append_batch(seqs.data(), n, at(bkapp_, 0), at(bvapp_, 0), true, &applied);
    } catch (...) {
        for (size_t i = 0; i < applied; ++i) cache_->truncate(seqs[i], positions[i]);  // all or nothing
        throw;
    }
    copy_logits(bands, n, logits_host);
}

bool DeviceModel::batched_widths() const {
    // the batched products tile K by 32 and the epilogues hold a row of up to
    // 16,384 in registers; other widths decode token by token
    const ModelConfig& c = cfg_;
    return c.hidden % 32 == 0 && c.intermediate % 32 == 0 && c.hidden <= 16384 && c.intermediate <= 16384;
}

void DeviceModel::stage_rows(const uint32_t* tokens, const size_t* positions, size_t n) {
    const ModelConfig& c = cfg_;
    hipStream_t s = cache_->stream();
    const int D = static_cast<int>(c.head_dim());
    // tokens and each row's (cos, sin) go up through one pinned staging area
    const size_t tok_bytes = (n * sizeof(uint32_t) + 15) / 16 * 16;
    auto* host = static_cast<char*>(bhost_.acquire(tok_bytes + n * c.head_dim() * sizeof(float)));
    std::memcpy(host, tokens, n * sizeof(uint32_t));
    auto* cs = reinterpret_cast<float*>(host + tok_bytes);
    // rotary()'s angle position / theta^(2i/D) (model.hpp:66-68), with the
    // power taken once per i (the same float values)
    std::vector<float> inv_freq(D / 2);
    for (int i = 0; i < D / 2; ++i) inv_freq[i] = std::pow(c.rope_theta, static_cast<float>(2 * i) / static_cast<float>(D));
    for (size_t j = 0; j < n; ++j)
        for (int i = 0; i < D / 2; ++i) {
            const float angle = static_cast<float>(positions[j]) / inv_freq[i];
            cs[j * D + 2 * i] = std::cos(angle);
            cs[j * D + 2 * i + 1] = std::sin(angle);
        }
    TVARA_HIP(hipMemcpyAsync(btok_.ptr, host, n * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    TVARA_HIP(hipMemcpyAsync(brope_.ptr, cs, n * c.head_dim() * sizeof(float), hipMemcpyHostToDevice, s));
    bhost_.release(s);
    const int N = static_cast<int>(n), H = static_cast<int>(c.hidden);
    if (embedding_.q8)
        launch_gather_embedding_q8(embedding_, static_cast<const uint32_t*>(btok_.ptr), 0, N, at(bx_, 0), s);
    else
        launch_gather_embedding(at(embedding_.f32, 0), static_cast<const uint32_t*>(btok_.ptr), N, H, at(bx_, 0), s);
}

void DeviceModel::layer_stack(size_t n, const Attend& attend) {
    const ModelConfig& c = cfg_;
    hipStream_t s = cache_->stream();
    const int N = static_cast<int>(n);
    const int H = static_cast<int>(c.hidden), I = static_cast<int>(c.intermediate), D = static_cast<int>(c.head_dim());
    float* x = at(bx_, 0);
    float* norm = at(bnorm_, 0);
    float* q = at(bq_, 0);
    float* attn = at(battn_, 0);
    float* gate = at(bgate_, 0);
    float* part = at(bpart_, 0);
    auto* halves = static_cast<_Float16*>(bhalves_.ptr);
    float* unscale = at(bunscale_, 0);
    // a Q8_0 product reads its input as halves, an f32 one as f32 rows
    auto halves_for = [&](const Weight& w) { return w.q8 ? halves : nullptr; };
    auto rows_for = [&](const Weight& w, float* rows) { return w.q8 ? nullptr : rows; };
    const Weight& logits_w = has_output_ ? output_ : embedding_;
    step_events_.ensure();
    // Per layer: the products write split sums, and each epilogue finishes
    // what follows its product (RoPE; the residual add with the next
    // RMSNorm; SwiGLU) and writes the next product's input.
    launch_resid_norm(nullptr, 0, x, at(layers_[0].attn_norm, 0), N, H, c.rms_epsilon, rows_for(layers_[0].qkv, norm),
                      halves_for(layers_[0].qkv), unscale, s);
    for (size_t l = 0; l < c.layers; ++l) {
        Layer& L = layers_[l];
        float* kl = at(bk_, l * n * c.kv_width());
        float* vl = at(bv_, l * n * c.kv_width());
        launch_batch_product(L.qkv, norm, halves, unscale, N, part, s);
        launch_qkv_epilogue(part, batch_splits(L.qkv, N), N, static_cast<int>(c.heads), static_cast<int>(c.kv_heads), D,
                            c.interleaved_rope, at(brope_, 0), q, kl, vl, s);
        attend(static_cast<int>(l), q, kl, vl, attn);
        if (l + 1 == c.layers) TVARA_HIP(hipEventRecord(step_events_.attn, s));
        if (L.out.q8) launch_split_halves(attn, N, H, halves, unscale, s);
        launch_batch_product(L.out, attn, halves, unscale, N, part, s);
        launch_resid_norm(part, batch_splits(L.out, N), x, at(L.ffn_norm, 0), N, H, c.rms_epsilon,
                          rows_for(L.gate_up, norm), halves_for(L.gate_up), unscale, s);
        launch_batch_product(L.gate_up, norm, halves, unscale, N, part, s);
        launch_swiglu_epilogue(part, batch_splits(L.gate_up, N), N, I, rows_for(L.down, gate), halves_for(L.down), unscale,
                               s, L.gate_up.interleaved);
        launch_batch_product(L.down, gate, halves, unscale, N, part, s);
        // after the last layer the rows stay too: the logits of chosen rows
        // are taken from them
        const bool last = l + 1 == c.layers;
        launch_resid_norm(part, batch_splits(L.down, N), x, last ? at(final_norm_, 0) : at(layers_[l + 1].attn_norm, 0), N,
                          H, c.rms_epsilon, last ? norm : rows_for(layers_[l + 1].qkv, norm),
                          halves_for(last ? logits_w : layers_[l + 1].qkv), unscale, s);
    }
}

DeviceModel::LogitsBands DeviceModel::launch_logits(size_t n, size_t row0) {
    const ModelConfig& c = cfg_;
    hipStream_t s = cache_->stream();
    const int N = static_cast<int>(n);
    const Weight& logits_w = has_output_ ? output_ : embedding_;
    const float* norm = at(bnorm_, row0 * c.hidden);
    auto* halves = static_cast<_Float16*>(bhalves_.ptr);
    float* unscale = at(bunscale_, 0);
    // rows after the first of the final norm: their halves again, from vector 0
    if (row0 && logits_w.q8) launch_split_halves(norm, N, static_cast<int>(c.hidden), halves, unscale, s);
    // Large logits (8 MiB and up, unsplit Q8_0) are computed in bands of row
    // tiles, each copied to the host while the next is computed.
    LogitsBands b;
    const int vocab = static_cast<int>(c.vocab);
    constexpr int kBands = StepEvents::kBands;
    b.banded = logits_w.q8 && batch_splits(logits_w, N) == 1 && n * c.vocab * sizeof(float) >= (size_t(8) << 20);
    if (b.banded) {
        const int tiles = logits_w.tiles(), per = (tiles + kBands - 1) / kBands;
        for (int t = 0; t < tiles; t += per) {
            launch_batch_product_tiles(logits_w, t, std::min(tiles, t + per), halves, unscale, N, at(blogits_, 0), s);
            TVARA_HIP(hipEventRecord(step_events_.band[b.bands], s));
            b.bounds[b.bands++] = static_cast<size_t>(t) * 16;
        }
        b.bounds[b.bands] = c.vocab;
    } else if (batch_splits(logits_w, N) == 1) {
        launch_batch_product(logits_w, norm, halves, unscale, N, at(blogits_, 0), s);
    } else {
        float* part = at(bpart_, 0);
        launch_batch_product(logits_w, norm, halves, unscale, N, part, s);
        launch_split_sum(part, batch_splits(logits_w, N), N, vocab, at(blogits_, 0), s);
    }
    return b;
}

void DeviceModel::copy_logits(const LogitsBands& b, size_t n, float* logits_host) {
    const ModelConfig& c = cfg_;
    hipStream_t s = cache_->stream();
    if (b.banded) {
        copier_.bands_from_device(logits_host, at(blogits_, 0), n, c.vocab, b.bounds, step_events_.band, b.bands,
                                  step_events_.copy);
        // calls that return host data leave the stream drained (work queued
        // behind the logits ended long before the last band's copy)
        TVARA_HIP(hipStreamSynchronize(s));
    } else
        copier_.from_device(logits_host, blogits_.ptr, n * c.vocab * sizeof(float), s);
}

void DeviceModel::decode_chunk(uint64_t sequence, const uint32_t* tokens, size_t n, float* logits_host,
                               bool last_only) {
    if (!n) return;
    const ModelConfig& c = cfg_;
    const size_t position = cache_->sequence(sequence).length;
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= c.vocab) throw std::invalid_argument("paged decode exceeds token/context limits");
    if (n > c.context || position > c.context - n)
        throw std::invalid_argument("paged decode exceeds token/context limits");
    if (n == 1 || !batched_widths()) {
        std::vector<float> scratch(last_only && n > 1 ? c.vocab : 0);
        for (size_t i = 0; i < n; ++i) {
            float* out = last_only ? (i + 1 == n ? logits_host : scratch.data()) : logits_host + i * c.vocab;
            decode(sequence, tokens[i], out);
        }
        return;
    }
    const size_t rows = std::min(n, kChunkRows);
    if (rows > static_cast<size_t>(std::numeric_limits<int>::max() / std::max<size_t>(c.vocab, c.hidden)))
        throw std::invalid_argument("decode batch too large");
    ensure_batch(rows);
    hipStream_t s = cache_->stream();
    const int heads = static_cast<int>(c.heads);
    std::vector<size_t> positions(rows);
    std::vector<uint64_t> seq_of_row(rows, sequence);
    // TVARA_CHUNK_ATTENTION=rows (read on every call) keeps the f32 rows, the
    // reference's arithmetic, for every layout
    const char* choice = std::getenv("TVARA_CHUNK_ATTENTION");
    const bool rows_only = choice && std::strcmp(choice, "rows") == 0;
    const bool tiles = !rows_only && prefill_x3_supported(cache_->layout(), 1);
    for (size_t c0 = 0; c0 < n; c0 += rows) {
        const size_t m = std::min(rows, n - c0);
        positions.resize(m);
        seq_of_row.resize(m);
        for (size_t j = 0; j < m; ++j) positions[j] = position + c0 + j;
        stage_rows(tokens + c0, positions.data(), m);
        // the chunk's tokens join the sequence now (their blocks zero-filled or
        // copied on write); every layer writes its K/V rows into their slots
        // before its attention reads them
        const RowOp* slots = cache_->reserve_tokens(sequence, m);
        const bool last = c0 + m == n, logits = !(last_only && !last);
        const size_t out_rows = last_only ? 1 : m;
        // One pass over the layers, the logits and their copy.  A pass on the
        // tiles returns false when their flag is raised: a query or key beyond
        // the fp16 range (or a non-finite input); the chunk is then staged
        // again and takes the f32 rows, which rewrite the same slots.
        auto pass = [&](bool on_tiles) {
            // row j sees the cached tokens and the chunk up to itself
            // (fused_prompt_attention, attention.hpp:85-89)
            std::function<void(hipEvent_t)> check;
            Attend attend;
            if (on_tiles) {
                const size_t start = position + c0;
                chunk_plan_.build(cache_.get(), &sequence, 1, c.heads, c.context, &start, &m, 2);
                chunk_plan_.use_pinned_error();
                attend = [&](int l, const float* q, float* kl, float* vl, float* attn) {
                    cache_->write_layer_rows(slots, m, l, kl, vl);
                    chunk_plan_.launch(l, q, attn, s);
                };
                check = [&](hipEvent_t e) { chunk_plan_.check_after(e); };
            } else {
                std::vector<size_t> lengths(m);
                for (size_t j = 0; j < m; ++j) lengths[j] = positions[j] + 1;
                batch_plan_.build(cache_.get(), seq_of_row, lengths, {}, heads, 0);
                attend = [&](int l, const float* q, float* kl, float* vl, float* attn) {
                    cache_->write_layer_rows(slots, m, l, kl, vl);
                    batch_plan_.launch(l, q, nullptr, nullptr, attn, s);
                };
                check = [&](hipEvent_t e) { batch_plan_.check_after(e); };
            }
            layer_stack(m, attend);
            LogitsBands bands;
            if (logits) bands = launch_logits(out_rows, m - out_rows);
            if (on_tiles) {
                try {
                    check(step_events_.attn);
                } catch (const std::invalid_argument&) {
                    TVARA_HIP(hipStreamSynchronize(s));
                    return false;
                }
            } else {
                check(step_events_.attn);
            }
            if (logits) copy_logits(bands, out_rows, last_only ? logits_host : logits_host + c0 * c.vocab);
            return true;
        };
        if (!pass(tiles)) {
            stage_rows(tokens + c0, positions.data(), m);
            pass(false);
        }
    }
}

}  // namespace tvara_amd
