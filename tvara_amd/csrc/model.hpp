// Llama decode executor over the device KV cache: the state behind the
// model-level C exports (core/include/tvara/c_api.h:13-24), restating
// PagedModelExecutor (core/include/tvara/paged_model.hpp:6-34) with weights
// in HBM and every step of a token on the GPU.
#pragma once

#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"
#include "host_copy.hpp"
#include "kv_cache.hpp"

namespace tvara_amd {

// output rows of one matvec launch that go to one buffer (as residual + y
// when `residual` is set)
struct MatvecSegment {
    float* out;
    int rows;
    const float* residual;
};

// A weight matrix in HBM: f32 rows, or Q8_0 kept quantised.  The Q8_0 form
// is tiled for the kernels that read it: rows are cut into tiles of 16
// (zero-padded) and the groups of 32 columns into pairs (an odd last group
// is paired with a zero group).  Per (tile, pair), lane l of a wave holds 16
// bytes: row l%16, columns 8(l/16) .. 8(l/16)+7 of the pair's first group
// then of its second -- each half is the operand a 16x16x32 MFMA lane reads
// for one group.  A separate plane holds, per (tile, pair), the 16 rows'
// fp16 scales of both groups ([row][2]).  Value = float(d) * q, as
// dequantize_q8_0 computes it (quant.hpp:39-49).
struct Weight {
    bool q8 = false;
    int rows = 0, cols = 0;
    DeviceBuffer f32;  // [rows][cols] floats
    DeviceBuffer q;    // int8 [tiles][pairs][64][16]
    DeviceBuffer d;    // fp16 bits [tiles][pairs][16][2]
    // a fused gate|up block stored with its rows interleaved (row 2i is gate
    // row i, 2i + 1 is up row i), so that the SwiGLU pairs meet in a tile
    bool interleaved = false;
    int tiles() const { return (rows + 15) / 16; }
    int groups() const { return cols / 32; }
    int pairs() const { return (groups() + 1) / 2; }
};

void launch_dequant(uint32_t type, const uint8_t* raw, size_t n, float* out, int* bad, hipStream_t s);
// GGUF Q8_0 rows [rows][cols/32][34 B] into rows row0.. of a tiled Weight;
// flags `bad` when a group scale is not finite (then so is a value)
// (rows row0, row0 + stride, ...); stride 2 interleaves two parts
void launch_q8_repack(const uint8_t* raw, int rows, int cols, int row0, int stride, Weight& w, int* bad,
                      hipStream_t s);
// y = W v; with norm_w set, v is rms_norm(x = the v argument) * norm_w,
// computed inside the launch; rope_cs (interleaved RoPE of the first
// rope_rows rows) and an interleaved gate|up weight (SwiGLU into seg[0])
// apply in the epilogue
void launch_matvec_q8(const Weight& w, const float* v, const MatvecSegment* seg, int nseg, hipStream_t s,
                      const float* norm_w = nullptr, float eps = 0.f, const float* rope_cs = nullptr,
                      int rope_dim = 0, int rope_rows = 0);
// Batched products for n vectors (one per sequence) write f32 sums per K
// split, out[split][n][rows]; batch_splits gives the split count.  Q8_0
// weights read the vectors as fp16 halves (launch_split_halves or an
// epilogue below writes them, with a power-of-two unscale per vector), f32
// weights read x [n][cols].
int batch_splits(const Weight& w, int n);
// the most splits any n gives (the size of a partial-sum buffer)
int batch_splits_max(const Weight& w);
void launch_batch_product(const Weight& w, const float* x, const _Float16* halves, const float* unscale, int n,
                          float* out, hipStream_t s);
// the rows of row tiles [tile0, tile1) of an unsplit Q8_0 product (out as for
// launch_batch_product, rows at their place), so a product can be issued in
// bands
void launch_batch_product_tiles(const Weight& w, int tile0, int tile1, const _Float16* halves, const float* unscale,
                                int n, float* out, hipStream_t s);
void launch_split_halves(const float* x, int n, int cols, _Float16* halves, float* unscale, hipStream_t s);
void launch_split_sum(const float* p, int splits, int n, int rows, float* out, hipStream_t s);
// the split sums of the fused QKV product into q, k (rotated by row j's
// (cos, sin) at cs + j*dim) and v
void launch_qkv_epilogue(const float* p, int splits, int n, int qheads, int kheads, int dim, bool interleaved,
                         const float* cs, float* q, float* k, float* v, hipStream_t s);
// x += the split sums (p may be null), then RMSNorm into norm and, when
// halves is given, into the next product's halves
void launch_resid_norm(const float* p, int splits, float* x, const float* w, int n, int h, float eps, float* norm,
                       _Float16* halves, float* unscale, hipStream_t s);
// SwiGLU of the fused gate|up sums into out and, when given, halves
void launch_swiglu_epilogue(const float* p, int splits, int n, int inter, float* out, _Float16* halves,
                            float* unscale, hipStream_t s, bool interleaved);
// out[j] = row idx[j] (or `row` when idx is null) of a Q8_0 table, dequantised
void launch_gather_embedding_q8(const Weight& w, const uint32_t* idx, uint32_t row, int n, float* out,
                                hipStream_t s);
// `rows` rows of a batch, each normalised on its own
void launch_rmsnorm(const float* x, const float* w, float* out, int n, float eps, hipStream_t s, int rows = 1);
void launch_matvec(const float* w, int rows, int cols, const float* v, const MatvecSegment* seg, int nseg,
                   hipStream_t s);
void launch_interleave_layers(const float* src, float* dst, int layers, int n, int kv, hipStream_t s);
void launch_gather_embedding(const float* table, const uint32_t* idx, int n, int h, float* out, hipStream_t s);
// row j of a batch rotates q + j*qheads*dim and k + j*kheads*dim by cs + j*dim
void launch_rope(float* q, int qheads, float* k, int kheads, int dim, const float* cs, bool interleaved,
                 hipStream_t s, int rows = 1);
void launch_swiglu(float* gate, const float* up, int n, hipStream_t s);

// ModelConfig (model.hpp:9-22)
struct ModelConfig {
    size_t vocab = 0, hidden = 0, intermediate = 0, layers = 0, heads = 0, kv_heads = 0, context = 0;
    float rms_epsilon = 1e-6f, rope_theta = 10000.f;
    bool interleaved_rope = true;
    void validate() const;
    size_t head_dim() const { return hidden / heads; }
    size_t kv_width() const { return head_dim() * kv_heads; }
};

class DeviceModel {
public:
    // load_weights (model.hpp:140-170) + the executor's cache (paged_model.hpp:8-9)
    DeviceModel(const std::string& path, size_t max_blocks, size_t block_tokens);
    const ModelConfig& config() const { return cfg_; }
    DeviceCache& cache() { return *cache_; }
    const std::string& metadata() const { return metadata_; }
    // PagedModelExecutor::decode (paged_model.hpp:12-28): logits of `token`
    // at the end of `sequence`, whose K/V are then appended
    void decode(uint64_t sequence, size_t token, float* logits_host);
    // one token for each of n distinct sequences in one pass: the logits of n
    // independent decode() calls; on failure no sequence changes
    void decode_many(const uint64_t* sequences, const uint32_t* tokens, size_t n, float* logits_host);
    // n consecutive tokens at the end of `sequence` in one pass per chunk of
    // up to kChunkRows tokens (the batched products, each layer's K/V written
    // into the cache, then the rows' causal attention over it): the logits of
    // n decode() calls, of every token or, with last_only, of the last one
    // only.  The attention runs as MFMA tiles with every f32 operand split
    // into two parts (queries and keys fp16, values and probabilities bf16;
    // three products each) where the cache layout allows it (blocks of 16
    // to 1,024 tokens, head_dim 64 or 128), else as f32 rows through the
    // decode kernels; a pass whose queries or keys leave the fp16 range runs
    // again on the rows.  On failure the sequence may hold part of the
    // tokens; the caller truncates it.
    void decode_chunk(uint64_t sequence, const uint32_t* tokens, size_t n, float* logits_host, bool last_only);
    static constexpr size_t kChunkRows = 512;

private:
    struct Layer {
        DeviceBuffer attn_norm, ffn_norm;
        Weight qkv, out, gate_up, down;
    };
    // y = W v, or W rms_norm(x) * norm_w when norm_w is given (v is then x)
    void matvec(const Weight& w, const float* v, const MatvecSegment* seg, int nseg, hipStream_t s,
                const float* norm_w = nullptr);

    ModelConfig cfg_;
    std::string metadata_;
    std::unique_ptr<DeviceCache> cache_;
    // the attention plans of a step, rebuilt per token into the same device
    // region (no allocation once it is large enough), and of a chunk pass
    AttnPlan step_plan_, batch_plan_;
    PrefillPlan chunk_plan_;
    Weight embedding_, output_;
    DeviceBuffer final_norm_;
    bool has_output_ = false;
    std::vector<Layer> layers_;
    // per-token work buffers
    DeviceBuffer x_, norm_, q_, kall_, vall_, attn_, gate_, up_, logits_, rope_, bad_;
    PinnedBuffer rope_host_;
    // batch work buffers, grown to the largest batch seen
    DeviceBuffer bx_, bnorm_, bq_, bk_, bv_, bkapp_, bvapp_, battn_, bgate_, blogits_, brope_, btok_, bpart_, bhalves_,
        bunscale_;
    size_t part_rows_ = 0;  // largest splits x rows of a batched product
    PinnedBuffer bhost_;
    HostCopier copier_;
    // the batched step's synchronisation: an event after the last layer's
    // attention (the plan's check waits on it, not on the whole stream), one
    // per band of the logits product, and the stream the bands' copies to the
    // host cross on while later bands are computed
    struct StepEvents {
        static constexpr int kBands = 4;
        hipStream_t copy = nullptr;
        hipEvent_t attn = nullptr, band[kBands] = {};
        void ensure();
        StepEvents() = default;
        StepEvents(const StepEvents&) = delete;
        StepEvents& operator=(const StepEvents&) = delete;
        ~StepEvents();
    };
    StepEvents step_events_;
    size_t batch_cap_ = 0;
    void ensure_batch(size_t n);
    // the widths the batched products and epilogues take
    bool batched_widths() const;
    // tokens and each row's (cos, sin) to the device, then the rows'
    // embeddings into bx_
    void stage_rows(const uint32_t* tokens, const size_t* positions, size_t n);
    // The layer stack over the n rows staged in bx_: per layer the fused QKV
    // product and its epilogue (q, k, v rows; RoPE), then attend(layer, q, k,
    // v, out), then the output, gate|up and down products with their
    // epilogues.  Records step_events_.attn after the last attention and
    // leaves every row's final RMSNorm in bnorm_ (halves for a Q8_0 logits
    // matrix).
    using Attend = std::function<void(int, const float*, float*, float*, float*)>;
    void layer_stack(size_t n, const Attend& attend);
    // the logits of final-norm rows row0 .. row0 + n - 1 into blogits_, in
    // bands of row tiles for large outputs
    struct LogitsBands {
        bool banded = false;
        int bands = 0;
        size_t bounds[StepEvents::kBands + 1] = {};
    };
    LogitsBands launch_logits(size_t n, size_t row0);
    // blogits_ [n][vocab] to the host (synchronous)
    void copy_logits(const LogitsBands& b, size_t n, float* logits_host);
};

}  // namespace tvara_amd
