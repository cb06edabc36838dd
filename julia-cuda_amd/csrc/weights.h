// The model's weights as the kernels read them (the reference's src/weights.rs): every matrix
// (and the embedding table) f16 in one arena, the GEMM matrices in MFMA fragment order
// (pack_frag), every vector (LayerNorm weights, biases, column
// sums, type embeddings, RoPE tables) f32 in another; each tensor is a Span into one of the two,
// 256-byte aligned. Prepared on the host once (`prepare`), uploaded with two copies.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <functional>
#include <string>
#include <vector>

namespace jh {

struct ModelConfig {
    int d = 768, layers = 22, inter = 1152, vocab = 50368, head_layers = 2, head_ff = 1536;
    int n_qtypes = 3, window = 64, global_every = 3, max_positions = 8192;
    int batch_rows = 0;  // rows of concatenated requests the engine holds (0: max_length)
    float norm_eps = 1e-5f, head_eps = 1e-5f, theta_global = 160000.0f, theta_local = 10000.0f;
    uint64_t seed = 42;
};

// "synthetic[:key=value,...]" -> a config; throws std::runtime_error on anything else.
ModelConfig parse_model_spec(const std::string& spec);

constexpr size_t ALIGN_BYTES = 256;

struct Span {
    size_t start = 0, len = 0;  // in elements of the arena
    bool present = false;
};

struct EncoderLayer {
    Span wqkv, qkv_colsum;  // LayerNorm folded from layer 1 (layer 0 has none: no colsum)
    Span wo;
    Span wi, wi_colsum;     // LayerNorm folded, rows GeGLU-interleaved
    Span wo_mlp;
    bool global = false;
};

struct HeadLayer {
    Span in_proj, in_proj_colsum, in_proj_b;  // norm1 folded (gamma into W, beta into the bias)
    Span out_proj, out_proj_b;
    Span linear1, linear1_colsum, linear1_b;  // norm2 folded
    Span linear2, linear2_b;
};

struct Scorer {
    Span lin1, lin1_colsum, lin1_b;  // the scorer's LayerNorm folded
    Span lin2;
    float lin2_b = 0.0f;
};

struct Layout {
    Span tok_embeddings, emb_norm, rope_global, rope_local;
    std::vector<EncoderLayer> layers;
    Span final_norm, type_emb;
    std::vector<HeadLayer> head;
    Scorer scorer;
};

struct HostWeights {
    Layout layout;
    std::vector<uint16_t> f16;
    std::vector<float> f32;
};

// Where the raw (unprepared) tensors come from: values start .. start + count of tensor `id` (the
// T_* ids below, in the checkpoint's own row-major layout) as f32 into `out`. Called from
// several threads at once.
using TensorSource = std::function<void(uint32_t id, size_t start, size_t count, float* out)>;

// The model for `c` from `src`, prepared (src/weights.rs:143-238).
HostWeights prepare(const ModelConfig& c, const TensorSource& src);

// The seeded synthetic model for `c`, prepared.
HostWeights prepare_synthetic(const ModelConfig& c);

// ---- the pieces (also behind the C ABI's julia_hip_prep_* for tests) ----
uint16_t f32_to_f16(float f);
float f16_to_f32(uint16_t h);
void synth(uint64_t seed, uint32_t id, uint64_t start, uint64_t count, double mean, double std,
           float* out);
void tensor_dist(uint32_t id, double* mean, double* std);
void fold_layernorm(const float* w, const float* gamma, int out, int k, uint16_t* w16,
                    float* colsum);
void fold_layernorm_bias(const float* w, const float* gamma, const float* beta, const float* b,
                         int out, int k, uint16_t* w16, float* colsum, float* bias);
void geglu_rows(int inter, int32_t* src);
// W [n][k] (n % 64 == 0, k % 32 == 0) <-> the GEMM kernels' MFMA fragment order: for 64-row
// group G, 32-column unit u, 16-row fragment j and lane l < 64, the 8 values
// W[64 G + 16 j + l % 16][32 u + 8 (l / 16) + e], e < 8, contiguous, in that nesting.
void pack_frag(const uint16_t* w, int n, int k, uint16_t* out);
void unpack_frag(const uint16_t* packed, int n, int k, uint16_t* w);
void rope_table(float theta, int npos, float* table);

// Tensor ids of the synthetic model (the generator's streams).
enum : uint32_t {
    T_TOK_EMB = 1, T_EMB_NORM = 2, T_FINAL_NORM = 3, T_TYPE_EMB = 4,
    T_LAYER = 100,   // + 16 l + {attn_norm, wqkv, wo, mlp_norm, wi, wo_mlp}
    T_HEAD = 1000,   // + 32 h + {norm1_w, norm1_b, in_proj_w, in_proj_b, out_proj_w, out_proj_b,
                     //           norm2_w, norm2_b, linear1_w, linear1_b, linear2_w, linear2_b}
    T_SCORER = 2000  // + {norm_w, norm_b, lin1_w, lin1_b, lin2_w, lin2_b}
};

}  // namespace jh
