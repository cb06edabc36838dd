// A checkpoint directory (the reference's src/checkpoint.rs:27-62): `model.safetensors` (the
// tensors, memory-mapped), `encoder/config.json` (the encoder's shapes, in the field names of
// Hugging Face's ModernBertConfig), optionally `julia_config.json` (the head's LayerNorm eps)
// and `julia_hip_names.json` (tensor names that differ from the defaults below). The head's
// sizes (layers, feed-forward width, question types) are read off the tensors' shapes.
//
// Tensor names: the reference reads them through julia-rs's safetensors parser, which is not
// vendored, so they are not known here. The defaults follow the public conventions of the
// pieces the model is made of: ModernBERT for the encoder ("{enc}layers.{l}.attn.Wqkv.weight",
// ...; {enc} is the prefix of the key that ends in "embeddings.tok_embeddings.weight"), torch's
// TransformerEncoderLayer for the head layers ("head.layers.{h}.self_attn.in_proj_weight",
// "...norm1.weight", "...linear1.weight", ...), and "type_emb.weight", "scorer.{norm,lin1,lin2}"
// for the rest. julia_hip_names.json maps a logical name (the keys of kNames in checkpoint.cpp,
// e.g. "layer.wqkv" or "head.norm1_w") to a pattern with {enc}, {l} and {h}, or sets
// "encoder_prefix".
#pragma once

#include <memory>
#include <string>

#include "weights.h"

namespace jh {

class Checkpoint {
public:
    // Opens and checks `dir`: every tensor the model needs is present, F32/F16/BF16, of the
    // shape the config implies, inside the file. Throws std::runtime_error naming what is wrong.
    explicit Checkpoint(const std::string& dir);
    ~Checkpoint();
    Checkpoint(const Checkpoint&) = delete;
    Checkpoint& operator=(const Checkpoint&) = delete;

    const ModelConfig& config() const { return cfg_; }
    // The tensors by T_* id as f32 (valid while this object lives).
    TensorSource source() const;

    // Whether `spec` names a checkpoint directory (anything but the synthetic model).
    static bool is_checkpoint(const std::string& spec);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
    ModelConfig cfg_;
};

}  // namespace jh
