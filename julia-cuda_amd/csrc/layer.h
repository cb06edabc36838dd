// The persistent layer kernel's host side (the reference's `layer` launch, src/forward.rs:
// 167-359, and `LayerPlan`, :737-757): one encoder layer as one cooperative launch, its five
// steps as phases separated by grid barriers, each phase a list of tasks the resident blocks
// stride over.
#pragma once

#include <stdint.h>

#include <string>

#include "kernels.h"

namespace jh {

// u32 words of device memory the grid barrier needs (zeroed once; every barrier leaves them zero).
constexpr int BAR_WORDS = 11 * 32;
// u64 words per block of the layer kernel's timestamps: (start, end) of phase p at 2p, 2p + 1
// (100 MHz clock), the block's CU id at 10.
constexpr int PROF_WORDS = 16;

struct LayerArgs {
    jh_half *x, *qkv, *o, *mid;
    float *stats_attn, *stats_mlp;  // wo writes stats_attn (wi reads it), wo_mlp stats_mlp
    const jh_half *wqkv, *wo, *wi, *wo_mlp;
    const float *qkv_colsum;  // null in layer 0: no LayerNorm before qkv
    const float *rope, *wi_colsum;
    int m, d, inter;
    float eps;
    int window;
    int rope_rows;
};

// src/forward.rs:737-757: per GEMM (qkv, wo, wi, wo_mlp) the tile height and split-K, and the
// key ranges per attention tile in global and sliding-window layers.
struct LayerPlan {
    int bm[4];
    int splits[4];
    int kv[2];
    std::string str() const;  // "qkv 32/1 wo 16/2 wi 32/1 wo_mlp 16/2 kv 3/1"
};

class LayerKernel {
public:
    void init(int cus);
    void bind(uint32_t* barrier) { bar_ = barrier; }
    LayerPlan default_plan(int m, int d, int inter, int window) const;
    size_t ws_floats(int max_m, int d, int inter) const;
    size_t counters(int max_m, int d, int inter) const;
    // Phases: bits 0-4 select qkv, attention, wo, wi, wo_mlp (0x1f: the whole layer).
    // prof: null, or PROF_WORDS u64 per block of the grid (grid()).
    void launch(const LayerArgs& a, const LayerPlan& plan, const Scratch& s, hipStream_t stream,
                unsigned phases = 0x1f, uint64_t* prof = nullptr);
    int grid(const LayerArgs& a, const LayerPlan& plan) const;
    // Whether a grid barrier gave up waiting since the last call (then clears the flag).
    // Synchronizes with the device.
    bool barrier_timed_out();
    int per_cu() const { return per_cu_; }
    bool available() const { return per_cu_ > 0; }

private:
    int cus_ = 0, per_cu_ = 0;
    uint32_t* bar_ = nullptr;  // BAR_WORDS words
};

}  // namespace jh
