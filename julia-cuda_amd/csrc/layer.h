// The persistent encoder kernel's host side (the reference's `layer` launch, src/forward.rs:
// 167-359, and `LayerPlan`, :737-757). The reference launches one cooperative kernel per layer;
// here one cooperative launch runs a range of layers (the whole encoder in the forward pass),
// each layer's five steps as phases separated by grid barriers, each phase a list of tasks the
// resident blocks stride over.
#pragma once

#include <stdint.h>

#include <string>

#include "kernels.h"

namespace jh {

// u32 words of device memory the grid barrier needs (zero between launches; a launch leaves
// them zero, and the host clears them after a barrier time-out).
constexpr int BAR_WORDS = 11 * 32;
// u64 words per block and layer of the kernel's timestamps: (start, end) of phase p at 2p,
// 2p + 1 (100 MHz clock), the block's CU id at 10; for the block's first attention task at 12 + i:
// its key range in LDS, its key loop done, its output stored; and for the block's first task of
// GEMM g (qkv, wo, wi, wo_mlp) at 16 + 4 g + i: its inputs in place (weights in LDS, activations
// in registers), its MFMAs done, its partial tiles reduced, its epilogue done.
constexpr int PROF_WORDS = 32;

// One layer's weights, as the kernel reads them (an array of these lives in device memory).
struct LayerDesc {
    const jh_half *wqkv, *wo, *wi, *wo_mlp;  // fragment order
    const float *qkv_colsum;                 // null in layer 0: no LayerNorm before qkv
    const float *wi_colsum, *rope;
    int window;                              // 0: global attention
    int pad_;
};

// The activations of a launch: every output of a phase that other blocks read through their
// caches goes to a buffer of its own, written once per launch (no L2 can hold a stale copy):
// layer l reads x_in (its first layer) or xa[2 l - 1], writes xa[2 l] (after wo) and
// xa[2 l + 1] (after wo_mlp), qkv into qa[l] and o into oa[l] (slots of x_stride, q_stride and
// o_stride elements; l is the absolute layer index). mid and the statistics, which several
// blocks write parts of per line, are single buffers read device-coherent.
struct LayerArgs {
    const jh_half* x_in;
    jh_half *xa, *qa, *oa, *mid;
    size_t x_stride, q_stride, o_stride;
    float *stats_attn, *stats_mlp;  // wo writes stats_attn (wi reads it), wo_mlp stats_mlp
    // Concatenated requests (nullable): each row's position in its request, and its request's
    // rows [first, one past last] (AttnParams::seg).
    const int32_t *pos, *seg;
    const LayerDesc* layers;        // device array, indexed by layer
    const LayerDesc* host_layers;   // the same on the host (for the plan and the checks)
    int first, count;               // the layers this launch runs
    int m, d, inter;
    float eps;
    int rope_rows;
};

// src/forward.rs:737-757: per GEMM (qkv, wo, wi, wo_mlp) the tile height and split-K, and the
// key ranges per attention tile in global and sliding-window layers.
struct LayerPlan {
    int bm[4];
    int splits[4];
    int kv[2];
    std::string str() const;  // "qkv 64/1 wo 16/1 wi 64/1 wo_mlp 16/1 kv 4/1"
};

class LayerKernel {
public:
    void init(int cus, int lds_bytes);
    void bind(uint32_t* barrier) { bar_ = barrier; }
    LayerPlan default_plan(int m, int d, int inter) const;
    size_t ws_floats(int max_m, int d, int inter) const;
    size_t counters(int max_m, int d, int inter) const;
    // Phases: bits 0-4 select qkv, attention, wo, wi, wo_mlp (0x1f: whole layers; a subset only
    // with one layer). prof: null, or PROF_WORDS u64 per block of the grid and layer run.
    void launch(const LayerArgs& a, const LayerPlan& plan, const Scratch& s, hipStream_t stream,
                unsigned phases = 0x1f, uint64_t* prof = nullptr);
    int grid(const LayerArgs& a, const LayerPlan& plan) const;
    // LDS bytes a plan needs on m rows (weight tile, reduction and attention share it).
    static int lds_bytes(const LayerPlan& plan, int d, int inter, int m, int window);
    // Whether a grid barrier gave up waiting since the last call (then clears the words).
    // Synchronizes with the device.
    bool barrier_timed_out();
    // Where the launch of `a` leaves the residual stream (x after its last layer).
    static jh_half* x_out(const LayerArgs& a) {
        return a.xa + (size_t)(2 * (a.first + a.count - 1) + 1) * a.x_stride;
    }
    int per_cu() const { return per_cu_; }
    bool available() const { return per_cu_ > 0; }
    // A plan for large batches: every GEMM on the 128 x 128 throughput tile and attention on the
    // 64-query tile, run by the kernel's large-batch instance (two blocks a CU).
    static bool is_big(const LayerPlan& plan, int m);
    static int big_mode(const LayerPlan& plan, int m);  // the kernel instance (layer.hip)

private:
    int cus_ = 0, per_cu_ = 0, per_cu_big_ = 0, per_cu_big256_ = 0, lds_max_ = 0;
    uint32_t* bar_ = nullptr;  // BAR_WORDS words
};

}  // namespace jh
