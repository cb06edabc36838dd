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
constexpr int BAR_WORDS = 19 * 32;
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

// One head layer's weights (a pre-LayerNorm encoder layer with biases, src/forward.rs:551-658),
// as the whole-model kernel reads them (an array of these lives in device memory).
struct HeadDesc {
    const jh_half *in_proj, *out_proj, *linear1, *linear2;  // fragment order, biases folded
    const float *in_proj_colsum, *in_proj_b, *out_proj_b, *linear1_colsum, *linear1_b, *linear2_b;
};

// The rest of the model around the encoder, for one launch of the whole forward pass (the
// reference's stated next step, README.md:12-13): embed writes the encoder's x_in first; after
// the last layer norm_add, the head layers, the scorer's lin1 and the score. Outputs that other
// blocks read through their caches have buffers of their own, as LayerArgs': the head's
// residual stream hxa (1 + 2 head_layers slots of x_stride: norm_add's output, then per head
// layer after out_proj and after linear2), each head layer's qkv (hqa, q_stride) and attention
// output (hoa, o_stride), the scorer's hidden rows hs; linear1's output goes to LayerArgs' mid.
struct ModelArgs {
    const uint32_t* ids;  // the rows' token ids (device)
    const jh_half* tok_emb;
    const float* emb_norm;
    int vocab;
    const HeadDesc* heads;       // device array of head_layers
    const HeadDesc* host_heads;  // the same on the host (for the checks)
    int head_layers, head_ff;
    float head_eps;
    const float* final_norm;
    // The type embedding added by norm_add: the request's row (row_type null), or the table,
    // each row adding row row_type[row] of it.
    const float* type_add;
    const int32_t* row_type;
    jh_half *hxa, *hqa, *hoa, *hs;
    const jh_half* lin1;
    const float *lin1_colsum, *lin1_b;
    const jh_half* lin2;
    float lin2_b;
    const uint32_t* markers;  // row indices (device)
    int n_markers;
    float* logits;  // n_markers (device)
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
    const ModelArgs* model = nullptr;  // the whole model: embed into x_in first, the head after
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
    // Split-K and key-range scratch for any m up to max_m (head_ff > 0: the whole-model
    // launch's head GEMMs too).
    size_t ws_floats(int max_m, int d, int inter, int head_ff = 0) const;
    size_t counters(int max_m, int d, int inter, int head_ff = 0) const;
    // Phases: bits 0-4 select qkv, attention, wo, wi, wo_mlp (0x1f: whole layers; a subset only
    // with one layer). prof: null, or PROF_WORDS u64 per block of the grid and layer run.
    // a.model: the whole forward pass (all layers and phases, from layer 0). Returns false,
    // having launched nothing, when the runtime refuses the cooperative launch (another process
    // holds the GPU's cooperative-launch resource): the caller runs the pass another way.
    [[nodiscard]] bool launch(const LayerArgs& a, const LayerPlan& plan, const Scratch& s,
                              hipStream_t stream, unsigned phases = 0x1f, uint64_t* prof = nullptr);
    int grid(const LayerArgs& a, const LayerPlan& plan) const;
    // LDS bytes a plan needs on m rows (weight tile, reduction and attention share it).
    static int lds_bytes(const LayerPlan& plan, int d, int inter, int m, int window);
    // Whether the whole-model launch takes this plan on m rows: its head GEMMs fit the plan's
    // kernel instance (the throughput instances need every head GEMM on their tile).
    bool model_fits(const LayerPlan& plan, int m, int d, int head_ff) const;
    // Whether a grid barrier gave up waiting since the last call (then clears the words).
    // Synchronizes with the device.
    bool barrier_timed_out();
    // Where the launch of `a` leaves the residual stream (x after its last layer).
    static jh_half* x_out(const LayerArgs& a) {
        return a.xa + (size_t)(2 * (a.first + a.count - 1) + 1) * a.x_stride;
    }
    int per_cu() const { return per_cu_; }
    size_t refused() const { return refused_; }  // cooperative launches the runtime refused
    bool available() const { return per_cu_ > 0; }
    // A plan for large batches: every GEMM on the 128 x 128 throughput tile and attention on the
    // 64-query tile, run by the kernel's large-batch instance (two blocks a CU).
    static bool is_big(const LayerPlan& plan, int m);
    static int big_mode(const LayerPlan& plan, int m);  // the kernel instance (layer.hip)

private:
    int cus_ = 0, per_cu_ = 0, per_cu_big_ = 0, per_cu_big256_ = 0, lds_max_ = 0;
    bool lat48_ok_ = false;  // the 48-row instance fits as many blocks a CU as the plain one
    uint32_t* bar_ = nullptr;  // BAR_WORDS words
    // Launch through hipLaunchCooperativeKernel (true), or as a plain launch of the same
    // resident grid when the environment sets JULIA_HIP_COOPERATIVE=0. The grid barrier is the
    // kernel's own (atomics with a bounded wait), so the plain launch runs the same code; a grid
    // that is not co-resident ends in the bounded wait's error.
    bool coop_ = true;
    // Tests of the barrier's time-out path only (JULIA_HIP_TEST_BARRIER_SKEW=1 when the engine
    // is loaded): every grid barrier waits for one generation more than its arrivals make, so
    // each block's bounded wait gives up (the non-co-resident case, forced from the host; every
    // block still runs to its end) and the host reports the error.
    uint32_t skew_ = 0;
    size_t refused_ = 0;
};

}  // namespace jh
