// The persistent encoder kernel (the reference's `layer`, kernels/src/main.rs:578-842, which runs
// one layer per cooperative launch): here one cooperative launch runs a range of layers, the
// whole encoder in the forward pass. Each layer's five steps are phases (qkv, attention, wo, wi,
// wo_mlp) with a grid barrier between two phases; every block strides over a phase's tasks. The
// grid is at most the number of blocks resident at once (the cooperative launch checks it).
// With EncParams::model the launch is the whole forward pass: embed before the first layer
// (a wave a row), then after the last layer norm_add, each head layer's in_proj, attention,
// out_proj, linear1 and linear2, the scorer's lin1 and the score, each a phase of its own.
//
// A GEMM task stages its weight tile in LDS (gemm_w_tile). The weights do not depend on the
// previous phase, so a block copies the weight tile of its first task in the next GEMM phase
// while it waits at the barrier (waves 1-3 issue the copy after the block has arrived, wave 0
// waits), and after the barrier only the activation loads stand before its MFMAs.
//
// The row statistics need no clearing phase: the resstats epilogue writes (not adds) one partial
// per row and 64-column group.
//
// Activations written once per launch (x after each residual step, each layer's qkv and o, each
// in its own buffer: LayerArgs) are read through the caches; mid and the statistics are read
// device-coherent. Every output is stored device-coherent (written through to memory).
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <stdexcept>
#include <string>

#include "attn_tile.h"
#include "gemm_big.h"
#include "gemm_tile.h"
#include "layer.h"
#include "rowops.h"

namespace jh {

struct EncParams {
    const LayerDesc* layers;
    int first, count;
    const jh_half* x_in;
    jh_half *xa, *qa, *oa, *mid;
    size_t x_stride, q_stride, o_stride;
    float *stats_attn, *stats_mlp;
    const int32_t *pos, *seg;
    int m, d, inter, rope_rows;
    float eps;
    int bm[4], splits[4], kv[2];
    float* ws;
    uint32_t* counters;
    unsigned phases;  // bits 0-4
    int barriers;     // grid barriers in this launch
    int lds_main;     // dynamic LDS bytes before the block's split-K flag
    int att_gkeys[2];  // keys the attention tile stages at once: global, window layers
    uint32_t* bar;    // the barrier's words (BAR_WORDS, zero between launches)
    uint32_t bar_skew;  // 0; 1 (tests of the time-out path): every barrier waits one too many
    uint64_t* prof;   // null, or PROF_WORDS per block and layer: see stamp()
    // The whole model (model != 0): ModelArgs, and the head GEMMs' tile heights and splits
    // (in_proj, out_proj, linear1, linear2, the scorer's lin1).
    int model;
    ModelArgs M;
    int hbm[5], hsplits[5];
};

// Per-phase timestamps (the reference's kernels/src/prof.rs): thread 0 of each block writes the
// GPU-wide constant-rate clock (100 MHz) at each phase's start (after the barrier before it)
// into word 2p and at its end (after the block's last task, before the barrier after it) into
// word 2p + 1, and its CU id into word 10.
__device__ __forceinline__ void stamp(uint64_t* prof, int slot) {
    if (prof && threadIdx.x == 0) prof[slot] = wall_clock64();
}

__device__ __forceinline__ void stamp_end(uint64_t* prof, int phase) {
    if (prof) {
        __syncthreads();  // the whole block is done with the phase (profiling only)
        stamp(prof, 2 * phase + 1);
    }
}

// The grid barrier's words, each on its own 128-byte line: BAR_NG group arrival counters, the
// count of groups complete, the generation, and the time-out flag.
constexpr int BAR_LINE = 32;
constexpr int BAR_NG = 16;  // arrival groups (8 and 32 measured slower on 256 blocks)
static_assert(BAR_WORDS == (BAR_NG + 3) * BAR_LINE, "the barrier's words");
constexpr int BAR_GROUPS = BAR_NG * BAR_LINE, BAR_GEN = (BAR_NG + 1) * BAR_LINE,
              BAR_TIMEOUT = (BAR_NG + 2) * BAR_LINE;

// Barrier nb (1, 2, ... within the launch) across the grid (the reference's is
// kernels/src/gemm.rs:435-489). Blocks arrive in BAR_NG groups (block b in group b % BAR_NG),
// so no counter sees more than a sixteenth of the arrivals (atomics on one word are served one
// at a time: a single counter for 256 blocks made a 293-token forward pass 15% slower); the arrival that
// completes group x's count for barrier nb counts the group, the one that completes the groups'
// count advances the generation. The counters only grow within a launch (targets nb * size),
// so an arrival is two dependent atomics at most and nobody resets anything on the way; block 0
// zeroes the counters after the launch's last barrier, when no arrival is left. The generation
// keeps growing across launches: each block reads it once at its start (before it arrives
// anywhere, so before any barrier of this launch can complete) and waits for g0 + nb.
//
// The phase outputs are stored device-coherent and read back through the coherent path, so the
// release is only each wave waiting for its stores to complete, and no cache needs invalidating
// after the barrier. `during` runs on waves 1-3 after the block has arrived (wave 0 waits): work
// that does not depend on the other blocks, the next phase's weight copy. The wait is bounded:
// past ~0.2 s (far beyond any real barrier) it gives up and raises the time-out flag, which the
// host turns into an error, so a broken launch cannot hang the GPU.
template <class F>
__device__ __forceinline__ void grid_sync(uint32_t* bar, uint32_t g0, uint32_t nb, bool last,
                                          bool& timed_out, F&& during) {
    release_wait();
    __syncthreads();
    if (threadIdx.x < 64) {
        if (threadIdx.x == 0) {
            const uint32_t grid = gridDim.x, x = blockIdx.x % BAR_NG;
            const uint32_t groups = grid < BAR_NG ? grid : BAR_NG, in_group = (grid - x + BAR_NG - 1) / BAR_NG;
            if (atomic_add_agent(bar + x * BAR_LINE, 1u) == nb * in_group - 1)
                if (atomic_add_agent(bar + BAR_GROUPS, 1u) == nb * groups - 1)
                    atomic_add_agent(bar + BAR_GEN, 1u);
            const uint32_t target = g0 + nb;
            const uint64_t t0 = wall_clock64();
            for (uint32_t it = 1; !timed_out && (int)(atomic_load_agent(bar + BAR_GEN) - target) < 0; it++) {
                __builtin_amdgcn_s_sleep(1);
                if (wall_clock64() - t0 > 20000000ull) {
                    atomic_store_agent(bar + BAR_TIMEOUT, 1u);
                    timed_out = true;  // the launch is lost: the remaining barriers do not wait
                } else if ((it & 63) == 0 && atomic_load_agent(bar + BAR_TIMEOUT)) {
                    timed_out = true;  // another block gave up: stop waiting at once
                }
            }
            if (last && blockIdx.x == 0) {
                for (int i = 0; i <= BAR_NG; i++) atomic_store_agent(bar + i * BAR_LINE, 0u);
            }
        }
    } else {
        during();
    }
    __syncthreads();
}

// Layer l's activation buffers (LayerArgs): x in, after wo, after wo_mlp; qkv; o.
__device__ __forceinline__ const jh_half* x_in_of(const EncParams& P, int l) {
    return l == P.first ? P.x_in : P.xa + (size_t)(2 * l - 1) * P.x_stride;
}
__device__ __forceinline__ jh_half* x_attn_of(const EncParams& P, int l) {
    return P.xa + (size_t)(2 * l) * P.x_stride;
}
__device__ __forceinline__ jh_half* x_out_of(const EncParams& P, int l) {
    return P.xa + (size_t)(2 * l + 1) * P.x_stride;
}

__device__ __forceinline__ GemmParams make_gemm(const EncParams& P, int g, const LayerDesc& L,
                                                int l) {
    GemmParams p{};
    p.m = P.m, p.eps = P.eps, p.ws = P.ws, p.counters = P.counters;
    p.splits = P.splits[g];
    if (g == 0) {
        p.a = x_in_of(P, l), p.w = L.wqkv, p.c = P.qa + (size_t)l * P.q_stride;
        p.n = 3 * P.d, p.k = P.d;
        p.rope = L.rope, p.rope_cols = 2 * P.d, p.rope_rows = P.rope_rows, p.pos = P.pos;
        if (L.qkv_colsum) p.stats_in = P.stats_mlp, p.colsum = L.qkv_colsum;
    } else if (g == 1) {
        p.a = P.oa + (size_t)l * P.o_stride, p.w = L.wo, p.c = x_attn_of(P, l), p.res = x_in_of(P, l);
        p.n = P.d, p.k = P.d, p.stats_out = P.stats_attn;
    } else if (g == 2) {
        p.a = x_attn_of(P, l), p.w = L.wi, p.c = P.mid, p.n = 2 * P.inter, p.k = P.d;
        p.stats_in = P.stats_attn, p.colsum = L.wi_colsum;
    } else {
        p.a = P.mid, p.w = L.wo_mlp, p.c = x_out_of(P, l), p.res = x_attn_of(P, l);
        p.n = P.d, p.k = P.inter, p.stats_out = P.stats_mlp;
    }
    p.tiles_n = p.n / (P.bm[g] >= 128 ? P.bm[g] : 64);
    p.tiles_m = (P.m + P.bm[g] - 1) / P.bm[g];
    return p;
}

// Head GEMM g (in_proj, out_proj, linear1, linear2; 4: the scorer's lin1) of head layer h, on
// the head's buffers (ModelArgs): hx slot 2h in, 2h + 1 after out_proj, 2h + 2 after linear2.
__device__ __forceinline__ GemmParams make_head_gemm(const EncParams& P, int g, const HeadDesc& H,
                                                     int h) {
    const ModelArgs& M = P.M;
    auto hx = [&](int i) { return M.hxa + (size_t)i * P.x_stride; };
    GemmParams p{};
    p.m = P.m, p.ws = P.ws, p.counters = P.counters, p.eps = M.head_eps;
    p.splits = P.hsplits[g];
    if (g == 0) {
        p.a = hx(2 * h), p.w = H.in_proj, p.c = M.hqa + (size_t)h * P.q_stride;
        p.n = 3 * P.d, p.k = P.d;
        p.stats_in = P.stats_attn, p.colsum = H.in_proj_colsum, p.bias = H.in_proj_b;
    } else if (g == 1) {
        p.a = M.hoa + (size_t)h * P.o_stride, p.w = H.out_proj, p.c = hx(2 * h + 1), p.res = hx(2 * h);
        p.n = P.d, p.k = P.d, p.bias = H.out_proj_b, p.stats_out = P.stats_mlp;
    } else if (g == 2) {
        p.a = hx(2 * h + 1), p.w = H.linear1, p.c = P.mid, p.n = M.head_ff, p.k = P.d;
        p.stats_in = P.stats_mlp, p.colsum = H.linear1_colsum, p.bias = H.linear1_b;
    } else if (g == 3) {
        p.a = P.mid, p.w = H.linear2, p.c = hx(2 * h + 2), p.res = hx(2 * h + 1);
        p.n = P.d, p.k = M.head_ff, p.bias = H.linear2_b, p.stats_out = P.stats_attn;
    } else {
        p.a = hx(2 * M.head_layers), p.w = M.lin1, p.c = M.hs, p.n = P.d, p.k = P.d;
        p.stats_in = P.stats_attn, p.colsum = M.lin1_colsum, p.bias = M.lin1_b;
    }
    p.tiles_n = p.n / (P.hbm[g] >= 128 ? P.hbm[g] : 64);
    p.tiles_m = (P.m + P.hbm[g] - 1) / P.hbm[g];
    return p;
}

__device__ __forceinline__ int gemm_tasks(const GemmParams& g) {
    return g.tiles_n * g.tiles_m * g.splits;
}

// The kernel's instances: MODE_LAT takes every plan (256 threads, one block a CU); MODE_BIG128
// and MODE_BIG256 the large-batch plans of 128 x 128 tiles (256 threads, two blocks a CU) and of
// 256 x 256 tiles (512 threads, one block a CU), with only the throughput tiles and the streaming
// attention tile compiled in.
constexpr int MODE_LAT = 0, MODE_BIG128 = 1, MODE_BIG256 = 2;
// MODE_LAT48: MODE_LAT with the 48-row latency tile compiled in for qkv and wi, for the plans
// that take it (an instance of its own: the code it adds shifts the register and spill layout
// of the whole kernel, which the other plans measured slower with).
constexpr int MODE_LAT48 = 3;

// The 48-row latency tile is compiled for qkv and wi only, in MODE_LAT48 (the plans give it to
// no other GEMM).
template <int EPI, int MODE>
constexpr bool T48 = MODE == MODE_LAT48 && (EPI == EPI_K_ROPE || EPI == EPI_K_LNROPE || EPI == EPI_K_LNGEGLU);

// bm 16/32/48/64: the latency tile with its weights in LDS; 128 and 256: the throughput tiles
// (large batches), which stage both operands themselves.
template <int EPI, bool AX, int MODE>
__device__ __forceinline__ void gemm_phase(const GemmParams& g, int bm, char* lds, bool pre,
                                           uint32_t* s_last, uint64_t* sub) {
    const int T = gemm_tasks(g);
    for (int t = blockIdx.x; t < T; t += gridDim.x) {
        const bool first = t == (int)blockIdx.x;
        const bool ready = pre && first;
        uint64_t* su = first ? sub : nullptr;
        if (MODE == MODE_BIG256)
            gemm_big_tile<256, 256, EPI, AX, true>(g, t, lds, su);
        else if (MODE == MODE_BIG128 || bm == 128)
            gemm_big_tile<128, 128, EPI, AX, true>(g, t, lds, su);
        else if (bm == 16)
            gemm_w_tile<16, EPI, AX>(g, t, lds, ready, s_last, su);
        else if (bm == 32)
            gemm_w_tile<32, EPI, AX>(g, t, lds, ready, s_last, su);
        else if (T48<EPI, MODE> && bm == 48)
            gemm_w_tile<T48<EPI, MODE> ? 48 : 64, EPI, AX>(g, t, lds, ready, s_last, su);
        else
            gemm_w_tile<64, EPI, AX>(g, t, lds, ready, s_last, su);
    }
}

template <int MODE>
__global__ __launch_bounds__(MODE == MODE_BIG256 ? 512 : 256, MODE == MODE_BIG128 ? 2 : 1)
void encoder_kernel(EncParams P) {
    constexpr bool BIG = MODE == MODE_BIG128 || MODE == MODE_BIG256;
    extern __shared__ __attribute__((aligned(16))) char lds[];
    uint32_t* s_last = (uint32_t*)(lds + P.lds_main);
    uint32_t g0 = 0, nb = 0;
    bool timed_out = false;
    if (threadIdx.x == 0) g0 = atomic_load_agent(P.bar + BAR_GEN) + P.bar_skew;
    auto on = [&](int ph) { return ((P.phases >> ph) & 1u) != 0; };
    auto sync = [&](auto&& during) {
        nb++;
        grid_sync(P.bar, g0, nb, (int)nb == P.barriers, timed_out, during);
    };
    auto nothing = [] {};
    // The next GEMM phase's weight copy for this block's first task in it (if it has one): the
    // barrier's `during`, issued by waves 1-3.
    f16* const wl = (f16*)lds;
    auto fetch_first = [wl](const GemmParams& g) {
        return [&g, wl] { w_tile_fetch(g, w_tile_of(g, blockIdx.x), wl, 1); };
    };
    // A block fetches its first weight tile during the barrier (latency tiles only).
    auto prefetch = [&](const GemmParams& g, int bm) {
        return !BIG && bm < 128 && (int)blockIdx.x < gemm_tasks(g);
    };

    // An attention phase: the tasks of the tile the plan and the instance take (qkv in a buffer of
    // its own, read through the caches).
    auto attend = [&](const AttnParams& at, uint64_t* su0) {
        const int heads = P.d >> 6;
        if (!BIG && at.chunks == 1 && !att_use_stream(P.m, at.window)) {
            const int T = ((P.m + 15) >> 4) * heads, gkeys = P.att_gkeys[at.window > 0 ? 1 : 0];
            for (int t = blockIdx.x; t < T; t += gridDim.x)
                attention_slice_tile<false, true>(at, t, lds, gkeys, t == (int)blockIdx.x ? su0 : nullptr);
        } else if (BIG || at.chunks == 1) {  // (the large-batch instances have one key range)
            constexpr int NW = MODE == MODE_BIG256 ? 8 : 4;
            const int T = ((P.m + 16 * NW - 1) / (16 * NW)) * heads;
            for (int t = blockIdx.x; t < T; t += gridDim.x)
                attention_stream_tile<true, NW>(at, t, lds);
        } else {
            const int T = ((P.m + 63) >> 6) * heads * at.chunks;
            for (int t = blockIdx.x; t < T; t += gridDim.x) {
                const int tile = t / at.chunks;
                attention_tile<true>(at, tile / heads, tile % heads, t % at.chunks, (f16*)lds, s_last);
            }
        }
    };
    // A row phase: a wave a row (or marker), the grid's waves striding over them.
    const int lane = threadIdx.x & 63, nwv = blockDim.x >> 6;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    LayerDesc L = P.layers[P.first];
    GemmParams gq = make_gemm(P, 0, L, P.first);
    bool pre = false;  // the weight tile of this block's first task in the coming phase is fetched
    if (P.model) {  // embed, into the first layer's x_in
        for (int r = blockIdx.x * nwv + wv; r < P.m; r += gridDim.x * nwv)
            embed_row<4, true>(P.M.ids, r, (const f16*)P.M.tok_emb, P.M.vocab, P.d, P.M.emb_norm,
                               P.eps, (f16*)P.x_in, lane);
        pre = prefetch(gq, P.bm[0]);
        if (pre) sync(fetch_first(gq)); else sync(nothing);
    }
    for (int li = 0; li < P.count; li++) {
        uint64_t* prof = P.prof ? P.prof + ((size_t)blockIdx.x * P.count + li) * PROF_WORDS : nullptr;
        if (prof && threadIdx.x == 0) prof[10] = __smid();
        auto sub = [prof](int g) { return prof ? prof + 16 + 4 * g : nullptr; };
        const int l = P.first + li;
        const GemmParams go = make_gemm(P, 1, L, l), gi = make_gemm(P, 2, L, l),
                         gm = make_gemm(P, 3, L, l);
        if (on(0)) {
            stamp(prof, 0);
            if (gq.colsum)
                gemm_phase<EPI_K_LNROPE, false, MODE>(gq, P.bm[0], lds, pre, s_last, sub(0));
            else
                gemm_phase<EPI_K_ROPE, false, MODE>(gq, P.bm[0], lds, pre, s_last, sub(0));
            pre = false;
            stamp_end(prof, 0);
            if (on(1)) sync(nothing);
        }
        if (on(1)) {
            stamp(prof, 2);
            const int chunks = L.window > 0 ? P.kv[1] : P.kv[0];
            attend(AttnParams{P.qa + (size_t)l * P.q_stride, P.oa + (size_t)l * P.o_stride, P.m,
                              P.d, L.window, chunks, P.ws, P.counters, P.seg},
                   prof ? prof + 12 : nullptr);
            stamp_end(prof, 1);
            if (on(2)) {
                pre = prefetch(go, P.bm[1]);
                if (pre) sync(fetch_first(go)); else sync(nothing);
            }
        }
        if (on(2)) {
            stamp(prof, 4);
            gemm_phase<EPI_K_RESSTATS, false, MODE>(go, P.bm[1], lds, pre, s_last, sub(1));
            pre = false;
            stamp_end(prof, 2);
            if (on(3)) {
                pre = prefetch(gi, P.bm[2]);
                if (pre) sync(fetch_first(gi)); else sync(nothing);
            }
        }
        if (on(3)) {
            stamp(prof, 6);
            gemm_phase<EPI_K_LNGEGLU, false, MODE>(gi, P.bm[2], lds, pre, s_last, sub(2));
            pre = false;
            stamp_end(prof, 3);
            if (on(4)) {
                pre = prefetch(gm, P.bm[3]);
                if (pre) sync(fetch_first(gm)); else sync(nothing);
            }
        }
        if (on(4)) {
            stamp(prof, 8);
            gemm_phase<EPI_K_RESSTATS, true, MODE>(gm, P.bm[3], lds, pre, s_last, sub(3));
            pre = false;
            stamp_end(prof, 4);
        }
        if (li + 1 < P.count) {  // whole layers only (the host checks)
            L = P.layers[l + 1];
            gq = make_gemm(P, 0, L, l + 1);
            pre = prefetch(gq, P.bm[0]);
            if (pre) sync(fetch_first(gq)); else sync(nothing);
        }
    }
    if (!P.model) return;

    // ---- the head (src/forward.rs:504-717): norm_add, the head layers, lin1, the score ----
    const ModelArgs& M = P.M;
    sync(nothing);  // the last layer's residual stream is complete
    {
        const jh_half* xl = x_out_of(P, P.first + P.count - 1);
        for (int r = blockIdx.x * nwv + wv; r < P.m; r += gridDim.x * nwv)
            norm_add_row<4, true>((const f16*)xl, r, P.d, M.final_norm, M.type_add, M.row_type,
                                  P.eps, (f16*)M.hxa, P.stats_attn, lane);
    }
    for (int h = 0; h < M.head_layers; h++) {
        const HeadDesc H = M.heads[h];
        const GemmParams gi = make_head_gemm(P, 0, H, h), go = make_head_gemm(P, 1, H, h),
                         g1 = make_head_gemm(P, 2, H, h), g2 = make_head_gemm(P, 3, H, h);
        pre = prefetch(gi, P.hbm[0]);
        if (pre) sync(fetch_first(gi)); else sync(nothing);
        gemm_phase<EPI_K_LNBIAS, false, MODE>(gi, P.hbm[0], lds, pre, s_last, nullptr);
        sync(nothing);
        attend(AttnParams{M.hqa + (size_t)h * P.q_stride, M.hoa + (size_t)h * P.o_stride, P.m, P.d,
                          0, P.kv[0], P.ws, P.counters, P.seg},
               nullptr);
        pre = prefetch(go, P.hbm[1]);
        if (pre) sync(fetch_first(go)); else sync(nothing);
        gemm_phase<EPI_K_BIASRESSTATS, false, MODE>(go, P.hbm[1], lds, pre, s_last, nullptr);
        pre = prefetch(g1, P.hbm[2]);
        if (pre) sync(fetch_first(g1)); else sync(nothing);
        gemm_phase<EPI_K_LNBIASRELU, false, MODE>(g1, P.hbm[2], lds, pre, s_last, nullptr);
        pre = prefetch(g2, P.hbm[3]);
        if (pre) sync(fetch_first(g2)); else sync(nothing);
        gemm_phase<EPI_K_BIASRESSTATS, true, MODE>(g2, P.hbm[3], lds, pre, s_last, nullptr);
    }
    const GemmParams gs = make_head_gemm(P, 4, HeadDesc{}, 0);
    pre = prefetch(gs, P.hbm[4]);
    if (pre) sync(fetch_first(gs)); else sync(nothing);
    gemm_phase<EPI_K_LNBIASGELU, false, MODE>(gs, P.hbm[4], lds, pre, s_last, nullptr);
    sync(nothing);
    for (int i = blockIdx.x * nwv + wv; i < M.n_markers; i += gridDim.x * nwv)
        score_row<4>((const f16*)M.hs, P.m, P.d, (const f16*)M.lin2, M.lin2_b, M.markers, i,
                     M.logits, lane);
}

// ---------------------------------------------------------------------------------------------
// Host side.

std::string LayerPlan::str() const {
    static const char* names[4] = {"qkv", "wo", "wi", "wo_mlp"};
    std::string s;
    for (int g = 0; g < 4; g++)
        s += std::string(names[g]) + " " + std::to_string(bm[g]) + "/" + std::to_string(splits[g]) + " ";
    return s + "kv " + std::to_string(kv[0]) + "/" + std::to_string(kv[1]);
}

static void shapes(int d, int inter, int cols[4], int ks[4]) {
    cols[0] = 3 * d, ks[0] = d;
    cols[1] = d, ks[1] = d;
    cols[2] = 2 * inter, ks[2] = d;
    cols[3] = d, ks[3] = inter;
}

static int red_bytes(int bm) { return 4 * bm * 68 * 4; }

int LayerKernel::lds_bytes(const LayerPlan& plan, int d, int inter, int m, int window) {
    int cols[4], ks[4];
    shapes(d, inter, cols, ks);
    int b = std::max({ATT_LDS_F16 * 2, att_lds_bytes(attention_gkeys(m, 0)),
                      att_lds_bytes(attention_gkeys(m, window))});
    if (att_use_stream(m, 0) || att_use_stream(m, window)) b = std::max(b, ATT_STREAM_LDS);
    for (int g = 0; g < 4; g++)
        b = plan.bm[g] >= 128 ? std::max(b, Big<128, 128>::LDS_BYTES)
                              : std::max({b, w_tile_bytes(ks[g], plan.splits[g]), red_bytes(plan.bm[g])});
    return (b + 15) / 16 * 16;
}

// The large-batch instances' LDS: the throughput tile or the streaming attention tile.
static int big_lds_bytes(int bm) {
    const int g = bm == 256 ? Big<256, 256>::LDS_BYTES : Big<128, 128>::LDS_BYTES;
    return (std::max<int>(g, ATT_STREAM_LDS) + 15) / 16 * 16;
}

void LayerKernel::init(int cus, int lds_max) {
    cus_ = cus > 0 ? cus : 256;
    const char* coop = getenv("JULIA_HIP_COOPERATIVE");
    coop_ = !(coop && strcmp(coop, "0") == 0);
    const char* skew = getenv("JULIA_HIP_TEST_BARRIER_SKEW");
    skew_ = skew && strcmp(skew, "1") == 0 ? 1u : 0u;
    lds_max_ = lds_max - 16;  // the split-K flag after the main area
    per_cu_ = per_cu_big_ = per_cu_big256_ = 0;
    auto occupancy = [](const void* k, int threads, int lds) {
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) {
            (void)hipGetLastError();
            return 0;
        }
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, threads, lds) != hipSuccess) n = 0;
        return n;
    };
    // with the largest LDS a plan may use: one block per CU
    per_cu_ = occupancy(reinterpret_cast<const void*>(encoder_kernel<MODE_LAT>), 256, lds_max);
    lat48_ok_ = per_cu_ > 0 &&
                occupancy(reinterpret_cast<const void*>(encoder_kernel<MODE_LAT48>), 256, lds_max) >= per_cu_;
    per_cu_big_ = occupancy(reinterpret_cast<const void*>(encoder_kernel<MODE_BIG128>), 256,
                            big_lds_bytes(128) + 16);
    per_cu_big256_ = occupancy(reinterpret_cast<const void*>(encoder_kernel<MODE_BIG256>), 512,
                               big_lds_bytes(256) + 16);
}

// Per GEMM the tile height and split-K with the least modelled time on a grid of one block per
// CU: a task waits for its activation tile (about 67 KB per us into one CU), its MFMAs, the
// cross-wave reduction and the epilogue; tasks run in rounds over the grid; the first round's
// weight tile is fetched during the barrier, later rounds fetch their own; a split costs a
// partial exchange. The weight tile must fit the LDS. Key ranges for global attention as the
// per-step attention's, none for sliding-window layers (src/forward.rs:173-189's rule).
// The latency tile's height and split-K for an m x cols x k GEMM (the cost model above).
static void lat_tile(int m, int cols, int k, int cus, int lds_max, int& bm_out, int& splits_out,
                     bool allow48 = false) {
    const double bw = 67e3;  // bytes per us into one CU
    double best = 1e30;
    bm_out = 16, splits_out = k / 32 >= 8 ? 2 : 1;
    for (int bm : {16, 32, 48, 64}) {
        if (bm == 48 && !allow48) continue;
        for (int s = 1; s <= 4; s++) {
            if (k / 32 < 4 * s) continue;  // every wave needs a K unit
            if (w_tile_bytes(k, s) > lds_max) continue;
            const long tasks = (long)(cols / 64) * ((m + bm - 1) / bm) * s;
            const long rounds = (tasks + cus - 1) / cus;
            const double a_us = (double)bm * (k / s) * 2 / bw;
            const double w_us = (double)w_tile_bytes(k, s) / bw;
            const double mma_us = (bm / 16) * (k / s / 32 / 4.0) * 4 * 16 / 2400.0;
            const double task = 1.2 + a_us + mma_us + 0.1 * (bm / 16) + 0.4;
            const double cost = rounds * task + (rounds - 1) * w_us + (s > 1 ? 1.5 : 0.0);
            if (cost < best - 1e-9) best = cost, bm_out = bm, splits_out = s;
        }
    }
}

// The head GEMMs' shapes (in_proj, out_proj, linear1, linear2, the scorer's lin1) and whether
// each has a LayerNorm epilogue.
static void head_shapes(int d, int ff, int cols[5], int ks[5], bool ln[5]) {
    const int c[5] = {3 * d, d, ff, d, d}, k[5] = {d, d, d, ff, d};
    const bool l[5] = {true, false, true, false, true};
    for (int g = 0; g < 5; g++) cols[g] = c[g], ks[g] = k[g], ln[g] = l[g];
}

// The head GEMMs' tiles under `plan` on m rows: the throughput instances' tile (every head GEMM
// must take it: false if one does not), else the latency tile's cost model.
static bool head_plan(const LayerPlan& plan, int m, int d, int ff, int cus, int lds_max,
                      int bm[5], int splits[5]) {
    int cols[5], ks[5];
    bool ln[5];
    head_shapes(d, ff, cols, ks, ln);
    const int mode = LayerKernel::big_mode(plan, m);
    for (int g = 0; g < 5; g++) {
        if (mode != MODE_LAT) {
            const int t = mode == MODE_BIG256 ? 256 : 128;
            if (cols[g] % t || ks[g] % 64 || (ln[g] && ks[g] > 128 * BIG_LN_SLOTS)) return false;
            bm[g] = t, splits[g] = 1;
        } else {
            lat_tile(m, cols[g], ks[g], cus, lds_max, bm[g], splits[g]);
            if (w_tile_bytes(ks[g], splits[g]) > lds_max) return false;
        }
    }
    return true;
}

bool LayerKernel::model_fits(const LayerPlan& plan, int m, int d, int head_ff) const {
    int bm[5], splits[5];
    return d <= 1024 && head_plan(plan, m, d, head_ff, cus_, lds_max_, bm, splits);
}

LayerPlan LayerKernel::default_plan(int m, int d, int inter) const {
    LayerPlan p{};
    int cols[4], ks[4];
    shapes(d, inter, cols, ks);
    for (int g = 0; g < 4; g++) {
        // Large batches: the throughput tile (LayerNorm epilogues, qkv and wi, need K <= 1024),
        // 256 x 256 where every GEMM's columns allow it (big_tiles below), else 128 x 128.
        const bool ln = g == 0 || g == 2;
        if (m > ATT_SLICE_ROWS && cols[g] % 128 == 0 && ks[g] % 64 == 0 &&
            (!ln || ks[g] <= 128 * BIG_LN_SLOTS) && Big<128, 128>::LDS_BYTES <= lds_max_) {
            p.bm[g] = 128, p.splits[g] = 1;
            continue;
        }
        lat_tile(m, cols[g], ks[g], cus_, lds_max_, p.bm[g], p.splits[g], lat48_ok_ && (g == 0 || g == 2));
    }
    p.kv[0] = attention_chunks(m, d, 0, cus_);
    p.kv[1] = 1;
    // All four on 256 x 256 tiles (one 512-thread block a CU) when they all take them.
    bool all256 = per_cu_big256_ > 0 && big_lds_bytes(256) <= lds_max_;
    for (int g = 0; g < 4; g++) all256 = all256 && p.bm[g] == 128 && cols[g] % 256 == 0;
    if (all256)
        for (int g = 0; g < 4; g++) p.bm[g] = 256;
    return p;
}

size_t LayerKernel::ws_floats(int max_m, int d, int inter, int head_ff) const {
    size_t ws = 0;
    int cols[4], ks[4], hc[5], hk[5];
    bool hl[5];
    shapes(d, inter, cols, ks);
    if (head_ff > 0) head_shapes(d, head_ff, hc, hk, hl);
    for (int m = 1; m <= max_m; m++) {
        const LayerPlan p = default_plan(m, d, inter);
        for (int g = 0; g < 4; g++)
            ws = std::max(ws, gemm_ws_floats(m, cols[g], GemmConfig{p.bm[g], p.splits[g]}));
        ws = std::max(ws, attention_ws_floats(m, d, p.kv[0]));
        int hbm[5], hsp[5];
        if (head_ff > 0 && head_plan(p, m, d, head_ff, cus_, lds_max_, hbm, hsp))
            for (int g = 0; g < 5; g++)
                ws = std::max(ws, gemm_ws_floats(m, hc[g], GemmConfig{hbm[g], hsp[g]}));
    }
    return ws;
}

size_t LayerKernel::counters(int max_m, int d, int inter, int head_ff) const {
    size_t c = attention_counters(max_m, d);
    int cols[4], ks[4], hc[5], hk[5];
    bool hl[5];
    shapes(d, inter, cols, ks);
    for (int g = 0; g < 4; g++) c = std::max(c, gemm_counters(max_m, cols[g], GemmConfig{16, 2}));
    if (head_ff > 0) {
        head_shapes(d, head_ff, hc, hk, hl);
        for (int g = 0; g < 5; g++) c = std::max(c, gemm_counters(max_m, hc[g], GemmConfig{16, 2}));
    }
    return c;
}

int LayerKernel::grid(const LayerArgs& a, const LayerPlan& plan) const {
    int cols[4], ks[4];
    shapes(a.d, a.inter, cols, ks);
    long most = (long)((a.m + 15) / 16) * (a.d / 64);  // attention slices
    most = std::max(most, (long)((a.m + 63) / 64) * (a.d / 64) * std::max(plan.kv[0], plan.kv[1]));
    for (int g = 0; g < 4; g++)
        most = std::max(most, (long)(cols[g] / (plan.bm[g] >= 128 ? plan.bm[g] : 64)) *
                                  ((a.m + plan.bm[g] - 1) / plan.bm[g]) * plan.splits[g]);
    // Enough blocks for the largest phase's tasks in one round if they fit (a multiple of 8, so
    // that the task-to-XCD map is even), else every resident block.
    const int mode = big_mode(plan, a.m);
    const int per_cu = mode == MODE_BIG256 ? per_cu_big256_ : mode == MODE_BIG128 ? per_cu_big_ : per_cu_;
    const long grid = std::min<long>((long)per_cu * cus_, (most + 7) / 8 * 8);
    return (int)std::max<long>(grid, 1);
}

bool LayerKernel::launch(const LayerArgs& a, const LayerPlan& plan, const Scratch& s,
                         hipStream_t stream, unsigned phases, uint64_t* prof) {
    auto fail = [&](const std::string& m) { throw std::runtime_error("layer: " + m); };
    if (per_cu_ <= 0) fail("the encoder kernel does not fit on a CU");
    if (!bar_) fail("no grid-barrier counter");
    if (!a.layers || !a.host_layers || a.count < 1) fail("no layers");
    if (phases == 0 || phases > 0x1f) fail("no phases selected");
    if (phases != 0x1f && a.count != 1) fail("a subset of the phases runs one layer only");
    for (int g = 0; g < 4; g++)
        if (!(plan.bm[g] == 16 || plan.bm[g] == 32 || (plan.bm[g] == 48 && lat48_ok_ && (g == 0 || g == 2)) ||
              plan.bm[g] == 64 || plan.bm[g] == 128 || plan.bm[g] == 256) ||
            plan.splits[g] < 1 || plan.splits[g] > 4 || (plan.bm[g] >= 128 && plan.splits[g] != 1))
            fail("no such plan: " + plan.str());
    if (plan.kv[0] < 1 || plan.kv[0] > 8 || plan.kv[1] < 1 || plan.kv[1] > 8)
        fail("no such plan: " + plan.str());
    if (a.seg && (plan.kv[0] != 1 || plan.kv[1] != 1))
        fail("concatenated sequences take one key range: " + plan.str());
    if ((a.pos == nullptr) != (a.seg == nullptr)) fail("positions go with sequence bounds");
    int window = 0;
    for (int li = 0; li < a.count; li++) window = std::max(window, a.host_layers[a.first + li].window);
    const int mode = big_mode(plan, a.m);
    bool any256 = false;
    for (int g = 0; g < 4; g++) any256 = any256 || plan.bm[g] == 256;
    if (any256 && mode != MODE_BIG256)
        fail("256 x 256 tiles take every GEMM, more than " + std::to_string(ATT_SLICE_ROWS) +
             " rows and one key range: " + plan.str());
    if ((mode == MODE_BIG128 && per_cu_big_ <= 0) || (mode == MODE_BIG256 && per_cu_big256_ <= 0))
        fail("the encoder kernel's large-batch instance does not fit on a CU");
    int lds = mode == MODE_BIG256   ? big_lds_bytes(256)
                    : mode == MODE_BIG128 ? big_lds_bytes(128)
                                          : lds_bytes(plan, a.d, a.inter, a.m, window);
    if (lds > lds_max_) fail("the plan's weight tiles do not fit the LDS: " + plan.str());

    // Every layer's GEMMs pass the per-step launcher's checks (the kernel builds the same ones).
    int cols[4], ks[4];
    shapes(a.d, a.inter, cols, ks);
    if (!a.x_in || !a.xa || !a.qa || !a.oa || !a.mid || ((uintptr_t)a.x_in % 16) ||
        a.x_stride < (size_t)a.m * a.d || a.q_stride < (size_t)a.m * 3 * a.d ||
        a.o_stride < (size_t)a.m * a.d || a.x_stride % 64 || a.q_stride % 64 || a.o_stride % 64)
        fail("bad activation buffers");
    for (int li = 0; li < a.count; li++) {
        const int l = a.first + li;
        const LayerDesc& L = a.host_layers[l];
        jh_half* x_in = l == a.first ? const_cast<jh_half*>(a.x_in) : a.xa + (2 * l - 1) * a.x_stride;
        jh_half* x_attn = a.xa + 2 * l * a.x_stride;
        jh_half* x_out = a.xa + (2 * l + 1) * a.x_stride;
        jh_half* qkv = a.qa + l * a.q_stride;
        jh_half* o = a.oa + l * a.o_stride;
        if (x_out == a.x_in || x_attn == a.x_in) fail("x_in is one of the launch's own buffers");
        Gemm g[4] = {};
        const bool ln0 = L.qkv_colsum != nullptr;
        g[0].epi = ln0 ? EPI_K_LNROPE : EPI_K_ROPE, g[0].a = x_in, g[0].w = L.wqkv, g[0].c = qkv;
        g[0].rope = L.rope, g[0].rope_rows = a.rope_rows, g[0].pos = a.pos;
        if (ln0) g[0].stats_in = a.stats_mlp, g[0].colsum = L.qkv_colsum;
        g[1].epi = EPI_K_RESSTATS, g[1].a = o, g[1].w = L.wo, g[1].c = x_attn, g[1].stats_out = a.stats_attn;
        g[2].epi = EPI_K_LNGEGLU, g[2].a = x_attn, g[2].w = L.wi, g[2].c = a.mid;
        g[2].stats_in = a.stats_attn, g[2].colsum = L.wi_colsum;
        g[3].epi = EPI_K_RESSTATS, g[3].a = a.mid, g[3].w = L.wo_mlp, g[3].c = x_out, g[3].stats_out = a.stats_mlp;
        for (int i = 0; i < 4; i++) {
            g[i].m = a.m, g[i].n = cols[i], g[i].k = ks[i], g[i].eps = a.eps;
            gemm_check(g[i], GemmConfig{plan.bm[i], plan.splits[i]}, s);
        }
        const int kv = L.window > 0 ? plan.kv[1] : plan.kv[0];
        if (kv > 1 && (attention_ws_floats(a.m, a.d, kv) > s.ws_floats ||
                       attention_counters(a.m, a.d) > s.n_counters))
            fail("the key-range scratch is too small for " + std::to_string(a.m) + " tokens");
    }

    // The whole model: embed before layer 0, the head after the last layer.
    int hbm[5] = {}, hsplits[5] = {};
    int lds_model = lds;
    const ModelArgs* M = a.model;
    if (M) {
        auto al16 = [](const void* q) { return ((uintptr_t)q % 16) == 0; };
        if (a.first != 0 || phases != 0x1f) fail("the whole model runs every phase from layer 0");
        if (a.d > 1024) fail("the whole model takes d up to 1024");
        if (!M->ids || !M->tok_emb || !M->emb_norm || M->vocab <= 0 || !M->final_norm ||
            !M->type_add || !M->hxa || !M->hs || !M->lin1 || !M->lin1_colsum || !M->lin1_b ||
            !M->lin2 || M->head_layers < 0 || M->head_ff <= 0 || M->n_markers < 0 ||
            (M->head_layers > 0 && (!M->heads || !M->host_heads || !M->hqa || !M->hoa)) ||
            (M->n_markers > 0 && (!M->markers || !M->logits)))
            fail("bad model arguments");
        if (!al16(M->tok_emb) || !al16(M->emb_norm) || !al16(M->final_norm) || !al16(M->type_add) ||
            !al16(M->hxa) || !al16(M->hs) || !al16(M->lin2))
            fail("the model's tables and buffers must be 16-byte aligned");
        if (!head_plan(plan, a.m, a.d, M->head_ff, cus_, lds_max_, hbm, hsplits))
            fail("the head's GEMMs do not take the plan's tiles: " + plan.str());
        int hc[5], hk[5];
        bool hl[5];
        head_shapes(a.d, M->head_ff, hc, hk, hl);
        auto hx = [&](int i) { return M->hxa + (size_t)i * a.x_stride; };
        auto check = [&](int g, int epi, const jh_half* in, const jh_half* w, jh_half* out,
                         const float* st_in, const float* colsum, const float* bias, float* st_out) {
            Gemm q{};
            q.epi = epi, q.a = in, q.w = w, q.c = out, q.m = a.m, q.n = hc[g], q.k = hk[g];
            q.stats_in = st_in, q.colsum = colsum, q.bias = bias, q.stats_out = st_out;
            q.eps = M->head_eps;
            gemm_check(q, GemmConfig{hbm[g], hsplits[g]}, s);
            if (mode == MODE_LAT)
                lds_model = std::max({lds_model, w_tile_bytes(hk[g], hsplits[g]), red_bytes(hbm[g])});
        };
        for (int h = 0; h < M->head_layers; h++) {
            const HeadDesc& H = M->host_heads[h];
            jh_half* hq = M->hqa + (size_t)h * a.q_stride;
            jh_half* ho = M->hoa + (size_t)h * a.o_stride;
            check(0, EPI_K_LNBIAS, hx(2 * h), H.in_proj, hq, a.stats_attn, H.in_proj_colsum,
                  H.in_proj_b, nullptr);
            check(1, EPI_K_BIASRESSTATS, ho, H.out_proj, hx(2 * h + 1), nullptr, nullptr,
                  H.out_proj_b, a.stats_mlp);
            check(2, EPI_K_LNBIASRELU, hx(2 * h + 1), H.linear1, a.mid, a.stats_mlp,
                  H.linear1_colsum, H.linear1_b, nullptr);
            check(3, EPI_K_BIASRESSTATS, a.mid, H.linear2, hx(2 * h + 2), nullptr, nullptr,
                  H.linear2_b, a.stats_attn);
        }
        check(4, EPI_K_LNBIASGELU, hx(2 * M->head_layers), M->lin1, M->hs, a.stats_attn,
              M->lin1_colsum, M->lin1_b, nullptr);
        lds_model = (lds_model + 15) / 16 * 16;
        if (lds_model > lds_max_) fail("the head's weight tiles do not fit the LDS");
    }

    EncParams P{};
    P.layers = a.layers, P.first = a.first, P.count = a.count;
    P.x_in = a.x_in, P.xa = a.xa, P.qa = a.qa, P.oa = a.oa, P.mid = a.mid;
    P.x_stride = a.x_stride, P.q_stride = a.q_stride, P.o_stride = a.o_stride;
    P.stats_attn = a.stats_attn, P.stats_mlp = a.stats_mlp;
    P.pos = a.pos, P.seg = a.seg;
    P.m = a.m, P.d = a.d, P.inter = a.inter, P.rope_rows = a.rope_rows, P.eps = a.eps;
    for (int g = 0; g < 4; g++) P.bm[g] = plan.bm[g], P.splits[g] = plan.splits[g];
    P.kv[0] = plan.kv[0], P.kv[1] = plan.kv[1];
    P.ws = s.ws, P.counters = s.counters;
    P.phases = phases;
    int barriers = 0;  // between two consecutive selected phases, and between layers
    for (int ph = 1; ph < 5; ph++)
        if (((phases >> ph) & 1) && ((phases >> (ph - 1)) & 1)) barriers++;
    P.barriers = barriers * a.count + (a.count - 1);
    if (M) {  // after embed, after the last layer, five a head layer, before lin1 and the score
        P.model = 1, P.M = *M;
        for (int g = 0; g < 5; g++) P.hbm[g] = hbm[g], P.hsplits[g] = hsplits[g];
        P.barriers += 4 + 5 * M->head_layers;
        lds = lds_model;
    }
    P.lds_main = lds;
    P.att_gkeys[0] = attention_gkeys(a.m, 0);
    P.att_gkeys[1] = attention_gkeys(a.m, window);
    P.bar = bar_;
    P.bar_skew = skew_;
    P.prof = prof;

    const int grid_blocks = grid(a, plan);
    const bool uses48 = mode == MODE_LAT && (plan.bm[0] == 48 || plan.bm[2] == 48);
    void* args[] = {&P};
    const void* kernel = mode == MODE_BIG256   ? reinterpret_cast<const void*>(encoder_kernel<MODE_BIG256>)
                         : mode == MODE_BIG128 ? reinterpret_cast<const void*>(encoder_kernel<MODE_BIG128>)
                         : uses48 ? reinterpret_cast<const void*>(encoder_kernel<MODE_LAT48>)
                                               : reinterpret_cast<const void*>(encoder_kernel<MODE_LAT>);
    const dim3 threads(mode == MODE_BIG256 ? 512 : 256);
    hipError_t e;
    if (coop_) {
        e = hipLaunchCooperativeKernel(kernel, dim3(grid_blocks), threads, args, lds + 16, stream);
        if (e == hipErrorIllegalState) {
            // Another process holds the cooperative-launch resource: nothing was launched, and
            // the caller runs this pass on the per-step kernels. The next pass tries again.
            (void)hipGetLastError();
            refused_++;
            return false;
        }
    } else {
        // JULIA_HIP_COOPERATIVE=0: plain launches of the same grid (at most the blocks resident
        // at once, as the occupancy query sized it; a grid that is not co-resident ends in the
        // barrier's bounded wait, which the host reports as an error, instead of hanging).
        e = hipLaunchKernel(kernel, dim3(grid_blocks), threads, args, lds + 16, stream);
    }
    if (e != hipSuccess) fail(std::string(hipGetErrorString(e)) + " (" + plan.str() + ", grid " +
                              std::to_string(grid_blocks) + ")");
    return true;
}

bool LayerKernel::is_big(const LayerPlan& plan, int m) { return big_mode(plan, m) != MODE_LAT; }

// The instance a plan runs on: the large-batch ones take plans of throughput tiles only, all of
// one size, over more than ATT_SLICE_ROWS rows with one key range.
int LayerKernel::big_mode(const LayerPlan& plan, int m) {
    if (m <= ATT_SLICE_ROWS || plan.kv[0] != 1 || plan.kv[1] != 1) return MODE_LAT;
    for (int g = 1; g < 4; g++)
        if (plan.bm[g] != plan.bm[0]) return MODE_LAT;
    return plan.bm[0] == 256 ? MODE_BIG256 : plan.bm[0] == 128 ? MODE_BIG128 : MODE_LAT;
}

bool LayerKernel::barrier_timed_out() {
    if (!bar_) return false;
    uint32_t flag = 0;
    if (hipMemcpy(&flag, bar_ + BAR_TIMEOUT, 4, hipMemcpyDeviceToHost) != hipSuccess) return true;
    if (flag && hipMemset(bar_, 0, BAR_WORDS * 4) != hipSuccess)  // its counts are stale
        return true;
    return flag != 0;
}

}  // namespace jh
