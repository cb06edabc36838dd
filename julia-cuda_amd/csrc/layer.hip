// The persistent layer kernel (the reference's `layer`, kernels/src/main.rs:578-842): one
// encoder layer as one cooperative launch. Its five steps are phases (qkv, attention, wo, wi,
// wo_mlp); every block strides over a phase's tasks (the per-step kernels' own tile functions,
// so the arithmetic is theirs), with a grid barrier between two selected phases. The grid is at
// most the number of blocks resident at once (the cooperative launch checks it), a multiple of
// 8 so that task t runs on XCD t % 8 as in the per-step kernels.
//
// The row statistics need no clearing phase here: the resstats epilogue writes (not adds) one
// partial per row and 64-column group.
#include <algorithm>
#include <stdexcept>
#include <string>

#include "attn_tile.h"
#include "gemm_tile.h"
#include "layer.h"

namespace jh {

struct LayerParams {
    GemmParams g[4];  // qkv, wo, wi, wo_mlp
    AttnParams at;
    int bm[4];
    int epi0;         // EPI_K_ROPE (layer 0) or EPI_K_LNROPE
    unsigned phases;  // bits 0-4
    uint32_t* bar;    // the barrier's words (BAR_WORDS, zero between launches)
    uint64_t* prof;   // null, or PROF_WORDS per block: see stamp()
};

// Per-phase timestamps (the reference's kernels/src/prof.rs): thread 0 of each block writes the
// GPU-wide constant-rate clock (100 MHz) at each phase's start (after the barrier before it)
// into word 2p and at its end (after the block's last task, before the barrier after it) into
// word 2p + 1, and its CU id into word 10.
__device__ __forceinline__ void stamp(uint64_t* prof, int slot) {
    if (prof && threadIdx.x == 0) prof[(size_t)blockIdx.x * PROF_WORDS + slot] = wall_clock64();
}

__device__ __forceinline__ void stamp_end(uint64_t* prof, int phase) {
    if (prof) {
        __syncthreads();  // the whole block is done with the phase (profiling only)
        stamp(prof, 2 * phase + 1);
    }
}

// The grid barrier's words, each on its own 128-byte line: eight group arrival counters, the
// count of groups complete, the generation, and the time-out flag.
constexpr int BAR_LINE = 32;
constexpr int BAR_GROUPS = 8 * BAR_LINE, BAR_GEN = 9 * BAR_LINE, BAR_TIMEOUT = 10 * BAR_LINE;

// A barrier across the grid (the reference's is kernels/src/gemm.rs:435-489): blocks arrive in
// eight groups (block b in group b % 8, which is the XCD it is dispatched to), so no counter sees
// more than an eighth of the arrivals; the last arrival of a group counts the group, the last
// group advances the generation that every block waits on, and each counter is reset by its
// last arrival, so the words are zero again at the end of every barrier.
//
// The phase outputs are stored device-coherent and read back through the coherent path (XG), so
// the release is only each wave waiting for its stores to complete, and no cache needs
// invalidating after the barrier (the weights other blocks share through L2 stay cached). The
// wait is bounded: past ~0.2 s (far beyond any real barrier) it gives up and raises the time-out
// flag, which the host turns into an error, so a broken launch cannot hang the GPU.
__device__ __forceinline__ void grid_sync(uint32_t* bar) {
    release_wait();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t grid = gridDim.x, x = blockIdx.x & 7;
        const uint32_t groups = grid < 8 ? grid : 8, in_group = (grid - x + 7) / 8;
        uint32_t* gen = bar + BAR_GEN;
        const uint32_t g0 = atomic_load_agent(gen);  // before arriving: it cannot move yet
        release_wait();
        if (atomic_add_agent(bar + x * BAR_LINE, 1u) == in_group - 1) {
            atomic_store_agent(bar + x * BAR_LINE, 0u);
            if (atomic_add_agent(bar + BAR_GROUPS, 1u) == groups - 1) {
                atomic_store_agent(bar + BAR_GROUPS, 0u);
                release_wait();  // the resets land before anyone can pass
                atomic_add_agent(gen, 1u);
            }
        }
        const uint64_t t0 = wall_clock64();
        while (atomic_load_agent(gen) == g0) {
            __builtin_amdgcn_s_sleep(1);
            if (wall_clock64() - t0 > 20000000ull) {
                atomic_store_agent(bar + BAR_TIMEOUT, 1u);
                break;
            }
        }
    }
    __syncthreads();
}

constexpr int LAYER_LDS_FLOATS = lat_lds_floats<32>();
static_assert(ATT_LDS_F16 / 2 <= LAYER_LDS_FLOATS, "attention tiles fit the GEMM's LDS");

template <int EPI>
__device__ __forceinline__ void gemm_phase(const GemmParams& g, int bm, float* lds,
                                           uint32_t* s_last) {
    const int T = g.tiles_n * g.tiles_m * g.splits;
    for (int t = blockIdx.x; t < T; t += gridDim.x) {
        if (bm == 16)
            gemm_lat_tile<16, EPI, true>(g, t, lds, s_last);
        else
            gemm_lat_tile<32, EPI, true>(g, t, lds, s_last);
    }
}

__global__ __launch_bounds__(256) void layer_kernel(LayerParams P) {
    __shared__ __attribute__((aligned(16))) float lds[LAYER_LDS_FLOATS];
    __shared__ uint32_t s_last;
    auto on = [&](int ph) { return (P.phases >> ph) & 1u; };
    auto sync_if = [&](int next) {
        if (on(next)) grid_sync(P.bar);
    };
    if (P.prof && threadIdx.x == 0) P.prof[(size_t)blockIdx.x * PROF_WORDS + 10] = __smid();
    if (on(0)) {
        stamp(P.prof, 0);
        if (P.epi0 == EPI_K_LNROPE)
            gemm_phase<EPI_K_LNROPE>(P.g[0], P.bm[0], lds, &s_last);
        else
            gemm_phase<EPI_K_ROPE>(P.g[0], P.bm[0], lds, &s_last);
        stamp_end(P.prof, 0);
        sync_if(1);
    }
    if (on(1)) {
        stamp(P.prof, 2);
        const AttnParams& a = P.at;
        const int heads = a.d >> 6, T = ((a.n + 63) >> 6) * heads * a.chunks;
        for (int t = blockIdx.x; t < T; t += gridDim.x) {
            const int tile = t / a.chunks;
            attention_tile<true>(a, tile / heads, tile % heads, t % a.chunks, (f16*)lds, &s_last);
        }
        stamp_end(P.prof, 1);
        sync_if(2);
    }
    if (on(2)) {
        stamp(P.prof, 4);
        gemm_phase<EPI_K_RESSTATS>(P.g[1], P.bm[1], lds, &s_last);
        stamp_end(P.prof, 2);
        sync_if(3);
    }
    if (on(3)) {
        stamp(P.prof, 6);
        gemm_phase<EPI_K_LNGEGLU>(P.g[2], P.bm[2], lds, &s_last);
        stamp_end(P.prof, 3);
        sync_if(4);
    }
    if (on(4)) {
        stamp(P.prof, 8);
        gemm_phase<EPI_K_RESSTATS>(P.g[3], P.bm[3], lds, &s_last);
        stamp_end(P.prof, 4);
    }
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

void LayerKernel::init(int cus) {
    cus_ = cus > 0 ? cus : 256;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(layer_kernel),
                                                     256, 0) != hipSuccess)
        n = 0;
    per_cu_ = n;
}

static void shapes(int d, int inter, int cols[4], int ks[4]) {
    cols[0] = 3 * d, ks[0] = d;
    cols[1] = d, ks[1] = d;
    cols[2] = 2 * inter, ks[2] = d;
    cols[3] = d, ks[3] = inter;
}

// Per GEMM the latency chooser's pick, limited to the layer kernel's tile heights (16 and 32
// rows, which keep the kernel's LDS at 34.8 KB); key ranges for global attention as the
// per-step attention's, none for sliding-window layers (src/forward.rs:173-189's rule).
LayerPlan LayerKernel::default_plan(int m, int d, int inter, int window) const {
    LayerPlan p{};
    int cols[4], ks[4];
    shapes(d, inter, cols, ks);
    for (int g = 0; g < 4; g++) {
        GemmConfig c = gemm_choose(std::min(m, 1024), cols[g], ks[g], cus_);
        if (c.bm > 32) c = GemmConfig{32, c.bm >= 128 ? 1 : c.splits};
        p.bm[g] = c.bm, p.splits[g] = c.splits;
    }
    p.kv[0] = attention_chunks(m, d, 0, cus_);
    p.kv[1] = 1;
    (void)window;
    return p;
}

size_t LayerKernel::ws_floats(int max_m, int d, int inter) const {
    size_t ws = 0;
    int cols[4], ks[4];
    shapes(d, inter, cols, ks);
    for (int m = 1; m <= max_m; m++) {
        const LayerPlan p = default_plan(m, d, inter, 0);
        for (int g = 0; g < 4; g++)
            ws = std::max(ws, gemm_ws_floats(m, cols[g], GemmConfig{p.bm[g], p.splits[g]}));
        ws = std::max(ws, attention_ws_floats(m, d, p.kv[0]));
    }
    return ws;
}

size_t LayerKernel::counters(int max_m, int d, int inter) const {
    size_t c = attention_counters(max_m, d);
    int cols[4], ks[4];
    shapes(d, inter, cols, ks);
    for (int g = 0; g < 4; g++) c = std::max(c, gemm_counters(max_m, cols[g], GemmConfig{16, 2}));
    return c;
}

static void fill(GemmParams& p, const Gemm& g, GemmConfig c, const Scratch& s) {
    p = GemmParams{};
    p.a = g.a, p.w = g.w, p.c = g.c, p.stats_in = g.stats_in, p.colsum = g.colsum;
    p.bias = g.bias, p.rope = g.rope, p.pos = g.pos, p.stats_out = g.stats_out;
    p.ws = s.ws, p.counters = s.counters;
    p.m = g.m, p.n = g.n, p.k = g.k, p.eps = g.eps;
    p.rope_cols = (g.epi & EPI_ROPE) ? 2 * (g.n / 3) : 0;
    p.rope_rows = g.rope_rows;
    p.splits = c.splits, p.tiles_n = g.n / 64, p.tiles_m = (g.m + c.bm - 1) / c.bm;
}

int LayerKernel::grid(const LayerArgs& a, const LayerPlan& plan) const {
    int cols[4], ks[4];
    shapes(a.d, a.inter, cols, ks);
    long most = (long)((a.m + 63) / 64) * (a.d / 64) * plan.kv[a.window > 0 ? 1 : 0];
    for (int g = 0; g < 4; g++)
        most = std::max(most, (long)(cols[g] / 64) * ((a.m + plan.bm[g] - 1) / plan.bm[g]) * plan.splits[g]);
    long grid = std::min<long>((long)per_cu_ * cus_, most);
    if (grid > 8) grid -= grid % 8;
    return (int)std::max<long>(grid, 1);
}

void LayerKernel::launch(const LayerArgs& a, const LayerPlan& plan, const Scratch& s,
                         hipStream_t stream, unsigned phases, uint64_t* prof) {
    auto fail = [&](const std::string& m) { throw std::runtime_error("layer: " + m); };
    if (per_cu_ <= 0) fail("the layer kernel does not fit on a CU");
    if (!bar_) fail("no grid-barrier counter");
    for (int g = 0; g < 4; g++)
        if (!(plan.bm[g] == 16 || plan.bm[g] == 32) || plan.splits[g] < 1 || plan.splits[g] > 4)
            fail("no such plan: " + plan.str());
    const int kv = plan.kv[a.window > 0 ? 1 : 0];
    if (kv < 1 || kv > 8) fail("no such plan: " + plan.str());
    if (phases == 0 || phases > 0x1f) fail("no phases selected");

    const bool ln0 = a.qkv_colsum != nullptr;
    Gemm g[4] = {};
    g[0].epi = ln0 ? EPI_K_LNROPE : EPI_K_ROPE, g[0].a = a.x, g[0].w = a.wqkv, g[0].c = a.qkv;
    g[0].m = a.m, g[0].n = 3 * a.d, g[0].k = a.d, g[0].eps = a.eps, g[0].rope = a.rope;
    g[0].rope_rows = a.rope_rows;
    if (ln0) g[0].stats_in = a.stats_mlp, g[0].colsum = a.qkv_colsum;
    g[1].epi = EPI_K_RESSTATS, g[1].a = a.o, g[1].w = a.wo, g[1].c = a.x, g[1].m = a.m;
    g[1].n = a.d, g[1].k = a.d, g[1].stats_out = a.stats_attn;
    g[2].epi = EPI_K_LNGEGLU, g[2].a = a.x, g[2].w = a.wi, g[2].c = a.mid, g[2].m = a.m;
    g[2].n = 2 * a.inter, g[2].k = a.d, g[2].stats_in = a.stats_attn, g[2].colsum = a.wi_colsum;
    g[2].eps = a.eps;
    g[3].epi = EPI_K_RESSTATS, g[3].a = a.mid, g[3].w = a.wo_mlp, g[3].c = a.x, g[3].m = a.m;
    g[3].n = a.d, g[3].k = a.inter, g[3].stats_out = a.stats_mlp;

    LayerParams P{};
    for (int i = 0; i < 4; i++) {
        const GemmConfig c{plan.bm[i], plan.splits[i]};
        gemm_check(g[i], c, s);
        fill(P.g[i], g[i], c, s);
        P.bm[i] = plan.bm[i];
    }
    if (kv > 1 && (attention_ws_floats(a.m, a.d, kv) > s.ws_floats ||
                   attention_counters(a.m, a.d) > s.n_counters))
        fail("the key-range scratch is too small for " + std::to_string(a.m) + " tokens");
    P.at = AttnParams{a.qkv, a.o, a.m, a.d, a.window, kv, s.ws, s.counters};
    P.epi0 = g[0].epi;
    P.phases = phases;
    P.bar = bar_;
    P.prof = prof;

    const int grid_blocks = grid(a, plan);
    // A barrier between two consecutive selected phases only (the kernel's sync_if).
    unsigned barriers = 0;
    for (int ph = 1; ph < 5; ph++)
        if (((phases >> ph) & 1) && ((phases >> (ph - 1)) & 1)) barriers++;
    void* args[] = {&P};
    hipError_t e;
    if (barriers > 0)
        e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(layer_kernel), dim3(grid_blocks),
                                       dim3(256), args, 0, stream);
    else
        e = hipLaunchKernel(reinterpret_cast<const void*>(layer_kernel), dim3(grid_blocks),
                            dim3(256), args, 0, stream);
    if (e != hipSuccess) fail(std::string(hipGetErrorString(e)) + " (" + plan.str() + ", grid " +
                              std::to_string(grid_blocks) + ")");
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
