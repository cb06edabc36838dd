// FlashAttention-2-style attention on MFMA (gfx950), global or sliding-window, heads of 64:
// o = softmax(q . k^T / 8) . v, keys |i - j| <= window (all keys when window is 0). The
// reference's kernel is kernels/src/main.rs:301-542 with attn.rs's building blocks.
//
// A block takes 64 queries of one head: four waves of 16. Keys go 64 at a time: K into an LDS
// tile [key][d], V transposed into [d][key]. Each wave computes S^T = K . Q^T (the MFMA's output
// gives lane l query l % 16 and 16 of the block's 64 keys), so the running max and sum need only
// in-lane work plus two cross-lane steps, and the lane's P values are exactly the B operand of
// O^T = V^T . P^T, whose output again gives lane l query l % 16 (16 of its 64 dimensions): the
// rescale by the new max is per lane. Softmax in the exp2 domain (scale log2(e) / 8); P rounded
// to f16 for P . V; f32 sums. Rows with no key in range get zeros.
//
// With `chunks` > 1 the key blocks of each (query block, head) tile are split into ranges, one
// block each; every range writes its unnormalised output, max and sum to the scratch and the
// last one of the tile to arrive merges them in range order (kernels/src/attn.rs:92-204).
// With one range, attention_launch picks the tile by measured crossovers (the table there):
// - one request of a few hundred tokens (a 16-query grid of at most a block a CU): the
//   streaming tile (attn_tile.h) with a task per 16-query slice and head and four single-wave
//   key groups, each taking every fourth 64-key block;
// - the shortest inputs, and windows up to 768 rows past that grid: the LDS-resident slice tile
//   (16 queries per block, the key range staged at once and split between the waves);
// - longer ones (config 5's concatenated requests among them): the streaming tile with 16 NW
//   queries a task and KS key groups, which loads each key once per 16 NW queries.
// (The persistent kernel chooses between the slice and the streaming tile itself:
// att_use_stream.)
#include <algorithm>
#include <stdexcept>
#include <string>

#include "attn_tile.h"

namespace jh {

// The streaming 64-query tile for long concatenated inputs (one key range).
__global__ __launch_bounds__(256) void attention_stream_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) char lds[ATT_STREAM_LDS];
    attention_stream_tile(p, blockIdx.x, lds);
}

// The streaming tile with KS key groups of NW waves (one long sequence on a grid of about a
// block a CU). Dynamic LDS: KS ATT_STREAM_LDS.
template <int NW, int KS>
__global__ __launch_bounds__(64 * NW * KS) void attention_streamk_kernel(AttnParams p) {
    extern __shared__ __attribute__((aligned(16))) char lds_dyn[];
    attention_stream_tile<false, NW, KS>(p, blockIdx.x, lds_dyn);
}

__global__ __launch_bounds__(256) void attention_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) f16 lds[ATT_LDS_F16];
    __shared__ uint32_t s_last;
    attention_tile(p, blockIdx.x, blockIdx.y, blockIdx.z, lds, &s_last);
}

// One block of NW waves per (16-query slice, head), the key range staged in LDS (dynamic,
// att_lds_bytes(gkeys, NW)). A step's chain of LDS reads, MFMAs, exponentials and cross-lane
// steps is latency-bound when a CU holds one block (one request's slices and heads number about
// one per CU): eight waves, two a SIMD, take the key steps in half the turns of four and hide
// each other's latencies (measured on MI355X: 293 tokens, global 6.2 -> 5.4 us, +-64 window
// 4.9 -> 4.5 us). Four where the slices' steps are few, or where eight would leave fewer blocks
// resident than the grid needs.
template <int NW>
__global__ __launch_bounds__(64 * NW) void attention_lds_kernel(AttnParams p, int gkeys) {
    extern __shared__ __attribute__((aligned(16))) char lds_dyn[];
    attention_slice_tile<false, false, NW>(p, blockIdx.x, lds_dyn, gkeys);
}

// Lets the LDS-resident kernels have their dynamic LDS (once per process; the engine calls it at
// load, before any graph capture).
bool attention_prepare() {
    static const bool ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(attention_lds_kernel<4>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, att_lds_bytes(512, 4)) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(attention_lds_kernel<8>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, att_lds_bytes(512, 8)) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(attention_streamk_kernel<1, 4>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 4 * ATT_STREAM_LDS) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(attention_streamk_kernel<2, 4>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 4 * ATT_STREAM_LDS) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(attention_streamk_kernel<4, 2>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 2 * ATT_STREAM_LDS) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(attention_streamk_kernel<4, 4>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 4 * ATT_STREAM_LDS) == hipSuccess;
    return ok;
}

// 32-key steps a 16-query slice takes over the keys it reaches (from a 32-aligned start; up to
// 512 keys at once).
int attention_slice_steps(int n, int window) {
    const int reach = window > 0 ? std::min(n, 16 + 2 * window) + 31 : n;
    return (std::min(reach, attention_gkeys(n, window)) + 31) / 32;
}

// Waves per block of the LDS-resident kernel: eight when a slice takes more than four key steps
// and the grid is at most a block a CU (measured: with two blocks on some CUs, eight-wave blocks
// lose to four-wave ones, e.g. a +-64 window over 448 rows, 5.2 against 4.8 us).
int attention_slice_waves(int n, int d, int window) {
    if (attention_slice_steps(n, window) <= 4) return 4;
    const long blocks = (long)(n + 15) / 16 * (d / 64);
    return blocks <= device_cus() ? 8 : 4;
}

// Keys the LDS holds at once for an attention over n rows: all a 16-query slice reaches (from a
// 32-aligned start, in steps of 32), up to 512.
int attention_gkeys(int n, int window) {
    const int reach = window > 0 ? std::min(n, 16 + 2 * window) + 31 : n;
    return std::max(32, std::min(512, (reach + 31) / 32 * 32));
}

size_t attention_ws_floats(int n, int d, int chunks) {
    if (chunks <= 1) return 0;
    return (size_t)((n + 63) / 64) * (d / 64) * chunks * ATT_PART * 256;
}

size_t attention_counters(int n, int d) { return (size_t)((n + 63) / 64) * (d / 64); }

// Key ranges per tile (the reference's default_plan splits global attention, src/forward.rs:
// 186-187). With the key range staged in LDS in one round trip, a tile's key loop is short and
// a split's merge (two more round trips through memory) costs more than it saves up to the
// longest requests: one range. Longer ranges go through LDS in groups of 512 keys.
int attention_chunks(int n, int d, int window, int cus) {
    (void)n, (void)d, (void)window, (void)cus;
    return 1;
}

void attention_launch(const jh_half* qkv, jh_half* o, int n, int d, int window, int chunks,
                      const Scratch& s, hipStream_t st, const int32_t* seg) {
    auto fail = [](const std::string& m) { throw std::runtime_error("attention: " + m); };
    if (n <= 0) fail("no rows");
    if (d <= 0 || d % 64) fail("d = " + std::to_string(d) + " is not a multiple of 64");
    if (window < 0) fail("negative window");
    if (!qkv || !o || ((uintptr_t)qkv % 16) || ((uintptr_t)o % 16)) fail("qkv and o must be 16-byte aligned");
    if (chunks < 1 || chunks > 16) fail(std::to_string(chunks) + " key ranges");
    if (chunks > 1 && (attention_ws_floats(n, d, chunks) > s.ws_floats ||
                       attention_counters(n, d) > s.n_counters || !s.ws || !s.counters))
        fail("the key-range scratch is too small for " + std::to_string(n) + " tokens");
    if (seg && chunks != 1) fail("concatenated sequences take one key range");
    if (seg && ((uintptr_t)seg % 8)) fail("seg must be 8-byte aligned");
    AttnParams p{qkv, o, n, d, window, chunks, s.ws, s.counters, seg};
    // One key range: the tile by measured crossovers (MI355X, one sequence, us). The slice
    // tile with 4 / 8 waves against the streaming tile with waves x key groups 1 x 4 / 2 x 2 /
    // 2 x 4 (d = 768 unless noted):
    //   global   72 rows  3.6 / 3.8 | 3.7 / 3.7 / 4.0     150 rows  4.3 / 4.1 | 3.9 / 4.3 / 4.5
    //            293 rows 5.5 / 5.1 | 4.7 / 5.1 / 5.2     336 rows  5.8 / 5.1 | 4.9 / 5.3 / 5.4
    //            352 rows 8.2 / 8.2 | 8.1 / 5.3 / 5.4     400 rows  9.5 / 8.8 | 8.5 / 5.9 / 5.7
    //            600 rows 2 x 2 / 2 x 4: 7.0 / 6.7        d = 384, 672 rows 8.5 / 6.7 | 6.2 / 7.4 / 6.8
    //   +-64     150 rows 4.2 / 4.1 | 3.9 / 4.3 / 4.5     293 rows  4.3 / 4.2 | 3.9 / 4.4 / 4.5
    //            400 rows 4.5 / 5.2 | 6.3 / 4.4 / 4.6     d = 384, 672 rows 4.3 / 4.2 | 3.9 / 4.4 / 4.5
    // so one wave of 16 queries a key group, four groups (a task per 16-query slice and head,
    // each group a quarter of the key blocks), wherever that grid fits the CUs and a slice takes
    // more than four 32-key steps. Past that grid (and from earlier measurements, slice tile
    // against the streaming tile's 2 x 2 / 4 x 2 / 4 x 1):
    //   global   1024 rows 28.3 / 21.2 | 10.7 / 10.8 / 12.7   2048 rows 98 / 68 | 30.1 / 27.5 / 28.8
    //            4096 rows (4 x 2 / 4 x 1) 85.4 / 82.5
    //   +-64     700 rows  4.9 / 6.6 | 5.0 / 5.1 / 5.0      1024 rows 5.3 / 7.1 | 5.3 / 5.3 / 5.0
    //            1536 rows 7.9 / 10.4 | 7.9 / 6.8 / 6.1
    // and four key groups of four waves (one 1024-thread block a CU) against 2 x 2 / 4 x 2:
    //   global   448 rows 6.9 against 5.6 / 6.7     768 rows 8.8 against 8.9 / 9.0
    //            1024 rows 10.5 against 11.1 / 11.0  1536 rows 25.4 against 24.1 / 22.4
    // so the slice tile for the shortest inputs (global) and up to 768 rows (window), else the
    // streaming tile: four key groups of two waves while that grid fits the CUs, then four
    // groups of four while their grid does, two of four while the four-wave grid is at most two
    // blocks a CU (global), one group of four otherwise (config 5's batch: 4 x 1 48 us a global
    // layer against 59 for 4 x 2).
    const int cus = device_cus();
    const long grid64 = (long)(n + 63) / 64 * (d / 64), grid32 = (long)(n + 31) / 32 * (d / 64);
    const long grid16 = (long)(n + 15) / 16 * (d / 64);
    const bool slice = chunks == 1 && (window == 0 ? n < 293 : n <= 768);
    if (chunks == 1 && grid16 <= cus && attention_slice_steps(n, window) > 4) {
        if (!attention_prepare()) fail("the multi-group streaming kernels cannot have their LDS");
        hipLaunchKernelGGL((attention_streamk_kernel<1, 4>), dim3(grid16), dim3(256), 4 * ATT_STREAM_LDS, st, p);
    } else if (slice) {
        if (!attention_prepare()) fail("the LDS-resident kernel cannot have its LDS");
        const int gkeys = attention_gkeys(n, window);
        const dim3 grid((n + 15) / 16 * (d / 64));
        if (attention_slice_waves(n, d, window) == 8)
            hipLaunchKernelGGL(attention_lds_kernel<8>, grid, dim3(512), att_lds_bytes(gkeys, 8), st, p, gkeys);
        else
            hipLaunchKernelGGL(attention_lds_kernel<4>, grid, dim3(256), att_lds_bytes(gkeys, 4), st, p, gkeys);
    } else if (chunks == 1) {
        if (!attention_prepare()) fail("the multi-group streaming kernels cannot have their LDS");
        if (window == 0 && grid32 <= cus)
            hipLaunchKernelGGL((attention_streamk_kernel<2, 4>), dim3(grid32), dim3(512), 4 * ATT_STREAM_LDS, st, p);
        else if (window == 0 && grid64 <= cus)
            hipLaunchKernelGGL((attention_streamk_kernel<4, 4>), dim3(grid64), dim3(1024), 4 * ATT_STREAM_LDS, st, p);
        else if (window == 0 && grid64 <= 2 * cus)
            hipLaunchKernelGGL((attention_streamk_kernel<4, 2>), dim3(grid64), dim3(512), 2 * ATT_STREAM_LDS, st, p);
        else
            hipLaunchKernelGGL(attention_stream_kernel, dim3(grid64), dim3(256), 0, st, p);
    } else {
        hipLaunchKernelGGL(attention_kernel, dim3((n + 63) / 64, d / 64, chunks), dim3(256), 0, st, p);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw std::runtime_error(std::string("attention: ") + hipGetErrorString(e));
}

}  // namespace jh
