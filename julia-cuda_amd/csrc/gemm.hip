// The fused-epilogue GEMM family on MFMA (gfx950): c = epilogue(a . w^T), f16 in, f32
// accumulate, f16 out. The reference's tensor-core GEMM (kernels/src/gemm.rs, gemm_tile in
// kernels/src/main.rs:886-1041) walks K through shared tiles with 4-8 warps each owning a
// piece of the output; here two kernels cover the two regimes of a 256-CU GPU:
//
//  - gemm_lat / gemm_lat1 (BM = 16/32/48/64 rows x 64 columns): the small-M, latency-bound
//    regime of one request (M = 72-1024). The block's waves split K between them and reduce
//    their partial tiles through LDS, so a tile's serial K loop is short and there are more
//    tiles to spread over 256 CUs. gemm_lat1, for grids of at most a block a CU (every latency
//    GEMM of a 293-token request), runs eight waves, copies each wave's range of a into LDS as
//    whole 128-byte lines and fixes the waves' K path per kernel instance (gemm_tile.h);
//    gemm_lat runs four waves streaming a and w fragments from L2 into registers, two blocks a
//    CU. Grid split-K on top is deterministic: the last block of a tile to arrive sums every
//    split's partial in split order.
//  - gemm_big (128 x 128, 192 x 256 or 256 x 256 tiles): the MFMA-bound regime (M >= 2048): a
//    and w tiles copied into four LDS stages by direct buffer -> LDS loads (gemm_big.h), four or
//    eight waves each owning a 64 x 64 (96 x 64, 128 x 64) output block on 32 x 32 x 16 MFMA, the
//    epilogue's column-wise part applied on the accumulators. A K split, the same deterministic
//    last-arriver sum, is there for completeness (config sweeps): at these sizes the chooser
//    never picks one.
//
// Both apply the epilogues of device.h (LayerNorm folding, bias, ReLU/GELU, RoPE, GeGLU,
// residual, output statistics) in the same order.
#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <string>

#include "gemm_big.h"
#include "gemm_tile.h"

namespace jh {

// ---------------------------------------------------------------------------------------------
// gemm_lat: grid = tiles_n * tiles_m * splits blocks (1-D, XCD-mapped), 256 threads, at most 256
// registers a lane so that two blocks share a CU (a CU with two tiles overlaps one's loads with
// the other's MFMAs and epilogue).
template <int BM, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_lat(GemmParams p) {
    __shared__ __attribute__((aligned(16))) float red[lat_lds_floats<BM>()];
    __shared__ uint32_t s_last;
    gemm_lat_tile<BM, EPI>(p, blockIdx.x, red, &s_last);
}

// gemm_lat for grids of at most one block a CU (one request's GEMMs up to ~300 tokens): eight
// waves split the tile's K steps, each issuing all of its three to five steps' loads at once. A
// CU takes in its operands from L2 faster with eight waves loading than with four (measured on
// MI355X: ~86-94 against ~55-79 GB/s), for twice the partial tiles to sum through LDS. KP: the
// waves' K path (LAT_KONE3 / 5 / 6, LAT_KLOOP), chosen by the host from K and BM. Dynamic LDS:
// lat_lds_floats<BM, 8>() floats.
template <int BM, int EPI, int KP>
__global__ __launch_bounds__(512, 1) void gemm_lat1(GemmParams p) {
    extern __shared__ __attribute__((aligned(16))) float red_dyn[];
    __shared__ uint32_t s_last;
    gemm_lat_tile<BM, EPI, false, false, 8, KP>(p, blockIdx.x, red_dyn, &s_last);
}

// ---------------------------------------------------------------------------------------------
// gemm_big: BM x BM tiles (BM = 128 or 256) for large M; see gemm_big.h. Dynamic LDS:
// Big<BM, BM>::LDS_BYTES.
// Persistent: the grid is the resident blocks (one 256 x 256 or two 128 x 128 a CU), and block
// b takes tasks b, b + grid, ...: a CU goes from one tile's epilogue to the next tile's copies
// without a block dispatch in between. (The grid is a multiple of 8, so a block's tasks stay on
// its XCD's range of xcd_task.)
// SPLIT: K split p.splits ways, the tile's last arriving split running the epilogue.
template <int BM, int EPI, bool SPLIT>
__global__ __launch_bounds__((Big<BM, big_bn(BM)>::THREADS)) void gemm_big(GemmParams p) {
    extern __shared__ __attribute__((aligned(16))) char lds_dyn[];
    const int T = p.tiles_n * p.tiles_m * (SPLIT ? p.splits : 1);
    for (int task = blockIdx.x; task < T; task += gridDim.x)  // each task ends with a block barrier
        gemm_big_tile<BM, big_bn(BM), EPI, false, false, SPLIT>(p, task, lds_dyn);
}

// ---------------------------------------------------------------------------------------------
// Host side.

namespace {

std::string cfg_str(GemmConfig c) {
    return std::to_string(c.bm) + "x" + std::to_string(c.bm >= 128 ? big_bn(c.bm) : 64) + " split " +
           std::to_string(c.splits);
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace

int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Split-K scratch: a tile's f32 partial per split, and an arrival counter per tile. A split
// latency tile runs on four waves (gemm_lat, gemm_w_tile: 256 threads, 32 rows an epilogue pass),
// and finish() stores whole passes: ceil(BM / 32) x 32 rows of 64 columns (16 -> 32, 48 -> 64).
// A throughput tile stores its BM x BN accumulators.
size_t gemm_ws_floats(int m, int n, GemmConfig cfg) {
    if (cfg.splits <= 1) return 0;
    const bool tput = cfg.bm >= 128;
    const int bn = tput ? big_bn(cfg.bm) : 64;
    const size_t tiles = (size_t)(n / bn) * ((m + cfg.bm - 1) / cfg.bm);
    const size_t rows = tput ? (size_t)cfg.bm : (size_t)(cfg.bm + LAT_SPLIT_PASS_ROWS - 1) /
                                                     LAT_SPLIT_PASS_ROWS * LAT_SPLIT_PASS_ROWS;
    return tiles * cfg.splits * rows * bn;
}

size_t gemm_counters(int m, int n, GemmConfig cfg) {
    if (cfg.splits <= 1) return 0;
    const int bn = cfg.bm >= 128 ? big_bn(cfg.bm) : 64;
    return (size_t)(n / bn) * ((m + cfg.bm - 1) / cfg.bm);
}

void gemm_check(const Gemm& g, GemmConfig cfg, const Scratch& s) {
    auto fail = [&](const std::string& msg) { throw std::runtime_error("gemm: " + msg); };
    if (g.k <= 0 || g.k % 64) fail("k = " + std::to_string(g.k) + " is not a multiple of 64");
    if (g.m <= 0) fail("no rows");
    if (g.n <= 0 || g.n % 64) fail("n = " + std::to_string(g.n) + " is not a multiple of 64");
    const bool tput = cfg.bm >= 128;
    if (!(cfg.bm == 16 || cfg.bm == 32 || cfg.bm == 48 || cfg.bm == 64 || cfg.bm == 128 ||
          cfg.bm == 192 || cfg.bm == 256))
        fail("no tile height " + std::to_string(cfg.bm));
    if (tput && g.n % big_bn(cfg.bm))
        fail("the " + cfg_str(cfg) + " tiles need n % " + std::to_string(big_bn(cfg.bm)) + " == 0");
    if (tput && (g.epi & EPI_LN) && g.k > 128 * BIG_LN_SLOTS)
        fail("the " + cfg_str(cfg) + " tiles take LayerNorm epilogues up to k = " +
             std::to_string(128 * BIG_LN_SLOTS));
    const int ksteps = g.k / 32;
    if (cfg.splits < 1 || cfg.splits > 8 || cfg.splits > ksteps)
        fail(std::to_string(cfg.splits) + " splits for " + std::to_string(ksteps) + " K steps");
    if (cfg.splits > 1 && (gemm_ws_floats(g.m, g.n, cfg) > s.ws_floats ||
                           gemm_counters(g.m, g.n, cfg) > s.n_counters || !s.ws || !s.counters))
        fail("the split-K scratch is too small for m = " + std::to_string(g.m));
    if (!g.a || !g.w || !g.c) fail("a, w or c is null");
    if (!aligned(g.a, 16) || !aligned(g.w, 16) || !aligned(g.c, 16))
        fail("a, w and c must be 16-byte aligned");
    if ((const void*)g.a == (const void*)g.c) fail("c may not alias a");
    if (g.res && (!(g.epi & EPI_RES) || !aligned(g.res, 16) || (const void*)g.res == (const void*)g.c))
        fail("a separate residual goes with the residual epilogues, 16-byte aligned, not c");
    const bool gather = g.epi & EPI_GATHER, score = g.epi & EPI_SCORE;
    if (gather != (g.rows != nullptr) || (gather && (tput || g.src_m < 1)))
        fail("gathered rows go with the gather epilogues on the latency tiles, from src_m >= 1 rows");
    if (gather && (g.epi & EPI_RES) && !g.res) fail("gathered rows need a separate residual");
    if (score != (g.score_w != nullptr && g.logits != nullptr))
        fail("score weights and logits go with the score epilogue");
    if (score && (tput || cfg.splits != 1 || (g.epi & (EPI_GEGLU | EPI_RES | EPI_STATS)) ||
                  !aligned(g.score_w, 8)))
        fail("the score takes latency tiles without a K split, no GeGLU, residual or statistics, "
             "and 8-byte aligned weights");
    if (score && ((size_t)g.m * (g.n / 64) > s.ws_floats || s.n_counters < 1 || !s.ws || !s.counters))
        fail("the score's partials need " + std::to_string((size_t)g.m * (g.n / 64)) +
             " floats of scratch and a counter");
    const bool ln = g.epi & EPI_LN;
    if (ln != (g.stats_in && g.colsum)) fail("LayerNorm inputs go with the ln epilogues");
    if (ln && (!aligned(g.colsum, 16) || !aligned(g.stats_in, 8)))
        fail("colsum must be 16-byte and stats 8-byte aligned");
    const bool rope = g.epi & EPI_ROPE;
    if (rope != (g.rope != nullptr)) fail("a RoPE table goes with the rope epilogues");
    if (rope && (g.n % 192 || g.rope_rows < 1 || (!g.pos && g.rope_rows < g.m) ||
                 !aligned(g.rope, 16)))
        fail("the RoPE table is too short for " + std::to_string(g.m) +
             " positions, or n = " + std::to_string(g.n) + " isn't qkv");
    const bool stats = g.epi & EPI_STATS;
    if (stats != (g.stats_out != nullptr)) fail("output statistics go with the resstats epilogues");
    if (stats && !aligned(g.stats_out, 8)) fail("stats_out must be 8-byte aligned");
    const bool bias = g.epi & EPI_BIAS;
    if (bias != (g.bias != nullptr)) fail("a bias goes with the bias epilogues");
    if (bias && !aligned(g.bias, 16)) fail("bias must be 16-byte aligned");
    if ((g.epi & EPI_GEGLU) && (g.epi & (EPI_RES | EPI_STATS | EPI_ROPE)))
        fail("GeGLU does not combine with a residual, statistics or RoPE");
    if (stats && (g.stats_out == g.stats_in)) fail("stats_out may not alias stats_in");
    if (tput && ((size_t)g.m * g.n * 2 > 0xFFFFFF00ull || (size_t)g.m * g.k * 2 > 0xFFFFFFFFull ||
                 (size_t)g.n * g.k * 2 > 0xFFFFFFFFull))  // buffer offsets: copies, epilogue
        fail("the throughput tiles take a, w and outputs up to 4 GB");
    if (!tput && (size_t)(gather ? g.src_m : g.m) * g.k * 2 > 0xFFFFFFFFull)  // the a copies' offsets
        fail("the latency tiles take a up to 4 GB");
    if (!tput && ksteps / cfg.splits < 4)  // each of the four waves takes a K step of every split
        fail(std::to_string(cfg.splits) + " splits leave a wave no K step of " + std::to_string(ksteps));
    if (tput && ksteps / cfg.splits < 2)  // the stage pipeline's first wait covers two stages
        fail(std::to_string(cfg.splits) + " splits leave a throughput tile fewer than two K steps of " +
             std::to_string(ksteps));
}

template <int B, int EPI, bool SPLIT>
static void launch_big(const GemmParams& p, hipStream_t st) {
    using C = Big<B, big_bn(B)>;
    static const bool lds_ok =  // once per instantiation, before its first launch
        hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_big<B, EPI, SPLIT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES) == hipSuccess;
    if (!lds_ok) throw std::runtime_error("gemm: the throughput kernel cannot have its LDS");
    const int blocks = p.tiles_n * p.tiles_m * p.splits;
    const int grid = std::min(blocks, (B == 128 ? 2 : 1) * device_cus());
    hipLaunchKernelGGL((gemm_big<B, EPI, SPLIT>), dim3(grid), dim3(C::THREADS), (C::LDS_BYTES), st, p);
}

template <int BM, int EPI, int KP>
static void launch_lat1(const GemmParams& p, int blocks, hipStream_t st) {
    constexpr int LDS = lat_lds_floats<BM, 8>() * 4;
    static const bool lds_ok =  // once per instantiation, before its first launch
        hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_lat1<BM, EPI, KP>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, LDS) == hipSuccess;
    if (!lds_ok) throw std::runtime_error("gemm: the one-block latency kernel cannot have its LDS");
    hipLaunchKernelGGL((gemm_lat1<BM, EPI, KP>), dim3(blocks), dim3(512), LDS, st, p);
}

// The eight-wave kernel's K path for K and the tile height: wave w of 8 takes K steps
// [w U / 8, (w + 1) U / 8) of U = K / 32, at most ceil(U / 8); six in one chunk for tiles of up
// to 32 rows (K = 1536: the head's linear2, 6.8 us on the chunked loop).
static int gemm_lat1_path(int k, int bm) {
    const int most = (k / 32 + 7) / 8;
    return most <= 3 ? LAT_KONE3 : most <= 5 ? LAT_KONE5 : most <= 6 && bm <= 32 ? LAT_KONE6 : LAT_KLOOP;
}

template <int BM, int EPI>
static void launch_lat(const GemmParams& p, hipStream_t st) {
    const int blocks = p.tiles_n * p.tiles_m * p.splits;
    // (Eight waves with a K step each: K >= 256.)
    if (p.splits == 1 && blocks <= device_cus() && p.k >= 256) {
        switch (gemm_lat1_path(p.k, BM)) {
            case LAT_KONE3: launch_lat1<BM, EPI, LAT_KONE3>(p, blocks, st); break;
            case LAT_KONE5: launch_lat1<BM, EPI, LAT_KONE5>(p, blocks, st); break;
            case LAT_KONE6:
                if constexpr (BM <= 32) launch_lat1<BM, EPI, LAT_KONE6>(p, blocks, st);
                break;
            default: launch_lat1<BM, EPI, LAT_KLOOP>(p, blocks, st); break;
        }
    } else {
        hipLaunchKernelGGL((gemm_lat<BM, EPI>), dim3(blocks), dim3(256), 0, st, p);
    }
}

template <int BM, int EPI>
static void launch_one(const GemmParams& p, hipStream_t st) {
    if (BM >= 128) {
        constexpr int B = BM >= 128 ? BM : 128;
        if (p.splits > 1) launch_big<B, EPI, true>(p, st);
        else launch_big<B, EPI, false>(p, st);
    } else {
        launch_lat<BM < 128 ? BM : 64, EPI>(p, st);
    }
}

// The epilogues only the latency tiles take (the score, gathered rows).
template <int EPI>
static void launch_epi_lat(const GemmParams& p, int bm, hipStream_t st) {
    switch (bm) {
        case 16: launch_lat<16, EPI>(p, st); break;
        case 32: launch_lat<32, EPI>(p, st); break;
        case 48: launch_lat<48, EPI>(p, st); break;
        default: launch_lat<64, EPI>(p, st); break;
    }
}

template <int EPI>
static void launch_epi(const GemmParams& p, int bm, hipStream_t st) {
    switch (bm) {
        case 16: launch_one<16, EPI>(p, st); break;
        case 32: launch_one<32, EPI>(p, st); break;
        case 48: launch_one<48, EPI>(p, st); break;
        case 64: launch_one<64, EPI>(p, st); break;
        case 128: launch_one<128, EPI>(p, st); break;
        case 192: launch_one<192, EPI>(p, st); break;
        default: launch_one<256, EPI>(p, st); break;
    }
}

void gemm_launch(const Gemm& g, GemmConfig cfg, const Scratch& s, hipStream_t st) {
    gemm_check(g, cfg, s);
    GemmParams p{};
    p.a = g.a, p.w = g.w, p.c = g.c;
    p.stats_in = g.stats_in, p.colsum = g.colsum, p.bias = g.bias, p.rope = g.rope, p.pos = g.pos;
    p.stats_out = g.stats_out, p.ws = s.ws, p.counters = s.counters, p.res = g.res;
    p.rows = g.rows, p.src_m = g.src_m;
    p.score_w = g.score_w, p.score_b = g.score_b, p.logits = g.logits;
    p.m = g.m, p.n = g.n, p.k = g.k, p.eps = g.eps;
    p.rope_cols = (g.epi & EPI_ROPE) ? 2 * (g.n / 3) : 0;
    p.rope_rows = g.rope_rows;
    p.splits = cfg.splits;
    p.tiles_n = g.n / (cfg.bm >= 128 ? big_bn(cfg.bm) : 64);
    p.tiles_m = (g.m + cfg.bm - 1) / cfg.bm;
    switch (g.epi) {
        case EPI_K_ROPE: launch_epi<EPI_K_ROPE>(p, cfg.bm, st); break;
        case EPI_K_LNROPE: launch_epi<EPI_K_LNROPE>(p, cfg.bm, st); break;
        case EPI_K_LNGEGLU: launch_epi<EPI_K_LNGEGLU>(p, cfg.bm, st); break;
        case EPI_K_RESSTATS: launch_epi<EPI_K_RESSTATS>(p, cfg.bm, st); break;
        case EPI_K_LNBIAS: launch_epi<EPI_K_LNBIAS>(p, cfg.bm, st); break;
        case EPI_K_LNBIASRELU: launch_epi<EPI_K_LNBIASRELU>(p, cfg.bm, st); break;
        case EPI_K_LNBIASGELU: launch_epi<EPI_K_LNBIASGELU>(p, cfg.bm, st); break;
        case EPI_K_BIASRESSTATS: launch_epi<EPI_K_BIASRESSTATS>(p, cfg.bm, st); break;
        case EPI_K_BIASRESSTATS | EPI_GATHER:
            launch_epi_lat<EPI_K_BIASRESSTATS | EPI_GATHER>(p, cfg.bm, st);
            break;
        case EPI_K_LNBIASGELU_SCORE: launch_epi_lat<EPI_K_LNBIASGELU_SCORE>(p, cfg.bm, st); break;
        case EPI_K_LNBIASGELU_SCORE | EPI_GATHER:
            launch_epi_lat<EPI_K_LNBIASGELU_SCORE | EPI_GATHER>(p, cfg.bm, st);
            break;
        case 0: launch_epi<0>(p, cfg.bm, st); break;
        default: throw std::runtime_error("gemm: no kernel for epilogue " + std::to_string(g.epi));
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        throw std::runtime_error(std::string("gemm (") + cfg_str(cfg) + "): " + hipGetErrorString(e));
}

// ---------------------------------------------------------------------------------------------
// The allocation-free entry (julia_hip_gemm_static): the split-K partials and arrival counters
// live in this file-scope device array instead of a caller's julia_hip_scratch, so a caller that
// cannot allocate (code under HIP graph capture, serving loops that forbid hipMalloc) can still
// launch split-K tilings. Every GPU the library runs on holds its own copy (32.06 MiB) until
// the process ends; every call on one GPU shares it, so calls that overlap on one GPU (two
// streams at once) race. The counters must start at zero: each split-K call clears the ones it
// uses with a fill kernel on its own stream before the GEMM (no hipMemsetAsync: the call may be
// under graph capture).
constexpr size_t STATIC_WS_FLOATS = size_t(8) << 20;  // f32 split-K partials (32 MiB)
constexpr size_t STATIC_COUNTERS = 16384;              // split-K tiles
static __device__ __align__(256) float scratch[STATIC_WS_FLOATS + STATIC_COUNTERS];

__global__ __launch_bounds__(256) void zero_words(uint32_t* p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

namespace {

// The array's device address on each GPU: host code never uses the name `scratch` itself (it is
// a host-side stand-in), only these addresses, looked up once per device with it current.
std::mutex static_mu;
float* static_addr[64] = {};

float* static_scratch() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        throw std::runtime_error("gemm_static: no current device (or more than 64)");
    std::lock_guard<std::mutex> lock(static_mu);
    if (!static_addr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            throw std::runtime_error(std::string("gemm_static: hipGetSymbolAddress: ") +
                                     hipGetErrorString(e));
        static_addr[dev] = (float*)ptr;
    }
    return static_addr[dev];
}

}  // namespace

size_t gemm_static_ws_floats() { return STATIC_WS_FLOATS; }
size_t gemm_static_counters() { return STATIC_COUNTERS; }

void gemm_launch_static(const Gemm& g, GemmConfig cfg, hipStream_t st) {
    if (cfg.splits > 1) {
        const size_t need = gemm_ws_floats(g.m, g.n, cfg), tiles = gemm_counters(g.m, g.n, cfg);
        if (need > STATIC_WS_FLOATS || tiles > STATIC_COUNTERS)
            throw std::runtime_error(
                "gemm_static: " + cfg_str(cfg) + " at m = " + std::to_string(g.m) + ", n = " +
                std::to_string(g.n) + " needs " + std::to_string(need) + " floats of split-K "
                "partials and " + std::to_string(tiles) + " counters; the static scratch holds " +
                std::to_string(STATIC_WS_FLOATS) + " and " + std::to_string(STATIC_COUNTERS));
    }
    float* base = static_scratch();
    uint32_t* counters = reinterpret_cast<uint32_t*>(base + STATIC_WS_FLOATS);
    const Scratch s{base, STATIC_WS_FLOATS, counters, STATIC_COUNTERS};
    gemm_check(g, cfg, s);
    if (cfg.splits > 1) {
        const int n = (int)gemm_counters(g.m, g.n, cfg);
        hipLaunchKernelGGL(zero_words, dim3((n + 255) / 256), dim3(256), 0, st, counters, n);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            throw std::runtime_error(std::string("gemm_static: clearing the counters: ") +
                                     hipGetErrorString(e));
    }
    gemm_launch(g, cfg, s, st);
}

// The tiling for a GEMM on a 256-CU GPU: the cheapest of the latency tiles and the three
// throughput tiles under a cost model fitted to MI355X sweeps (M = 72 .. 18752, the encoder's
// four shapes; microseconds, random operands, weights rotating through the layers).
//  - Latency tiles (BM = 16/32/48/64 x 64): bound by how fast a CU takes in its tiles'
//    operands: a fixed ~4 us (launch, first round trip, reduction, epilogue) plus the busiest
//    CU's operand bytes, ceil(tiles / CUs) x (BM + 64) x K x 2, at about 55 GB/s into one CU.
//    Ties go to the shorter tile.
//  - 128 x 128 tiles (two a CU): ~2 us plus ~8.5 us (K = 768) per tile on the busiest CU,
//    ceil(tiles / CUs) of them (measured 10.1-11.8 us at one a CU, 17.5-19.9 at two, 27.6 at
//    three, 35.7-43.9 at four and five).
//  - 256 x 256 tiles (one a CU): ~2 us plus ~26.5 us per round of tiles (measured 21.6-29 us
//    for one round, 48.7-55 for two, 82 for three).
//  - 192 x 256 tiles (one a CU): ~2 us plus ~21.7 us per round (0.82 of the 256-row round:
//    23.3-24.4, 42.5-45.9, 66.1, 89.5 us for one to four rounds).
// The throughput tiles enter from 640 rows (below, the latency tiles win by the model and by
// measurement: qkv at 448 rows 6.7 us on 64-row tiles against 10.5 on 128 x 128; at 600 level).
// Measured winners it reproduces: 48-row tiles for qkv and wi at 293 tokens, 16-row for wo and
// wo_mlp; 64-row for qkv and wi at 448; 128 x 128 for qkv and wi at 800 rows (10.7 us against
// 12.3 for 64-row latency tiles) and 1024-3072 and 8192, and for wo and wo_mlp from 2048 to 8192;
// 192 x 256 for qkv and wi at 4096; 256 x 256 at 6144 and 12288 (qkv, wi) and everything at
// 18752.
GemmConfig gemm_choose(int m, int n, int k, int cus, int epi) {
    static_assert(GEMM_BIG_LN_MAX_K == 128 * BIG_LN_SLOTS, "the LayerNorm limit of the throughput tiles");
    if (cus <= 0) cus = 256;
    GemmConfig best{32, 1};
    double best_cost = 1e30;
    for (int bm : {16, 32, 48, 64}) {
        const long tiles = (long)(n / 64) * ((m + bm - 1) / bm);
        const long per_cu = (tiles + cus - 1) / cus;
        const double cost = 4.0 + (double)per_cu * (bm + 64) * k * 2 / 55e3;
        if (cost < best_cost - 0.05) best_cost = cost, best = GemmConfig{bm, 1};
    }
    if (m >= 640 && n % 128 == 0 && k % 64 == 0 && !((epi & EPI_LN) && k > GEMM_BIG_LN_MAX_K)) {
        const double ks = (double)k / 768.0;
        const long l128 = ((long)(n / 128) * ((m + 127) / 128) + cus - 1) / cus;
        const double c128 = 2.0 + 8.5 * ks * (double)l128;
        if (c128 < best_cost) best_cost = c128, best = GemmConfig{128, 1};
        if (n % 256 == 0) {
            const long l256 = ((long)(n / 256) * ((m + 255) / 256) + cus - 1) / cus;
            const double c256 = 2.0 + 26.5 * ks * (double)l256;
            if (c256 < best_cost) best_cost = c256, best = GemmConfig{256, 1};
            const long l192 = ((long)(n / 256) * ((m + 191) / 192) + cus - 1) / cus;
            const double c192 = 2.0 + 21.7 * ks * (double)l192;
            if (c192 < best_cost) best_cost = c192, best = GemmConfig{192, 1};
        }
    }
    return best;
}

}  // namespace jh
