// The kernels' parameter blocks and the host-side launchers (each checks what its kernel
// assumes and throws std::runtime_error otherwise, as the reference's launchers `ensure!` it:
// src/gemm.rs:262-329, src/attn.rs:28-38, src/lib.rs:189-195). Shared by the HIP translation
// units (kernels) and the host-only C++ (engine, capi).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

// f16 storage as its bit pattern in every interface (the device code views it as _Float16),
// so the host-only and the HIP translation units agree on the types.
typedef uint16_t jh_half;

// Epilogue flags (the reference's EPI_* set, kernels/src/main.rs:870-877).
enum {
    EPI_RES = 1,
    EPI_GEGLU = 2,
    EPI_LN = 4,
    EPI_STATS = 8,
    EPI_ROPE = 16,
    EPI_BIAS = 32,
    EPI_RELU = 64,
    EPI_GELU = 128,
    // Not in the reference's set: the score folded into the scorer's lin1 (each row's logit,
    // the dot product of its f16 outputs with one weight row, plus a bias; the outputs are not
    // stored). Latency tiles without a K split only.
    EPI_SCORE = 256,
    // Not in the reference's set either: the rows of a, the residual and the input statistics
    // gathered through an index list (GemmParams::rows). Latency tiles only.
    EPI_GATHER = 512,
};

// The eight epilogue combinations the model uses (src/gemm.rs:56-124).
enum {
    EPI_K_ROPE = EPI_ROPE,
    EPI_K_LNROPE = EPI_LN | EPI_ROPE,
    EPI_K_LNGEGLU = EPI_LN | EPI_GEGLU,
    EPI_K_RESSTATS = EPI_RES | EPI_STATS,
    EPI_K_LNBIAS = EPI_LN | EPI_BIAS,
    EPI_K_LNBIASRELU = EPI_LN | EPI_BIAS | EPI_RELU,
    EPI_K_LNBIASGELU = EPI_LN | EPI_BIAS | EPI_GELU,
    EPI_K_BIASRESSTATS = EPI_BIAS | EPI_RES | EPI_STATS,
    EPI_K_LNBIASGELU_SCORE = EPI_K_LNBIASGELU | EPI_SCORE,
};

// c = epilogue(a . w^T): a [m][k], w [n][k], c [m][n] ([m][n/2] with GeGLU), f16; f32 math.
// Row statistics are (sum, sum of squares) pairs per row and 64-column group:
// stats_in [m][k/64][2], stats_out [m][n/64][2].
struct GemmParams {
    const jh_half* a;
    const jh_half* w;
    jh_half* c;
    const jh_half* res;     // residual rows [m][n] (null: c itself, updated in place)
    const float* stats_in;
    const float* colsum;
    const float* bias;
    const float* rope;      // [positions][32][2] (cos, sin)
    const int32_t* pos;     // per-row positions, or null: row r is position r
    float* stats_out;
    float* ws;              // split-K partials
    uint32_t* counters;     // split-K arrivals, one per output tile, zero between launches
    int m, n, k;
    float eps;
    int rope_cols;          // RoPE applies to columns below this (2 d for qkv)
    int rope_rows;          // positions in the RoPE table (positions are clamped to it)
    int splits;
    int tiles_n, tiles_m;
    // EPI_GATHER: row r of a, of the residual and of stats_in is row rows[r] of those buffers
    // (src_m rows each, indices clamped to them); c and stats_out keep row r.
    const uint32_t* rows;
    int src_m;
    // EPI_SCORE: logits[r] = (f16 row r of the output) . score_w + score_b. Each tile leaves
    // its rows' partial dot products in ws ([m][tiles_n]); the last tile to finish (counters[0],
    // reset by it) sums them in column order.
    const jh_half* score_w;
    float score_b;
    float* logits;
};

// Attention over qkv [n][3 d] (heads of 64, rows [q | k | v]) into o [n][d].
struct AttnParams {
    const jh_half* qkv;
    jh_half* o;
    int n, d;
    int window;          // keys with |i - j| <= window; 0: all
    int chunks;          // key ranges per (64 queries, head) tile
    float* ws;           // key-range partials
    uint32_t* counters;  // one per (query block, head), zero between launches
    // Concatenated sequences (the batched forward): for each row, the first row of its sequence
    // and one past its last ([n][2]); keys outside a query's own sequence are masked. Null: one
    // sequence of n rows.
    const int32_t* seg;
};

namespace jh {

struct GemmConfig {
    int bm;      // rows per tile: 16, 32, 48, 64 (latency kernel) or 128, 192, 256 (throughput kernel)
    int splits;  // K splits, 1-8
};

// Device scratch the split-K GEMMs and split-KV attention share (never at the same time).
struct Scratch {
    float* ws;
    size_t ws_floats;
    uint32_t* counters;
    size_t n_counters;
};

// What a GEMM computes; the launcher fills in the tiling.
struct Gemm {
    int epi;
    const jh_half* a;
    const jh_half* w;
    jh_half* c;
    int m, n, k;
    const float* stats_in;
    const float* colsum;
    float eps;
    const float* bias;
    const float* rope;
    const int32_t* pos;
    int rope_rows;  // positions in the RoPE table
    float* stats_out;
    const jh_half* res = nullptr;     // the residual rows (null: c, updated in place)
    const uint32_t* rows = nullptr;   // GemmParams::rows, over src_m rows
    int src_m = 0;
    const jh_half* score_w = nullptr;  // EPI_SCORE (GemmParams)
    float score_b = 0.0f;
    float* logits = nullptr;
};

// Throws std::runtime_error when g or cfg break what the kernels assume.
void gemm_check(const Gemm& g, GemmConfig cfg, const Scratch& s);
void gemm_launch(const Gemm& g, GemmConfig cfg, const Scratch& s, hipStream_t stream);
// The tile height and split-K for an m x n x k GEMM with epilogue `epi` on `cus` compute units
// (the throughput tiles only where they take the epilogue: LayerNorm up to k = GEMM_BIG_LN_MAX_K).
GemmConfig gemm_choose(int m, int n, int k, int cus, int epi = 0);
constexpr int GEMM_BIG_LN_MAX_K = 1024;
// Compute units of the current device (queried once per device; 256 if the query fails).
int device_cus();
size_t gemm_ws_floats(int m, int n, GemmConfig cfg);
size_t gemm_counters(int m, int n, GemmConfig cfg);
// gemm_launch with the split-K partials and counters in the library's static device scratch
// (no allocation); throws when the tiling needs more than it holds.
void gemm_launch_static(const Gemm& g, GemmConfig cfg, hipStream_t stream);
size_t gemm_static_ws_floats();
size_t gemm_static_counters();

void attention_launch(const jh_half* qkv, jh_half* o, int n, int d, int window, int chunks,
                      const Scratch& s, hipStream_t stream, const int32_t* seg = nullptr);
size_t attention_ws_floats(int n, int d, int chunks);
size_t attention_counters(int n, int d);
int attention_chunks(int n, int d, int window, int cus);
int attention_gkeys(int n, int window);
bool attention_prepare();
int attention_slice_waves(int n, int d, int window);  // 4 or 8 (needs the device)
int attention_slice_steps(int n, int window);

void embed_launch(const uint32_t* ids, int n, const jh_half* table, int vocab, int d,
                  const float* gamma, float eps, jh_half* x, hipStream_t stream);
// row_type (nullable): each row's question type; the row adds add + row_type[row] * d (the
// caller has checked the types against the table), else add.
void norm_add_launch(const jh_half* x, int n, int d, const float* gamma, const float* add,
                     float eps, jh_half* out, float* stats, hipStream_t stream,
                     const int32_t* row_type = nullptr);
// Rows markers[i] (i < k) of a, and of b and the row statistics when given, into row i of
// a_out (b_out, stats_out).
void gather_rows_launch(const jh_half* a, const jh_half* b, const float* stats, int n, int d,
                        const uint32_t* markers, int k, jh_half* a_out, jh_half* b_out,
                        float* stats_out, hipStream_t stream);
// logits[i] = y[markers[i]] . w + b for i < k; markers null: row i.
void score_launch(const jh_half* y, int n, int d, const jh_half* w, float b,
                  const uint32_t* markers, int k, float* logits, hipStream_t stream);
void stream_copy_launch(void* dst, const void* src, size_t bytes, hipStream_t stream);

}  // namespace jh
