/*
 * julia-hip: the MI355X (gfx950) encoder hot path of arnu515/julia-cuda, as a C-ABI shared
 * library (libjulia_hip.so).
 *
 * Part 1 is the drop-in boundary: the five functions of the reference's C interface
 * (src/capi.rs), same names, arguments, ownership and error behaviour, so a caller that binds
 * libjulia_cuda with ctypes can bind this library unchanged.
 *
 * Part 2 is the reference's internal per-op surface, which its --check/--time drivers call
 * (src/gemm.rs gemm::launch, src/attn.rs attn::launch, src/lib.rs embed_into, src/forward.rs
 * GpuHead::launch_input / launch_score, src/timing.rs): each op on caller-owned device memory
 * (plain device pointers) and a HIP stream (hipStream_t as void*; NULL = the null stream).
 *
 * Part 3 is host-only: the weight preparation (src/prep.rs), the synthetic weight generator,
 * the tile choosers (src/gemm.rs:146-172, src/forward.rs:759-806) and engine introspection.
 *
 * Every int-returning function returns 0 or -1; on -1 the error is in `err` (err_len bytes,
 * NUL-terminated, truncated). Nothing unwinds across the boundary (src/capi.rs:36-54).
 */
#ifndef JULIA_HIP_H
#define JULIA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ================= Part 1: the reference's C interface (src/capi.rs) ================== */

typedef struct Engine Engine;

/* src/capi.rs:58-62: the code-object tier this library was built with, static: "gfx950". */
const char *julia_cuda_tier(void);

/* src/capi.rs:70-84 (Engine::load, src/engine.rs:124-161): opens the model in `dir` on GPU 0.
 * `dir` is a checkpoint directory, as in the reference (src/checkpoint.rs:27-62):
 * model.safetensors (F32, F16 or BF16 tensors, memory-mapped), encoder/config.json
 * (ModernBertConfig's fields hidden_size, num_hidden_layers, intermediate_size, vocab_size,
 * max_position_embeddings, num_attention_heads, global_rope_theta, local_rope_theta,
 * global_attn_every_n_layers, local_attention, norm_eps), optionally julia_config.json
 * (head_norm_eps) and julia_hip_names.json (tensor-name overrides: the reference's names come
 * from julia-rs, which is not vendored; the defaults follow ModernBERT for the encoder and
 * torch's TransformerEncoderLayer for the head, see csrc/checkpoint.h). Or the seeded
 * synthetic Julia-1-shaped model named by a spec "synthetic[:key=value,...]" with keys d,
 * layers, inter, vocab, head_layers, head_ff, window, global_every, max_positions, seed,
 * batch_rows (defaults: the ModernBERT-base shapes d=768, layers=22, inter=1152, vocab=50368,
 * head_ff=1536, seed=42). `max_length` sizes the activation buffers and scratch; 0 means the
 * model's maximum. Returns NULL with the error in `err` on failure. */
Engine *julia_cuda_load(const char *dir, size_t max_length, char *err, size_t err_len);

/* src/capi.rs:91-96: frees an engine from julia_cuda_load (NULL is fine). */
void julia_cuda_free(Engine *engine);

/* src/capi.rs:103-106: the GPU's name into buf (len bytes, NUL-terminated). */
void julia_cuda_device(const Engine *engine, char *buf, size_t len);

/* src/capi.rs:120-190 (Engine::run, src/engine.rs:170-196): runs b sequences back to back.
 * Sequence i is lens[i] token ids (all concatenated in ids) with n_markers[i] marker positions
 * (concatenated in markers) and question type qtypes[i] (0 choice, 1 score, 2 noul). Writes each
 * sequence's logits, one per marker, concatenated into logits, and its GPU time in ms (embed to
 * logits) into gpu_ms[i]. layer_fused: the persistent kernels instead of the per-step ones (the
 * whole model in one launch where julia_hip_model_kernel says so). Requests are queued 16 at a
 * time and waited for once per 16. Not thread-safe per
 * engine (the reference's contract). Returns 0, or -1 with the error in err. */
int julia_cuda_run(const Engine *engine, size_t b, const uint32_t *ids, const size_t *lens,
                   const uint32_t *markers, const size_t *n_markers, const uint32_t *qtypes,
                   int layer_fused, float *logits, float *gpu_ms, char *err, size_t err_len);

/* layer_fused = 1 runs the whole forward pass (embed, every layer, the head, the score) as one
 * cooperative launch, the reference's stated next step (README.md:12-13), when the plan's kernel
 * instance takes the head's GEMMs; otherwise the encoder kernel and the head's own launches.
 * Returns 1 if the one-launch path takes `rows` rows (a request's tokens, or a batched pass's),
 * else 0. */
int julia_hip_model_kernel(const Engine *engine, size_t rows);

/* Multi-request throughput (the varlen batching the reference plans beyond Engine::run,
 * src/engine.rs:170-196, which queues requests one by one). */
/* julia_cuda_load with room for batch_rows concatenated rows (0: max_length, or the synthetic
 * spec's batch_rows): the most rows julia_hip_run_batched puts into one pass. */
Engine *julia_hip_load(const char *dir, size_t max_length, size_t batch_rows, char *err,
                       size_t err_len);
/* julia_cuda_run's arguments, checks and outputs, but consecutive requests are packed into
 * passes of at most the engine's rows (julia_hip_load's batch_rows), each run as one forward
 * pass over the concatenated rows: RoPE positions restart in every request, attention (the
 * encoder's and the head's) stays within each request, every row adds its request's type
 * embedding. gpu_ms[i] is the GPU time of the pass request i ran in (shared by the requests of
 * a pass). Results equal julia_cuda_run's within the logit tolerance (the GEMMs' tiles, and so
 * their summation order, depend on the rows). Returns 0, or -1 with the error in err. */
int julia_hip_run_batched(const Engine *engine, size_t b, const uint32_t *ids, const size_t *lens,
                          const uint32_t *markers, const size_t *n_markers,
                          const uint32_t *qtypes, int layer_fused, float *logits, float *gpu_ms,
                          char *err, size_t err_len);

/* ================= Part 2: the per-op surface (device pointers) ======================== */

/* Epilogue flags (kernels/src/main.rs:870-877) and the eight combinations (src/gemm.rs:56-124). */
enum {
    JULIA_HIP_EPI_RES = 1,
    JULIA_HIP_EPI_GEGLU = 2,
    JULIA_HIP_EPI_LN = 4,
    JULIA_HIP_EPI_STATS = 8,
    JULIA_HIP_EPI_ROPE = 16,
    JULIA_HIP_EPI_BIAS = 32,
    JULIA_HIP_EPI_RELU = 64,
    JULIA_HIP_EPI_GELU = 128
};

/* One GEMM (src/gemm.rs:226-245 `Gemm`): c = epilogue(a . w^T), a [m][k], w [n][k], c [m][n]
 * ([m][n/2] with GeGLU), all f16; w is passed packed in MFMA fragment order
 * (julia_hip_prep_pack_frag; the engine's weights are stored so). Row statistics are (sum, sum of squares) f32 pairs per row and
 * 64-column group: stats_in [m][k/64][2] (the LayerNorm epilogues), stats_out [m][n/64][2]
 * (the residual epilogues; written, no clearing needed). colsum and bias have n floats, rope is
 * [rope_rows][32][2] (cos, sin), positions (nullable) gives each row's position. */
typedef struct {
    int epi;
    const void *a;
    const void *w;
    void *c;
    int m, n, k;
    const float *stats_in;
    const float *colsum;
    float eps;
    const float *bias;
    const float *rope;
    const int32_t *positions;
    int rope_rows;
    float *stats_out;
} julia_hip_gemm_args;

/* src/gemm.rs:126-137 `Config`: tile height (16, 32, 48, 64: the latency tiles, 64 columns
 * wide; 128, 192, 256: the throughput tiles, 128, 256 and 256 wide) and K splits (1-8; at least
 * four K steps of 32 a split on the latency tiles, two on the throughput tiles). */
typedef struct {
    int bm;
    int splits;
} julia_hip_gemm_config;

/* src/gemm.rs:199-216 `Scratch`: split-K / key-range partials and arrival counters. */
typedef struct julia_hip_scratch julia_hip_scratch;
julia_hip_scratch *julia_hip_scratch_new(size_t ws_floats, size_t counters, char *err,
                                         size_t err_len);
void julia_hip_scratch_free(julia_hip_scratch *s);

/* src/gemm.rs:254-392 `gemm::launch`: checks, then launches. cfg.bm == 0: the chooser's pick. */
int julia_hip_gemm(const julia_hip_gemm_args *g, julia_hip_gemm_config cfg,
                   const julia_hip_scratch *s, void *stream, char *err, size_t err_len);

/* No counterpart in the reference: julia_hip_gemm for callers that cannot allocate (code under
 * HIP graph capture, serving loops that forbid hipMalloc). It takes no scratch: split-K
 * partials and arrival counters live in a static device array of the library (32 MiB of
 * partials and 16384 counters, held on every GPU it runs on until the process ends), and it
 * calls no allocating routine. A tiling that needs more is rejected with -1 and the sizes.
 * Calls on one GPU share the array: calls that overlap on one GPU (several streams at once)
 * race. The counters a call uses are cleared by a fill kernel on its stream first. */
int julia_hip_gemm_static(const julia_hip_gemm_args *g, julia_hip_gemm_config cfg, void *stream,
                          char *err, size_t err_len);

/* src/attn.rs:20-56 `attn::launch` (+ the layer kernel's key ranges): o [n][d] from qkv
 * [n][3d], heads of 64; window 0 = global; chunks = key ranges per tile (0: the chooser's). */
int julia_hip_attention(const void *qkv, void *o, int n, int d, int window, int chunks,
                        const julia_hip_scratch *s, void *stream, char *err, size_t err_len);

/* julia_hip_attention over concatenated sequences (config 5's batch): seg [n][2] (int32, on
 * the device) holds each row's sequence start and end, and a query sees only the keys of its
 * own sequence. No counterpart in the reference: its batch runs requests one at a time.
 * chunks must be 1. */
int julia_hip_attention_seg(const void *qkv, void *o, int n, int d, int window,
                            const int32_t *seg, const julia_hip_scratch *s, void *stream,
                            char *err, size_t err_len);

/* src/lib.rs:177-219 `embed_into`: x [n][d] = LN(table[ids]) . gamma (ids on the device). */
int julia_hip_embed(const uint32_t *ids, int n, const void *table, int vocab, int d,
                    const float *gamma, float eps, void *x, void *stream, char *err,
                    size_t err_len);

/* src/forward.rs:504-548 `GpuHead::launch_input`: out = LN(x) . gamma + add, and stats
 * [n][d/64][2] of the stored values. */
int julia_hip_norm_add(const void *x, int n, int d, const float *gamma, const float *add,
                       float eps, void *out, float *stats, void *stream, char *err,
                       size_t err_len);

/* src/forward.rs:693-717 (the `score` launch): logits[i] = y[markers[i]] . w + b. */
int julia_hip_score(const void *y, int n, int d, const void *w, float b, const uint32_t *markers,
                    int k, float *logits, void *stream, char *err, size_t err_len);

/* src/timing.rs:43-74 `timing::time` for one GEMM: `warmup` calls, then `batches` batches of
 * `per_batch` back-to-back calls between HIP events; min and median microseconds per call. */
int julia_hip_time_gemm(const julia_hip_gemm_args *g, julia_hip_gemm_config cfg,
                        const julia_hip_scratch *s, int warmup, int batches, int per_batch,
                        float *min_us, float *median_us, char *err, size_t err_len);
int julia_hip_time_attention(const void *qkv, void *o, int n, int d, int window, int chunks,
                             const julia_hip_scratch *s, int warmup, int batches, int per_batch,
                             float *min_us, float *median_us, char *err, size_t err_len);

/* A plain device copy kernel of `bytes` (16-byte multiple) between two fresh buffers, timed as
 * julia_hip_time_gemm: the achievable-bandwidth reference for the bandwidth-bound kernels and the
 * known-size kernel rocprofv3's byte counters are calibrated against. */
int julia_hip_time_copy(size_t bytes, int warmup, int batches, int per_batch, float *min_us,
                        float *median_us, char *err, size_t err_len);

/* hipMemcpy / hipMalloc helpers for callers without a HIP binding of their own (tests and the
 * benchmark, which then run on this library's HIP runtime alone). */
int julia_hip_copy(void *dst, const void *src, size_t bytes, int kind, char *err, size_t err_len);
int julia_hip_device_count(void);
void *julia_hip_device_alloc(size_t bytes, char *err, size_t err_len);
void julia_hip_device_free(void *p);
int julia_hip_device_sync(char *err, size_t err_len);

/* ================= Part 3: host-side logic ============================================== */

/* src/prep.rs:22-35: W' = f16(W . diag(gamma)) and colsum[j] = sum_k W'[j][k] (f64 sum of the
 * rounded weights). w [out][k] f32; w16 [out][k] f16 bits. */
void julia_hip_prep_fold_layernorm(const float *w, const float *gamma, int out, int k,
                                   uint16_t *w16, float *colsum);
/* src/prep.rs:41-59: as above, and bias = b + W . beta (f64). */
void julia_hip_prep_fold_layernorm_bias(const float *w, const float *gamma, const float *beta,
                                        const float *b, int out, int k, uint16_t *w16,
                                        float *colsum, float *bias);
/* The GeGLU row interleave of this library's epilogue (the reference's is src/prep.rs:61-77):
 * src[p] = the checkpoint row of Wi that packed row p holds. */
void julia_hip_prep_geglu_rows(int inter, int32_t *src);
/* w [n][k] f16 bits (n % 64 == 0, k % 32 == 0) <-> the GEMM kernels' fragment order: for
 * 64-row group G, 32-column unit u, 16-row fragment j and lane l < 64, the 8 values
 * w[64 G + 16 j + l % 16][32 u + 8 (l / 16) + e], e < 8, contiguous, in that nesting. A layout
 * transform of this library's, like the reference's row permutations (src/prep.rs:61-101). */
void julia_hip_prep_pack_frag(const uint16_t *w, int n, int k, uint16_t *out);
void julia_hip_prep_unpack_frag(const uint16_t *packed, int n, int k, uint16_t *w);
/* src/prep.rs:103-118: RoPE (cos, sin) [npos][32][2]. */
void julia_hip_prep_rope_table(float theta, int npos, float *table);
/* The synthetic generator: elements start..start+count of tensor `id`, mean + std * N(0, 1). */
void julia_hip_synth(uint64_t seed, uint32_t id, uint64_t start, uint64_t count, double mean,
                     double std, float *out);
/* f32 -> f16 bits, round to nearest even. */
void julia_hip_round_f16(const float *in, uint16_t *out, size_t n);

/* This library's tile and split-K chooser for a 256-CU GPU (replaces src/gemm.rs:153-163);
 * epi: the epilogue flags (the throughput tiles take LayerNorm epilogues up to k = 1024). */
julia_hip_gemm_config julia_hip_gemm_choose(int m, int n, int k, int cus, int epi);
/* The launcher's precondition checks alone (src/gemm.rs:262-329), on the host: 0, or -1 and the
 * reason. The pointers are checked for null and alignment only; the scratch is described by its
 * sizes. */
int julia_hip_gemm_check(const julia_hip_gemm_args *g, julia_hip_gemm_config cfg,
                         size_t ws_floats, size_t counters, char *err, size_t err_len);
/* The reference's layer-kernel plan for a 2080 Ti, kept for provenance and tested against its
 * golden picks: src/forward.rs:759-806 (gemm_plan, phase_cost). */
void julia_hip_gemm_plan_2080ti(int n, int cols, int k, int sms, int per_sm, int *bm,
                                int *splits);
/* The reference's per-step rule, src/gemm.rs:153-172 (choose, splits). */
julia_hip_gemm_config julia_hip_gemm_choose_2080ti(int m, int n, int k, int sms);

/* julia-rs `head::answer` (src/serve.rs:58), as the reference's tools/torch_baseline.py:214-226
 * states it for results tools/score.py compares: probabilities[i] = softmax(logits)[i] (f64);
 * value = the most probable option's index (qtype 0, choice; the first of equal ones), the
 * expected index sum_i i p_i (1, score) or p[1] (2, noul: the "true" option; n >= 2).
 * Returns 0, or -1 and the reason. */
int julia_hip_answer(uint32_t qtype, const float *logits, size_t n, double *probabilities,
                     double *value, char *err, size_t err_len);
/* src/serve.rs:78-115 `report`'s figures over n > 0 values: out[5] = mean, then the values at
 * index round((n - 1) p) (half away from zero) of the sorted values for p = 0.5, 0.9, 0.99, 1. */
int julia_hip_latency_summary(const double *v, size_t n, double *out);

/* Engine introspection (tests, bench). */
typedef struct {
    int d, layers, inter, vocab, head_layers, head_ff, n_qtypes, window, global_every;
    int max_positions, max_length, cus;
    float norm_eps, head_eps;
    uint64_t seed;
    size_t weight_bytes_f16, weight_bytes_f32;
    /* persistent-kernel launches the runtime refused since the engine was loaded (another
     * process held the GPU's cooperative-launch resource); those passes ran per-step */
    size_t coop_refused;
} julia_hip_engine_info;
int julia_hip_engine_info_get(const Engine *e, julia_hip_engine_info *out);
/* src/checkpoint.rs:27-62 `Checkpoint::open` (without a GPU): opens and checks a checkpoint
 * directory (model.safetensors, encoder/config.json; tensor names as documented with
 * julia_cuda_load) and fills the model fields of *out (the engine fields stay zero). */
int julia_hip_checkpoint_config(const char *dir, julia_hip_engine_info *out, char *err,
                                size_t err_len);
/* A prepared weight tensor's device address and size in bytes: name is one of tok_emb,
 * emb_norm, rope_global, rope_local, wqkv, qkv_colsum, wo, wi, wi_colsum, wo_mlp, final_norm,
 * type_emb, in_proj, in_proj_colsum, in_proj_b, out_proj, out_proj_b, linear1, linear1_colsum,
 * linear1_b, linear2, linear2_b, lin1, lin1_colsum, lin1_b, lin2; index = the layer. */
const void *julia_hip_engine_tensor(const Engine *e, const char *name, int index, size_t *bytes);
/* src/timing.rs / the reference's --time (src/main.rs:234-453): one encoder step of the engine
 * on m rows, timed as julia_hip_time_gemm does, rotating through the layers' weights from call
 * to call so they are not L2-resident (src/main.rs:307-312). step: 0 qkv, 1 attention (the
 * layers' own global/window mix), 2 wo, 3 wi, 4 wo_mlp, 5 global attention; the row kernels:
 * 6 embed (m ids), 7 norm_add (m rows), 8 score (every one of m rows). bm = 0: the chooser's
 * tiling. */
int julia_hip_time_encoder_step(const Engine *e, int step, int m, int bm, int splits, int warmup,
                                int batches, int per_batch, float *min_us, float *median_us,
                                char *err, size_t err_len);
/* src/profile.rs:84-241 with kernels/src/prof.rs's stamps: runs the encoder up to `layer` on n
 * tokens (per-step), then that layer with the persistent encoder kernel recording, per block,
 * the 100 MHz clock at each phase's start and end (32 u64 per block: phase p at 2p, 2p + 1; the
 * CU at 10; the stages of the block's first task of GEMM g at 16 + 4 g .. + 3: inputs in place,
 * MFMAs done, partials reduced, epilogue done). layer -1: the whole encoder as the forward pass
 * runs it, one launch, stamps [block][layer][32]. plan: NULL for the default, else 10 ints
 * (bm[4], splits[4], kv[2]); plan_out (nullable) receives the plan used, grid the block count;
 * stamps holds max_rows rows of 32. */
int julia_hip_profile_layer(const Engine *e, int n, int layer, const int *plan, uint64_t *stamps,
                            int max_rows, int *grid, int *plan_out, char *err, size_t err_len);
/* Config 5's batched variant (the reference runs one request at a time): b requests' ids
 * concatenated (lens[i] each, at most max_length; the sum at most the engine's rows, which the
 * model spec's batch_rows raises) through embed and the encoder as one set of rows: positions
 * restart at 0 in every request and attention stays within each request (and its window).
 * x_out (nullable) receives the residual stream after the last layer, [rows][d] f16 bits;
 * gpu_ms the GPU time from embed to the encoder's end (HIP events). No head: the batched
 * variant measures the encoder. */
int julia_hip_encode_batch(const Engine *e, size_t b, const uint32_t *ids, const size_t *lens,
                           int layer_fused, uint16_t *x_out, float *gpu_ms, char *err,
                           size_t err_len);

/* The same batch through the per-step kernels with a HIP event between every two steps: the GPU
 * ms of each step summed over the layers, phase_ms[5] = qkv, attention, wo, wi, wo_mlp (config
 * 5's per-phase timings; the reference's --layer-fused profile is src/profile.rs). */
int julia_hip_encode_batch_phases(const Engine *e, size_t b, const uint32_t *ids,
                                  const size_t *lens, float *phase_ms, char *err, size_t err_len);

/* One request with the residual stream copied out after every encoder layer (x_trace, f16 bits
 * [layers][n][d], nullable) and the head's stream after its last layer (head_x, [n][d],
 * nullable): for step-by-step parity checks. */
int julia_hip_run_trace(const Engine *e, const uint32_t *ids, size_t n, const uint32_t *markers,
                        size_t n_markers, uint32_t qtype, int layer_fused, float *logits,
                        uint16_t *x_trace, uint16_t *head_x, char *err, size_t err_len);

#ifdef __cplusplus
}
#endif
#endif
