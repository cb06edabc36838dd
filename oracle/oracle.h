/*
 * CPU oracle for the julia-hip encoder hot path.  TEST INFRASTRUCTURE ONLY: tests/, the
 * smoke check in __graft_entry__.py and bench.py's cpu_baseline leg load it as the checker.
 * The product library (julia-cuda_amd/) never links, loads or calls anything here.
 *
 * Two tiers, both restated from the reference's own checking code (paths are relative to the
 * reference repository, arnu515/julia-cuda):
 *
 *   - the f32 forward pass over UNFOLDED weights, LayerNorms in f64, as src/check.rs `trace`
 *     (:177-224) and `head_trace` (:484-548) describe julia-rs's computation;
 *   - an f16 emulation of each kernel's arithmetic (f16 inputs and outputs, exact products
 *     summed in f64, the epilogues in f32), as src/check.rs `HostEncoder` (:879-1076) and
 *     `emulate_embed` (:62-83) do, for ulp-level kernel checks.
 *
 * The synthetic weight generator (a counter-based splitmix64 + Box-Muller stream per tensor)
 * and the weight preparation (src/prep.rs) are restated here independently of the product's
 * own copies, so a test can check the product's prepared weights bit for bit.
 */
#ifndef JULIA_HIP_ORACLE_H
#define JULIA_HIP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numerics ------------------------------------------------------------------------- */
uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);
void oracle_round_f16(const float *in, uint16_t *out, size_t n);
void oracle_widen_f16(const uint16_t *in, float *out, size_t n);
float oracle_gelu(float x);

/* ---- synthetic weights ---------------------------------------------------------------- */
void oracle_synth(uint64_t seed, uint32_t id, uint64_t start, uint64_t count, double mean,
                  double std, float *out);

/* Tensor ids and their distributions (mean, std) for the synthetic Julia-1-shaped model. */
enum {
    ORACLE_TOK_EMB = 1,
    ORACLE_EMB_NORM = 2,
    ORACLE_FINAL_NORM = 3,
    ORACLE_TYPE_EMB = 4,
    ORACLE_LAYER_BASE = 100,  /* + 16*layer + slot */
    ORACLE_HEAD_BASE = 1000,  /* + 32*head layer + slot */
    ORACLE_SCORER_BASE = 2000 /* + slot */
};
enum { ORACLE_L_ATTN_NORM, ORACLE_L_WQKV, ORACLE_L_WO, ORACLE_L_MLP_NORM, ORACLE_L_WI, ORACLE_L_WO_MLP };
enum {
    ORACLE_H_NORM1_W, ORACLE_H_NORM1_B, ORACLE_H_IN_PROJ_W, ORACLE_H_IN_PROJ_B,
    ORACLE_H_OUT_PROJ_W, ORACLE_H_OUT_PROJ_B, ORACLE_H_NORM2_W, ORACLE_H_NORM2_B,
    ORACLE_H_LINEAR1_W, ORACLE_H_LINEAR1_B, ORACLE_H_LINEAR2_W, ORACLE_H_LINEAR2_B
};
enum { ORACLE_S_NORM_W, ORACLE_S_NORM_B, ORACLE_S_LIN1_W, ORACLE_S_LIN1_B, ORACLE_S_LIN2_W, ORACLE_S_LIN2_B };
/* Fills mean/std for tensor `id`; returns 0, or -1 for an unknown id. */
int oracle_tensor_dist(uint32_t id, double *mean, double *std);

/* ---- weight preparation (src/prep.rs) --------------------------------------------------- */
void oracle_fold_layernorm(const float *w, const float *gamma, int out, int k, uint16_t *w16,
                           float *colsum);
void oracle_fold_layernorm_bias(const float *w, const float *gamma, const float *beta,
                                const float *b, int out, int k, uint16_t *w16, float *colsum,
                                float *bias);
/* For the GeGLU-interleaved Wi: src[p] = the checkpoint row that packed row p holds. */
void oracle_geglu_rows(int inter, int *src);
void oracle_rope_table(float theta, int npos, float *table);

/* ---- f32 operations --------------------------------------------------------------------- */
void oracle_layernorm_rows(const float *x, const float *gamma, const float *beta, float eps,
                           int rows, int k, float *out);
void oracle_linear(const float *x, const float *w, const float *b, int rows, int in, int out,
                   float *y);
void oracle_rope_apply(float *qkv, int n, int d, const float *table, const int32_t *pos);
void oracle_attention(const float *q, int q_stride, const float *kv, int kv_stride, int n,
                      int d, int window, float *o);
void oracle_geglu(const float *hh, int rows, int inter, float *m);
void oracle_row_stats(const uint16_t *x, int rows, int k, float *stats);

/* ---- the model -------------------------------------------------------------------------- */
typedef struct {
    int32_t d, layers, inter, vocab, head_layers, head_ff, n_qtypes, window, global_every,
        max_positions;
    float norm_eps, head_eps, theta_global, theta_local;
    uint64_t seed;
} oracle_cfg;

void *oracle_model_new(const oracle_cfg *cfg);
void oracle_model_free(void *model);
/* The f32 forward pass on one request.  x_trace (nullable) gets the residual stream after
 * each encoder layer, [layers][n][d]; head_x (nullable) the head's stream after its last
 * layer, [n][d].  Returns 0, or -1 on bad arguments. */
int oracle_model_forward(void *model, const uint32_t *ids, int n, int qtype,
                         const uint32_t *markers, int nm, float *logits, float *x_trace,
                         float *head_x);
/* The embedding rows of `ids` as the model generates them (f32, [n][d]). */
void oracle_model_embed_rows(void *model, const uint32_t *ids, int n, float *out);

/* ---- f16 emulation of the kernels -------------------------------------------------------- */
/* Epilogue flags, the product's: */
enum {
    ORACLE_EPI_RES = 1, ORACLE_EPI_GEGLU = 2, ORACLE_EPI_LN = 4, ORACLE_EPI_STATS = 8,
    ORACLE_EPI_ROPE = 16, ORACLE_EPI_BIAS = 32, ORACLE_EPI_RELU = 64, ORACLE_EPI_GELU = 128
};
void oracle_emu_embed(const uint16_t *table, const float *gamma, const uint32_t *ids, int n,
                      int d, float eps, uint16_t *x);
/* c = epi(a . w^T); a [m][k], w [n][k] f16.  stats_in/stats_out hold `k/64` (resp. `n/64`)
 * (sum, sum of squares) pairs per row.  c is read first when EPI_RES is set. */
void oracle_emu_gemm(const uint16_t *a, const uint16_t *w, int m, int n, int k, int epi,
                     const float *stats_in, const float *colsum, float eps, const float *bias,
                     const float *rope, const int32_t *pos, int rope_cols, uint16_t *c,
                     float *stats_out);
void oracle_emu_attention(const uint16_t *qkv, int n, int d, int window, uint16_t *o);
void oracle_emu_norm_add(const uint16_t *x, const float *gamma, const float *add, int n, int d,
                         float eps, uint16_t *out, float *stats);

#ifdef __cplusplus
}
#endif
#endif
