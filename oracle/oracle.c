/*
 * CPU oracle for the julia-hip encoder hot path.  TEST INFRASTRUCTURE ONLY (see oracle.h):
 * it is the checker that tests/, the smoke check and bench.py's cpu_baseline load; the
 * product never links or calls it.
 *
 * Reference citations are paths in arnu515/julia-cuda.  Every function here is pinned by a
 * test in tests/test_oracle.py against something it does not share code with: numpy/torch
 * library routines (LayerNorm, matmul, scaled-dot-product attention, erf), closed forms
 * (RoPE's rotation, the LayerNorm fold identity), brute force on tiny inputs, or the
 * reference's own known-answer tests.  Parity against julia-rs itself (an un-vendored git
 * dependency, rev 6006d2bc, whose checkpoint-gated tests cannot run here) stays unpinned.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- numerics ------------------------------------------------------------------------- */

/* IEEE binary16, round to nearest even (the rounding of cvt.rn.f16.f32, which the reference's
 * `pack` uses: kernels/src/gemm.rs:77-85). */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal */
        uint32_t e = ax >> 23;
        if (e < 102) return (uint16_t)sign;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax >> 13) - (112u << 10);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            uint32_t s = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                s++;
            }
            x = sign | ((113u - s) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void oracle_round_f16(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_f32_to_f16(in[i]);
}

void oracle_widen_f16(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_f16_to_f32(in[i]);
}

static float h2f(uint16_t h) { return oracle_f16_to_f32(h); }
static uint16_t f2h(float f) { return oracle_f32_to_f16(f); }
static float rnd16(float f) { return h2f(f2h(f)); }

/* GELU(x) = x * Phi(x), Phi(x) = (1 + erf(x / sqrt 2)) / 2, with erf from Abramowitz & Stegun
 * 7.1.26 (|error| <= 1.5e-7): erf(y) ~ 1 - (a1 t + ... + a5 t^5) exp(-y^2), t = 1/(1 + p y).
 * The reference uses this approximation (kernels/src/gemm.rs:139-150, "as in julia-rs"). */
static double gelu64(double x) {
    const double p = 0.3275911, a1 = 0.254829592, a2 = -0.284496736, a3 = 1.421413741,
                 a4 = -1.453152027, a5 = 1.061405429;
    double y = fabs(x) * 0.70710678118654752440;
    double t = 1.0 / (1.0 + p * y);
    double poly = ((((a5 * t + a4) * t + a3) * t + a2) * t + a1) * t;
    double q = 0.5 * poly * exp(-y * y); /* = 1 - Phi(|x|) */
    return x * (x >= 0 ? 1.0 - q : q);
}

float oracle_gelu(float x) { return (float)gelu64(x); }

/* ---- synthetic weights ---------------------------------------------------------------- */

static uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Element e of tensor `id`: elements 2p and 2p+1 are the Box-Muller pair of counter p of
 * the tensor's splitmix64 stream, so any element is computable on its own. */
static float synth_one(uint64_t stream, uint64_t e, double mean, double std) {
    uint64_t h1 = mix64(stream + (e >> 1));
    uint64_t h2 = mix64(h1);
    double u1 = ((double)(h1 >> 11) + 0.5) * 0x1.0p-53;
    double u2 = (double)(h2 >> 11) * 0x1.0p-53;
    double r = sqrt(-2.0 * log(u1));
    double a = 6.283185307179586 * u2;
    double z = (e & 1) ? r * sin(a) : r * cos(a);
    return (float)(mean + std * z);
}

void oracle_synth(uint64_t seed, uint32_t id, uint64_t start, uint64_t count, double mean,
                  double std, float *out) {
    uint64_t stream = mix64(seed ^ ((uint64_t)id << 32));
#pragma omp parallel for schedule(static) if (count > 65536)
    for (int64_t i = 0; i < (int64_t)count; i++)
        out[i] = synth_one(stream, start + (uint64_t)i, mean, std);
}

int oracle_tensor_dist(uint32_t id, double *mean, double *std) {
    double m = 0.0, s = 0.02; /* linear weights and biases */
    if (id == ORACLE_TOK_EMB) {
        s = 1.0;
    } else if (id == ORACLE_EMB_NORM || id == ORACLE_FINAL_NORM) {
        m = 1.0, s = 0.1;
    } else if (id == ORACLE_TYPE_EMB) {
        s = 0.1;
    } else if (id >= ORACLE_LAYER_BASE && id < ORACLE_HEAD_BASE) {
        uint32_t slot = (id - ORACLE_LAYER_BASE) % 16;
        if (slot > ORACLE_L_WO_MLP) return -1;
        if (slot == ORACLE_L_ATTN_NORM || slot == ORACLE_L_MLP_NORM) m = 1.0, s = 0.1;
    } else if (id >= ORACLE_HEAD_BASE && id < ORACLE_SCORER_BASE) {
        uint32_t slot = (id - ORACLE_HEAD_BASE) % 32;
        if (slot > ORACLE_H_LINEAR2_B) return -1;
        if (slot == ORACLE_H_NORM1_W || slot == ORACLE_H_NORM2_W) m = 1.0, s = 0.1;
        if (slot == ORACLE_H_NORM1_B || slot == ORACLE_H_NORM2_B) s = 0.05;
    } else if (id >= ORACLE_SCORER_BASE && id <= ORACLE_SCORER_BASE + ORACLE_S_LIN2_B) {
        uint32_t slot = id - ORACLE_SCORER_BASE;
        if (slot == ORACLE_S_NORM_W) m = 1.0, s = 0.1;
        if (slot == ORACLE_S_NORM_B) s = 0.05;
    } else {
        return -1;
    }
    *mean = m;
    *std = s;
    return 0;
}

static float *synth_new(uint64_t seed, uint32_t id, size_t count) {
    double m, s;
    if (oracle_tensor_dist(id, &m, &s)) return NULL;
    float *p = (float *)malloc(count * sizeof(float));
    if (p) oracle_synth(seed, id, 0, count, m, s, p);
    return p;
}

/* ---- weight preparation (src/prep.rs) --------------------------------------------------- */

/* src/prep.rs:22-35: W' = f16(W * gamma) per column; colsum[j] = sum_k W'[j][k] of the ROUNDED
 * weights, in f64, stored as f32. */
void oracle_fold_layernorm(const float *w, const float *gamma, int out, int k, uint16_t *w16,
                           float *colsum) {
    for (int j = 0; j < out; j++) {
        double s = 0.0;
        for (int i = 0; i < k; i++) {
            uint16_t h = f2h(w[(size_t)j * k + i] * gamma[i]);
            w16[(size_t)j * k + i] = h;
            s += (double)h2f(h);
        }
        colsum[j] = (float)s;
    }
}

/* src/prep.rs:41-59: the LayerNorm's beta goes into the bias, b' = b + W.beta (f32 W, f64 sum). */
void oracle_fold_layernorm_bias(const float *w, const float *gamma, const float *beta,
                                const float *b, int out, int k, uint16_t *w16, float *colsum,
                                float *bias) {
    for (int j = 0; j < out; j++) {
        double s = 0.0;
        for (int i = 0; i < k; i++) s += (double)w[(size_t)j * k + i] * (double)beta[i];
        bias[j] = (float)((double)b[j] + s);
    }
    oracle_fold_layernorm(w, gamma, out, k, w16, colsum);
}

/* The GeGLU row order of the product's epilogue (the reference's is src/prep.rs:66-77, for its
 * mma.sync fragments): in each block of 64 packed rows t, rows 64t + e (e < 32) are input
 * rows 32t + e and rows 64t + 32 + e the matching gate rows (inter + 32t + e). */
void oracle_geglu_rows(int inter, int *src) {
    for (int p = 0; p < 2 * inter; p++) {
        int t = p / 64, s = (p % 64) / 32, e = p % 32;
        src[p] = 32 * t + e + (s ? inter : 0);
    }
}

/* src/prep.rs:105-118: (cos, sin) per position and pair j < 32; inv = 1 / theta^(2j/64) and the
 * angle in f32. */
void oracle_rope_table(float theta, int npos, float *table) {
    float inv[32];
    for (int j = 0; j < 32; j++) inv[j] = 1.0f / powf(theta, (float)(2 * j) / 64.0f);
    for (int p = 0; p < npos; p++)
        for (int j = 0; j < 32; j++) {
            float a = (float)p * inv[j];
            table[((size_t)p * 32 + j) * 2] = cosf(a);
            table[((size_t)p * 32 + j) * 2 + 1] = sinf(a);
        }
}

/* ---- f32 operations --------------------------------------------------------------------- */

/* src/check.rs:227-242: LayerNorm per row in f64 (two-pass variance), optional beta. */
void oracle_layernorm_rows(const float *x, const float *gamma, const float *beta, float eps,
                           int rows, int k, float *out) {
#pragma omp parallel for schedule(static) if (rows > 16)
    for (int r = 0; r < rows; r++) {
        const float *row = x + (size_t)r * k;
        double mean = 0.0, var = 0.0;
        for (int i = 0; i < k; i++) mean += row[i];
        mean /= k;
        for (int i = 0; i < k; i++) var += ((double)row[i] - mean) * ((double)row[i] - mean);
        var /= k;
        double rs = 1.0 / sqrt(var + (double)eps);
        for (int i = 0; i < k; i++) {
            double b = beta ? (double)beta[i] : 0.0;
            out[(size_t)r * k + i] = (float)(((double)row[i] - mean) * rs * (double)gamma[i] + b);
        }
    }
}

static float dot_f32(const float *a, const float *b, int k) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= k; i += 8)
        for (int j = 0; j < 8; j++) acc[j] += a[i + j] * b[i + j];
    float s = 0.0f;
    for (; i < k; i++) s += a[i] * b[i];
    return s + ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
}

/* y = x . W^T + b, W [out][in] as the checkpoint stores it (julia-rs `linear`). */
void oracle_linear(const float *x, const float *w, const float *b, int rows, int in, int out,
                   float *y) {
#pragma omp parallel for schedule(dynamic, 8)
    for (int o = 0; o < out; o++) {
        const float *wr = w + (size_t)o * in;
        float bias = b ? b[o] : 0.0f;
        for (int r = 0; r < rows; r++) y[(size_t)r * out + o] = dot_f32(x + (size_t)r * in, wr, in) + bias;
    }
}

/* RoPE on the q and k thirds of qkv rows ([n][3d], heads of 64): the pair (i, i + 32) of each
 * head, rotate-half, x1' = x1 c - x2 s, x2' = x2 c + x1 s (kernels/src/main.rs:977-979). Row r
 * is position pos[r] (or r). */
void oracle_rope_apply(float *qkv, int n, int d, const float *table, const int32_t *pos) {
    for (int r = 0; r < n; r++) {
        int p = pos ? pos[r] : r;
        for (int h = 0; h < 2 * d / 64; h++) {
            float *v = qkv + (size_t)r * 3 * d + h * 64;
            for (int i = 0; i < 32; i++) {
                float c = table[((size_t)p * 32 + i) * 2], s = table[((size_t)p * 32 + i) * 2 + 1];
                float x1 = v[i], x2 = v[i + 32];
                v[i] = x1 * c - x2 * s;
                v[i + 32] = x2 * c + x1 * s;
            }
        }
    }
}

/* softmax(q . k^T / 8) . v per head of 64, keys |i - j| <= window (all keys when window is 0);
 * f64 throughout.  q rows at stride q_stride; k at kv and v at kv + d, rows at kv_stride. */
void oracle_attention(const float *q, int q_stride, const float *kv, int kv_stride, int n,
                      int d, int window, float *o) {
    int heads = d / 64;
#pragma omp parallel for schedule(dynamic, 4) collapse(2)
    for (int h = 0; h < heads; h++)
        for (int i = 0; i < n; i++) {
            double *s = (double *)malloc(sizeof(double) * (size_t)n);
            const float *qi = q + (size_t)i * q_stride + h * 64;
            int j0 = 0, j1 = n;
            if (window > 0) {
                j0 = i - window < 0 ? 0 : i - window;
                j1 = i + window + 1 > n ? n : i + window + 1;
            }
            double mx = -INFINITY;
            for (int j = j0; j < j1; j++) {
                const float *kj = kv + (size_t)j * kv_stride + h * 64;
                double acc = 0.0;
                for (int e = 0; e < 64; e++) acc += (double)qi[e] * (double)kj[e];
                s[j] = acc / 8.0;
                if (s[j] > mx) mx = s[j];
            }
            double sum = 0.0, out[64];
            for (int e = 0; e < 64; e++) out[e] = 0.0;
            for (int j = j0; j < j1; j++) {
                double p = exp(s[j] - mx);
                sum += p;
                const float *vj = kv + (size_t)j * kv_stride + d + h * 64;
                for (int e = 0; e < 64; e++) out[e] += p * (double)vj[e];
            }
            for (int e = 0; e < 64; e++) o[(size_t)i * d + h * 64 + e] = (float)(out[e] / sum);
            free(s);
        }
}

/* julia-rs `geglu`: m = GELU(hh[:, :inter]) * hh[:, inter:]. */
void oracle_geglu(const float *hh, int rows, int inter, float *m) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < inter; c++)
            m[(size_t)r * inter + c] =
                oracle_gelu(hh[(size_t)r * 2 * inter + c]) * hh[(size_t)r * 2 * inter + inter + c];
}

/* Per row and 64-column group: (sum, sum of squares) of f16 values, f64 sums (src/check.rs
 * `row_stats` :268-279 sums a whole row; the product keeps one pair per 64 columns). */
void oracle_row_stats(const uint16_t *x, int rows, int k, float *stats) {
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < k / 64; g++) {
            double s = 0.0, q = 0.0;
            for (int i = 0; i < 64; i++) {
                double v = h2f(x[(size_t)r * k + g * 64 + i]);
                s += v;
                q += v * v;
            }
            stats[((size_t)r * (k / 64) + g) * 2] = (float)s;
            stats[((size_t)r * (k / 64) + g) * 2 + 1] = (float)q;
        }
}

/* ---- the model -------------------------------------------------------------------------- */

typedef struct {
    float *attn_norm, *wqkv, *wo, *mlp_norm, *wi, *wo_mlp;
    int global;
} o_layer;

typedef struct {
    float *n1w, *n1b, *ipw, *ipb, *opw, *opb, *n2w, *n2b, *l1w, *l1b, *l2w, *l2b;
} o_head;

typedef struct {
    oracle_cfg c;
    float *emb_norm, *final_norm, *type_emb;
    o_layer *layers;
    o_head *head;
    float *s_nw, *s_nb, *s_l1w, *s_l1b, *s_l2w, *s_l2b;
    float *rope_g, *rope_l;
} o_model;

void oracle_model_free(void *mp) {
    o_model *m = (o_model *)mp;
    if (!m) return;
    free(m->emb_norm), free(m->final_norm), free(m->type_emb);
    for (int l = 0; m->layers && l < m->c.layers; l++) {
        o_layer *L = &m->layers[l];
        free(L->attn_norm), free(L->wqkv), free(L->wo), free(L->mlp_norm), free(L->wi), free(L->wo_mlp);
    }
    for (int h = 0; m->head && h < m->c.head_layers; h++) {
        o_head *H = &m->head[h];
        free(H->n1w), free(H->n1b), free(H->ipw), free(H->ipb), free(H->opw), free(H->opb);
        free(H->n2w), free(H->n2b), free(H->l1w), free(H->l1b), free(H->l2w), free(H->l2b);
    }
    free(m->layers), free(m->head);
    free(m->s_nw), free(m->s_nb), free(m->s_l1w), free(m->s_l1b), free(m->s_l2w), free(m->s_l2b);
    free(m->rope_g), free(m->rope_l);
    free(m);
}

void *oracle_model_new(const oracle_cfg *cfg) {
    if (cfg->d <= 0 || cfg->d % 64 || cfg->layers <= 0 || cfg->inter <= 0 || cfg->vocab <= 0 ||
        cfg->head_ff <= 0 || cfg->head_layers < 0 || cfg->n_qtypes <= 0 || cfg->max_positions <= 0 ||
        cfg->global_every <= 0)
        return NULL;
    o_model *m = (o_model *)calloc(1, sizeof(o_model));
    if (!m) return NULL;
    m->c = *cfg;
    size_t d = (size_t)cfg->d, I = (size_t)cfg->inter, F = (size_t)cfg->head_ff;
    uint64_t s = cfg->seed;
    m->emb_norm = synth_new(s, ORACLE_EMB_NORM, d);
    m->final_norm = synth_new(s, ORACLE_FINAL_NORM, d);
    m->type_emb = synth_new(s, ORACLE_TYPE_EMB, (size_t)cfg->n_qtypes * d);
    m->layers = (o_layer *)calloc((size_t)cfg->layers, sizeof(o_layer));
    for (int l = 0; l < cfg->layers; l++) {
        uint32_t b = ORACLE_LAYER_BASE + 16u * (uint32_t)l;
        o_layer *L = &m->layers[l];
        L->attn_norm = l == 0 ? NULL : synth_new(s, b + ORACLE_L_ATTN_NORM, d);
        L->wqkv = synth_new(s, b + ORACLE_L_WQKV, 3 * d * d);
        L->wo = synth_new(s, b + ORACLE_L_WO, d * d);
        L->mlp_norm = synth_new(s, b + ORACLE_L_MLP_NORM, d);
        L->wi = synth_new(s, b + ORACLE_L_WI, 2 * I * d);
        L->wo_mlp = synth_new(s, b + ORACLE_L_WO_MLP, d * I);
        L->global = l % cfg->global_every == 0;
    }
    m->head = (o_head *)calloc((size_t)(cfg->head_layers ? cfg->head_layers : 1), sizeof(o_head));
    for (int h = 0; h < cfg->head_layers; h++) {
        uint32_t b = ORACLE_HEAD_BASE + 32u * (uint32_t)h;
        o_head *H = &m->head[h];
        H->n1w = synth_new(s, b + ORACLE_H_NORM1_W, d);
        H->n1b = synth_new(s, b + ORACLE_H_NORM1_B, d);
        H->ipw = synth_new(s, b + ORACLE_H_IN_PROJ_W, 3 * d * d);
        H->ipb = synth_new(s, b + ORACLE_H_IN_PROJ_B, 3 * d);
        H->opw = synth_new(s, b + ORACLE_H_OUT_PROJ_W, d * d);
        H->opb = synth_new(s, b + ORACLE_H_OUT_PROJ_B, d);
        H->n2w = synth_new(s, b + ORACLE_H_NORM2_W, d);
        H->n2b = synth_new(s, b + ORACLE_H_NORM2_B, d);
        H->l1w = synth_new(s, b + ORACLE_H_LINEAR1_W, F * d);
        H->l1b = synth_new(s, b + ORACLE_H_LINEAR1_B, F);
        H->l2w = synth_new(s, b + ORACLE_H_LINEAR2_W, d * F);
        H->l2b = synth_new(s, b + ORACLE_H_LINEAR2_B, d);
    }
    uint32_t sb = ORACLE_SCORER_BASE;
    m->s_nw = synth_new(s, sb + ORACLE_S_NORM_W, d);
    m->s_nb = synth_new(s, sb + ORACLE_S_NORM_B, d);
    m->s_l1w = synth_new(s, sb + ORACLE_S_LIN1_W, d * d);
    m->s_l1b = synth_new(s, sb + ORACLE_S_LIN1_B, d);
    m->s_l2w = synth_new(s, sb + ORACLE_S_LIN2_W, d);
    m->s_l2b = synth_new(s, sb + ORACLE_S_LIN2_B, 1);
    m->rope_g = (float *)malloc(sizeof(float) * (size_t)cfg->max_positions * 64);
    m->rope_l = (float *)malloc(sizeof(float) * (size_t)cfg->max_positions * 64);
    if (!m->rope_g || !m->rope_l || !m->s_l2b) {
        oracle_model_free(m);
        return NULL;
    }
    oracle_rope_table(cfg->theta_global, cfg->max_positions, m->rope_g);
    oracle_rope_table(cfg->theta_local, cfg->max_positions, m->rope_l);
    return m;
}

void oracle_model_embed_rows(void *mp, const uint32_t *ids, int n, float *out) {
    o_model *m = (o_model *)mp;
    size_t d = (size_t)m->c.d;
    double mean, std;
    oracle_tensor_dist(ORACLE_TOK_EMB, &mean, &std);
    for (int r = 0; r < n; r++)
        oracle_synth(m->c.seed, ORACLE_TOK_EMB, (uint64_t)ids[r] * d, d, mean, std, out + (size_t)r * d);
}

/* The forward pass: src/check.rs `trace` (:177-224) for the encoder, then `head_trace`
 * (:484-548) for the head (final norm with the encoder's eps, the type embedding, pre-LN head
 * layers with biases and ReLU, global attention without RoPE, the scorer on the marker rows). */
int oracle_model_forward(void *mp, const uint32_t *ids, int n, int qtype, const uint32_t *markers,
                         int nm, float *logits, float *x_trace, float *head_x) {
    o_model *m = (o_model *)mp;
    const oracle_cfg *c = &m->c;
    if (n <= 0 || n > c->max_positions || qtype < 0 || qtype >= c->n_qtypes || nm < 0) return -1;
    for (int i = 0; i < n; i++)
        if (ids[i] >= (uint32_t)c->vocab) return -1;
    for (int i = 0; i < nm; i++)
        if (markers[i] >= (uint32_t)n) return -1;
    size_t d = (size_t)c->d, I = (size_t)c->inter, F = (size_t)c->head_ff, N = (size_t)n;
    float *x = (float *)malloc(sizeof(float) * N * d);
    float *h = (float *)malloc(sizeof(float) * N * d);
    float *t = (float *)malloc(sizeof(float) * N * d);
    float *o = (float *)malloc(sizeof(float) * N * d);
    float *qkv = (float *)malloc(sizeof(float) * N * 3 * d);
    size_t big = 2 * I > F ? 2 * I : F;
    float *hh = (float *)malloc(sizeof(float) * N * big);
    float *mm = (float *)malloc(sizeof(float) * N * I);
    if (!x || !h || !t || !o || !qkv || !hh || !mm) {
        free(x), free(h), free(t), free(o), free(qkv), free(hh), free(mm);
        return -1;
    }
    oracle_model_embed_rows(m, ids, n, t);
    oracle_layernorm_rows(t, m->emb_norm, NULL, c->norm_eps, n, (int)d, x);
    for (int l = 0; l < c->layers; l++) {
        o_layer *L = &m->layers[l];
        if (L->attn_norm)
            oracle_layernorm_rows(x, L->attn_norm, NULL, c->norm_eps, n, (int)d, h);
        else
            memcpy(h, x, sizeof(float) * N * d);
        oracle_linear(h, L->wqkv, NULL, n, (int)d, (int)(3 * d), qkv);
        oracle_rope_apply(qkv, n, (int)d, L->global ? m->rope_g : m->rope_l, NULL);
        oracle_attention(qkv, (int)(3 * d), qkv + d, (int)(3 * d), n, (int)d,
                         L->global ? 0 : c->window, o);
        oracle_linear(o, L->wo, NULL, n, (int)d, (int)d, t);
        for (size_t i = 0; i < N * d; i++) x[i] += t[i];
        oracle_layernorm_rows(x, L->mlp_norm, NULL, c->norm_eps, n, (int)d, h);
        oracle_linear(h, L->wi, NULL, n, (int)d, (int)(2 * I), hh);
        oracle_geglu(hh, n, (int)I, mm);
        oracle_linear(mm, L->wo_mlp, NULL, n, (int)I, (int)d, t);
        for (size_t i = 0; i < N * d; i++) x[i] += t[i];
        if (x_trace) memcpy(x_trace + (size_t)l * N * d, x, sizeof(float) * N * d);
    }
    /* head */
    oracle_layernorm_rows(x, m->final_norm, NULL, c->norm_eps, n, (int)d, h);
    for (size_t r = 0; r < N; r++)
        for (size_t i = 0; i < d; i++) x[r * d + i] = h[r * d + i] + m->type_emb[(size_t)qtype * d + i];
    for (int hl = 0; hl < c->head_layers; hl++) {
        o_head *H = &m->head[hl];
        oracle_layernorm_rows(x, H->n1w, H->n1b, c->head_eps, n, (int)d, h);
        oracle_linear(h, H->ipw, H->ipb, n, (int)d, (int)(3 * d), qkv);
        oracle_attention(qkv, (int)(3 * d), qkv + d, (int)(3 * d), n, (int)d, 0, o);
        oracle_linear(o, H->opw, H->opb, n, (int)d, (int)d, t);
        for (size_t i = 0; i < N * d; i++) x[i] += t[i];
        oracle_layernorm_rows(x, H->n2w, H->n2b, c->head_eps, n, (int)d, h);
        oracle_linear(h, H->l1w, H->l1b, n, (int)d, (int)F, hh);
        for (size_t i = 0; i < N * F; i++) hh[i] = hh[i] > 0.0f ? hh[i] : 0.0f;
        oracle_linear(hh, H->l2w, H->l2b, n, (int)F, (int)d, t);
        for (size_t i = 0; i < N * d; i++) x[i] += t[i];
    }
    if (head_x) memcpy(head_x, x, sizeof(float) * N * d);
    for (int i = 0; i < nm; i++) {
        float z[4096], zn[4096], y[4096];
        if (d > 4096) break;
        memcpy(z, x + (size_t)markers[i] * d, sizeof(float) * d);
        oracle_layernorm_rows(z, m->s_nw, m->s_nb, c->head_eps, 1, (int)d, zn);
        oracle_linear(zn, m->s_l1w, m->s_l1b, 1, (int)d, (int)d, y);
        for (size_t e = 0; e < d; e++) y[e] = oracle_gelu(y[e]);
        oracle_linear(y, m->s_l2w, m->s_l2b, 1, (int)d, 1, &logits[i]);
    }
    free(x), free(h), free(t), free(o), free(qkv), free(hh), free(mm);
    return 0;
}

/* ---- f16 emulation of the kernels -------------------------------------------------------- */

/* src/check.rs:62-83: the f16 table row, a two-pass LayerNorm in f32, rounded to f16. */
void oracle_emu_embed(const uint16_t *table, const float *gamma, const uint32_t *ids, int n,
                      int d, float eps, uint16_t *x) {
    for (int r = 0; r < n; r++) {
        const uint16_t *row = table + (size_t)ids[r] * d;
        float mean = 0.0f, var = 0.0f;
        for (int i = 0; i < d; i++) mean += h2f(row[i]);
        mean /= (float)d;
        for (int i = 0; i < d; i++) var += (h2f(row[i]) - mean) * (h2f(row[i]) - mean);
        var /= (float)d;
        float rs = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < d; i++) x[(size_t)r * d + i] = f2h((h2f(row[i]) - mean) * rs * gamma[i]);
    }
}

/* The GEMM with its epilogues as the kernels compute them (src/check.rs HostEncoder :901-951;
 * kernels/src/main.rs gemm_tile :931-1038): acc = f64 sums of exact f16 products, as f32; then
 * LN (stats_in), bias, ReLU, GELU, RoPE (pairs c, c + 32 of each 64-column head in the first
 * rope_cols columns), then GeGLU (the product's 64-row interleave) or the store with the
 * residual, rounded to f16, and the stored values' statistics per 64 columns. */
void oracle_emu_gemm(const uint16_t *a, const uint16_t *w, int m, int n, int k, int epi,
                     const float *stats_in, const float *colsum, float eps, const float *bias,
                     const float *rope, const int32_t *pos, int rope_cols, uint16_t *c,
                     float *stats_out) {
    float *wf = (float *)malloc(sizeof(float) * (size_t)n * k);
    oracle_widen_f16(w, wf, (size_t)n * k);
#pragma omp parallel for schedule(dynamic, 4)
    for (int r = 0; r < m; r++) {
        float *af = (float *)malloc(sizeof(float) * (size_t)k);
        float *v = (float *)malloc(sizeof(float) * (size_t)n);
        oracle_widen_f16(a + (size_t)r * k, af, (size_t)k);
        for (int j = 0; j < n; j++) {
            double s = 0.0;
            const float *wr = wf + (size_t)j * k;
            for (int i = 0; i < k; i++) s += (double)(af[i] * wr[i]);
            v[j] = (float)s;
        }
        if (epi & ORACLE_EPI_LN) {
            float S = 0.0f, Q = 0.0f;
            for (int g = 0; g < k / 64; g++) {
                S += stats_in[((size_t)r * (k / 64) + g) * 2];
                Q += stats_in[((size_t)r * (k / 64) + g) * 2 + 1];
            }
            float mean = S / (float)k, var = Q / (float)k - mean * mean;
            float rs = 1.0f / sqrtf((var > 0.0f ? var : 0.0f) + eps);
            for (int j = 0; j < n; j++) v[j] = rs * (v[j] - mean * colsum[j]);
        }
        if (epi & ORACLE_EPI_BIAS)
            for (int j = 0; j < n; j++) v[j] += bias[j];
        if (epi & ORACLE_EPI_RELU)
            for (int j = 0; j < n; j++) v[j] = v[j] > 0.0f ? v[j] : 0.0f;
        if (epi & ORACLE_EPI_GELU)
            for (int j = 0; j < n; j++) v[j] = (float)gelu64(v[j]);
        if (epi & ORACLE_EPI_ROPE) {
            int p = pos ? pos[r] : r;
            for (int j = 0; j < rope_cols; j++) {
                if (j % 64 >= 32) continue;
                int i = j % 64;
                float cs = rope[((size_t)p * 32 + i) * 2], sn = rope[((size_t)p * 32 + i) * 2 + 1];
                float x1 = v[j], x2 = v[j + 32];
                v[j] = x1 * cs - x2 * sn;
                v[j + 32] = x2 * cs + x1 * sn;
            }
        }
        if (epi & ORACLE_EPI_GEGLU) {
            for (int t = 0; t < n / 64; t++)
                for (int e = 0; e < 32; e++)
                    c[(size_t)r * (n / 2) + 32 * t + e] =
                        f2h((float)gelu64(v[64 * t + e]) * v[64 * t + 32 + e]);
        } else {
            for (int j = 0; j < n; j++) {
                float o = v[j];
                if (epi & ORACLE_EPI_RES) o += h2f(c[(size_t)r * n + j]);
                c[(size_t)r * n + j] = f2h(o);
            }
            if (epi & ORACLE_EPI_STATS) oracle_row_stats(c + (size_t)r * n, 1, n, stats_out + (size_t)r * (n / 64) * 2);
        }
        free(af), free(v);
    }
    free(wf);
}

/* src/check.rs:995-1029: scores in f32 from f16 q and k, / 8, softmax with exp in f32, P rounded
 * to f16 for P.V, f32 sums, rounded to f16.  A row with no key in range gets zeros. */
void oracle_emu_attention(const uint16_t *qkv, int n, int d, int window, uint16_t *o) {
    int heads = d / 64;
#pragma omp parallel for schedule(dynamic, 4) collapse(2)
    for (int h = 0; h < heads; h++)
        for (int i = 0; i < n; i++) {
            float *s = (float *)malloc(sizeof(float) * (size_t)n);
            float q[64], acc[64];
            for (int e = 0; e < 64; e++) q[e] = h2f(qkv[(size_t)i * 3 * d + h * 64 + e]), acc[e] = 0.0f;
            int j0 = 0, j1 = n;
            if (window > 0) {
                j0 = i - window < 0 ? 0 : i - window;
                j1 = i + window + 1 > n ? n : i + window + 1;
            }
            float mx = -INFINITY, sum = 0.0f;
            for (int j = j0; j < j1; j++) {
                float dot = 0.0f;
                for (int e = 0; e < 64; e++) dot += q[e] * h2f(qkv[(size_t)j * 3 * d + d + h * 64 + e]);
                s[j] = dot / 8.0f;
                if (s[j] > mx) mx = s[j];
            }
            for (int j = j0; j < j1; j++) {
                float p = expf(s[j] - mx);
                sum += p;
                float p16 = rnd16(p);
                for (int e = 0; e < 64; e++) acc[e] += p16 * h2f(qkv[(size_t)j * 3 * d + 2 * d + h * 64 + e]);
            }
            for (int e = 0; e < 64; e++)
                o[(size_t)i * d + h * 64 + e] = f2h(sum > 0.0f ? acc[e] / sum : 0.0f);
            free(s);
        }
}

/* kernels/src/main.rs:108-176: LN(x) . gamma + add in f32 (two-pass), rounded to f16, and the
 * stored values' statistics (here per 64 columns). */
void oracle_emu_norm_add(const uint16_t *x, const float *gamma, const float *add, int n, int d,
                         float eps, uint16_t *out, float *stats) {
    for (int r = 0; r < n; r++) {
        const uint16_t *row = x + (size_t)r * d;
        float mean = 0.0f, var = 0.0f;
        for (int i = 0; i < d; i++) mean += h2f(row[i]);
        mean /= (float)d;
        for (int i = 0; i < d; i++) var += (h2f(row[i]) - mean) * (h2f(row[i]) - mean);
        var /= (float)d;
        float rs = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < d; i++) out[(size_t)r * d + i] = f2h((h2f(row[i]) - mean) * rs * gamma[i] + add[i]);
    }
    oracle_row_stats(out, n, d, stats);
}
