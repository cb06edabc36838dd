// Weight preparation and the synthetic model (host only). The transforms restate the
// reference's src/prep.rs; the layout follows src/weights.rs:143-238, with two changes for the
// gfx950 kernels: Wqkv keeps the checkpoint's row order (this library's GEMM epilogue holds
// columns i and i + 32 of a head in one thread without a permutation), and Wi's GeGLU interleave
// is re-derived for that epilogue (geglu_rows).
#include "weights.h"

#include <immintrin.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <functional>
#include <stdexcept>
#include <thread>

namespace jh {

// ---- f16 conversion: the CPU's F16C instructions, round to nearest even. ----
uint16_t f32_to_f16(float f) { return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }
float f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }

// ---- the synthetic generator ----
// A counter-based stream per tensor: element e is half of the Box-Muller pair of counter e / 2
// of splitmix64 seeded with (seed, tensor id), so any element can be generated on its own and
// the tensors in parallel. Doubles throughout; the result rounded to f32 once.
static inline uint64_t splitmix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void synth(uint64_t seed, uint32_t id, uint64_t start, uint64_t count, double mean, double std,
           float* out) {
    const uint64_t stream = splitmix(seed ^ ((uint64_t)id << 32));
    for (uint64_t i = 0; i < count; i++) {
        const uint64_t e = start + i;
        const uint64_t h1 = splitmix(stream + (e >> 1)), h2 = splitmix(h1);
        const double u1 = ((double)(h1 >> 11) + 0.5) * 0x1.0p-53;
        const double u2 = (double)(h2 >> 11) * 0x1.0p-53;
        const double r = sqrt(-2.0 * log(u1)), a = 6.283185307179586 * u2;
        const double z = (e & 1) ? r * sin(a) : r * cos(a);
        out[i] = (float)(mean + std * z);
    }
}

// Distributions: the embedding table N(0, 1); LayerNorm weights 1 + N(0, 0.1), their biases
// N(0, 0.05); the type embeddings N(0, 0.1); linear weights and biases N(0, 0.02).
void tensor_dist(uint32_t id, double* mean, double* std) {
    double m = 0.0, s = 0.02;
    if (id == T_TOK_EMB) {
        s = 1.0;
    } else if (id == T_EMB_NORM || id == T_FINAL_NORM) {
        m = 1.0, s = 0.1;
    } else if (id == T_TYPE_EMB) {
        s = 0.1;
    } else if (id >= T_LAYER && id < T_HEAD) {
        const uint32_t slot = (id - T_LAYER) % 16;
        if (slot == 0 || slot == 3) m = 1.0, s = 0.1;
    } else if (id >= T_HEAD && id < T_SCORER) {
        const uint32_t slot = (id - T_HEAD) % 32;
        if (slot == 0 || slot == 6) m = 1.0, s = 0.1;
        if (slot == 1 || slot == 7) s = 0.05;
    } else if (id >= T_SCORER) {
        const uint32_t slot = id - T_SCORER;
        if (slot == 0) m = 1.0, s = 0.1;
        if (slot == 1) s = 0.05;
    }
    *mean = m;
    *std = s;
}

// ---- src/prep.rs ----
// src/prep.rs:22-35: W' = f16(W . diag(gamma)); colsum[j] = sum_k W'[j][k] of the rounded values
// in f64 (so mu . colsum cancels the mean part of x . W'^T as the GEMM computes it).
void fold_layernorm(const float* w, const float* gamma, int out, int k, uint16_t* w16,
                    float* colsum) {
    for (int j = 0; j < out; j++) {
        double s = 0.0;
        for (int i = 0; i < k; i++) {
            const uint16_t q = f32_to_f16(w[(size_t)j * k + i] * gamma[i]);
            w16[(size_t)j * k + i] = q;
            s += (double)f16_to_f32(q);
        }
        colsum[j] = (float)s;
    }
}

// src/prep.rs:41-59: LN(x) . W^T + b = rstd (x . W'^T - mu colsum) + (b + W . beta).
void fold_layernorm_bias(const float* w, const float* gamma, const float* beta, const float* b,
                         int out, int k, uint16_t* w16, float* colsum, float* bias) {
    for (int j = 0; j < out; j++) {
        double s = (double)b[j];
        for (int i = 0; i < k; i++) s += (double)w[(size_t)j * k + i] * (double)beta[i];
        bias[j] = (float)s;
    }
    fold_layernorm(w, gamma, out, k, w16, colsum);
}

// The epilogue's thread holds columns c and c + 32 of a 64-column group; for GeGLU those are an
// input and its gate: packed rows 64 t + e hold input row 32 t + e, and 64 t + 32 + e the gate
// row inter + 32 t + e (e < 32); output column 32 t + e.
void geglu_rows(int inter, int32_t* src) {
    for (int p = 0; p < 2 * inter; p++) {
        const int t = p >> 6, half = (p >> 5) & 1, e = p & 31;
        src[p] = 32 * t + e + half * inter;
    }
}

// Each wave load of a GEMM tile's weights then reads 1 KB contiguous (16 rows x 64 bytes of the
// row-major matrix otherwise, which costs the CU's memory pipeline about twice as long).
void pack_frag(const uint16_t* w, int n, int k, uint16_t* out) {
    const int U = k / 32;
    size_t o = 0;
    for (int G = 0; G < n / 64; G++)
        for (int u = 0; u < U; u++)
            for (int j = 0; j < 4; j++)
                for (int l = 0; l < 64; l++, o += 8)
                    memcpy(out + o, w + (size_t)(64 * G + 16 * j + l % 16) * k + 32 * u + 8 * (l / 16), 16);
}

void unpack_frag(const uint16_t* packed, int n, int k, uint16_t* w) {
    const int U = k / 32;
    size_t o = 0;
    for (int G = 0; G < n / 64; G++)
        for (int u = 0; u < U; u++)
            for (int j = 0; j < 4; j++)
                for (int l = 0; l < 64; l++, o += 8)
                    memcpy(w + (size_t)(64 * G + 16 * j + l % 16) * k + 32 * u + 8 * (l / 16), packed + o, 16);
}

// src/prep.rs:103-118: cos and sin of p . theta^(-2j/64) for pairs j < 32, in f32.
void rope_table(float theta, int npos, float* table) {
    float inv[32];
    for (int j = 0; j < 32; j++) inv[j] = 1.0f / powf(theta, (float)(2 * j) / 64.0f);
    for (int p = 0; p < npos; p++)
        for (int j = 0; j < 32; j++) {
            const float a = (float)p * inv[j];
            table[((size_t)p * 32 + j) * 2] = cosf(a);
            table[((size_t)p * 32 + j) * 2 + 1] = sinf(a);
        }
}

// ---- the model spec ----
ModelConfig parse_model_spec(const std::string& spec) {
    ModelConfig c;
    const std::string head = "synthetic";
    if (spec.compare(0, head.size(), head) != 0)
        throw std::runtime_error(
            "no model at '" + spec +
            "': this build loads the seeded synthetic model, \"synthetic[:key=value,...]\" "
            "(checkpoint loading is not built)");
    std::string rest = spec.substr(head.size());
    if (!rest.empty()) {
        if (rest[0] != ':') throw std::runtime_error("bad model spec '" + spec + "'");
        rest = rest.substr(1);
    }
    size_t at = 0;
    while (at < rest.size()) {
        size_t end = rest.find(',', at);
        if (end == std::string::npos) end = rest.size();
        const std::string kv = rest.substr(at, end - at);
        at = end + 1;
        if (kv.empty()) continue;
        const size_t eq = kv.find('=');
        if (eq == std::string::npos) throw std::runtime_error("bad model spec entry '" + kv + "'");
        const std::string k = kv.substr(0, eq), v = kv.substr(eq + 1);
        char* stop = nullptr;
        const long long x = strtoll(v.c_str(), &stop, 10);
        if (!stop || *stop || v.empty()) throw std::runtime_error("bad value in '" + kv + "'");
        if (k == "d") c.d = (int)x;
        else if (k == "layers") c.layers = (int)x;
        else if (k == "inter") c.inter = (int)x;
        else if (k == "vocab") c.vocab = (int)x;
        else if (k == "head_layers") c.head_layers = (int)x;
        else if (k == "head_ff") c.head_ff = (int)x;
        else if (k == "window") c.window = (int)x;
        else if (k == "global_every") c.global_every = (int)x;
        else if (k == "max_positions") c.max_positions = (int)x;
        else if (k == "seed") c.seed = (uint64_t)x;
        else if (k == "batch_rows") c.batch_rows = (int)x;
        else throw std::runtime_error("unknown model spec key '" + k + "'");
    }
    auto bad = [](const std::string& m) { throw std::runtime_error("model spec: " + m); };
    if (c.d <= 0 || c.d % 128 || c.d > 4096) bad("d must be a multiple of 128 up to 4096");
    if (c.layers <= 0 || c.layers > 256) bad("layers must be 1-256");
    if (c.inter <= 0 || c.inter % 64) bad("inter must be a multiple of 64");
    if (c.head_ff <= 0 || c.head_ff % 128) bad("head_ff must be a multiple of 128");
    if (c.vocab <= 0 || c.head_layers < 0 || c.head_layers > 16 || c.window < 0 ||
        c.global_every <= 0 || c.max_positions <= 0 || c.max_positions > (1 << 20))
        bad("vocab, head_layers, window, global_every or max_positions out of range");
    if (c.batch_rows < 0 || c.batch_rows > (1 << 20)) bad("batch_rows out of range");
    return c;
}

// ---- preparation ----
namespace {

struct Arena {
    size_t n16 = 0, n32 = 0;
    Span h(size_t len) {
        Span s;
        s.start = (n16 + ALIGN_BYTES / 2 - 1) / (ALIGN_BYTES / 2) * (ALIGN_BYTES / 2);
        s.len = len, s.present = true;
        n16 = s.start + len;
        return s;
    }
    Span f(size_t len) {
        Span s;
        s.start = (n32 + ALIGN_BYTES / 4 - 1) / (ALIGN_BYTES / 4) * (ALIGN_BYTES / 4);
        s.len = len, s.present = true;
        n32 = s.start + len;
        return s;
    }
};

void run_parallel(std::vector<std::function<void()>>& tasks) {
    unsigned nt = std::thread::hardware_concurrency();
    nt = std::max(1u, std::min(nt, 32u));
    std::atomic<size_t> next{0};
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < nt; t++)
        pool.emplace_back([&] {
            for (size_t i = next++; i < tasks.size(); i = next++) tasks[i]();
        });
    for (auto& th : pool) th.join();
}

}  // namespace

HostWeights prepare(const ModelConfig& c, const TensorSource& src) {
    HostWeights hw;
    Layout& L = hw.layout;
    Arena a;
    const size_t d = c.d, I = c.inter, F = c.head_ff;
    L.tok_embeddings = a.h((size_t)c.vocab * d);
    L.emb_norm = a.f(d);
    L.rope_global = a.f((size_t)c.max_positions * 64);
    L.rope_local = a.f((size_t)c.max_positions * 64);
    L.layers.resize(c.layers);
    for (int l = 0; l < c.layers; l++) {
        EncoderLayer& e = L.layers[l];
        e.wqkv = a.h(3 * d * d);
        if (l > 0) e.qkv_colsum = a.f(3 * d);
        e.wo = a.h(d * d);
        e.wi = a.h(2 * I * d);
        e.wi_colsum = a.f(2 * I);
        e.wo_mlp = a.h(d * I);
        e.global = l % c.global_every == 0;
    }
    L.final_norm = a.f(d);
    L.type_emb = a.f((size_t)c.n_qtypes * d);
    L.head.resize(c.head_layers);
    for (auto& h : L.head) {
        h.in_proj = a.h(3 * d * d), h.in_proj_colsum = a.f(3 * d), h.in_proj_b = a.f(3 * d);
        h.out_proj = a.h(d * d), h.out_proj_b = a.f(d);
        h.linear1 = a.h(F * d), h.linear1_colsum = a.f(F), h.linear1_b = a.f(F);
        h.linear2 = a.h(d * F), h.linear2_b = a.f(d);
    }
    L.scorer.lin1 = a.h(d * d), L.scorer.lin1_colsum = a.f(d), L.scorer.lin1_b = a.f(d);
    L.scorer.lin2 = a.h(d);
    hw.f16.assign(a.n16, 0);
    hw.f32.assign(a.n32, 0.0f);

    uint16_t* H = hw.f16.data();
    float* Fv = hw.f32.data();
    std::vector<std::function<void()>> tasks;
    auto gen = [&src](uint32_t id, size_t count) {
        std::vector<float> v(count);
        src(id, 0, count, v.data());
        return v;
    };
    auto conv16 = [&](Span s, uint32_t id) {
        tasks.push_back([=, &gen] {
            const std::vector<float> v = gen(id, s.len);
            for (size_t i = 0; i < s.len; i++) H[s.start + i] = f32_to_f16(v[i]);
        });
    };
    auto copy32 = [&](Span s, uint32_t id) {
        tasks.push_back([=, &src] { src(id, 0, s.len, Fv + s.start); });
    };
    // The embedding table in row blocks: it is most of the work.
    {
        const size_t rows = c.vocab, per = 512, emb0 = L.tok_embeddings.start;
        for (size_t r0 = 0; r0 < rows; r0 += per) {
            const size_t r1 = std::min(rows, r0 + per);
            tasks.push_back([=, &src] {
                std::vector<float> v((r1 - r0) * d);
                src(T_TOK_EMB, r0 * d, v.size(), v.data());
                for (size_t i = 0; i < v.size(); i++) H[emb0 + r0 * d + i] = f32_to_f16(v[i]);
            });
        }
    }
    copy32(L.emb_norm, T_EMB_NORM);
    {
        float* rg = Fv + L.rope_global.start;
        float* rl = Fv + L.rope_local.start;
        const float tg = c.theta_global, tl = c.theta_local;
        const int np = c.max_positions;
        tasks.push_back([=] { rope_table(tg, np, rg); });
        tasks.push_back([=] { rope_table(tl, np, rl); });
    }
    for (int l = 0; l < c.layers; l++) {
        const EncoderLayer e = L.layers[l];
        const uint32_t b = T_LAYER + 16u * (uint32_t)l;
        if (l == 0) {
            conv16(e.wqkv, b + 1);  // no attention LayerNorm in layer 0: converted only
        } else {
            tasks.push_back([=, &gen] {
                const std::vector<float> w = gen(b + 1, 3 * d * d), g = gen(b + 0, d);
                fold_layernorm(w.data(), g.data(), (int)(3 * d), (int)d, H + e.wqkv.start,
                               Fv + e.qkv_colsum.start);
            });
        }
        conv16(e.wo, b + 2);
        tasks.push_back([=, &gen] {
            const std::vector<float> w = gen(b + 4, 2 * I * d), g = gen(b + 3, d);
            std::vector<uint16_t> w16(2 * I * d);
            std::vector<float> cs(2 * I);
            fold_layernorm(w.data(), g.data(), (int)(2 * I), (int)d, w16.data(), cs.data());
            std::vector<int32_t> src(2 * I);
            geglu_rows((int)I, src.data());
            for (size_t p = 0; p < 2 * I; p++) {
                memcpy(H + e.wi.start + p * d, w16.data() + (size_t)src[p] * d, d * 2);
                Fv[e.wi_colsum.start + p] = cs[src[p]];
            }
        });
        conv16(e.wo_mlp, b + 5);
    }
    copy32(L.final_norm, T_FINAL_NORM);
    copy32(L.type_emb, T_TYPE_EMB);
    for (int hl = 0; hl < c.head_layers; hl++) {
        const HeadLayer h = L.head[hl];
        const uint32_t b = T_HEAD + 32u * (uint32_t)hl;
        tasks.push_back([=, &gen] {
            const std::vector<float> w = gen(b + 2, 3 * d * d), g = gen(b + 0, d),
                                     be = gen(b + 1, d), bi = gen(b + 3, 3 * d);
            fold_layernorm_bias(w.data(), g.data(), be.data(), bi.data(), (int)(3 * d), (int)d,
                                H + h.in_proj.start, Fv + h.in_proj_colsum.start, Fv + h.in_proj_b.start);
        });
        conv16(h.out_proj, b + 4);
        copy32(h.out_proj_b, b + 5);
        tasks.push_back([=, &gen] {
            const std::vector<float> w = gen(b + 8, F * d), g = gen(b + 6, d),
                                     be = gen(b + 7, d), bi = gen(b + 9, F);
            fold_layernorm_bias(w.data(), g.data(), be.data(), bi.data(), (int)F, (int)d,
                                H + h.linear1.start, Fv + h.linear1_colsum.start, Fv + h.linear1_b.start);
        });
        conv16(h.linear2, b + 10);
        copy32(h.linear2_b, b + 11);
    }
    {
        const Scorer s = L.scorer;
        tasks.push_back([=, &gen] {
            const std::vector<float> w = gen(T_SCORER + 2, d * d), g = gen(T_SCORER + 0, d),
                                     be = gen(T_SCORER + 1, d), bi = gen(T_SCORER + 3, d);
            fold_layernorm_bias(w.data(), g.data(), be.data(), bi.data(), (int)d, (int)d,
                                H + s.lin1.start, Fv + s.lin1_colsum.start, Fv + s.lin1_b.start);
        });
        conv16(s.lin2, T_SCORER + 4);
    }
    run_parallel(tasks);
    // The GEMM matrices into fragment order, in place.
    tasks.clear();
    auto pack = [&](Span s, int n, int k) {
        tasks.push_back([=] {
            const std::vector<uint16_t> w(H + s.start, H + s.start + s.len);
            pack_frag(w.data(), n, k, H + s.start);
        });
    };
    for (const EncoderLayer& e : L.layers) {
        pack(e.wqkv, (int)(3 * d), (int)d);
        pack(e.wo, (int)d, (int)d);
        pack(e.wi, (int)(2 * I), (int)d);
        pack(e.wo_mlp, (int)d, (int)I);
    }
    for (const HeadLayer& h : L.head) {
        pack(h.in_proj, (int)(3 * d), (int)d);
        pack(h.out_proj, (int)d, (int)d);
        pack(h.linear1, (int)F, (int)d);
        pack(h.linear2, (int)d, (int)F);
    }
    pack(L.scorer.lin1, (int)d, (int)d);
    run_parallel(tasks);
    L.scorer.lin2_b = gen(T_SCORER + 5, 1)[0];
    return hw;
}

HostWeights prepare_synthetic(const ModelConfig& c) {
    const uint64_t seed = c.seed;
    return prepare(c, [seed](uint32_t id, size_t start, size_t count, float* out) {
        double m, sd;
        tensor_dist(id, &m, &sd);
        synth(seed, id, start, count, m, sd, out);
    });
}

}  // namespace jh
