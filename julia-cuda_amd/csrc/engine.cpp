// The engine and the C ABI (host only). Engine mirrors the reference's src/engine.rs (the model
// on GPU 0, one stream, weights, scratch; `launch` queues one request, `run` queues 16 and waits
// once), Encoder/Head mirror src/forward.rs's GpuEncoder and GpuHead, and the extern "C"
// functions mirror src/capi.rs. Unlike the reference, the activation buffers are allocated once
// at load for max_length rows (no allocation per request), and the row statistics are per
// 64-column partial sums (deterministic; no clearing between GEMMs).
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <memory>
#include <stdexcept>
#include <tuple>
#include <string>
#include <vector>

#include "../../include/julia_hip.h"
#include "kernels.h"
#include "layer.h"
#include "weights.h"
#include "checkpoint.h"

using namespace jh;

namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

template <typename T>
T* dalloc(size_t count, const char* what) {
    void* p = nullptr;
    hip_check(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)), what);
    return (T*)p;
}

constexpr int QUEUE = 16;  // requests queued before waiting (src/engine.rs:26)

// One request of julia_cuda_run: its ids, markers (row indices < n) and question type.
struct Request {
    const uint32_t* ids;
    size_t n;
    const uint32_t* markers;
    size_t nm;
    uint32_t qtype;
};

}  // namespace

struct Engine {
    int device = 0, cus = 256;
    std::string name;
    hipStream_t stream = nullptr;
    ModelConfig cfg;
    Layout layout;
    jh_half* w16 = nullptr;
    float* w32 = nullptr;
    size_t n16 = 0, n32 = 0;
    int max_length = 0;
    int rows = 0;  // activation rows: max_length, or more for concatenated requests (batch_rows)
    // The batched encoder's inputs: ids, each row's position in its request and its request's
    // rows (first, one past last).
    // Batched requests also carry each row's question type.
    uint32_t* bids_d = nullptr;
    int32_t *pos_d = nullptr, *seg_d = nullptr, *qt_d = nullptr;
    // Activations for max_length rows.
    jh_half *x = nullptr, *qkv = nullptr, *o = nullptr, *mid = nullptr, *hx = nullptr;
    float *stats_a = nullptr, *stats_b = nullptr;
    // Per queued request: ids (max_length each), on the device and in pinned host memory; the
    // queued requests' markers and logits, mcap of each (grown on demand: a request may repeat
    // markers, so its count has no bound).
    uint32_t *ids_d = nullptr, *markers_d = nullptr, *ids_h = nullptr, *markers_h = nullptr;
    float *logits_d = nullptr, *logits_h = nullptr;
    size_t mcap = 0;
    hipEvent_t ev_start[QUEUE] = {}, ev_end[QUEUE] = {};
    Scratch scratch{};
    LayerKernel layer_kernel;
    // Every layer's weights for the persistent encoder kernel, on the device and the host.
    LayerDesc* layers_d = nullptr;
    std::vector<LayerDesc> layers_h;
    // Its write-once activation buffers (LayerArgs): x after each residual step, each layer's
    // qkv and o, max_length rows each.
    jh_half *xa = nullptr, *qa = nullptr, *oa = nullptr;
    // The whole-model launch's own buffers (ModelArgs): the head's residual stream, its layers'
    // qkv and attention outputs, the scorer's hidden rows; and the head-layer table.
    jh_half *hxa = nullptr, *hqa = nullptr, *hoa = nullptr, *hs = nullptr;
    HeadDesc* heads_d = nullptr;
    std::vector<HeadDesc> heads_h;
    // The per-step forward pass as HIP graphs, one per (tokens, markers, question type): 124
    // launches submitted as one. They read the request from fixed buffers (gin: ids, then
    // markers at max_length) and write glogits; stream order keeps queued requests apart.
    bool use_graphs = true;
    uint32_t* gin = nullptr;
    float* glogits = nullptr;
    std::map<std::tuple<int, int, int>, hipGraphExec_t> graphs;

    const jh_half* h(const Span& s) const { return s.present ? w16 + s.start : nullptr; }
    const float* f(const Span& s) const { return s.present ? w32 + s.start : nullptr; }

    // Room for `need` markers and logits (waits for the stream before it reallocates).
    void ensure_markers(size_t need) {
        if (need <= mcap) return;
        hip_check(hipStreamSynchronize(stream), "markers");
        const size_t cap = std::max(need, 2 * mcap);
        hip_check(hipFree(markers_d), "hipFree"), markers_d = nullptr;
        hip_check(hipFree(logits_d), "hipFree"), logits_d = nullptr;
        hip_check(hipHostFree(markers_h), "hipHostFree"), markers_h = nullptr;
        hip_check(hipHostFree(logits_h), "hipHostFree"), logits_h = nullptr;
        mcap = 0;
        markers_d = dalloc<uint32_t>(cap, "markers");
        logits_d = dalloc<float>(cap, "logits");
        hip_check(hipHostMalloc((void**)&markers_h, cap * 4, hipHostMallocDefault), "pinned markers");
        hip_check(hipHostMalloc((void**)&logits_h, cap * 4, hipHostMallocDefault), "pinned logits");
        mcap = cap;
    }

    ~Engine() {
        if (device >= 0) hipSetDevice(device);
        if (stream) hipStreamSynchronize(stream);
        for (auto& kv : graphs) hipGraphExecDestroy(kv.second);
        if (gin) hipFree(gin);
        if (glogits) hipFree(glogits);
        for (int i = 0; i < QUEUE; i++) {
            if (ev_start[i]) hipEventDestroy(ev_start[i]);
            if (ev_end[i]) hipEventDestroy(ev_end[i]);
        }
        for (void* p : {(void*)w16, (void*)w32, (void*)x, (void*)qkv, (void*)o, (void*)mid,
                        (void*)hx, (void*)stats_a, (void*)stats_b, (void*)ids_d,
                        (void*)markers_d, (void*)logits_d, (void*)scratch.ws,
                        (void*)scratch.counters, (void*)layers_d, (void*)xa, (void*)qa,
                        (void*)oa, (void*)bids_d, (void*)pos_d, (void*)seg_d, (void*)qt_d,
                        (void*)hxa, (void*)hqa, (void*)hoa, (void*)hs, (void*)heads_d})
            if (p) hipFree(p);
        if (ids_h) hipHostFree(ids_h);
        if (markers_h) hipHostFree(markers_h);
        if (logits_h) hipHostFree(logits_h);
        if (stream) hipStreamDestroy(stream);
    }

    // ---- the encoder (src/forward.rs GpuEncoder) -------------------------------------------
    void gemm(int epi, const jh_half* a, const jh_half* w, jh_half* c, int m, int n, int k,
              const float* stats_in, const float* colsum, float eps, const float* bias,
              const float* rope, float* stats_out, const int32_t* pos = nullptr) {
        Gemm g{};
        g.epi = epi, g.a = a, g.w = w, g.c = c, g.m = m, g.n = n, g.k = k;
        g.stats_in = stats_in, g.colsum = colsum, g.eps = eps, g.bias = bias;
        g.rope = rope, g.pos = pos, g.rope_rows = cfg.max_positions, g.stats_out = stats_out;
        gemm_launch(g, gemm_choose(m, n, k, cus, epi), scratch, stream);
    }

    // Layer l's five steps as five launches (src/forward.rs:105-165, 361-424): qkv (RoPE; the
    // LayerNorm folded in from layer 1, from the statistics wo_mlp left in stats_b), attention,
    // wo (+ residual, statistics into stats_a), wi (LayerNorm from stats_a, GeGLU), wo_mlp
    // (+ residual, statistics into stats_b). pos and seg (nullable): concatenated requests' row
    // positions and sequence bounds.
    // ev (profiling): six events, recorded before each of the five steps and after the last.
    void launch_layer(int l, int n, const int32_t* pos = nullptr, const int32_t* seg = nullptr,
                      hipEvent_t* ev = nullptr) {
        const EncoderLayer& L = layout.layers[l];
        const int d = cfg.d, I = cfg.inter;
        const float* rope = f(L.global ? layout.rope_global : layout.rope_local);
        auto mark = [&](int i) {
            if (ev) hip_check(hipEventRecord(ev[i], stream), "hipEventRecord");
        };
        mark(0);
        if (L.qkv_colsum.present)
            gemm(EPI_K_LNROPE, x, h(L.wqkv), qkv, n, 3 * d, d, stats_b, f(L.qkv_colsum),
                 cfg.norm_eps, nullptr, rope, nullptr, pos);
        else
            gemm(EPI_K_ROPE, x, h(L.wqkv), qkv, n, 3 * d, d, nullptr, nullptr, 0.0f, nullptr, rope,
                 nullptr, pos);
        mark(1);
        const int window = L.global ? 0 : cfg.window;
        attention_launch(qkv, o, n, d, window, attention_chunks(n, d, window, cus), scratch, stream,
                         seg);
        mark(2);
        gemm(EPI_K_RESSTATS, o, h(L.wo), x, n, d, d, nullptr, nullptr, 0.0f, nullptr, nullptr, stats_a);
        mark(3);
        gemm(EPI_K_LNGEGLU, x, h(L.wi), mid, n, 2 * I, d, stats_a, f(L.wi_colsum), cfg.norm_eps,
             nullptr, nullptr, nullptr);
        mark(4);
        gemm(EPI_K_RESSTATS, mid, h(L.wo_mlp), x, n, d, I, nullptr, nullptr, 0.0f, nullptr, nullptr,
             stats_b);
        mark(5);
    }

    // Config 5's batched input: the sequences' ids, positions restarting per sequence, and each
    // row's sequence bounds, on the device. Returns the rows.
    int prepare_batch(size_t b, const uint32_t* ids, const size_t* lens) {
        if (b == 0 || !ids || !lens) throw std::runtime_error("no requests");
        size_t n = 0;
        for (size_t i = 0; i < b; i++) {
            if (lens[i] == 0 || lens[i] > (size_t)max_length)
                throw std::runtime_error("sequence " + std::to_string(i) + ": " +
                                         std::to_string(lens[i]) + " tokens, not 1 to " +
                                         std::to_string(max_length));
            n += lens[i];
        }
        if (n > (size_t)rows)
            throw std::runtime_error(std::to_string(n) + " rows are over the engine's " +
                                     std::to_string(rows) + " (load with batch_rows)");
        for (size_t j = 0; j < n; j++)
            if (ids[j] >= (uint32_t)cfg.vocab)
                throw std::runtime_error("token id " + std::to_string(ids[j]) + " is past the vocabulary");
        std::vector<Request> reqs(b);
        for (size_t i = 0, at = 0; i < b; at += lens[i], i++)
            reqs[i] = Request{ids + at, lens[i], nullptr, 0, 0};
        return upload_batch(reqs.data(), b).first;
    }

    // Checked requests r[0, b) as one set of concatenated rows on the device: ids (bids_d), each
    // row's position in its request (pos_d), its request's rows [first, last) (seg_d) and
    // question type (qt_d), and the markers as row indices (markers_d, after ensure_markers).
    // Returns (rows, markers); the rows fit (the caller has checked).
    std::pair<int, size_t> upload_batch(const Request* r, size_t b) {
        size_t n = 0, nm = 0;
        for (size_t i = 0; i < b; i++) n += r[i].n, nm += r[i].nm;
        std::vector<uint32_t> ids(n), marks(nm);
        std::vector<int32_t> pos(n), seg(2 * n), qt(n);
        for (size_t i = 0, r0 = 0, m0 = 0; i < b; r0 += r[i].n, m0 += r[i].nm, i++) {
            memcpy(ids.data() + r0, r[i].ids, r[i].n * 4);
            for (size_t j = 0; j < r[i].nm; j++) marks[m0 + j] = (uint32_t)(r0 + r[i].markers[j]);
            for (size_t k = r0; k < r0 + r[i].n; k++) {
                pos[k] = (int32_t)(k - r0), qt[k] = (int32_t)r[i].qtype;
                seg[2 * k] = (int32_t)r0, seg[2 * k + 1] = (int32_t)(r0 + r[i].n);
            }
        }
        hip_check(hipMemcpy(bids_d, ids.data(), n * 4, hipMemcpyHostToDevice), "ids");
        hip_check(hipMemcpy(pos_d, pos.data(), n * 4, hipMemcpyHostToDevice), "positions");
        hip_check(hipMemcpy(seg_d, seg.data(), n * 8, hipMemcpyHostToDevice), "sequences");
        hip_check(hipMemcpy(qt_d, qt.data(), n * 4, hipMemcpyHostToDevice), "question types");
        if (nm) {
            ensure_markers(nm);
            hip_check(hipMemcpy(markers_d, marks.data(), nm * 4, hipMemcpyHostToDevice), "markers");
        }
        return {(int)n, nm};
    }

    // The persistent encoder kernel: layers [first, first + count) as one cooperative launch,
    // from the residual stream in x_in.
    LayerArgs layer_args(int first, int count, int n, const jh_half* x_in,
                         const int32_t* pos = nullptr, const int32_t* seg = nullptr) const {
        LayerArgs a{};
        const size_t ml = (size_t)rows, d = cfg.d;
        a.pos = pos, a.seg = seg;
        a.x_in = x_in, a.xa = xa, a.qa = qa, a.oa = oa, a.mid = mid;
        a.x_stride = ml * d, a.q_stride = ml * 3 * d, a.o_stride = ml * d;
        a.stats_attn = stats_a, a.stats_mlp = stats_b;
        a.layers = layers_d, a.host_layers = layers_h.data(), a.first = first, a.count = count;
        a.m = n, a.d = cfg.d, a.inter = cfg.inter, a.eps = cfg.norm_eps;
        a.rope_rows = cfg.max_positions;
        return a;
    }

    // Returns where the residual stream is after the launch. When the runtime refuses the
    // cooperative launch (another process holds its resource), the layers run on the per-step
    // kernels instead, in place on x.
    const jh_half* launch_encoder_fused(int first, int count, int n, const jh_half* x_in,
                                        const int32_t* pos = nullptr, const int32_t* seg = nullptr) {
        const LayerArgs a = layer_args(first, count, n, x_in, pos, seg);
        if (layer_kernel.launch(a, layer_kernel.default_plan(n, cfg.d, cfg.inter), scratch, stream))
            return LayerKernel::x_out(a);
        if (x_in != x)
            hip_check(hipMemcpyAsync(x, x_in, (size_t)n * cfg.d * 2, hipMemcpyDeviceToDevice, stream),
                      "the residual stream");
        for (int l = first; l < first + count; l++) launch_layer(l, n, pos, seg);
        return x;
    }

    // The whole forward pass as one cooperative launch (embed, every layer, the head, the score)
    // when the plan's kernel instance takes the head's GEMMs; false if not, or if the runtime
    // refused the launch (the caller then runs the encoder kernel, or the per-step layers, and
    // the head's own launches). ids, markers: device, row indices.
    bool launch_model(const uint32_t* ids, int n, int qtype, const uint32_t* markers, int nm,
                      float* logits, const int32_t* pos = nullptr, const int32_t* seg = nullptr,
                      const int32_t* row_type = nullptr) {
        const LayerPlan plan = layer_kernel.default_plan(n, cfg.d, cfg.inter);
        if (!layer_kernel.model_fits(plan, n, cfg.d, cfg.head_ff)) return false;
        const Scorer& S = layout.scorer;
        ModelArgs M{};
        M.ids = ids, M.tok_emb = h(layout.tok_embeddings), M.emb_norm = f(layout.emb_norm);
        M.vocab = cfg.vocab;
        M.heads = heads_d, M.host_heads = heads_h.data(), M.head_layers = (int)heads_h.size();
        M.head_ff = cfg.head_ff, M.head_eps = cfg.head_eps, M.final_norm = f(layout.final_norm);
        M.type_add = f(layout.type_emb) + (row_type ? 0 : (size_t)qtype * cfg.d);
        M.row_type = row_type;
        M.hxa = hxa, M.hqa = hqa, M.hoa = hoa, M.hs = hs;
        M.lin1 = h(S.lin1), M.lin1_colsum = f(S.lin1_colsum), M.lin1_b = f(S.lin1_b);
        M.lin2 = h(S.lin2), M.lin2_b = S.lin2_b;
        M.markers = markers, M.n_markers = nm, M.logits = logits;
        LayerArgs a = layer_args(0, cfg.layers, n, x, pos, seg);
        a.model = &M;
        return layer_kernel.launch(a, plan, scratch, stream);  // false: refused, nothing ran
    }

    // ---- the head (src/forward.rs GpuHead) -------------------------------------------------
    // The final norm + type embedding (statistics into stats_a), the head layers (in_proj: LN
    // with bias from stats_a; global attention, no RoPE; out_proj + bias + residual, statistics
    // into stats_b; linear1: LN from stats_b, bias, ReLU; linear2 + bias + residual, statistics
    // into stats_a), the scorer's lin1 (LN from stats_a, bias, GELU) and the score.
    // Concatenated requests: seg bounds each row's attention to its request, row_type gives its
    // question type (qtype is then unused) and the markers are row indices into the whole set.
    // After the last head layer's attention every step is row-wise and only the marker rows are
    // scored, so unless all_rows (or the markers are not fewer than the rows) those steps run on
    // the marker rows alone, gathered into rows 0 .. nm - 1 of spare buffers: the same values
    // for those rows (up to the GEMM tiles' summation order, which depends on the row count).
    // Without markers (and without all_rows) the head is not run at all.
    void launch_head(const jh_half* xin, int n, int qtype, const uint32_t* markers, int nm,
                     float* logits, const int32_t* seg = nullptr,
                     const int32_t* row_type = nullptr, bool all_rows = false) {
        if (nm <= 0 && !all_rows) return;  // no marker: nothing the head computes is read
        const int d = cfg.d, F = cfg.head_ff;
        const float* add = f(layout.type_emb) + (row_type ? 0 : (size_t)qtype * d);
        norm_add_launch(xin, n, d, f(layout.final_norm), add, cfg.norm_eps, hx, stats_a, stream,
                        row_type);
        const bool compact = !all_rows && nm < n;
        const size_t L = layout.head.size();
        const Scorer& S = layout.scorer;
        // With fewer markers than rows the head's last steps run on the marker rows alone. The
        // GEMM that first reads them gathers them itself (EPI_GATHER: out_proj of the last head
        // layer, or the scorer's lin1 without head layers), and the score rides on lin1's
        // epilogue (EPI_SCORE), where the chooser gives those GEMMs latency tiles (lin1 without
        // a K split); otherwise a gather kernel and a score kernel run.
        auto lat = [&](GemmConfig c) { return c.bm < 128; };
        const GemmConfig cs = compact ? gemm_choose(nm, d, d, cus, EPI_K_LNBIASGELU) : GemmConfig{};
        const bool fold = compact && lat(cs) && cs.splits == 1 &&
                          (L == 0 || lat(gemm_choose(nm, d, d, cus, EPI_K_BIASRESSTATS)));
        // The marker rows' residual stream: x is free once norm_add has read the encoder's
        // output; their attention output goes to qkv (free once attention has read it).
        jh_half* hr = hx;
        int m = n;
        if (compact && L == 0 && !fold) {  // straight into the scorer: its LN statistics go along
            gather_rows_launch(hx, nullptr, stats_a, n, d, markers, nm, x, nullptr, stats_b, stream);
            hr = x, m = nm;
        }
        for (size_t i = 0; i < L; i++) {
            const HeadLayer& H = layout.head[i];
            gemm(EPI_K_LNBIAS, hx, h(H.in_proj), qkv, n, 3 * d, d, stats_a, f(H.in_proj_colsum),
                 cfg.head_eps, f(H.in_proj_b), nullptr, nullptr);
            attention_launch(qkv, o, n, d, 0, attention_chunks(n, d, 0, cus), scratch, stream,
                             seg);
            if (compact && i + 1 == L && fold) {  // out_proj on the marker rows of o and hx
                Gemm g{};
                g.epi = EPI_K_BIASRESSTATS | EPI_GATHER, g.a = o, g.w = h(H.out_proj), g.c = x;
                g.m = nm, g.n = d, g.k = d, g.bias = f(H.out_proj_b), g.stats_out = stats_b;
                g.res = hx, g.rows = markers, g.src_m = n;
                gemm_launch(g, gemm_choose(nm, d, d, cus, g.epi), scratch, stream);
                hr = x, m = nm;
            } else {
                const jh_half* ao = o;
                if (compact && i + 1 == L) {
                    gather_rows_launch(o, hx, nullptr, n, d, markers, nm, qkv, x, nullptr, stream);
                    ao = qkv, hr = x, m = nm;
                }
                gemm(EPI_K_BIASRESSTATS, ao, h(H.out_proj), hr, m, d, d, nullptr, nullptr, 0.0f,
                     f(H.out_proj_b), nullptr, stats_b);
            }
            gemm(EPI_K_LNBIASRELU, hr, h(H.linear1), mid, m, F, d, stats_b, f(H.linear1_colsum),
                 cfg.head_eps, f(H.linear1_b), nullptr, nullptr);
            gemm(EPI_K_BIASRESSTATS, mid, h(H.linear2), hr, m, d, F, nullptr, nullptr, 0.0f,
                 f(H.linear2_b), nullptr, stats_a);
        }
        if (fold) {  // lin1 and the score in one launch (without head layers: from hx's rows)
            Gemm g{};
            g.epi = EPI_K_LNBIASGELU_SCORE | (L == 0 ? EPI_GATHER : 0), g.a = L == 0 ? hx : hr;
            g.w = h(S.lin1), g.c = o, g.m = nm, g.n = d, g.k = d, g.stats_in = stats_a;
            g.colsum = f(S.lin1_colsum), g.eps = cfg.head_eps, g.bias = f(S.lin1_b);
            g.score_w = h(S.lin2), g.score_b = S.lin2_b, g.logits = logits;
            if (L == 0) g.rows = markers, g.src_m = n;
            gemm_launch(g, cs, scratch, stream);
            return;
        }
        const float* st = compact && L == 0 ? stats_b : stats_a;
        gemm(EPI_K_LNBIASGELU, hr, h(S.lin1), o, m, d, d, st, f(S.lin1_colsum), cfg.head_eps,
             f(S.lin1_b), nullptr, nullptr);
        score_launch(o, m, d, h(S.lin2), S.lin2_b, compact ? nullptr : markers, nm, logits, stream);
    }

    // The per-step forward pass for (n, nm, qtype) as an executable graph (captured and
    // instantiated on first use), reading gin and writing glogits.
    hipGraphExec_t graph_for(int n, int nm, int qtype) {
        const auto key = std::make_tuple(n, nm, qtype);
        auto it = graphs.find(key);
        if (it != graphs.end()) return it->second;
        if (graphs.size() >= 512) {  // bound the cache: drop everything, start over
            hip_check(hipStreamSynchronize(stream), "graph cache");
            for (auto& kv : graphs) hipGraphExecDestroy(kv.second);
            graphs.clear();
        }
        hipGraph_t g = nullptr;
        hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "capture");
        try {
            launch(gin, n, qtype, gin + max_length, nm, glogits, false);
        } catch (...) {
            hipStreamEndCapture(stream, &g);
            if (g) hipGraphDestroy(g);
            throw;
        }
        hip_check(hipStreamEndCapture(stream, &g), "capture");
        hipGraphExec_t ex = nullptr;
        const hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        hip_check(e, "hipGraphInstantiate");
        graphs[key] = ex;
        return ex;
    }

    // One request's forward pass (src/engine.rs:66-112 `launch`): ids already on the device.
    void launch(const uint32_t* ids, int n, int qtype, const uint32_t* markers, int nm,
                float* logits, bool fused) {
        if (fused && launch_model(ids, n, qtype, markers, nm, logits)) return;
        embed_launch(ids, n, h(layout.tok_embeddings), cfg.vocab, cfg.d, f(layout.emb_norm),
                     cfg.norm_eps, x, stream);
        const jh_half* xf = x;
        if (fused)
            xf = launch_encoder_fused(0, cfg.layers, n, x);
        else
            for (int l = 0; l < cfg.layers; l++) launch_layer(l, n);
        launch_head(xf, n, qtype, markers, nm, logits);
    }
};

namespace {

Engine* load_engine(const char* dir, size_t max_length, size_t batch_rows = 0) {
    if (!dir) throw std::runtime_error("no model given");
    // A checkpoint directory, or the seeded synthetic model (checked before any device work).
    std::unique_ptr<Checkpoint> ck;
    if (Checkpoint::is_checkpoint(dir)) ck.reset(new Checkpoint(dir));
    const ModelConfig spec = ck ? ck->config() : parse_model_spec(dir);
    if (batch_rows > (1u << 20)) throw std::runtime_error("batch_rows out of range");
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        throw std::runtime_error("no HIP device is available");
    std::unique_ptr<Engine> e(new Engine());
    e->device = 0;
    hip_check(hipSetDevice(0), "hipSetDevice");
    hipDeviceProp_t prop;
    hip_check(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties");
    const std::string arch = prop.gcnArchName;
    if (arch.compare(0, 6, "gfx950") != 0)
        throw std::runtime_error(std::string("this library has gfx950 kernels, but ") + prop.name +
                                 " is " + arch);
    e->name = prop.name;
    if (e->name.empty()) e->name = "AMD GPU (" + arch + ")";  // a runtime without the name table
    e->cus = prop.multiProcessorCount;
    e->cfg = spec;
    const ModelConfig& c = e->cfg;
    const size_t ml = max_length ? max_length : (size_t)c.max_positions;
    if (ml > (size_t)c.max_positions)
        throw std::runtime_error("max_length " + std::to_string(ml) + " is over the model's " +
                                 std::to_string(c.max_positions));
    e->max_length = (int)ml;
    e->rows = (int)std::max({ml, (size_t)c.batch_rows, batch_rows});
    HostWeights hw = ck ? prepare(c, ck->source()) : prepare_synthetic(c);
    ck.reset();  // the mapping is no longer needed
    e->layout = hw.layout;
    e->n16 = hw.f16.size(), e->n32 = hw.f32.size();
    hip_check(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking), "hipStreamCreate");
    e->w16 = dalloc<jh_half>(e->n16, "weights (f16)");
    e->w32 = dalloc<float>(e->n32, "weights (f32)");
    hip_check(hipMemcpy(e->w16, hw.f16.data(), e->n16 * 2, hipMemcpyHostToDevice), "upload");
    hip_check(hipMemcpy(e->w32, hw.f32.data(), e->n32 * 4, hipMemcpyHostToDevice), "upload");

    const size_t n = e->rows, d = c.d, wide = std::max<size_t>(c.inter, c.head_ff);
    e->x = dalloc<jh_half>(n * d, "x");
    e->qkv = dalloc<jh_half>(n * 3 * d, "qkv");
    e->o = dalloc<jh_half>(n * d, "o");
    e->mid = dalloc<jh_half>(n * std::max(wide, d), "mid");
    e->hx = dalloc<jh_half>(n * d, "hx");
    e->stats_a = dalloc<float>(n * (d / 64) * 2, "stats");
    e->stats_b = dalloc<float>(n * (d / 64) * 2, "stats");
    e->ids_d = dalloc<uint32_t>(QUEUE * ml, "ids");
    e->markers_d = dalloc<uint32_t>(QUEUE * ml, "markers");
    e->logits_d = dalloc<float>(QUEUE * ml, "logits");
    e->gin = dalloc<uint32_t>(2 * ml, "graph input");
    e->glogits = dalloc<float>(ml, "graph logits");
    e->bids_d = dalloc<uint32_t>(n, "batch ids");
    e->pos_d = dalloc<int32_t>(n, "batch positions");
    e->seg_d = dalloc<int32_t>(2 * n, "batch sequences");
    e->qt_d = dalloc<int32_t>(n, "batch question types");
    if (const char* g = getenv("JULIA_HIP_GRAPHS")) e->use_graphs = strcmp(g, "0") != 0;
    hip_check(hipHostMalloc((void**)&e->ids_h, QUEUE * ml * 4, hipHostMallocDefault), "pinned ids");
    hip_check(hipHostMalloc((void**)&e->markers_h, QUEUE * ml * 4, hipHostMallocDefault), "pinned markers");
    hip_check(hipHostMalloc((void**)&e->logits_h, QUEUE * ml * 4, hipHostMallocDefault), "pinned logits");
    e->mcap = QUEUE * ml;
    for (int i = 0; i < QUEUE; i++) {
        hip_check(hipEventCreate(&e->ev_start[i]), "hipEventCreate");
        hip_check(hipEventCreate(&e->ev_end[i]), "hipEventCreate");
    }

    // Scratch for the largest split-K / key-range partials any request up to max_length needs.
    size_t ws = 0, counters = 0;
    const int shapes[][3] = {{3 * (int)d, (int)d, EPI_LN}, {(int)d, (int)d, 0},
                             {2 * c.inter, (int)d, EPI_LN}, {(int)d, c.inter, 0},
                             {c.head_ff, (int)d, EPI_LN},   {(int)d, c.head_ff, 0}};
    for (int m = 1; m <= (int)n; m++) {
        for (auto& s : shapes) {
            const GemmConfig cfg = gemm_choose(m, s[0], s[1], e->cus, s[2]);
            ws = std::max(ws, gemm_ws_floats(m, s[0], cfg));
            counters = std::max(counters, gemm_counters(m, s[0], cfg));
        }
        const int ch = attention_chunks(m, (int)d, 0, e->cus);
        ws = std::max(ws, attention_ws_floats(m, (int)d, ch));
        counters = std::max(counters, attention_counters(m, (int)d));
    }
    // The per-layer weight table of the persistent kernel.
    for (const EncoderLayer& L : e->layout.layers) {
        LayerDesc ld{};
        ld.wqkv = e->h(L.wqkv), ld.wo = e->h(L.wo), ld.wi = e->h(L.wi), ld.wo_mlp = e->h(L.wo_mlp);
        ld.qkv_colsum = e->f(L.qkv_colsum), ld.wi_colsum = e->f(L.wi_colsum);
        ld.rope = e->f(L.global ? e->layout.rope_global : e->layout.rope_local);
        ld.window = L.global ? 0 : c.window;
        e->layers_h.push_back(ld);
    }
    e->layers_d = dalloc<LayerDesc>(e->layers_h.size(), "layer table");
    e->xa = dalloc<jh_half>(2 * (size_t)c.layers * n * d, "encoder activations");
    e->qa = dalloc<jh_half>((size_t)c.layers * n * 3 * d, "encoder activations");
    e->oa = dalloc<jh_half>((size_t)c.layers * n * d, "encoder activations");
    const size_t H = e->layout.head.size();
    e->hxa = dalloc<jh_half>((1 + 2 * H) * n * d, "head activations");
    e->hqa = dalloc<jh_half>(H * n * 3 * d, "head activations");
    e->hoa = dalloc<jh_half>(H * n * d, "head activations");
    e->hs = dalloc<jh_half>(n * d, "scorer activations");
    for (const HeadLayer& L : e->layout.head) {
        HeadDesc hd{};
        hd.in_proj = e->h(L.in_proj), hd.out_proj = e->h(L.out_proj);
        hd.linear1 = e->h(L.linear1), hd.linear2 = e->h(L.linear2);
        hd.in_proj_colsum = e->f(L.in_proj_colsum), hd.in_proj_b = e->f(L.in_proj_b);
        hd.out_proj_b = e->f(L.out_proj_b), hd.linear1_colsum = e->f(L.linear1_colsum);
        hd.linear1_b = e->f(L.linear1_b), hd.linear2_b = e->f(L.linear2_b);
        e->heads_h.push_back(hd);
    }
    e->heads_d = dalloc<HeadDesc>(std::max<size_t>(H, 1), "head table");
    if (H)
        hip_check(hipMemcpy(e->heads_d, e->heads_h.data(), H * sizeof(HeadDesc),
                            hipMemcpyHostToDevice), "head table");
    hip_check(hipMemcpy(e->layers_d, e->layers_h.data(), e->layers_h.size() * sizeof(LayerDesc),
                        hipMemcpyHostToDevice), "layer table");
    e->layer_kernel.init(e->cus, (int)prop.sharedMemPerBlock);
    if (!attention_prepare()) throw std::runtime_error("attention: cannot set the kernel's LDS size");
    ws = std::max(ws, e->layer_kernel.ws_floats((int)n, (int)d, c.inter, c.head_ff));
    counters = std::max(counters, e->layer_kernel.counters((int)n, (int)d, c.inter, c.head_ff));
    ws = std::max(ws, n * (d / 64));  // the score's partials: up to a marker a row
    counters = std::max<size_t>(counters, 1);
    e->scratch.ws = dalloc<float>(ws, "scratch");
    e->scratch.ws_floats = ws;
    counters = (counters + 31) / 32 * 32;  // the barrier's words start on a 128-byte line
    e->scratch.counters = dalloc<uint32_t>(counters + BAR_WORDS, "counters");
    e->scratch.n_counters = counters;
    hip_check(hipMemset(e->scratch.counters, 0, (counters + BAR_WORDS) * 4), "hipMemset");
    e->layer_kernel.bind(e->scratch.counters + counters);  // the grid barrier's counter
    hip_check(hipDeviceSynchronize(), "load");
    return e.release();
}

void check_request(const Engine& e, const Request& r, size_t i) {
    if (r.qtype > 2 || (int)r.qtype >= e.cfg.n_qtypes)
        throw std::runtime_error("sequence " + std::to_string(i) + ": no question type " +
                                 std::to_string(r.qtype));
    if (r.n == 0 || r.n > (size_t)e.max_length)
        throw std::runtime_error("sequence " + std::to_string(i) + ": " + std::to_string(r.n) +
                                 " tokens, not 1 to " + std::to_string(e.max_length));
    for (size_t j = 0; j < r.nm; j++)
        if (r.markers[j] >= r.n) throw std::runtime_error("a marker is past the sequence");
    for (size_t j = 0; j < r.n; j++)
        if (r.ids[j] >= (uint32_t)e.cfg.vocab)
            throw std::runtime_error("sequence " + std::to_string(i) + ": token id " +
                                     std::to_string(r.ids[j]) + " is past the vocabulary");
}

// src/engine.rs:170-196 `Engine::run`: chunks of QUEUE requests, queued back to back (copy in,
// start event, forward, end event, logits out), then one wait per chunk. Every request is
// checked before the first runs (src/capi.rs:150-170), so a bad one runs nothing.
void run_requests(Engine& e, const std::vector<Request>& reqs, bool fused, float* logits_out,
                  float* gpu_ms) {
    hip_check(hipSetDevice(e.device), "hipSetDevice");
    for (size_t i = 0; i < reqs.size(); i++) check_request(e, reqs[i], i);
    size_t out_at = 0;
    for (size_t c0 = 0; c0 < reqs.size(); c0 += QUEUE) {
        const size_t c1 = std::min(reqs.size(), c0 + QUEUE);
        size_t chunk_markers = 0;
        for (size_t i = c0; i < c1; i++) chunk_markers += reqs[i].nm;
        e.ensure_markers(chunk_markers);  // the stream is idle here
        for (size_t i = c0, m0 = 0; i < c1; m0 += reqs[i].nm, i++) {
            const Request& r = reqs[i];
            const size_t q = i - c0, slot = q * e.max_length;
            memcpy(e.ids_h + slot, r.ids, r.n * 4);
            if (r.nm) memcpy(e.markers_h + m0, r.markers, r.nm * 4);
            // The graph reads its request from gin (ids, then up to max_length markers) and
            // writes glogits; otherwise the request has its own ids slot and marker range.
            const bool graph = e.use_graphs && !fused && r.nm <= (size_t)e.max_length;
            uint32_t* ids_dst = graph ? e.gin : e.ids_d + slot;
            uint32_t* markers_dst = graph ? e.gin + e.max_length : e.markers_d + m0;
            float* logits_src = graph ? e.glogits : e.logits_d + m0;
            hipGraphExec_t ex = graph ? e.graph_for((int)r.n, (int)r.nm, (int)r.qtype) : nullptr;
            hip_check(hipMemcpyAsync(ids_dst, e.ids_h + slot, r.n * 4, hipMemcpyHostToDevice,
                                     e.stream), "ids");
            if (r.nm)
                hip_check(hipMemcpyAsync(markers_dst, e.markers_h + m0, r.nm * 4,
                                         hipMemcpyHostToDevice, e.stream), "markers");
            hip_check(hipEventRecord(e.ev_start[q], e.stream), "hipEventRecord");
            if (graph)
                hip_check(hipGraphLaunch(ex, e.stream), "hipGraphLaunch");
            else
                e.launch(ids_dst, (int)r.n, (int)r.qtype, markers_dst, (int)r.nm, logits_src, fused);
            hip_check(hipEventRecord(e.ev_end[q], e.stream), "hipEventRecord");
            if (r.nm)
                hip_check(hipMemcpyAsync(e.logits_h + m0, logits_src, r.nm * 4,
                                         hipMemcpyDeviceToHost, e.stream), "logits");
        }
        hip_check(hipStreamSynchronize(e.stream), "the forward pass");
        if (fused && e.layer_kernel.barrier_timed_out())
            throw std::runtime_error("layer: a grid barrier timed out (blocks not co-resident)");
        for (size_t i = c0, m0 = 0; i < c1; m0 += reqs[i].nm, i++) {
            const Request& r = reqs[i];
            const size_t q = i - c0;
            float ms = 0.0f;
            hip_check(hipEventElapsedTime(&ms, e.ev_start[q], e.ev_end[q]), "hipEventElapsedTime");
            for (size_t j = 0; j < r.nm; j++)
                if (!std::isfinite(e.logits_h[m0 + j]))
                    throw std::runtime_error("inference returned nonfinite logits");
            if (r.nm) memcpy(logits_out + out_at, e.logits_h + m0, r.nm * 4);
            out_at += r.nm;
            if (gpu_ms) gpu_ms[i] = ms;
        }
    }
}

// Multi-request throughput: the requests and outputs of run_requests, but consecutive requests
// are packed into sets of at most e.rows rows and each set runs as one forward pass over its
// concatenated rows: RoPE at each row's position in its request, attention (encoder and head)
// bounded to the row's request, norm_add with the row's question type, markers as row indices.
// Each request's gpu_ms is the time of the pass it ran in.
void run_batched(Engine& e, const std::vector<Request>& reqs, bool fused, float* logits_out,
                 float* gpu_ms) {
    hip_check(hipSetDevice(e.device), "hipSetDevice");
    for (size_t i = 0; i < reqs.size(); i++) check_request(e, reqs[i], i);
    size_t out_at = 0;
    for (size_t b0 = 0; b0 < reqs.size();) {
        size_t b1 = b0, rows = 0;  // every request fits alone: n <= max_length <= e.rows
        while (b1 < reqs.size() && rows + reqs[b1].n <= (size_t)e.rows) rows += reqs[b1++].n;
        const std::pair<int, size_t> nr = e.upload_batch(reqs.data() + b0, b1 - b0);
        const int n = nr.first;
        const size_t nm = nr.second;
        hip_check(hipEventRecord(e.ev_start[0], e.stream), "hipEventRecord");
        if (!fused || !e.launch_model(e.bids_d, n, 0, e.markers_d, (int)nm, e.logits_d, e.pos_d,
                                      e.seg_d, e.qt_d)) {
            embed_launch(e.bids_d, n, e.h(e.layout.tok_embeddings), e.cfg.vocab, e.cfg.d,
                         e.f(e.layout.emb_norm), e.cfg.norm_eps, e.x, e.stream);
            const jh_half* xf = e.x;
            if (fused)
                xf = e.launch_encoder_fused(0, e.cfg.layers, n, e.x, e.pos_d, e.seg_d);
            else
                for (int l = 0; l < e.cfg.layers; l++) e.launch_layer(l, n, e.pos_d, e.seg_d);
            e.launch_head(xf, n, 0, e.markers_d, (int)nm, e.logits_d, e.seg_d, e.qt_d);
        }
        hip_check(hipEventRecord(e.ev_end[0], e.stream), "hipEventRecord");
        if (nm)
            hip_check(hipMemcpyAsync(e.logits_h, e.logits_d, nm * 4, hipMemcpyDeviceToHost,
                                     e.stream), "logits");
        hip_check(hipStreamSynchronize(e.stream), "the forward pass");
        if (fused && e.layer_kernel.barrier_timed_out())
            throw std::runtime_error("layer: a grid barrier timed out (blocks not co-resident)");
        float ms = 0.0f;
        hip_check(hipEventElapsedTime(&ms, e.ev_start[0], e.ev_end[0]), "hipEventElapsedTime");
        for (size_t j = 0; j < nm; j++)
            if (!std::isfinite(e.logits_h[j]))
                throw std::runtime_error("inference returned nonfinite logits");
        if (nm) memcpy(logits_out + out_at, e.logits_h, nm * 4);
        out_at += nm;
        for (size_t i = b0; i < b1; i++)
            if (gpu_ms) gpu_ms[i] = ms;
        b0 = b1;
    }
}

// julia_cuda_run's arguments as requests (src/capi.rs:134-177); checks the pointers.
std::vector<Request> gather_requests(size_t b, const uint32_t* ids, const size_t* lens,
                                     const uint32_t* markers, const size_t* n_markers,
                                     const uint32_t* qtypes, const float* logits) {
    if (!ids || !lens || !n_markers || !qtypes) throw std::runtime_error("null argument");
    std::vector<Request> reqs(b);
    size_t at_id = 0, at_m = 0;
    for (size_t i = 0; i < b; i++) {
        reqs[i] = Request{ids + at_id, lens[i], markers ? markers + at_m : nullptr, n_markers[i],
                          qtypes[i]};
        if (n_markers[i] && !markers) throw std::runtime_error("null markers");
        at_id += lens[i];
        at_m += n_markers[i];
    }
    if (at_m && !logits) throw std::runtime_error("null logits");
    return reqs;
}

void report(char* err, size_t len, const std::string& msg) {
    if (!err || len == 0) return;
    const size_t n = std::min(msg.size(), len - 1);
    memcpy(err, msg.data(), n);
    err[n] = 0;
}

template <typename F>
int guarded(char* err, size_t len, F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& ex) {
        report(err, len, ex.what());
    } catch (...) {
        report(err, len, "julia-hip: unknown exception");
    }
    return -1;
}

// src/timing.rs:43-74: warm-up calls, then batches of back-to-back calls between two events,
// one wait at the end; min and median per call.
template <typename F>
void time_calls(F&& launch, int warmup, int batches, int per_batch, hipStream_t st,
                       float* min_us, float* median_us) {
    if (batches <= 0 || per_batch <= 0) throw std::runtime_error("time: no batches");
    for (int i = 0; i < warmup; i++) launch();
    std::vector<hipEvent_t> ev(2 * batches);
    for (auto& e : ev) hip_check(hipEventCreate(&e), "hipEventCreate");
    for (int b = 0; b < batches; b++) {
        hip_check(hipEventRecord(ev[2 * b], st), "hipEventRecord");
        for (int i = 0; i < per_batch; i++) launch();
        hip_check(hipEventRecord(ev[2 * b + 1], st), "hipEventRecord");
    }
    hip_check(hipStreamSynchronize(st), "time");
    std::vector<float> us(batches);
    for (int b = 0; b < batches; b++) {
        float ms = 0.0f;
        hip_check(hipEventElapsedTime(&ms, ev[2 * b], ev[2 * b + 1]), "hipEventElapsedTime");
        us[b] = ms * 1000.0f / per_batch;
    }
    for (auto& e : ev) hipEventDestroy(e);
    std::sort(us.begin(), us.end());
    if (min_us) *min_us = us[0];
    if (median_us) *median_us = us[us.size() / 2];
}

}  // namespace

struct julia_hip_scratch {
    Scratch s;
};

extern "C" {

// ---------------------------------------------------------------- Part 1: src/capi.rs
const char* julia_cuda_tier(void) { return "gfx950"; }

Engine* julia_cuda_load(const char* dir, size_t max_length, char* err, size_t err_len) {
    Engine* e = nullptr;
    guarded(err, err_len, [&] { e = load_engine(dir, max_length); });
    return e;
}

void julia_cuda_free(Engine* engine) { delete engine; }

void julia_cuda_device(const Engine* engine, char* buf, size_t len) {
    if (engine) report(buf, len, engine->name);
}

int julia_cuda_run(const Engine* engine, size_t b, const uint32_t* ids, const size_t* lens,
                   const uint32_t* markers, const size_t* n_markers, const uint32_t* qtypes,
                   int layer_fused, float* logits, float* gpu_ms, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!engine) throw std::runtime_error("no engine");
        if (b == 0) return;
        const std::vector<Request> reqs =
            gather_requests(b, ids, lens, markers, n_markers, qtypes, logits);
        run_requests(*const_cast<Engine*>(engine), reqs, layer_fused != 0, logits, gpu_ms);
    });
}

Engine* julia_hip_load(const char* dir, size_t max_length, size_t batch_rows, char* err,
                       size_t err_len) {
    Engine* e = nullptr;
    guarded(err, err_len, [&] { e = load_engine(dir, max_length, batch_rows); });
    return e;
}

int julia_hip_run_batched(const Engine* engine, size_t b, const uint32_t* ids, const size_t* lens,
                          const uint32_t* markers, const size_t* n_markers,
                          const uint32_t* qtypes, int layer_fused, float* logits, float* gpu_ms,
                          char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!engine) throw std::runtime_error("no engine");
        if (b == 0) return;
        const std::vector<Request> reqs =
            gather_requests(b, ids, lens, markers, n_markers, qtypes, logits);
        run_batched(*const_cast<Engine*>(engine), reqs, layer_fused != 0, logits, gpu_ms);
    });
}

// ---------------------------------------------------------------- Part 2: per-op surface
julia_hip_scratch* julia_hip_scratch_new(size_t ws_floats, size_t counters, char* err,
                                         size_t err_len) {
    julia_hip_scratch* s = nullptr;
    guarded(err, err_len, [&] {
        std::unique_ptr<julia_hip_scratch> p(new julia_hip_scratch());
        p->s.ws = dalloc<float>(ws_floats, "scratch");
        p->s.ws_floats = ws_floats;
        p->s.counters = dalloc<uint32_t>(counters, "counters");
        p->s.n_counters = counters;
        hip_check(hipMemset(p->s.counters, 0, std::max<size_t>(counters, 1) * 4), "hipMemset");
        hip_check(hipDeviceSynchronize(), "scratch");
        s = p.release();
    });
    return s;
}

void julia_hip_scratch_free(julia_hip_scratch* s) {
    if (!s) return;
    if (s->s.ws) hipFree(s->s.ws);
    if (s->s.counters) hipFree(s->s.counters);
    delete s;
}

static Gemm to_gemm(const julia_hip_gemm_args* g) {
    if (!g) throw std::runtime_error("gemm: no arguments");
    Gemm x{};
    x.epi = g->epi, x.a = (const jh_half*)g->a, x.w = (const jh_half*)g->w, x.c = (jh_half*)g->c;
    x.m = g->m, x.n = g->n, x.k = g->k, x.stats_in = g->stats_in, x.colsum = g->colsum;
    x.eps = g->eps, x.bias = g->bias, x.rope = g->rope, x.pos = g->positions;
    x.rope_rows = g->rope_rows, x.stats_out = g->stats_out;
    return x;
}

static Scratch scratch_of(const julia_hip_scratch* s) { return s ? s->s : Scratch{}; }

int julia_hip_gemm(const julia_hip_gemm_args* g, julia_hip_gemm_config cfg,
                   const julia_hip_scratch* s, void* stream, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        const Gemm x = to_gemm(g);
        GemmConfig c{cfg.bm, cfg.splits};
        if (c.bm == 0) c = gemm_choose(x.m, x.n, x.k, device_cus(), x.epi);
        gemm_launch(x, c, scratch_of(s), (hipStream_t)stream);
    });
}

int julia_hip_gemm_static(const julia_hip_gemm_args* g, julia_hip_gemm_config cfg, void* stream,
                          char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        const Gemm x = to_gemm(g);
        GemmConfig c{cfg.bm, cfg.splits};
        if (c.bm == 0) c = gemm_choose(x.m, x.n, x.k, device_cus(), x.epi);
        gemm_launch_static(x, c, (hipStream_t)stream);
    });
}

int julia_hip_attention(const void* qkv, void* o, int n, int d, int window, int chunks,
                        const julia_hip_scratch* s, void* stream, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        const int ch = chunks > 0 ? chunks : attention_chunks(n, d, window, device_cus());
        attention_launch((const jh_half*)qkv, (jh_half*)o, n, d, window, ch, scratch_of(s),
                         (hipStream_t)stream);
    });
}

int julia_hip_attention_seg(const void* qkv, void* o, int n, int d, int window,
                            const int32_t* seg, const julia_hip_scratch* s, void* stream, char* err,
                            size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!seg) throw std::runtime_error("attention: no sequence bounds");
        attention_launch((const jh_half*)qkv, (jh_half*)o, n, d, window, 1, scratch_of(s),
                         (hipStream_t)stream, seg);
    });
}

int julia_hip_embed(const uint32_t* ids, int n, const void* table, int vocab, int d,
                    const float* gamma, float eps, void* x, void* stream, char* err,
                    size_t err_len) {
    return guarded(err, err_len, [&] {
        embed_launch(ids, n, (const jh_half*)table, vocab, d, gamma, eps, (jh_half*)x,
                     (hipStream_t)stream);
    });
}

int julia_hip_norm_add(const void* x, int n, int d, const float* gamma, const float* add,
                       float eps, void* out, float* stats, void* stream, char* err,
                       size_t err_len) {
    return guarded(err, err_len, [&] {
        norm_add_launch((const jh_half*)x, n, d, gamma, add, eps, (jh_half*)out, stats,
                        (hipStream_t)stream);
    });
}

int julia_hip_score(const void* y, int n, int d, const void* w, float b, const uint32_t* markers,
                    int k, float* logits, void* stream, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        score_launch((const jh_half*)y, n, d, (const jh_half*)w, b, markers, k, logits,
                     (hipStream_t)stream);
    });
}

int julia_hip_time_gemm(const julia_hip_gemm_args* g, julia_hip_gemm_config cfg,
                        const julia_hip_scratch* s, int warmup, int batches, int per_batch,
                        float* min_us, float* median_us, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        const Gemm x = to_gemm(g);
        GemmConfig c{cfg.bm, cfg.splits};
        if (c.bm == 0) c = gemm_choose(x.m, x.n, x.k, device_cus(), x.epi);
        const Scratch sc = scratch_of(s);
        gemm_check(x, c, sc);
        hipStream_t st = nullptr;
        hip_check(hipStreamCreate(&st), "hipStreamCreate");
        try {
            time_calls([&] { gemm_launch(x, c, sc, st); }, warmup, batches, per_batch, st, min_us,
                       median_us);
        } catch (...) {
            hipStreamSynchronize(st);
            hipStreamDestroy(st);
            throw;
        }
        hipStreamDestroy(st);
    });
}

int julia_hip_time_attention(const void* qkv, void* o, int n, int d, int window, int chunks,
                             const julia_hip_scratch* s, int warmup, int batches, int per_batch,
                             float* min_us, float* median_us, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        const int ch = chunks > 0 ? chunks : attention_chunks(n, d, window, device_cus());
        const Scratch sc = scratch_of(s);
        hipStream_t st = nullptr;
        hip_check(hipStreamCreate(&st), "hipStreamCreate");
        try {
            time_calls([&] {
                attention_launch((const jh_half*)qkv, (jh_half*)o, n, d, window, ch, sc, st);
            }, warmup, batches, per_batch, st, min_us, median_us);
        } catch (...) {
            hipStreamSynchronize(st);
            hipStreamDestroy(st);
            throw;
        }
        hipStreamDestroy(st);
    });
}

int julia_hip_time_copy(size_t bytes, int warmup, int batches, int per_batch, float* min_us,
                        float* median_us, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        void *a = nullptr, *b = nullptr;
        hipStream_t st = nullptr;
        hip_check(hipMalloc(&a, bytes), "copy buffer");
        try {
            hip_check(hipMalloc(&b, bytes), "copy buffer");
            hip_check(hipMemset(a, 1, bytes), "hipMemset");
            hip_check(hipStreamCreate(&st), "hipStreamCreate");
            time_calls([&] { stream_copy_launch(b, a, bytes, st); }, warmup, batches, per_batch, st,
                       min_us, median_us);
        } catch (...) {
            if (st) hipStreamSynchronize(st), hipStreamDestroy(st);
            hipFree(a);
            if (b) hipFree(b);
            throw;
        }
        hipStreamDestroy(st);
        hipFree(a);
        hipFree(b);
    });
}

int julia_hip_copy(void* dst, const void* src, size_t bytes, int kind, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        const hipMemcpyKind k = kind == 1 ? hipMemcpyHostToDevice
                                : kind == 2 ? hipMemcpyDeviceToHost
                                : kind == 3 ? hipMemcpyDeviceToDevice
                                            : hipMemcpyDefault;
        hip_check(hipMemcpy(dst, src, bytes, k), "hipMemcpy");
    });
}

int julia_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

void* julia_hip_device_alloc(size_t bytes, char* err, size_t err_len) {
    void* p = nullptr;
    guarded(err, err_len, [&] { p = dalloc<uint8_t>(bytes, "julia_hip_device_alloc"); });
    return p;
}

void julia_hip_device_free(void* p) {
    if (p) hipFree(p);
}

int julia_hip_device_sync(char* err, size_t err_len) {
    return guarded(err, err_len, [&] { hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize"); });
}

// ---------------------------------------------------------------- Part 3: host-side logic
void julia_hip_prep_fold_layernorm(const float* w, const float* gamma, int out, int k,
                                   uint16_t* w16, float* colsum) {
    fold_layernorm(w, gamma, out, k, w16, colsum);
}

void julia_hip_prep_fold_layernorm_bias(const float* w, const float* gamma, const float* beta,
                                        const float* b, int out, int k, uint16_t* w16,
                                        float* colsum, float* bias) {
    fold_layernorm_bias(w, gamma, beta, b, out, k, w16, colsum, bias);
}

void julia_hip_prep_geglu_rows(int inter, int32_t* src) { geglu_rows(inter, src); }

void julia_hip_prep_pack_frag(const uint16_t* w, int n, int k, uint16_t* out) {
    if (n > 0 && k > 0 && n % 64 == 0 && k % 32 == 0) pack_frag(w, n, k, out);
}

void julia_hip_prep_unpack_frag(const uint16_t* packed, int n, int k, uint16_t* w) {
    if (n > 0 && k > 0 && n % 64 == 0 && k % 32 == 0) unpack_frag(packed, n, k, w);
}

void julia_hip_prep_rope_table(float theta, int npos, float* table) {
    rope_table(theta, npos, table);
}

void julia_hip_synth(uint64_t seed, uint32_t id, uint64_t start, uint64_t count, double mean,
                     double std, float* out) {
    synth(seed, id, start, count, mean, std, out);
}

void julia_hip_round_f16(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f32_to_f16(in[i]);
}

julia_hip_gemm_config julia_hip_gemm_choose(int m, int n, int k, int cus, int epi) {
    const GemmConfig c = gemm_choose(m, n, k, cus, epi);
    return julia_hip_gemm_config{c.bm, c.splits};
}

int julia_hip_gemm_check(const julia_hip_gemm_args* g, julia_hip_gemm_config cfg,
                         size_t ws_floats, size_t counters, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        // Stand-in scratch of the stated sizes: the check reads only the sizes and non-null.
        static float ws_probe;
        static uint32_t counter_probe;
        const Scratch s{ws_floats ? &ws_probe : nullptr, ws_floats,
                        counters ? &counter_probe : nullptr, counters};
        gemm_check(to_gemm(g), GemmConfig{cfg.bm, cfg.splits}, s);
    });
}

// src/forward.rs:771-806 `phase_cost`, the 2080 Ti latency model: a task costs 5 us (10 with
// 64-row tiles) plus 0.35 us per 32-deep K step; c tasks at once on an SM take 1 + 0.2 (c - 1)
// times one; split tiles add 0.4 us per split and 32 rows; the busiest SM has ceil(tasks / SMs).
static double phase_cost_2080ti(int n, int cols, int k, int bm, int z, int sms, int per_sm) {
    const long tasks = (long)(cols / 64) * ((n + bm - 1) / bm) * z;
    const double steps = (double)(k / 32) / z;
    const double task = (bm == 32 ? 5.0 : 10.0) + 0.35 * steps;
    auto at_once = [](long c) { return 1.0 + 0.2 * ((double)c - 1.0); };
    const long on_sm = (tasks + sms - 1) / sms;
    const long rounds = on_sm / per_sm, rest = on_sm % per_sm;
    double t = (double)rounds * at_once(per_sm) * task;
    if (rest > 0) t += at_once(rest) * task;
    if (z > 1) t += 0.4 * z * (bm / 32);
    return t;
}

// src/forward.rs:759-769 `gemm_plan`: the (bm in {32, 64}, z in 1-4, at least 3 K steps a split)
// with the lowest phase_cost; ties keep the first.
void julia_hip_gemm_plan_2080ti(int n, int cols, int k, int sms, int per_sm, int* bm, int* splits) {
    double best = 1e300;
    int bb = 32, bz = 1;
    for (int b : {32, 64})
        for (int z = 1; z <= 4; z++) {
            if (k / 32 / z < 3) continue;
            const double c = phase_cost_2080ti(n, cols, k, b, z, sms, per_sm);
            if (c < best) best = c, bb = b, bz = z;
        }
    if (bm) *bm = bb;
    if (splits) *splits = bz;
}

// src/gemm.rs:153-172: tile height by m, and 4 splits only while there are at most half as many
// tiles as SMs (each split at least 3 K steps).
julia_hip_gemm_config julia_hip_gemm_choose_2080ti(int m, int n, int k, int sms) {
    const int bm = m <= 200 ? 32 : (m <= 400 ? 64 : 128);
    const long tiles = (long)(n / 64) * ((m + bm - 1) / bm);
    int z = 2 * tiles > sms ? 1 : 4;
    z = std::min(z, std::max(k / 32 / 3, 1));
    return julia_hip_gemm_config{bm, z};
}

int julia_hip_checkpoint_config(const char* dir, julia_hip_engine_info* out, char* err,
                                size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!dir || !out) throw std::runtime_error("no directory or output");
        const Checkpoint ck(dir);
        const ModelConfig& c = ck.config();
        *out = julia_hip_engine_info{};
        out->d = c.d, out->layers = c.layers, out->inter = c.inter, out->vocab = c.vocab;
        out->head_layers = c.head_layers, out->head_ff = c.head_ff, out->n_qtypes = c.n_qtypes;
        out->window = c.window, out->global_every = c.global_every;
        out->max_positions = c.max_positions;
        out->norm_eps = c.norm_eps, out->head_eps = c.head_eps;
    });
}

int julia_hip_model_kernel(const Engine* e, size_t rows) {
    if (!e || rows == 0 || rows > (size_t)e->rows) return 0;
    const int n = (int)rows;
    const LayerPlan plan = e->layer_kernel.default_plan(n, e->cfg.d, e->cfg.inter);
    return e->layer_kernel.model_fits(plan, n, e->cfg.d, e->cfg.head_ff) ? 1 : 0;
}

int julia_hip_engine_info_get(const Engine* e, julia_hip_engine_info* out) {
    if (!e || !out) return -1;
    const ModelConfig& c = e->cfg;
    out->d = c.d, out->layers = c.layers, out->inter = c.inter, out->vocab = c.vocab;
    out->head_layers = c.head_layers, out->head_ff = c.head_ff, out->n_qtypes = c.n_qtypes;
    out->window = c.window, out->global_every = c.global_every;
    out->max_positions = c.max_positions, out->max_length = e->max_length, out->cus = e->cus;
    out->norm_eps = c.norm_eps, out->head_eps = c.head_eps, out->seed = c.seed;
    out->weight_bytes_f16 = e->n16 * 2, out->weight_bytes_f32 = e->n32 * 4;
    out->coop_refused = e->layer_kernel.refused();
    return 0;
}

const void* julia_hip_engine_tensor(const Engine* e, const char* name, int index, size_t* bytes) {
    if (!e || !name) return nullptr;
    const std::string nm = name;
    const Layout& L = e->layout;
    const Span* s16 = nullptr;
    const Span* s32 = nullptr;
    const bool lok = index >= 0 && index < (int)L.layers.size();
    const bool hok = index >= 0 && index < (int)L.head.size();
    if (nm == "tok_emb") s16 = &L.tok_embeddings;
    else if (nm == "emb_norm") s32 = &L.emb_norm;
    else if (nm == "rope_global") s32 = &L.rope_global;
    else if (nm == "rope_local") s32 = &L.rope_local;
    else if (nm == "final_norm") s32 = &L.final_norm;
    else if (nm == "type_emb") s32 = &L.type_emb;
    else if (nm == "wqkv" && lok) s16 = &L.layers[index].wqkv;
    else if (nm == "qkv_colsum" && lok) s32 = &L.layers[index].qkv_colsum;
    else if (nm == "wo" && lok) s16 = &L.layers[index].wo;
    else if (nm == "wi" && lok) s16 = &L.layers[index].wi;
    else if (nm == "wi_colsum" && lok) s32 = &L.layers[index].wi_colsum;
    else if (nm == "wo_mlp" && lok) s16 = &L.layers[index].wo_mlp;
    else if (nm == "in_proj" && hok) s16 = &L.head[index].in_proj;
    else if (nm == "in_proj_colsum" && hok) s32 = &L.head[index].in_proj_colsum;
    else if (nm == "in_proj_b" && hok) s32 = &L.head[index].in_proj_b;
    else if (nm == "out_proj" && hok) s16 = &L.head[index].out_proj;
    else if (nm == "out_proj_b" && hok) s32 = &L.head[index].out_proj_b;
    else if (nm == "linear1" && hok) s16 = &L.head[index].linear1;
    else if (nm == "linear1_colsum" && hok) s32 = &L.head[index].linear1_colsum;
    else if (nm == "linear1_b" && hok) s32 = &L.head[index].linear1_b;
    else if (nm == "linear2" && hok) s16 = &L.head[index].linear2;
    else if (nm == "linear2_b" && hok) s32 = &L.head[index].linear2_b;
    else if (nm == "lin1") s16 = &L.scorer.lin1;
    else if (nm == "lin1_colsum") s32 = &L.scorer.lin1_colsum;
    else if (nm == "lin1_b") s32 = &L.scorer.lin1_b;
    else if (nm == "lin2") s16 = &L.scorer.lin2;
    if (s16 && s16->present) {
        if (bytes) *bytes = s16->len * 2;
        return e->w16 + s16->start;
    }
    if (s32 && s32->present) {
        if (bytes) *bytes = s32->len * 4;
        return e->w32 + s32->start;
    }
    if (nm == "lin2_b") {
        if (bytes) *bytes = 0;
        return nullptr;
    }
    return nullptr;
}

int julia_hip_time_encoder_step(const Engine* ce, int step, int m, int bm, int splits, int warmup,
                                int batches, int per_batch, float* min_us, float* median_us,
                                char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!ce) throw std::runtime_error("no engine");
        Engine& e = *const_cast<Engine*>(ce);
        hip_check(hipSetDevice(e.device), "hipSetDevice");
        if (m <= 0 || m > e.max_length) throw std::runtime_error("time: m out of range");
        if (step < 0 || step > 8) throw std::runtime_error("time: no step " + std::to_string(step));
        const int d = e.cfg.d, I = e.cfg.inter, L = e.cfg.layers;
        // A real residual stream and statistics to run on: embed ids 0..m-1 and one layer.
        std::vector<uint32_t> ids(m);
        for (int i = 0; i < m; i++) ids[i] = (uint32_t)(i * 7919 % e.cfg.vocab);
        hip_check(hipMemcpy(e.ids_d, ids.data(), m * 4, hipMemcpyHostToDevice), "ids");
        embed_launch(e.ids_d, m, e.h(e.layout.tok_embeddings), e.cfg.vocab, d, e.f(e.layout.emb_norm),
                     e.cfg.norm_eps, e.x, e.stream);
        e.launch_layer(0, m);
        hip_check(hipStreamSynchronize(e.stream), "time");
        int l = 0;
        auto gemm_cfg = [&](int n, int k, int epi) {
            return bm > 0 ? GemmConfig{bm, splits} : gemm_choose(m, n, k, e.cus, epi);
        };
        // Rotate through the layers' weights, as the reference's --time does (src/main.rs:
        // 307-312), so the weights are not the last call's, still in L2. Layer 0 has no
        // attention LayerNorm: the qkv step uses layers 1.. when there are more than one.
        auto launch = [&] {
            const int lo = (step == 0 && L > 1) ? 1 : 0;
            l = lo + (l + 1 - lo) % (L - lo);
            const EncoderLayer& Ly = e.layout.layers[l];
            const float* rope = e.f(Ly.global ? e.layout.rope_global : e.layout.rope_local);
            // The row kernels: embed of the m ids, the final norm + type embedding of the
            // residual stream, the score of every row (identity markers).
            if (step == 6) {
                embed_launch(e.ids_d, m, e.h(e.layout.tok_embeddings), e.cfg.vocab, d,
                             e.f(e.layout.emb_norm), e.cfg.norm_eps, e.hx, e.stream);
                return;
            }
            if (step == 7) {
                norm_add_launch(e.x, m, d, e.f(e.layout.final_norm), e.f(e.layout.type_emb),
                                e.cfg.norm_eps, e.hx, e.stats_a, e.stream);
                return;
            }
            if (step == 8) {
                score_launch(e.x, m, d, e.h(e.layout.scorer.lin2), e.layout.scorer.lin2_b, nullptr,
                             m, e.logits_d, e.stream);
                return;
            }
            Gemm g{};
            g.m = m, g.rope_rows = e.cfg.max_positions, g.eps = e.cfg.norm_eps;
            switch (step) {
                case 0:
                    g.epi = Ly.qkv_colsum.present ? EPI_K_LNROPE : EPI_K_ROPE, g.a = e.x;
                    g.w = e.h(Ly.wqkv), g.c = e.qkv, g.n = 3 * d, g.k = d, g.rope = rope;
                    if (Ly.qkv_colsum.present) g.stats_in = e.stats_b, g.colsum = e.f(Ly.qkv_colsum);
                    break;
                case 2:
                    g.epi = EPI_K_RESSTATS, g.a = e.o, g.w = e.h(Ly.wo), g.c = e.hx, g.n = d, g.k = d;
                    g.stats_out = e.stats_a;
                    break;
                case 3:
                    g.epi = EPI_K_LNGEGLU, g.a = e.x, g.w = e.h(Ly.wi), g.c = e.mid, g.n = 2 * I;
                    g.k = d, g.stats_in = e.stats_a, g.colsum = e.f(Ly.wi_colsum);
                    break;
                case 4:
                    g.epi = EPI_K_RESSTATS, g.a = e.mid, g.w = e.h(Ly.wo_mlp), g.c = e.hx, g.n = d;
                    g.k = I, g.stats_out = e.stats_b;
                    break;
                default: {
                    const int window = (step == 1 && !Ly.global) ? e.cfg.window : 0;
                    attention_launch(e.qkv, e.o, m, d, window,
                                     attention_chunks(m, d, window, e.cus), e.scratch, e.stream);
                    return;
                }
            }
            gemm_launch(g, gemm_cfg(g.n, g.k, g.epi), e.scratch, e.stream);
        };
        time_calls(launch, warmup, batches, per_batch, e.stream, min_us, median_us);
    });
}

int julia_hip_profile_layer(const Engine* ce, int n, int layer, const int* plan, uint64_t* stamps,
                            int max_rows, int* grid, int* plan_out, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!ce) throw std::runtime_error("no engine");
        Engine& e = *const_cast<Engine*>(ce);
        hip_check(hipSetDevice(e.device), "hipSetDevice");
        if (n <= 0 || n > e.rows) throw std::runtime_error("profile: n out of range");
        if (layer < -1 || layer >= e.cfg.layers) throw std::runtime_error("profile: no such layer");
        std::vector<uint32_t> ids(n);
        for (int i = 0; i < n; i++) ids[i] = (uint32_t)(i * 7919 % e.cfg.vocab);
        uint32_t* ids_d = n > e.max_length ? e.bids_d : e.ids_d;  // (one sequence of n rows)
        hip_check(hipMemcpy(ids_d, ids.data(), n * 4, hipMemcpyHostToDevice), "ids");
        embed_launch(ids_d, n, e.h(e.layout.tok_embeddings), e.cfg.vocab, e.cfg.d,
                     e.f(e.layout.emb_norm), e.cfg.norm_eps, e.x, e.stream);
        // One layer (after the ones before it, per step) or, with layer -1, the whole encoder.
        const int first = layer < 0 ? 0 : layer, count = layer < 0 ? e.cfg.layers : 1;
        for (int l = 0; l < first; l++) e.launch_layer(l, n);
        const LayerArgs a = e.layer_args(first, count, n, e.x);
        LayerPlan p = e.layer_kernel.default_plan(n, e.cfg.d, e.cfg.inter);
        if (plan) {
            for (int g = 0; g < 4; g++) p.bm[g] = plan[g], p.splits[g] = plan[4 + g];
            p.kv[0] = plan[8], p.kv[1] = plan[9];
        }
        const int gb = e.layer_kernel.grid(a, p);
        if (grid) *grid = gb;
        if (plan_out) {
            for (int g = 0; g < 4; g++) plan_out[g] = p.bm[g], plan_out[4 + g] = p.splits[g];
            plan_out[8] = p.kv[0], plan_out[9] = p.kv[1];
        }
        const size_t rows = (size_t)gb * count;
        if (rows > (size_t)std::max(max_rows, 0))
            throw std::runtime_error("profile: the stamps buffer is too small");
        uint64_t* prof = dalloc<uint64_t>(rows * PROF_WORDS, "profile");
        try {
            hip_check(hipMemset(prof, 0, rows * PROF_WORDS * 8), "hipMemset");
            if (!e.layer_kernel.launch(a, p, e.scratch, e.stream, 0x1f, prof))
                throw std::runtime_error("profile: the runtime refused the cooperative launch "
                                         "(another process holds its resource)");
            hip_check(hipStreamSynchronize(e.stream), "profile");
            if (e.layer_kernel.barrier_timed_out())
                throw std::runtime_error("layer: a grid barrier timed out");
            hip_check(hipMemcpy(stamps, prof, rows * PROF_WORDS * 8, hipMemcpyDeviceToHost),
                      "profile");
        } catch (...) {
            hipFree(prof);
            throw;
        }
        hipFree(prof);
    });
}

int julia_hip_encode_batch(const Engine* ce, size_t b, const uint32_t* ids, const size_t* lens,
                           int layer_fused, uint16_t* x_out, float* gpu_ms, char* err,
                           size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!ce) throw std::runtime_error("no engine");
        Engine& e = *const_cast<Engine*>(ce);
        hip_check(hipSetDevice(e.device), "hipSetDevice");
        const int n = e.prepare_batch(b, ids, lens);
        const size_t rows = (size_t)n;
        hip_check(hipEventRecord(e.ev_start[0], e.stream), "hipEventRecord");
        embed_launch(e.bids_d, n, e.h(e.layout.tok_embeddings), e.cfg.vocab, e.cfg.d,
                     e.f(e.layout.emb_norm), e.cfg.norm_eps, e.x, e.stream);
        const jh_half* xf = e.x;
        if (layer_fused)
            xf = e.launch_encoder_fused(0, e.cfg.layers, n, e.x, e.pos_d, e.seg_d);
        else
            for (int l = 0; l < e.cfg.layers; l++) e.launch_layer(l, n, e.pos_d, e.seg_d);
        hip_check(hipEventRecord(e.ev_end[0], e.stream), "hipEventRecord");
        hip_check(hipStreamSynchronize(e.stream), "the batched encoder");
        if (layer_fused && e.layer_kernel.barrier_timed_out())
            throw std::runtime_error("layer: a grid barrier timed out (blocks not co-resident)");
        if (gpu_ms) hip_check(hipEventElapsedTime(gpu_ms, e.ev_start[0], e.ev_end[0]), "hipEventElapsedTime");
        if (x_out) hip_check(hipMemcpy(x_out, xf, rows * e.cfg.d * 2, hipMemcpyDeviceToHost), "x");
    });
}

int julia_hip_encode_batch_phases(const Engine* ce, size_t b, const uint32_t* ids,
                                  const size_t* lens, float* phase_ms, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!ce) throw std::runtime_error("no engine");
        if (!phase_ms) throw std::runtime_error("no output");
        Engine& e = *const_cast<Engine*>(ce);
        hip_check(hipSetDevice(e.device), "hipSetDevice");
        const int n = e.prepare_batch(b, ids, lens);
        embed_launch(e.bids_d, n, e.h(e.layout.tok_embeddings), e.cfg.vocab, e.cfg.d,
                     e.f(e.layout.emb_norm), e.cfg.norm_eps, e.x, e.stream);
        for (int i = 0; i < 5; i++) phase_ms[i] = 0.0f;
        for (int l = 0; l < e.cfg.layers; l++) {
            e.launch_layer(l, n, e.pos_d, e.seg_d, e.ev_start);
            hip_check(hipStreamSynchronize(e.stream), "the batched encoder");
            for (int i = 0; i < 5; i++) {
                float ms = 0.0f;
                hip_check(hipEventElapsedTime(&ms, e.ev_start[i], e.ev_start[i + 1]), "hipEventElapsedTime");
                phase_ms[i] += ms;
            }
        }
    });
}

int julia_hip_run_trace(const Engine* ce, const uint32_t* ids, size_t n, const uint32_t* markers,
                        size_t n_markers, uint32_t qtype, int layer_fused, float* logits,
                        uint16_t* x_trace, uint16_t* head_x, char* err, size_t err_len) {
    return guarded(err, err_len, [&] {
        if (!ce) throw std::runtime_error("no engine");
        Engine& e = *const_cast<Engine*>(ce);
        hip_check(hipSetDevice(e.device), "hipSetDevice");
        const Request r{ids, n, markers, n_markers, qtype};
        check_request(e, r, 0);
        hip_check(hipMemcpy(e.ids_d, ids, n * 4, hipMemcpyHostToDevice), "ids");
        if (n_markers) hip_check(hipMemcpy(e.markers_d, markers, n_markers * 4, hipMemcpyHostToDevice), "markers");
        const size_t d = e.cfg.d;
        embed_launch(e.ids_d, (int)n, e.h(e.layout.tok_embeddings), e.cfg.vocab, e.cfg.d,
                     e.f(e.layout.emb_norm), e.cfg.norm_eps, e.x, e.stream);
        const jh_half* xl = e.x;  // the residual stream after each layer
        for (int l = 0; l < e.cfg.layers; l++) {
            if (layer_fused)
                xl = e.launch_encoder_fused(l, 1, (int)n, xl);
            else
                e.launch_layer(l, (int)n);
            if (x_trace) {
                hip_check(hipMemcpyAsync(x_trace + (size_t)l * n * d, xl, n * d * 2,
                                         hipMemcpyDeviceToHost, e.stream), "trace");
                hip_check(hipStreamSynchronize(e.stream), "trace");
            }
        }
        e.launch_head(xl, (int)n, (int)qtype, e.markers_d, (int)n_markers, e.logits_d, nullptr,
                      nullptr, head_x != nullptr);
        hip_check(hipStreamSynchronize(e.stream), "forward");
        if (layer_fused && e.layer_kernel.barrier_timed_out())
            throw std::runtime_error("layer: a grid barrier timed out (blocks not co-resident)");
        if (head_x) hip_check(hipMemcpy(head_x, e.hx, n * d * 2, hipMemcpyDeviceToHost), "head_x");
        if (n_markers) hip_check(hipMemcpy(logits, e.logits_d, n_markers * 4, hipMemcpyDeviceToHost), "logits");
    });
}

}  // extern "C"
