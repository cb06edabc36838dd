// The serve loop's host-side pieces behind the C ABI (host only, no device): the answer to a
// question from its marker logits, and the latency summary the serve loop reports.
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/julia_hip.h"

namespace {

void put(char* err, size_t len, const std::string& msg) {
    if (!err || len == 0) return;
    const size_t n = std::min(msg.size(), len - 1);
    memcpy(err, msg.data(), n);
    err[n] = 0;
}

}  // namespace

extern "C" {

// julia-rs `head::answer`, as the reference's own baseline tool states it for results that
// tools/score.py compares with the engine's (tools/torch_baseline.py:214-226): the options'
// probabilities are the softmax of their logits (in f64, shifted by the largest); a choice
// question answers the most probable option (the first of equal ones), a score question the
// expected option index sum_i i p_i, a noul question p[1] (the "true" option).
int julia_hip_answer(uint32_t qtype, const float* logits, size_t n, double* probabilities,
                     double* value, char* err, size_t err_len) {
    try {
        if (!logits || !probabilities || !value) throw std::runtime_error("null argument");
        if (qtype > 2) throw std::runtime_error("no question type " + std::to_string(qtype));
        if (n == 0) throw std::runtime_error("no options");
        if (qtype == 2 && n < 2) throw std::runtime_error("a noul question has two options");
        double mx = -INFINITY;
        for (size_t i = 0; i < n; i++) {
            if (!std::isfinite(logits[i])) throw std::runtime_error("nonfinite logit");
            mx = std::max(mx, (double)logits[i]);
        }
        double sum = 0.0;
        for (size_t i = 0; i < n; i++) sum += (probabilities[i] = exp((double)logits[i] - mx));
        for (size_t i = 0; i < n; i++) probabilities[i] /= sum;
        if (qtype == 0) {
            size_t best = 0;
            for (size_t i = 1; i < n; i++)
                if (probabilities[i] > probabilities[best]) best = i;
            *value = (double)best;
        } else if (qtype == 1) {
            double s = 0.0;
            for (size_t i = 0; i < n; i++) s += (double)i * probabilities[i];
            *value = s;
        } else {
            *value = probabilities[1];
        }
        return 0;
    } catch (const std::exception& ex) {
        put(err, err_len, ex.what());
        return -1;
    }
}

// src/serve.rs:78-115 `report`'s figures over n values: mean, then the values at index
// round((n - 1) p) of the sorted values for p = 0.5, 0.9, 0.99 and 1 (the maximum).
int julia_hip_latency_summary(const double* v, size_t n, double* out) {
    if (!v || !out || n == 0) return -1;
    std::vector<double> s(v, v + n);
    std::sort(s.begin(), s.end());
    double sum = 0.0;
    for (double x : s) sum += x;
    out[0] = sum / (double)n;
    const double ps[4] = {0.5, 0.9, 0.99, 1.0};
    for (int i = 0; i < 4; i++) out[1 + i] = s[(size_t)llround((double)(n - 1) * ps[i])];
    return 0;
}

}  // extern "C"
