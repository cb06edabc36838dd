// julia-serve: requests from stdin, results to stdout, one JSON object per line (the reference's
// serve loop, src/serve.rs:25-75), through the drop-in C ABI alone (julia_cuda_load /
// julia_cuda_run, one request at a time), with the latency report on stderr at the end
// (src/serve.rs:78-115).
//
//   julia-serve MODEL [--max-length N] [--head-length N] [--layer-fused] < requests.jsonl
//
// MODEL is a checkpoint directory or "synthetic[:key=value,...]". This build has no tokenizer
// (the reference tokenizes with julia-rs, which is not part of it): a request carries its tokens,
//   {"ids": [..], "markers": [..], "type": "choice" | "score" | "noul", "truncated": false}
// (markers: the row of each option's marker token; truncated is passed through). --head-length
// belongs to tokenization and is accepted and unused. A result is
//   {"logits": [..], "probabilities": [..], "truncated": .., "choice" | "score" | "noul": ..}
// as the reference writes it.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <iostream>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/julia_hip.h"

namespace {

// A JSON value: the subset a request line needs (objects, arrays, numbers, strings, booleans,
// null), parsed by recursive descent.
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;
};

struct Parser {
    const char* p;
    const char* end;

    [[noreturn]] void fail(const char* what) { throw std::runtime_error(std::string("json: ") + what); }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char* s) {
        const size_t n = strlen(s);
        if ((size_t)(end - p) >= n && memcmp(p, s, n) == 0) return p += n, true;
        return false;
    }
    std::string string() {
        if (*p != '"') fail("expected a string");
        p++;
        std::string out;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end) fail("bad escape");
                c = *p++;
                switch (c) {
                    case 'n': out += '\n'; break;
                    case 't': out += '\t'; break;
                    case 'r': out += '\r'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'u':  // kept as written: keys and values here are ASCII
                        if (end - p < 4) fail("bad \\u escape");
                        out += "\\u", out.append(p, 4), p += 4;
                        break;
                    default: out += c;
                }
            } else {
                out += c;
            }
        }
        if (p >= end) fail("unterminated string");
        p++;
        return out;
    }
    Json value(int depth = 0) {
        if (depth > 64) fail("nested too deeply");
        ws();
        if (p >= end) fail("unexpected end");
        Json v;
        if (*p == '{') {
            v.kind = Json::Obj, p++, ws();
            if (p < end && *p == '}') return p++, v;
            for (;;) {
                ws();
                std::string k = string();
                ws();
                if (p >= end || *p != ':') fail("expected ':'");
                p++;
                v.obj[k] = value(depth + 1);
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == '}') { p++; break; }
                fail("expected ',' or '}'");
            }
        } else if (*p == '[') {
            v.kind = Json::Arr, p++, ws();
            if (p < end && *p == ']') return p++, v;
            for (;;) {
                v.arr.push_back(value(depth + 1));
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == ']') { p++; break; }
                fail("expected ',' or ']'");
            }
        } else if (*p == '"') {
            v.kind = Json::Str, v.str = string();
        } else if (lit("true")) {
            v.kind = Json::Bool, v.b = true;
        } else if (lit("false")) {
            v.kind = Json::Bool, v.b = false;
        } else if (lit("null")) {
            v.kind = Json::Null;
        } else {
            char* e = nullptr;
            v.kind = Json::Num, v.num = strtod(p, &e);
            if (e == p) fail("unexpected character");
            p = e;
        }
        return v;
    }
};

Json parse(const std::string& line) {
    Parser ps{line.data(), line.data() + line.size()};
    Json v = ps.value();
    ps.ws();
    if (ps.p != ps.end) ps.fail("trailing characters");
    return v;
}

std::vector<uint32_t> u32_array(const Json& o, const char* key) {
    auto it = o.obj.find(key);
    if (it == o.obj.end() || it->second.kind != Json::Arr)
        throw std::runtime_error(std::string("no \"") + key + "\" array");
    std::vector<uint32_t> out;
    for (const Json& x : it->second.arr) {
        if (x.kind != Json::Num || x.num < 0 || x.num > 4294967295.0 || x.num != (double)(uint32_t)x.num)
            throw std::runtime_error(std::string("\"") + key + "\" holds a value that is not a u32");
        out.push_back((uint32_t)x.num);
    }
    return out;
}

const char* kTypes[3] = {"choice", "score", "noul"};

uint32_t qtype_of(const Json& o) {
    auto it = o.obj.find("type");
    if (it == o.obj.end()) return 0;  // julia-rs's default question type
    if (it->second.kind != Json::Str) throw std::runtime_error("\"type\" is not a string");
    for (uint32_t t = 0; t < 3; t++)
        if (it->second.str == kTypes[t]) return t;
    throw std::runtime_error("no question type \"" + it->second.str + "\"");
}

void put_floats(std::string& s, const char* key, const float* v, size_t n) {
    s += '"', s += key, s += "\":[";
    char buf[32];
    for (size_t i = 0; i < n; i++) {
        snprintf(buf, sizeof buf, "%s%.9g", i ? "," : "", (double)v[i]);
        s += buf;
    }
    s += ']';
}

void put_doubles(std::string& s, const char* key, const double* v, size_t n) {
    s += '"', s += key, s += "\":[";
    char buf[40];
    for (size_t i = 0; i < n; i++) {
        snprintf(buf, sizeof buf, "%s%.17g", i ? "," : "", v[i]);
        s += buf;
    }
    s += ']';
}

std::string pct(const std::vector<double>& v) {
    double o[5];
    julia_hip_latency_summary(v.data(), v.size(), o);
    char buf[160];
    snprintf(buf, sizeof buf, "mean %.3f, p50 %.3f, p90 %.3f, p99 %.3f, max %.3f ms", o[0], o[1],
             o[2], o[3], o[4]);
    return buf;
}

// src/serve.rs:78-115: over the requests after the first (which also builds the graphs).
void report(const std::vector<size_t>& tokens, const std::vector<double>& wall,
            const std::vector<double>& gpu) {
    if (tokens.empty()) {
        fprintf(stderr, "no requests\n");
        return;
    }
    size_t sum = 0, lo = tokens[0], hi = tokens[0];
    for (size_t t : tokens) sum += t, lo = std::min(lo, t), hi = std::max(hi, t);
    fprintf(stderr,
            "%zu requests, %zu tokens on average (%zu-%zu); the first took %.1f ms (wall, "
            "building its graph)\n",
            tokens.size(), sum / tokens.size(), lo, hi, wall[0]);
    if (tokens.size() < 2) return;
    const std::vector<double> w(wall.begin() + 1, wall.end()), g(gpu.begin() + 1, gpu.end());
    fprintf(stderr, "  per request, wall (parse, upload, run, download): %s\n", pct(w).c_str());
    fprintf(stderr, "  per request, GPU (embed to logits):                %s\n", pct(g).c_str());
}

const char* kUsage =
    "usage: julia-serve MODEL [--max-length N] [--head-length N] [--layer-fused] < requests.jsonl\n"
    "  MODEL: a checkpoint directory or synthetic[:key=value,...]. One request per line,\n"
    "  {\"ids\": [..], \"markers\": [..], \"type\": \"choice\"|\"score\"|\"noul\"}; one result per\n"
    "  line on stdout; the latency report on stderr.\n";

int serve(int argc, char** argv) {
    if (argc < 2 || argv[1][0] == '-') {
        fputs(kUsage, stderr);
        return 2;
    }
    const char* model = argv[1];
    size_t max_length = 0;
    bool fused = false;
    for (int i = 2; i < argc; i++) {
        const std::string f = argv[i];
        if ((f == "--max-length" || f == "--head-length") && i + 1 < argc) {
            char* e = nullptr;
            const unsigned long long v = strtoull(argv[++i], &e, 10);
            if (!*argv[i] || *e) {
                fprintf(stderr, "%s %s: not a number\n", f.c_str(), argv[i]);
                return 2;
            }
            if (f == "--max-length") max_length = (size_t)v;
        } else if (f == "--layer-fused") {
            fused = true;
        } else {
            fputs(kUsage, stderr);
            return 2;
        }
    }
    char err[1024] = {0};
    std::unique_ptr<Engine, void (*)(Engine*)> eng(julia_cuda_load(model, max_length, err, sizeof err),
                                                   julia_cuda_free);
    if (!eng) {
        fprintf(stderr, "julia-serve: %s\n", err);
        return 1;
    }
    char dev[256] = {0};
    julia_cuda_device(eng.get(), dev, sizeof dev);
    fprintf(stderr, "%s (%s)%s\n", dev, julia_cuda_tier(), fused ? ", layer-fused" : "");
    std::vector<size_t> tokens;
    std::vector<double> wall, gpu;
    std::string line, out;
    for (size_t no = 1; std::getline(std::cin, line); no++) {
        if (line.find_first_not_of(" \t\r") == std::string::npos) continue;
        const auto t0 = std::chrono::steady_clock::now();
        try {
            const Json req = parse(line);
            if (req.kind != Json::Obj) throw std::runtime_error("a request is a JSON object");
            if (!req.obj.count("ids"))
                throw std::runtime_error(
                    "no \"ids\": this build has no tokenizer, so requests carry their tokens "
                    "(ids, markers, type)");
            const std::vector<uint32_t> ids = u32_array(req, "ids");
            const std::vector<uint32_t> markers = u32_array(req, "markers");
            const uint32_t qt = qtype_of(req);
            bool truncated = false;
            auto tr = req.obj.find("truncated");
            if (tr != req.obj.end() && tr->second.kind == Json::Bool) truncated = tr->second.b;
            const size_t n = ids.size(), nm = markers.size();
            std::vector<float> logits(std::max<size_t>(nm, 1));
            float ms = 0.0f;
            if (julia_cuda_run(eng.get(), 1, ids.data(), &n, markers.data(), &nm, &qt,
                               fused ? 1 : 0, logits.data(), &ms, err, sizeof err) != 0)
                throw std::runtime_error(err);
            std::vector<double> p(std::max<size_t>(nm, 1));
            double value = 0.0;
            if (julia_hip_answer(qt, logits.data(), nm, p.data(), &value, err, sizeof err) != 0)
                throw std::runtime_error(err);
            out.clear();
            out += '{';
            put_floats(out, "logits", logits.data(), nm);
            out += ',';
            put_doubles(out, "probabilities", p.data(), nm);
            out += truncated ? ",\"truncated\":true," : ",\"truncated\":false,";
            char buf[64];
            if (qt == 0)
                snprintf(buf, sizeof buf, "\"choice\":%zu}", (size_t)value);
            else
                snprintf(buf, sizeof buf, "\"%s\":%.17g}", kTypes[qt], value);
            out += buf;
            fwrite(out.data(), 1, out.size(), stdout);
            fputc('\n', stdout);
            tokens.push_back(n);
            wall.push_back(std::chrono::duration<double, std::milli>(
                               std::chrono::steady_clock::now() - t0).count());
            gpu.push_back(ms);
        } catch (const std::exception& ex) {
            fflush(stdout);
            fprintf(stderr, "julia-serve: line %zu: %s\n", no, ex.what());
            return 1;
        }
    }
    fflush(stdout);
    julia_hip_engine_info info{};
    if (fused && julia_hip_engine_info_get(eng.get(), &info) == 0 && info.coop_refused)
        fprintf(stderr, "layer-fused: the runtime refused %zu cooperative launches (another process "
                "holds the resource); those requests ran on the per-step kernels\n", info.coop_refused);
    report(tokens, wall, gpu);
    return 0;
}

}  // namespace

int main(int argc, char** argv) { return serve(argc, argv); }
