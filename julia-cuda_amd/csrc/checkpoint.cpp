// Checkpoint directories: safetensors + config (see checkpoint.h).
#include "checkpoint.h"

#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <fstream>
#include <map>
#include <sstream>
#include <stdexcept>
#include <vector>

namespace jh {

// ---- a small JSON reader: objects, arrays, strings, numbers, true/false/null ----------------
namespace {

struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;

    const Json* get(const std::string& k) const {
        if (kind != Obj) return nullptr;
        auto it = obj.find(k);
        return it == obj.end() ? nullptr : &it->second;
    }
};

class JsonParser {
public:
    JsonParser(const char* p, size_t n, const std::string& what) : p_(p), end_(p + n), what_(what) {}
    Json parse() {
        Json v = value(0);
        ws();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

private:
    const char* p_;
    const char* end_;
    std::string what_;

    [[noreturn]] void fail(const std::string& m) { throw std::runtime_error(what_ + ": bad JSON (" + m + ")"); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool eat(char c) {
        ws();
        if (p_ < end_ && *p_ == c) {
            p_++;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!eat(c)) fail(std::string("expected '") + c + "'");
    }
    Json value(int depth) {
        if (depth > 64) fail("nested too deeply");
        ws();
        if (p_ >= end_) fail("unexpected end");
        Json v;
        const char c = *p_;
        if (c == '{') {
            p_++;
            v.kind = Json::Obj;
            if (eat('}')) return v;
            do {
                ws();
                if (p_ >= end_ || *p_ != '"') fail("expected a key");
                std::string k = string();
                expect(':');
                v.obj[k] = value(depth + 1);
            } while (eat(','));
            expect('}');
        } else if (c == '[') {
            p_++;
            v.kind = Json::Arr;
            if (eat(']')) return v;
            do v.arr.push_back(value(depth + 1));
            while (eat(','));
            expect(']');
        } else if (c == '"') {
            v.kind = Json::Str;
            v.str = string();
        } else if (word("true")) {
            v.kind = Json::Bool, v.b = true;
        } else if (word("false")) {
            v.kind = Json::Bool, v.b = false;
        } else if (word("null")) {
            v.kind = Json::Null;
        } else {
            v.kind = Json::Num;
            const char* s = p_;
            while (p_ < end_ && (isdigit((unsigned char)*p_) || *p_ == '-' || *p_ == '+' || *p_ == '.' ||
                                 *p_ == 'e' || *p_ == 'E'))
                p_++;
            if (s == p_) fail("unexpected character");
            const std::string t(s, p_);
            char* stop = nullptr;
            v.num = strtod(t.c_str(), &stop);
            if (!stop || *stop) fail("bad number '" + t + "'");
        }
        return v;
    }
    bool word(const char* w) {
        const size_t n = strlen(w);
        if ((size_t)(end_ - p_) >= n && memcmp(p_, w, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    std::string string() {
        p_++;  // the opening quote
        std::string s;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c == '\\') {
                if (p_ >= end_) fail("bad escape");
                const char e = *p_++;
                switch (e) {
                    case '"': s += '"'; break;
                    case '\\': s += '\\'; break;
                    case '/': s += '/'; break;
                    case 'b': s += '\b'; break;
                    case 'f': s += '\f'; break;
                    case 'n': s += '\n'; break;
                    case 'r': s += '\r'; break;
                    case 't': s += '\t'; break;
                    case 'u': {  // kept as UTF-8 for code points below 0x800 (names are ASCII)
                        if (end_ - p_ < 4) fail("bad \\u escape");
                        const unsigned cp = (unsigned)strtoul(std::string(p_, p_ + 4).c_str(), nullptr, 16);
                        p_ += 4;
                        if (cp < 0x80) {
                            s += (char)cp;
                        } else if (cp < 0x800) {
                            s += (char)(0xC0 | (cp >> 6));
                            s += (char)(0x80 | (cp & 0x3F));
                        } else {
                            s += (char)(0xE0 | (cp >> 12));
                            s += (char)(0x80 | ((cp >> 6) & 0x3F));
                            s += (char)(0x80 | (cp & 0x3F));
                        }
                        break;
                    }
                    default: fail("bad escape");
                }
            } else {
                s += c;
            }
        }
        if (p_ >= end_) fail("unterminated string");
        p_++;
        return s;
    }
};

std::string read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot read " + path);
    std::stringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

bool exists(const std::string& path) {
    struct stat st;
    return stat(path.c_str(), &st) == 0;
}

Json parse_file(const std::string& path) {
    const std::string text = read_file(path);
    return JsonParser(text.data(), text.size(), path).parse();
}

// ---- the logical tensors and their default names ----------------------------------------------
struct NameDef {
    const char* key;  // logical name (the override file's keys)
    const char* pattern;
};
const NameDef kNames[] = {
    {"tok_embeddings", "{enc}embeddings.tok_embeddings.weight"},
    {"emb_norm", "{enc}embeddings.norm.weight"},
    {"final_norm", "{enc}final_norm.weight"},
    {"type_emb", "type_emb.weight"},
    {"layer.attn_norm", "{enc}layers.{l}.attn_norm.weight"},
    {"layer.wqkv", "{enc}layers.{l}.attn.Wqkv.weight"},
    {"layer.wo", "{enc}layers.{l}.attn.Wo.weight"},
    {"layer.mlp_norm", "{enc}layers.{l}.mlp_norm.weight"},
    {"layer.wi", "{enc}layers.{l}.mlp.Wi.weight"},
    {"layer.wo_mlp", "{enc}layers.{l}.mlp.Wo.weight"},
    {"head.norm1_w", "head.layers.{h}.norm1.weight"},
    {"head.norm1_b", "head.layers.{h}.norm1.bias"},
    {"head.in_proj_w", "head.layers.{h}.self_attn.in_proj_weight"},
    {"head.in_proj_b", "head.layers.{h}.self_attn.in_proj_bias"},
    {"head.out_proj_w", "head.layers.{h}.self_attn.out_proj.weight"},
    {"head.out_proj_b", "head.layers.{h}.self_attn.out_proj.bias"},
    {"head.norm2_w", "head.layers.{h}.norm2.weight"},
    {"head.norm2_b", "head.layers.{h}.norm2.bias"},
    {"head.linear1_w", "head.layers.{h}.linear1.weight"},
    {"head.linear1_b", "head.layers.{h}.linear1.bias"},
    {"head.linear2_w", "head.layers.{h}.linear2.weight"},
    {"head.linear2_b", "head.layers.{h}.linear2.bias"},
    {"scorer.norm_w", "scorer.norm.weight"},
    {"scorer.norm_b", "scorer.norm.bias"},
    {"scorer.lin1_w", "scorer.lin1.weight"},
    {"scorer.lin1_b", "scorer.lin1.bias"},
    {"scorer.lin2_w", "scorer.lin2.weight"},
    {"scorer.lin2_b", "scorer.lin2.bias"},
};

// Logical key of a T_* id (layer and head slots as in weights.h).
const char* key_of(uint32_t id, int* layer, int* head) {
    static const char* lslot[6] = {"layer.attn_norm", "layer.wqkv", "layer.wo", "layer.mlp_norm",
                                   "layer.wi", "layer.wo_mlp"};
    static const char* hslot[12] = {"head.norm1_w", "head.norm1_b", "head.in_proj_w", "head.in_proj_b",
                                    "head.out_proj_w", "head.out_proj_b", "head.norm2_w", "head.norm2_b",
                                    "head.linear1_w", "head.linear1_b", "head.linear2_w", "head.linear2_b"};
    static const char* sslot[6] = {"scorer.norm_w", "scorer.norm_b", "scorer.lin1_w", "scorer.lin1_b",
                                   "scorer.lin2_w", "scorer.lin2_b"};
    *layer = *head = 0;
    if (id == T_TOK_EMB) return "tok_embeddings";
    if (id == T_EMB_NORM) return "emb_norm";
    if (id == T_FINAL_NORM) return "final_norm";
    if (id == T_TYPE_EMB) return "type_emb";
    if (id >= T_LAYER && id < T_HEAD && (id - T_LAYER) % 16 < 6) {
        *layer = (int)((id - T_LAYER) / 16);
        return lslot[(id - T_LAYER) % 16];
    }
    if (id >= T_HEAD && id < T_SCORER && (id - T_HEAD) % 32 < 12) {
        *head = (int)((id - T_HEAD) / 32);
        return hslot[(id - T_HEAD) % 32];
    }
    if (id >= T_SCORER && id < T_SCORER + 6) return sslot[id - T_SCORER];
    return nullptr;
}

std::string subst(std::string s, const std::string& enc, int l, int h) {
    auto put = [&s](const std::string& from, const std::string& to) {
        for (size_t at = s.find(from); at != std::string::npos; at = s.find(from, at + to.size()))
            s.replace(at, from.size(), to);
    };
    put("{enc}", enc);
    put("{l}", std::to_string(l));
    put("{h}", std::to_string(h));
    return s;
}

enum DType { F32, F16, BF16 };

struct TensorInfo {
    DType dtype;
    std::vector<int64_t> shape;
    size_t begin = 0, end = 0;  // byte offsets in the data section
};

float bf16_to_f32(uint16_t v) {
    const uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

}  // namespace

// ---- the checkpoint ---------------------------------------------------------------------------
struct Checkpoint::Impl {
    int fd = -1;
    void* map = nullptr;
    size_t size = 0;
    const uint8_t* data = nullptr;  // the data section
    size_t data_len = 0;
    std::map<std::string, TensorInfo> tensors;
    std::map<std::string, std::string> patterns;  // logical key -> pattern
    std::string enc;                              // the encoder's key prefix
    std::map<uint32_t, std::pair<std::string, size_t>> by_id;  // id -> (name, elements)

    ~Impl() {
        if (map && map != MAP_FAILED) munmap(map, size);
        if (fd >= 0) close(fd);
    }
    std::string name(uint32_t id) const {
        int l, h;
        const char* k = key_of(id, &l, &h);
        if (!k) throw std::runtime_error("checkpoint: no tensor id " + std::to_string(id));
        return subst(patterns.at(k), enc, l, h);
    }
    const TensorInfo* find(const std::string& n) const {
        auto it = tensors.find(n);
        return it == tensors.end() ? nullptr : &it->second;
    }
};

bool Checkpoint::is_checkpoint(const std::string& spec) { return spec.compare(0, 9, "synthetic") != 0; }

Checkpoint::Checkpoint(const std::string& dir) : impl_(new Impl) {
    Impl& I = *impl_;
    auto fail = [&](const std::string& m) { throw std::runtime_error("checkpoint " + dir + ": " + m); };
    const std::string st_path = dir + "/model.safetensors", cfg_path = dir + "/encoder/config.json";
    if (!exists(st_path) || !exists(cfg_path))
        throw std::runtime_error("no model at '" + dir + "': a checkpoint directory holds model.safetensors and "
                                 "encoder/config.json (or use \"synthetic[:key=value,...]\")");

    // The safetensors file: u64 header length, the JSON header, the data section.
    I.fd = open(st_path.c_str(), O_RDONLY);
    if (I.fd < 0) fail("cannot open model.safetensors");
    struct stat stt;
    if (fstat(I.fd, &stt) != 0) fail("cannot stat model.safetensors");
    I.size = (size_t)stt.st_size;
    if (I.size < 8) fail("model.safetensors is too short");
    I.map = mmap(nullptr, I.size, PROT_READ, MAP_PRIVATE, I.fd, 0);
    if (I.map == MAP_FAILED) fail("cannot map model.safetensors");
    const uint8_t* base = (const uint8_t*)I.map;
    uint64_t hlen = 0;
    memcpy(&hlen, base, 8);  // little-endian, as the host
    if (hlen > I.size - 8) fail("model.safetensors header length " + std::to_string(hlen) + " exceeds the file");
    I.data = base + 8 + hlen;
    I.data_len = I.size - 8 - (size_t)hlen;
    const Json header = JsonParser((const char*)base + 8, (size_t)hlen, "model.safetensors header").parse();
    if (header.kind != Json::Obj) fail("the safetensors header is not an object");
    for (const auto& kv : header.obj) {
        if (kv.first == "__metadata__") continue;
        const Json& t = kv.second;
        const Json *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
        if (!dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !off || off->kind != Json::Arr ||
            off->arr.size() != 2)
            fail("tensor '" + kv.first + "': no dtype, shape or data_offsets");
        TensorInfo ti;
        if (dt->str == "F32") ti.dtype = F32;
        else if (dt->str == "F16") ti.dtype = F16;
        else if (dt->str == "BF16") ti.dtype = BF16;
        else ti.dtype = (DType)-1;  // checked when the model uses the tensor
        for (const Json& x : sh->arr) ti.shape.push_back((int64_t)x.num);
        ti.begin = (size_t)off->arr[0].num, ti.end = (size_t)off->arr[1].num;
        if (ti.begin > ti.end || ti.end > I.data_len) fail("tensor '" + kv.first + "' lies outside the file");
        I.tensors[kv.first] = ti;
    }

    // Names: defaults, the override file, the encoder prefix.
    for (const NameDef& nd : kNames) I.patterns[nd.key] = nd.pattern;
    bool prefix_set = false;
    if (exists(dir + "/julia_hip_names.json")) {
        const Json names = parse_file(dir + "/julia_hip_names.json");
        if (names.kind != Json::Obj) fail("julia_hip_names.json is not an object");
        for (const auto& kv : names.obj) {
            if (kv.second.kind != Json::Str) fail("julia_hip_names.json: '" + kv.first + "' is not a string");
            if (kv.first == "encoder_prefix") {
                I.enc = kv.second.str, prefix_set = true;
            } else {
                if (!I.patterns.count(kv.first)) fail("julia_hip_names.json: unknown tensor '" + kv.first + "'");
                I.patterns[kv.first] = kv.second.str;
            }
        }
    }
    if (!prefix_set) {
        const std::string tail = "embeddings.tok_embeddings.weight";
        for (const auto& kv : I.tensors)
            if (kv.first.size() >= tail.size() &&
                kv.first.compare(kv.first.size() - tail.size(), tail.size(), tail) == 0) {
                I.enc = kv.first.substr(0, kv.first.size() - tail.size());
                break;
            }
    }

    // The encoder's config (ModernBertConfig's field names).
    const Json ec = parse_file(cfg_path);
    auto num = [&](const char* k, bool required, double dflt) {
        const Json* v = ec.get(k);
        if (!v || v->kind != Json::Num) {
            if (required) fail(std::string("encoder/config.json has no number '") + k + "'");
            return dflt;
        }
        return v->num;
    };
    ModelConfig& c = cfg_;
    c.d = (int)num("hidden_size", true, 0);
    c.layers = (int)num("num_hidden_layers", true, 0);
    c.inter = (int)num("intermediate_size", true, 0);
    c.vocab = (int)num("vocab_size", true, 0);
    c.max_positions = (int)num("max_position_embeddings", true, 0);
    c.theta_global = (float)num("global_rope_theta", false, 160000.0);
    c.theta_local = (float)num("local_rope_theta", false, 10000.0);
    c.global_every = (int)num("global_attn_every_n_layers", false, 3);
    c.window = (int)num("local_attention", false, 128) / 2;
    c.norm_eps = (float)num("norm_eps", false, 1e-5);
    const int heads = (int)num("num_attention_heads", false, c.d / 64);
    if (heads * 64 != c.d) fail("heads of 64 only: hidden_size " + std::to_string(c.d) + ", " +
                                std::to_string(heads) + " heads");
    if (const Json* nb = ec.get("norm_bias"); nb && nb->kind == Json::Bool && nb->b)
        fail("encoder LayerNorms with a bias are not supported (norm_bias: true)");
    if (const Json* act = ec.get("hidden_activation"); act && act->kind == Json::Str && act->str != "gelu")
        fail("the MLP activation must be gelu, not " + act->str);
    c.head_eps = 1e-5f;
    if (exists(dir + "/julia_config.json")) {
        const Json jc = parse_file(dir + "/julia_config.json");
        if (const Json* v = jc.get("head_norm_eps"); v && v->kind == Json::Num) c.head_eps = (float)v->num;
    }
    c.seed = 0;

    // The head's sizes from the tensors.
    c.head_layers = 0;
    while (c.head_layers < 16 && I.find(I.name(T_HEAD + 32u * (uint32_t)c.head_layers + 2))) c.head_layers++;
    if (const TensorInfo* t = I.find(I.name(T_TYPE_EMB)); t && t->shape.size() == 2) c.n_qtypes = (int)t->shape[0];
    if (c.head_layers > 0) {
        const TensorInfo* t = I.find(I.name(T_HEAD + 8));
        if (t && t->shape.size() == 2) c.head_ff = (int)t->shape[0];
    }
    if (c.d <= 0 || c.d % 128 || c.d > 4096) fail("hidden_size must be a multiple of 128 up to 4096");
    if (c.layers <= 0 || c.layers > 256) fail("num_hidden_layers must be 1-256");
    if (c.inter <= 0 || c.inter % 64) fail("intermediate_size must be a multiple of 64");
    if (c.head_ff <= 0 || c.head_ff % 128) fail("the head's feed-forward width must be a multiple of 128");
    if (c.vocab <= 0 || c.window < 0 || c.global_every <= 0 || c.max_positions <= 0 ||
        c.max_positions > (1 << 20) || c.n_qtypes <= 0)
        fail("vocab, window, global layers, positions or question types out of range");

    // Every tensor the model reads, with its shape.
    const int64_t d = c.d, inter = c.inter, F = c.head_ff;
    auto need = [&](uint32_t id, std::vector<int64_t> shape) {
        const std::string n = I.name(id);
        const TensorInfo* t = I.find(n);
        if (!t) fail("no tensor '" + n + "'");
        if (t->dtype != F32 && t->dtype != F16 && t->dtype != BF16) fail("tensor '" + n + "': F32, F16 or BF16 only");
        // a [1, n] or [n] vector either way
        std::vector<int64_t> got = t->shape;
        if (shape.size() == 1 && got.size() == 2 && got[0] == 1) got.erase(got.begin());
        if (got != shape) {
            std::string a, b;
            for (int64_t x : t->shape) a += (a.empty() ? "" : ", ") + std::to_string(x);
            for (int64_t x : shape) b += (b.empty() ? "" : ", ") + std::to_string(x);
            fail("tensor '" + n + "' is [" + a + "], the config says [" + b + "]");
        }
        size_t count = 1;
        for (int64_t x : shape) count *= (size_t)x;
        const size_t esz = t->dtype == F32 ? 4 : 2;
        if (t->end - t->begin != count * esz) fail("tensor '" + n + "': its bytes do not match its shape");
        I.by_id[id] = {n, count};
    };
    need(T_TOK_EMB, {c.vocab, d});
    need(T_EMB_NORM, {d});
    for (int l = 0; l < c.layers; l++) {
        const uint32_t b = T_LAYER + 16u * (uint32_t)l;
        if (l > 0) need(b + 0, {d});  // layer 0 has no attention LayerNorm (ModernBERT)
        need(b + 1, {3 * d, d});
        need(b + 2, {d, d});
        need(b + 3, {d});
        need(b + 4, {2 * inter, d});
        need(b + 5, {d, inter});
    }
    need(T_FINAL_NORM, {d});
    need(T_TYPE_EMB, {c.n_qtypes, d});
    for (int h = 0; h < c.head_layers; h++) {
        const uint32_t b = T_HEAD + 32u * (uint32_t)h;
        need(b + 0, {d}), need(b + 1, {d});
        need(b + 2, {3 * d, d}), need(b + 3, {3 * d});
        need(b + 4, {d, d}), need(b + 5, {d});
        need(b + 6, {d}), need(b + 7, {d});
        need(b + 8, {F, d}), need(b + 9, {F});
        need(b + 10, {d, F}), need(b + 11, {d});
    }
    need(T_SCORER + 0, {d}), need(T_SCORER + 1, {d});
    need(T_SCORER + 2, {d, d}), need(T_SCORER + 3, {d});
    need(T_SCORER + 4, {1, d}), need(T_SCORER + 5, {1});
}

Checkpoint::~Checkpoint() = default;

TensorSource Checkpoint::source() const {
    const Impl* I = impl_.get();
    return [I](uint32_t id, size_t start, size_t count, float* out) {
        auto it = I->by_id.find(id);
        if (it == I->by_id.end()) throw std::runtime_error("checkpoint: the model reads no tensor " + std::to_string(id));
        if (start + count > it->second.second)
            throw std::runtime_error("checkpoint: reading past tensor '" + it->second.first + "'");
        const TensorInfo& t = I->tensors.at(it->second.first);
        const uint8_t* p = I->data + t.begin;
        if (t.dtype == F32) {
            memcpy(out, p + start * 4, count * 4);
        } else if (t.dtype == F16) {
            for (size_t i = 0; i < count; i++) {
                uint16_t v;
                memcpy(&v, p + (start + i) * 2, 2);
                out[i] = f16_to_f32(v);
            }
        } else {
            for (size_t i = 0; i < count; i++) {
                uint16_t v;
                memcpy(&v, p + (start + i) * 2, 2);
                out[i] = bf16_to_f32(v);
            }
        }
    };
}

}  // namespace jh
