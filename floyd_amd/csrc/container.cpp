// container.cpp -- config.json / safetensors reader for the Moonlight container.
#include "container.h"

#include <dirent.h>
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>

namespace mlh {

// ---------------------------------------------------------------------------
// minimal JSON (objects, arrays, strings, numbers, true/false/null)
// ---------------------------------------------------------------------------

struct JsonValue {
    enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
    bool boolean = false;
    double number = 0.0;
    std::string text;
    std::vector<std::unique_ptr<JsonValue>> items;  // array items / object values
    std::vector<std::string> keys;                   // object keys

    const JsonValue *get(const char *key) const {
        if (kind != kObject) return nullptr;
        for (size_t i = 0; i < keys.size(); ++i)
            if (keys[i] == key) return items[i].get();
        return nullptr;
    }
};

class JsonParser {
public:
    explicit JsonParser(const std::string &s) : p_(s.c_str()), end_(s.c_str() + s.size()) {}

    std::unique_ptr<JsonValue> parse(std::string *error) {
        auto v = value();
        skip();
        if (!v || (p_ != end_ && *p_)) {
            if (error) *error = "invalid JSON";
            return nullptr;
        }
        return v;
    }

private:
    const char *p_;
    const char *end_;

    void skip() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }

    bool literal(const char *word) {
        size_t n = strlen(word);
        if ((size_t)(end_ - p_) < n || strncmp(p_, word, n)) return false;
        p_ += n;
        return true;
    }

    static void put_utf8(std::string &out, unsigned cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }

    bool hex4(unsigned *out) {
        if (end_ - p_ < 4) return false;
        unsigned v = 0;
        for (int i = 0; i < 4; ++i) {
            char c = p_[i];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return false;
        }
        p_ += 4;
        *out = v;
        return true;
    }

    bool string(std::string *out) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c != '\\') {
                *out += c;
                continue;
            }
            if (p_ >= end_) return false;
            char e = *p_++;
            switch (e) {
            case '"': *out += '"'; break;
            case '\\': *out += '\\'; break;
            case '/': *out += '/'; break;
            case 'b': *out += '\b'; break;
            case 'f': *out += '\f'; break;
            case 'n': *out += '\n'; break;
            case 'r': *out += '\r'; break;
            case 't': *out += '\t'; break;
            case 'u': {
                unsigned cp;
                if (!hex4(&cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' &&
                    p_[1] == 'u') {
                    p_ += 2;
                    unsigned lo;
                    if (!hex4(&lo)) return false;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                put_utf8(*out, cp);
                break;
            }
            default: return false;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }

    std::unique_ptr<JsonValue> value() {
        skip();
        if (p_ >= end_) return nullptr;
        auto v = std::make_unique<JsonValue>();
        char c = *p_;
        if (c == '{') {
            ++p_;
            v->kind = JsonValue::kObject;
            skip();
            if (p_ < end_ && *p_ == '}') { ++p_; return v; }
            for (;;) {
                skip();
                std::string key;
                if (!string(&key)) return nullptr;
                skip();
                if (p_ >= end_ || *p_ != ':') return nullptr;
                ++p_;
                auto item = value();
                if (!item) return nullptr;
                v->keys.push_back(std::move(key));
                v->items.push_back(std::move(item));
                skip();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == '}') { ++p_; return v; }
                return nullptr;
            }
        }
        if (c == '[') {
            ++p_;
            v->kind = JsonValue::kArray;
            skip();
            if (p_ < end_ && *p_ == ']') { ++p_; return v; }
            for (;;) {
                auto item = value();
                if (!item) return nullptr;
                v->items.push_back(std::move(item));
                skip();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == ']') { ++p_; return v; }
                return nullptr;
            }
        }
        if (c == '"') {
            v->kind = JsonValue::kString;
            if (!string(&v->text)) return nullptr;
            return v;
        }
        if (literal("true")) { v->kind = JsonValue::kBool; v->boolean = true; return v; }
        if (literal("false")) { v->kind = JsonValue::kBool; return v; }
        if (literal("null")) return v;
        char *stop = nullptr;
        std::string num;
        while (p_ + num.size() < end_ && strchr("+-0123456789.eE", p_[num.size()]))
            num += p_[num.size()];
        if (num.empty()) return nullptr;
        v->kind = JsonValue::kNumber;
        v->number = strtod(num.c_str(), &stop);
        if (!stop || *stop) return nullptr;
        p_ += num.size();
        return v;
    }
};

// read_config (moonlight_model.c:26-110): missing or non-numeric ints read as
// 0, floats fall back to their defaults, rope_theta falls back to
// rope_parameters.rope_theta while it still equals the 10000 default.
static int json_int(const JsonValue *root, const char *key) {
    const JsonValue *v = root->get(key);
    return v && v->kind == JsonValue::kNumber ? (int)v->number : 0;
}

static float json_float(const JsonValue *root, const char *key, float fallback) {
    const JsonValue *v = root->get(key);
    return v && v->kind == JsonValue::kNumber ? (float)v->number : fallback;
}

static int json_bool(const JsonValue *root, const char *key, int fallback) {
    const JsonValue *v = root->get(key);
    return v && v->kind == JsonValue::kBool ? (v->boolean ? 1 : 0) : fallback;
}

bool parse_config_json(const std::string &text, ModelConfig *c, std::string *error) {
    JsonParser parser(text);
    auto root = parser.parse(error);
    if (!root || root->kind != JsonValue::kObject) {
        if (error) *error = "invalid JSON";
        return false;
    }
    *c = ModelConfig();
    c->hidden_size = json_int(root.get(), "hidden_size");
    c->layer_count = json_int(root.get(), "num_hidden_layers");
    c->head_count = json_int(root.get(), "num_attention_heads");
    c->expert_count = json_int(root.get(), "n_routed_experts");
    c->experts_per_token = json_int(root.get(), "num_experts_per_tok");
    c->dense_intermediate_size = json_int(root.get(), "intermediate_size");
    c->moe_intermediate_size = json_int(root.get(), "moe_intermediate_size");
    c->first_dense_layer_count = json_int(root.get(), "first_k_dense_replace");
    c->q_lora_rank = json_int(root.get(), "q_lora_rank");
    c->kv_lora_rank = json_int(root.get(), "kv_lora_rank");
    c->qk_nope_dim = json_int(root.get(), "qk_nope_head_dim");
    c->qk_rope_dim = json_int(root.get(), "qk_rope_head_dim");
    c->value_dim = json_int(root.get(), "v_head_dim");
    c->shared_expert_count = json_int(root.get(), "n_shared_experts");
    c->normalize_topk = json_bool(root.get(), "norm_topk_prob", 1);
    c->vocab_size = json_int(root.get(), "vocab_size");
    c->rms_norm_epsilon = json_float(root.get(), "rms_norm_eps", 1e-5f);
    c->rope_theta = json_float(root.get(), "rope_theta", 10000.0f);
    c->routed_scale = json_float(root.get(), "routed_scaling_factor", 1.0f);
    if (c->rope_theta == 10000.0f) {
        const JsonValue *rp = root->get("rope_parameters");
        if (rp) c->rope_theta = json_float(rp, "rope_theta", 10000.0f);
    }
    if (c->hidden_size <= 0 || c->layer_count <= 0 || c->head_count <= 0 ||
        c->expert_count <= 0 || c->experts_per_token <= 0 || c->kv_lora_rank <= 0 ||
        c->qk_rope_dim <= 0 || c->vocab_size <= 0) {
        if (error) *error = "unsupported Moonlight config";
        return false;
    }
    return true;
}

// ---------------------------------------------------------------------------
// safetensors
// ---------------------------------------------------------------------------

static int dtype_code(const std::string &s) {
    if (s == "BF16") return kDtypeBF16;
    if (s == "F16") return kDtypeF16;
    if (s == "F32") return kDtypeF32;
    if (s == "U8" || s == "I8") return kDtypeU8;
    if (s == "I64") return kDtypeI64;
    if (s == "F8_E8M0") return kDtypeF8E8M0;
    if (s == "F8_E4M3") return kDtypeF8E4M3;
    return -1;
}

static bool read_file(const std::string &path, std::string *out) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof(buf), f)) > 0) out->append(buf, n);
    bool ok = !ferror(f);
    fclose(f);
    return ok;
}

Container::~Container() {
    for (int fd : fds_)
        if (fd >= 0) close(fd);
}

bool Container::open(const std::string &dir, std::string *error) {
    std::string text;
    const std::string config_path = dir + "/config.json";
    if (!read_file(config_path, &text)) {
        *error = "cannot open " + config_path;
        return false;
    }
    std::string why;
    if (!parse_config_json(text, &config_, &why)) {
        *error = why == "invalid JSON" ? "invalid JSON in " + config_path
                                       : "unsupported Moonlight config in " + config_path;
        return false;
    }
    std::vector<std::string> files;
    if (DIR *d = opendir(dir.c_str())) {
        while (struct dirent *e = readdir(d)) {
            const char *dot = strrchr(e->d_name, '.');
            if (dot && !strcmp(dot, ".safetensors")) files.push_back(dir + "/" + e->d_name);
        }
        closedir(d);
    }
    std::sort(files.begin(), files.end());
    if (files.empty()) {
        *error = "no safetensors found in " + dir;
        return false;
    }
    for (const std::string &path : files) {
        int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) {
            *error = "cannot open " + path;
            return false;
        }
        fds_.push_back(fd);
        uint64_t hlen = 0;
        if (pread(fd, &hlen, 8, 0) != 8 || hlen > (1ull << 31)) {
            *error = "bad safetensors header in " + path;
            return false;
        }
        std::string header(hlen, '\0');
        if (pread(fd, &header[0], hlen, 8) != (ssize_t)hlen) {
            *error = "short safetensors header in " + path;
            return false;
        }
        JsonParser parser(header);
        auto root = parser.parse(&why);
        if (!root || root->kind != JsonValue::kObject) {
            *error = "invalid safetensors header in " + path;
            return false;
        }
        const int64_t data_start = 8 + (int64_t)hlen;
        for (size_t i = 0; i < root->keys.size(); ++i) {
            if (root->keys[i] == "__metadata__") continue;
            const JsonValue *m = root->items[i].get();
            const JsonValue *dt = m->get("dtype");
            const JsonValue *off = m->get("data_offsets");
            const JsonValue *shape = m->get("shape");
            if (!dt || dt->kind != JsonValue::kString || !off ||
                off->kind != JsonValue::kArray || off->items.size() != 2 || !shape ||
                shape->kind != JsonValue::kArray) {
                *error = "malformed tensor entry " + root->keys[i] + " in " + path;
                return false;
            }
            TensorEntry t;
            t.name = root->keys[i];
            t.dtype = dtype_code(dt->text);
            if (t.dtype < 0) {
                *error = "unsupported dtype " + dt->text + " for " + t.name;
                return false;
            }
            int64_t a = (int64_t)off->items[0]->number, b = (int64_t)off->items[1]->number;
            t.numel = 1;
            for (auto &dim : shape->items) t.numel *= (int64_t)dim->number;
            t.nbytes = b - a;
            t.file = (int)fds_.size() - 1;
            t.offset = data_start + a;
            total_bytes_ += (uint64_t)t.nbytes;
            if (!index_.count(t.name)) index_[t.name] = (int)tensors_.size();
            tensors_.push_back(std::move(t));
        }
    }
    return true;
}

int Container::find(const std::string &name) const {
    auto it = index_.find(name);
    return it == index_.end() ? -1 : it->second;
}

bool Container::read(int index, void *dst, size_t capacity) const {
    if (index < 0 || index >= (int)tensors_.size() || !dst) return false;
    const TensorEntry &t = tensors_[index];
    if (t.nbytes < 0 || (uint64_t)t.nbytes > capacity) return false;
    char *out = static_cast<char *>(dst);
    int64_t done = 0;
    while (done < t.nbytes) {
        ssize_t n = pread(fds_[t.file], out + done, (size_t)(t.nbytes - done), t.offset + done);
        if (n <= 0) return false;
        done += n;
    }
    return true;
}

bool Container::read_slice(int index, int64_t offset, size_t n, void *dst) const {
    if (index < 0 || index >= (int)tensors_.size() || !dst || offset < 0) return false;
    const TensorEntry &t = tensors_[index];
    if (offset + (int64_t)n > t.nbytes) return false;
    char *out = static_cast<char *>(dst);
    size_t done = 0;
    while (done < n) {
        ssize_t got = pread(fds_[t.file], out + done, n - done, t.offset + offset + (int64_t)done);
        if (got <= 0) return false;
        done += (size_t)got;
    }
    return true;
}

}  // namespace mlh
