// checkpoint.hip -- Model::open from a checkpoint directory (src/model.rs:418-451):
// config.json (Config::read, src/model.rs:29-73) and the memory-mapped
// safetensors shards (Weights::open, src/checkpoint.rs:310-414), with the
// reference's checks and messages.  Only the tensors of the autoregressive
// decode path are read (embedding, the AR pathway of every layer, the final
// norm, the LM head); the NAR pathway, latent and VAE tensors are not
// needed on this path and are ignored.  BF16 matrices are uploaded straight
// from the mapping; F32 and F16 ones are rounded to BF16 as the reference's
// converted weights are (src/tensor.rs:436-438, Linear with bf16 = true).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <array>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/yue2_hip.h"
#include "runtime.h"
#include "vae.h"
#include "y2_math.h"

using namespace y2;

namespace {

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) ------

struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const std::string& k) const {
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct Parser {
    const char* p;
    const char* end;
    std::string err;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    bool literal(const char* s) {
        const size_t n = std::strlen(s);
        if ((size_t)(end - p) < n || std::strncmp(p, s, n) != 0) return fail("Invalid JSON literal");
        p += n;
        return true;
    }
    bool string(std::string* out) {
        if (p >= end || *p != '"') return fail("Expected JSON string");
        ++p;
        out->clear();
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end) return fail("Invalid JSON escape");
                const char e = *p++;
                switch (e) {
                    case '"': case '\\': case '/': out->push_back(e); break;
                    case 'b': out->push_back('\b'); break;
                    case 'f': out->push_back('\f'); break;
                    case 'n': out->push_back('\n'); break;
                    case 'r': out->push_back('\r'); break;
                    case 't': out->push_back('\t'); break;
                    case 'u': {
                        if (end - p < 4) return fail("Invalid JSON escape");
                        unsigned v = 0;
                        for (int i = 0; i < 4; ++i) {
                            const char h = *p++;
                            v <<= 4;
                            if (h >= '0' && h <= '9') v |= h - '0';
                            else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
                            else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
                            else return fail("Invalid JSON escape");
                        }
                        // names in these files are ASCII; other code points keep a placeholder
                        out->push_back(v < 0x80 ? (char)v : '?');
                        break;
                    }
                    default: return fail("Invalid JSON escape");
                }
            } else {
                out->push_back(c);
            }
        }
        if (p >= end) return fail("Unterminated JSON string");
        ++p;
        return true;
    }
    bool value(Json* v, int depth) {
        if (depth > 64) return fail("JSON nesting too deep");
        ws();
        if (p >= end) return fail("Unexpected end of JSON");
        const char c = *p;
        if (c == '{') {
            ++p;
            v->kind = Json::OBJ;
            ws();
            if (p < end && *p == '}') {
                ++p;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (!string(&k)) return false;
                ws();
                if (p >= end || *p != ':') return fail("Expected ':' in JSON object");
                ++p;
                Json item;
                if (!value(&item, depth + 1)) return false;
                v->obj.emplace_back(std::move(k), std::move(item));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    return true;
                }
                return fail("Expected ',' or '}' in JSON object");
            }
        }
        if (c == '[') {
            ++p;
            v->kind = Json::ARR;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return true;
            }
            for (;;) {
                Json item;
                if (!value(&item, depth + 1)) return false;
                v->arr.push_back(std::move(item));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    return true;
                }
                return fail("Expected ',' or ']' in JSON array");
            }
        }
        if (c == '"') {
            v->kind = Json::STR;
            return string(&v->str);
        }
        if (c == 't') {
            v->kind = Json::BOOL;
            v->b = true;
            return literal("true");
        }
        if (c == 'f') {
            v->kind = Json::BOOL;
            return literal("false");
        }
        if (c == 'n') return literal("null");
        const char* q = p;
        if (q < end && (*q == '-' || *q == '+')) ++q;
        while (q < end && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' || *q == '-' || *q == '+'))
            ++q;
        if (q == p) return fail("Invalid JSON value");
        const std::string text(p, q);
        char* stop = nullptr;
        v->kind = Json::NUM;
        v->num = std::strtod(text.c_str(), &stop);
        if (!stop || *stop) return fail("Invalid JSON number");
        p = q;
        return true;
    }
};

bool parse_json(const char* data, size_t n, Json* out, std::string* err) {
    Parser ps{data, data + n, {}};
    if (!ps.value(out, 0)) {
        *err = ps.err;
        return false;
    }
    ps.ws();
    if (ps.p != ps.end) {
        *err = "Trailing characters after JSON";
        return false;
    }
    return true;
}

bool read_file(const std::string& path, std::string* out) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[65536];
    size_t n;
    out->clear();
    while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) out->append(buf, n);
    std::fclose(f);
    return true;
}

// A non-negative integer JSON value (a usize in the reference).
bool as_size(const Json& v, size_t* out) {
    if (v.kind != Json::NUM || !(v.num >= 0.0) || v.num != std::floor(v.num) || v.num > 9007199254740992.0)
        return false;
    *out = (size_t)v.num;
    return true;
}

// ---- safetensors ----------------------------------------------------------

enum DType { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

struct Mapping {
    void* ptr = nullptr;
    size_t len = 0;
    ~Mapping() {
        if (ptr) munmap(ptr, len);
    }
};

struct Tensor {
    std::shared_ptr<Mapping> map;
    size_t offset = 0;  // bytes from the start of the mapping
    std::vector<size_t> shape;
    DType dtype = DT_BF16;
    size_t count() const {
        size_t c = 1;
        for (size_t s : shape) c *= s;
        return c;
    }
    const uint8_t* bytes() const { return static_cast<const uint8_t*>(map->ptr) + offset; }
};

struct Checkpoint {
    Yue2Config config{};
    bool tie = false;
    std::map<std::string, Tensor> tensors;
};

int invalid(const std::string& msg) { return fail(YUE2_ERR_CONFIG, msg); }

std::string shape_text(const std::vector<size_t>& s) {
    std::string t = "[";
    for (size_t i = 0; i < s.size(); ++i) t += (i ? ", " : "") + std::to_string(s[i]);
    return t + "]";
}

// Weights::open (src/checkpoint.rs:310-386).
int open_shard(const std::string& dir, const std::string& file, Checkpoint* ck) {
    if (file.empty() || file.find('/') != std::string::npos || file == "." || file == "..")
        return invalid("Invalid shard path");
    const std::string path = dir + "/" + file;
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return fail(YUE2_ERR_ARG, "cannot open " + path + ": " + std::strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        ::close(fd);
        return fail(YUE2_ERR_ARG, "cannot stat " + path);
    }
    auto map = std::make_shared<Mapping>();
    map->len = (size_t)sb.st_size;
    if (map->len < 8) {
        ::close(fd);
        return invalid("Short safetensors file");
    }
    void* ptr = mmap(nullptr, map->len, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (ptr == MAP_FAILED) return fail(YUE2_ERR_ARG, "cannot map " + path);
    map->ptr = ptr;
    const uint8_t* bytes = static_cast<const uint8_t*>(ptr);
    uint64_t header = 0;
    for (int i = 7; i >= 0; --i) header = (header << 8) | bytes[i];
    if (header > 100000000ull || header > map->len - 8) return invalid("Invalid safetensors header size");
    const size_t data = 8 + (size_t)header;
    Json root;
    std::string err;
    if (!parse_json(reinterpret_cast<const char*>(bytes + 8), (size_t)header, &root, &err)) return invalid(err);
    if (root.kind != Json::OBJ) return invalid("Expected JSON object");
    std::vector<std::pair<size_t, size_t>> ranges;
    for (const auto& kv : root.obj) {
        const std::string& name = kv.first;
        if (name == "__metadata__") continue;
        const Json& v = kv.second;
        const Json* dt = v.get("dtype");
        const Json* sh = v.get("shape");
        const Json* of = v.get("data_offsets");
        if (!dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !of || of->kind != Json::ARR)
            return invalid("Invalid tensor entry " + name);
        Tensor t;
        if (dt->str == "F32") t.dtype = DT_F32;
        else if (dt->str == "BF16") t.dtype = DT_BF16;
        else if (dt->str == "F16") t.dtype = DT_F16;
        else return invalid("Unsupported dtype " + dt->str + " for " + name);
        for (const Json& d : sh->arr) {
            size_t s;
            if (!as_size(d, &s)) return invalid("Invalid tensor shape " + name);
            t.shape.push_back(s);
        }
        if (of->arr.size() != 2) return invalid("Invalid tensor offsets");
        size_t a, b;
        if (!as_size(of->arr[0], &a) || !as_size(of->arr[1], &b)) return invalid("Invalid tensor offsets");
        size_t count = 1;
        for (size_t s : t.shape) {
            if (s != 0 && count > SIZE_MAX / s) return invalid("Tensor size overflow");
            count *= s;
        }
        const size_t width = t.dtype == DT_F32 ? 4 : 2;
        if (count > SIZE_MAX / width) return invalid("Tensor bytes overflow");
        if (b < a || b > map->len - data || b - a != count * width) return invalid("Invalid tensor extent " + name);
        ranges.emplace_back(a, b);
        t.map = map;
        t.offset = data + a;
        if (!ck->tensors.emplace(name, std::move(t)).second) return invalid("Duplicate tensor " + name);
    }
    std::sort(ranges.begin(), ranges.end());
    for (size_t i = 1; i < ranges.size(); ++i)
        if (ranges[i - 1].second > ranges[i].first) return invalid("Overlapping safetensors tensors");
    return YUE2_OK;
}

// Config::read (src/model.rs:29-73): every field with the reference's
// defaults and checks.  A present key of the wrong JSON kind is an error with
// the reference's message (Value::string / usize / f64 / boolean,
// src/json.rs:26-66), never a fallback to the default.
int read_config(const std::string& dir, Checkpoint* ck) {
    std::string text, err;
    if (!read_file(dir + "/config.json", &text)) return fail(YUE2_ERR_ARG, "cannot read " + dir + "/config.json");
    Json v;
    if (!parse_json(text.data(), text.size(), &v, &err)) return invalid(err);
    if (v.kind != Json::OBJ) return invalid("Expected JSON object");
    const char* bad = nullptr;  // the first wrong-kind message
    auto text_or = [&](const char* k, const char* d) {
        const Json* j = v.get(k);
        if (j && j->kind != Json::STR && !bad) bad = "Expected JSON string";
        return j && j->kind == Json::STR ? j->str : std::string(d);
    };
    const std::string model_type = text_or("model_type", "yue2"), latent_type = text_or("latent_type", "vae");
    if (bad) return invalid(bad);
    if (model_type != "yue2" || latent_type != "vae") return invalid("Expected YuE2 VAE-latent model");
    auto size_or = [&](const char* k, size_t d) -> int32_t {
        const Json* j = v.get(k);
        size_t s = d;
        if (j && j->kind != Json::NUM && !bad) bad = "Expected unsigned JSON integer";
        if (j && j->kind == Json::NUM && !as_size(*j, &s) && !bad) bad = "invalid digit found in string";
        if (s > 0x7fffffff && !bad) bad = "Invalid transformer configuration";
        return (int32_t)s;
    };
    auto float_or = [&](const char* k, double d) {
        const Json* j = v.get(k);
        if (j && j->kind != Json::NUM && !bad) bad = "Expected JSON number";
        return (float)(j && j->kind == Json::NUM ? j->num : d);
    };
    Yue2Config& c = ck->config;
    c.hidden_size = size_or("hidden_size", 2048);
    c.num_hidden_layers = size_or("num_hidden_layers", 28);
    c.num_attention_heads = size_or("num_attention_heads", 16);
    c.num_key_value_heads = size_or("num_key_value_heads", 8);
    c.head_dim = size_or("head_dim", 128);
    c.intermediate_size = size_or("intermediate_size", 6144);
    c.vocab_size = size_or("vocab_size", 184704);
    c.rms_norm_eps = float_or("rms_norm_eps", 1e-6);
    c.rope_theta = float_or("rope_theta", 1e6);
    c.max_position_embeddings = size_or("max_position_embeddings", 24576);
    // the NAR pathway's fields, read and checked here as the reference does
    // although the decode path does not use them
    const int32_t latent_dim = size_or("latent_dim", 64);
    const int32_t max_latent_frames = size_or("max_latent_frames", 24576);
    const float timestep_shift = float_or("timestep_shift", 1.0);
    const Json* tie = v.get("tie_word_embeddings");
    if (tie && tie->kind != Json::BOOL && !bad) bad = "Expected JSON boolean";
    ck->tie = tie && tie->kind == Json::BOOL && tie->b;
    if (bad) return invalid(bad);
    if (yue2_hip_config_validate(&c) != YUE2_OK || latent_dim == 0 || max_latent_frames == 0 ||
        !(timestep_shift > 0.0f) || !std::isfinite(timestep_shift))
        return invalid("Invalid transformer configuration");
    return YUE2_OK;
}

int open_checkpoint(const char* dir_c, Checkpoint* ck) {
    if (!dir_c) return fail(YUE2_ERR_ARG, "null checkpoint directory");
    const std::string dir(dir_c);
    if (int rc = read_config(dir, ck)) return rc;
    std::set<std::string> files;
    std::string index;
    if (read_file(dir + "/model.safetensors.index.json", &index)) {
        Json v;
        std::string err;
        if (!parse_json(index.data(), index.size(), &v, &err)) return invalid(err);
        const Json* wm = v.get("weight_map");
        if (!wm || wm->kind != Json::OBJ) return invalid("Missing weight_map");
        for (const auto& kv : wm->obj) {
            if (kv.second.kind != Json::STR) return invalid("Invalid weight_map entry");
            files.insert(kv.second.str);
        }
    } else {
        files.insert("model.safetensors");
    }
    for (const std::string& f : files)
        if (int rc = open_shard(dir, f, ck)) return rc;
    return YUE2_OK;
}

// Weights::checked (src/checkpoint.rs:405-409).
int checked(const Checkpoint& ck, const std::string& name, std::vector<size_t> shape, const Tensor** out) {
    auto it = ck.tensors.find(name);
    if (it == ck.tensors.end()) return invalid("Missing checkpoint tensor " + name);
    if (it->second.shape != shape)
        return invalid("Tensor " + name + ": expected " + shape_text(shape) + ", found " + shape_text(it->second.shape));
    *out = &it->second;
    return YUE2_OK;
}

struct ArTensors {
    const Tensor *embed = nullptr, *lm_head = nullptr, *final_norm = nullptr;
    std::vector<std::array<const Tensor*, 11>> layers;  // q k v o gate up down, in q_norm k_norm post
};

// The tensors of the decode path with their shapes (src/model.rs:79-94,
// 108-118, 193-205, 247-263, 418-440).
int ar_tensors(const Checkpoint& ck, ArTensors* t) {
    const Yue2Config& c = ck.config;
    const size_t H = c.hidden_size, D = c.head_dim, I = c.intermediate_size, V = c.vocab_size;
    const size_t qd = (size_t)c.num_attention_heads * D, kd = (size_t)c.num_key_value_heads * D;
    if (int rc = checked(ck, "model.embed_tokens.weight", {V, H}, &t->embed)) return rc;
    if (ck.tie) t->lm_head = t->embed;
    else if (int rc = checked(ck, "lm_head.weight", {V, H}, &t->lm_head)) return rc;
    if (int rc = checked(ck, "model.norm.weight", {H}, &t->final_norm)) return rc;
    t->layers.resize(c.num_hidden_layers);
    for (int l = 0; l < c.num_hidden_layers; ++l) {
        const std::string p = "model.layers." + std::to_string(l);
        const std::string a = p + ".self_attn", m = p + ".mlp";
        auto& L = t->layers[l];
        const struct {
            std::string name;
            std::vector<size_t> shape;
        } want[11] = {{a + ".q_proj.weight", {qd, H}},    {a + ".k_proj.weight", {kd, H}},
                      {a + ".v_proj.weight", {kd, H}},    {a + ".o_proj.weight", {H, qd}},
                      {m + ".gate_proj.weight", {I, H}},  {m + ".up_proj.weight", {I, H}},
                      {m + ".down_proj.weight", {H, I}},  {p + ".input_layernorm.weight", {H}},
                      {a + ".q_norm.weight", {D}},        {a + ".k_norm.weight", {D}},
                      {p + ".post_attention_layernorm.weight", {H}}};
        for (int i = 0; i < 11; ++i)
            if (int rc = checked(ck, want[i].name, want[i].shape, &L[i])) return rc;
    }
    return YUE2_OK;
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const int e = (h >> 10) & 31;
    const uint32_t m = h & 1023u;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {  // subnormal: normalise
            int shift = 0;
            uint32_t mm = m;
            while (!(mm & 0x400u)) {
                mm <<= 1;
                ++shift;
            }
            bits = sign | ((uint32_t)(113 - shift) << 23) | ((mm & 1023u) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((uint32_t)(e + 112) << 23) | (m << 13);
    }
    return u2f(bits);
}

float value_at(const Tensor& t, size_t i) {
    const uint8_t* b = t.bytes();
    if (t.dtype == DT_F32) {
        float v;
        std::memcpy(&v, b + 4 * i, 4);
        return v;
    }
    uint16_t h;
    std::memcpy(&h, b + 2 * i, 2);
    return t.dtype == DT_BF16 ? u2f((uint32_t)h << 16) : f16_to_f32(h);
}

// A matrix as BF16 bits: the mapping itself when BF16, else rounded values.
const uint16_t* bf16_data(const Tensor& t, std::vector<std::vector<uint16_t>>* keep) {
    if (t.dtype == DT_BF16) return reinterpret_cast<const uint16_t*>(t.bytes());
    keep->emplace_back(t.count());
    std::vector<uint16_t>& out = keep->back();
    for (size_t i = 0; i < out.size(); ++i) out[i] = (uint16_t)(f2u(rb(value_at(t, i))) >> 16);
    return out.data();
}

const float* f32_data(const Tensor& t, std::vector<std::vector<float>>* keep) {
    keep->emplace_back(t.count());
    std::vector<float>& out = keep->back();
    for (size_t i = 0; i < out.size(); ++i) out[i] = value_at(t, i);
    return out.data();
}

}  // namespace

namespace y2 {

// Vae::open (src/vae.rs:635-669) with network(.., decoder = true)
// (:470-546), Conv::load (:67-146) and Activation::load (:268-281).
int vae_read(const char* dir_c, VaeHost* out) {
    if (!dir_c || !out) return fail(YUE2_ERR_ARG, "null VAE directory");
    const std::string dir(dir_c);
    std::string text, err;
    if (!read_file(dir + "/config.json", &text)) return fail(YUE2_ERR_ARG, "cannot read " + dir + "/config.json");
    Json v;
    if (!parse_json(text.data(), text.size(), &v, &err)) return invalid(err);
    if (v.kind != Json::OBJ) return invalid("Expected JSON object");
    bool ok = true;
    auto text_or = [&](const Json& o, const char* k, const char* d) {
        const Json* j = o.get(k);
        if (j && j->kind != Json::STR) ok = false;
        return j && j->kind == Json::STR ? j->str : std::string(d);
    };
    auto size_or = [&](const Json& o, const char* k, size_t d) -> int {
        const Json* j = o.get(k);
        size_t s = d;
        if (j && !as_size(*j, &s)) ok = false;
        if (s > 0x7fffffff) ok = false;
        return (int)s;
    };
    auto bool_or = [&](const Json& o, const char* k, bool d) {
        const Json* j = o.get(k);
        if (j && j->kind != Json::BOOL) ok = false;
        return j && j->kind == Json::BOOL ? j->b : d;
    };
    auto sizes = [&](const Json& o, const char* k, std::vector<int>* r) {
        const Json* j = o.get(k);
        if (!j || j->kind != Json::ARR) return false;
        for (const Json& e : j->arr) {
            size_t s;
            if (!as_size(e, &s) || s > 0x7fffffff) return false;
            r->push_back((int)s);
        }
        return true;
    };
    if (text_or(v, "model_type", "yue2_vae") != "yue2_vae") return invalid("Expected YuE2 VAE checkpoint");
    const Json* dc = v.get("decoder_config");
    if (!dc || dc->kind != Json::OBJ) return invalid("Missing key decoder_config");
    out->ratio = size_or(v, "downsampling_ratio", 1920);
    out->latent_dim = size_or(v, "latent_dim", 64);
    out->sample_rate = size_or(v, "sample_rate", 48000);
    out->audio_channels = size_or(v, "audio_channels", 2);
    out->core_frames = size_or(v, "decode_core_frames", 1024);
    out->halo_frames = size_or(v, "decode_halo_frames", 16);
    std::vector<int> strides, mults{1}, cm;
    if (!sizes(*dc, "strides", &strides) || !sizes(*dc, "c_mults", &cm)) return invalid("Invalid VAE channel list");
    mults.insert(mults.end(), cm.begin(), cm.end());
    long prod = 1;
    for (int st : strides) prod = std::min<long>(prod * st, 1L << 40);
    if (prod != out->ratio || size_or(*dc, "latent_dim", 32) != out->latent_dim ||
        size_or(*dc, "out_channels", 2) != out->audio_channels || out->sample_rate == 0)
        return invalid("VAE configuration mismatch");
    const int base = size_or(*dc, "channels", 128);
    if (strides.size() + 1 != mults.size() || std::count(strides.begin(), strides.end(), 0) ||
        std::count(mults.begin(), mults.end(), 0) || base == 0)
        return invalid("Invalid Oobleck channel/stride configuration");
    for (const char* k : {"antialias_activation", "use_filter", "use_nearest_upsample"})
        if (bool_or(*dc, k, false)) return invalid(std::string("Unsupported VAE option ") + k);
    const bool snake = bool_or(*dc, "use_snake", false);
    if (snake && text_or(*dc, "snake_type", "vanilla") != "vanilla") return invalid("Expected vanilla SnakeBeta");
    const int out_ch = size_or(*dc, "out_channels", 2);
    const bool final_tanh = bool_or(*dc, "final_tanh", true);
    if (!ok) return invalid("Invalid configuration value");
    // Weights::open over the VAE directory
    Checkpoint ck;
    std::set<std::string> files;
    std::string index_json;
    if (read_file(dir + "/model.safetensors.index.json", &index_json)) {
        Json iv;
        if (!parse_json(index_json.data(), index_json.size(), &iv, &err)) return invalid(err);
        const Json* wm = iv.get("weight_map");
        if (!wm || wm->kind != Json::OBJ) return invalid("Missing weight_map");
        for (const auto& kv : wm->obj) {
            if (kv.second.kind != Json::STR) return invalid("Invalid weight_map entry");
            files.insert(kv.second.str);
        }
    } else {
        files.insert("model.safetensors");
    }
    for (const std::string& f : files)
        if (int rc = open_shard(dir, f, &ck)) return rc;
    auto f32 = [](const Tensor& t) {
        std::vector<float> r(t.count());
        std::memcpy(r.data(), t.bytes(), r.size() * 4);
        return r;
    };
    auto conv = [&](const std::string& name, int in, int outc, int k, int stride, int pad, int dil, bool tr,
                    bool bias) -> int {
        const std::vector<size_t> shape = tr ? std::vector<size_t>{(size_t)in, (size_t)outc, (size_t)k}
                                             : std::vector<size_t>{(size_t)outc, (size_t)in, (size_t)k};
        const Tensor *tv, *tg;
        if (int rc = checked(ck, name + ".weight_v", shape, &tv)) return rc;
        if (int rc = checked(ck, name + ".weight_g", {shape[0], 1, 1}, &tg)) return rc;
        if (tv->dtype != DT_F32 || tg->dtype != DT_F32) return invalid("VAE weights must remain FP32");
        VaeOpHost op;
        op.kind = tr ? VAE_CONVT : VAE_CONV;
        op.cin = in;
        op.cout = outc;
        op.kernel = k;
        op.stride = stride;
        op.padding = pad;
        op.dilation = dil;
        op.w = f32(*tv);
        const std::vector<float> gain = f32(*tg);
        const size_t cols = shape[1] * (size_t)k;
        for (size_t r = 0; r < shape[0]; ++r) {
            float* row = op.w.data() + r * cols;
            float ss = 0.0f;  // the sequential f32 sum of squares (src/vae.rs:89)
            for (size_t q = 0; q < cols; ++q) ss += row[q] * row[q];
            const float norm = std::sqrt(ss);
            if (!std::isfinite(norm) || norm == 0.0f) return invalid("Invalid VAE weight normalization");
            const float f = gain[r] / norm;
            for (size_t q = 0; q < cols; ++q) row[q] *= f;
        }
        if (bias) {
            const Tensor* tb;
            if (int rc = checked(ck, name + ".bias", {(size_t)outc}, &tb)) return rc;
            if (tb->dtype != DT_F32) return invalid("VAE bias must be FP32");
            op.b = f32(*tb);
        }
        out->ops.push_back(std::move(op));
        return YUE2_OK;
    };
    auto act = [&](const std::string& name, int c) -> int {
        VaeOpHost op;
        if (!snake) {
            op.kind = VAE_ELU;
            out->ops.push_back(std::move(op));
            return YUE2_OK;
        }
        const Tensor *ta, *tb;
        if (int rc = checked(ck, name + ".alpha", {(size_t)c}, &ta)) return rc;
        if (int rc = checked(ck, name + ".beta", {(size_t)c}, &tb)) return rc;
        if (ta->dtype != DT_F32 || tb->dtype != DT_F32) return invalid("VAE activation must be FP32");
        op.kind = VAE_SNAKE;
        op.cin = op.cout = c;
        op.a = f32(*ta);
        op.ib = f32(*tb);
        for (float& x : op.a) x = expf(x);
        for (float& x : op.ib) x = 1.0f / (expf(x) + 1e-9f);
        out->ops.push_back(std::move(op));
        return YUE2_OK;
    };
    out->ops.clear();
    const std::string d = "decoder";
    if (int rc = conv(d + ".layers.0", out->latent_dim, base * mults.back(), 7, 1, 3, 1, false, true)) return rc;
    int index = 1;
    for (int i = (int)mults.size() - 1; i >= 1; --i) {
        const int in = base * mults[i], oc = base * mults[i - 1], st = strides[i - 1];
        const std::string p = d + ".layers." + std::to_string(index) + ".layers";
        if (int rc = act(p + ".0", in)) return rc;
        if (int rc = conv(p + ".1", in, oc, 2 * st, st, (st + 1) / 2, 1, true, true)) return rc;
        const int dils[3] = {1, 3, 9};
        for (int r = 0; r < 3; ++r) {
            // residual (src/vae.rs:427-466)
            const std::string rp = p + "." + std::to_string(r + 2) + ".layers";
            out->ops.push_back(VaeOpHost{VAE_RES_BEGIN});
            if (int rc = act(rp + ".0", oc)) return rc;
            if (int rc = conv(rp + ".1", oc, oc, 7, 1, 3 * dils[r], dils[r], false, true)) return rc;
            if (int rc = act(rp + ".2", oc)) return rc;
            if (int rc = conv(rp + ".3", oc, oc, 1, 1, 0, 1, false, true)) return rc;
            out->ops.push_back(VaeOpHost{VAE_RES_END});
        }
        ++index;
    }
    if (int rc = act(d + ".layers." + std::to_string(index), base)) return rc;
    if (int rc = conv(d + ".layers." + std::to_string(index + 1), base, out_ch, 7, 1, 3, 1, false, false)) return rc;
    if (final_tanh) out->ops.push_back(VaeOpHost{VAE_TANH});
    return YUE2_OK;
}

}  // namespace y2

extern "C" int32_t yue2_hip_checkpoint_config(const char* dir, Yue2Config* out) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    Checkpoint ck;
    if (int rc = open_checkpoint(dir, &ck)) return rc;
    ArTensors t;
    if (int rc = ar_tensors(ck, &t)) return rc;
    if (out) *out = ck.config;
    return YUE2_OK;
}

extern "C" Yue2Model* yue2_hip_model_open_dir(const char* dir) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    Checkpoint ck;
    if (open_checkpoint(dir, &ck) != YUE2_OK) return nullptr;
    ArTensors t;
    if (ar_tensors(ck, &t) != YUE2_OK) return nullptr;
    std::vector<std::vector<uint16_t>> keep16;
    std::vector<std::vector<float>> keep32;
    keep16.reserve(3 + 7 * t.layers.size());
    keep32.reserve(1 + 4 * t.layers.size());
    const uint16_t* embed = bf16_data(*t.embed, &keep16);
    const uint16_t* head = t.lm_head == t.embed ? embed : bf16_data(*t.lm_head, &keep16);
    const float* fnorm = f32_data(*t.final_norm, &keep32);
    std::vector<Yue2LayerWeights> layers(t.layers.size());
    for (size_t l = 0; l < t.layers.size(); ++l) {
        const auto& L = t.layers[l];
        Yue2LayerWeights& w = layers[l];
        w.q_proj = bf16_data(*L[0], &keep16);
        w.k_proj = bf16_data(*L[1], &keep16);
        w.v_proj = bf16_data(*L[2], &keep16);
        w.o_proj = bf16_data(*L[3], &keep16);
        w.gate_proj = bf16_data(*L[4], &keep16);
        w.up_proj = bf16_data(*L[5], &keep16);
        w.down_proj = bf16_data(*L[6], &keep16);
        w.input_layernorm = f32_data(*L[7], &keep32);
        w.q_norm = f32_data(*L[8], &keep32);
        w.k_norm = f32_data(*L[9], &keep32);
        w.post_attention_layernorm = f32_data(*L[10], &keep32);
    }
    // the weights are copied into device memory; the mappings close on return
    return yue2_hip_model_open(&ck.config, embed, head, fnorm, layers.data());
}
