// Hugging Face checkpoints for the engine: config.json and safetensors
// files (one, or the shards model.safetensors.index.json lists) of a
// Llama-family model, read into the host weight layout of
// tsl_weights_random (src/llm/safetensors.rs:190-358), and written back in
// the same layout Hugging Face uses (src/llm/safetensors.rs:362-444).
//
// Host code only: the tensors are converted to f16 bits on the CPU and the
// caller hands them to tsl_engine_new.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/tessel.h"

int tsl_fail(int code, const std::string& msg);

namespace {

typedef uint16_t u16;

// ---------------------------------------------------------------- JSON
// A JSON value; object members keep their file order.
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const std::string& k) const {
        if (kind != OBJ) return nullptr;
        for (auto& m : obj)
            if (m.first == k) return &m.second;
        return nullptr;
    }
};

struct JsonParser {
    const std::string& s;
    size_t i = 0;
    std::string err;

    explicit JsonParser(const std::string& text) : s(text) {}

    bool fail(const char* what) {
        if (err.empty()) err = std::string("json: ") + what + " at byte " + std::to_string(i);
        return false;
    }
    void skip() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) i++;
    }
    static void utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xc0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += (char)(0xe0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3f));
            out += (char)(0x80 | (cp & 0x3f));
        } else {
            out += (char)(0xf0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3f));
            out += (char)(0x80 | ((cp >> 6) & 0x3f));
            out += (char)(0x80 | (cp & 0x3f));
        }
    }
    bool hex4(uint32_t& v) {
        if (i + 4 > s.size()) return fail("short \\u escape");
        v = 0;
        for (int k = 0; k < 4; k++) {
            const char c = s[i++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string& out) {  // at the opening quote
        i++;
        while (true) {
            if (i >= s.size()) return fail("unterminated string");
            const char c = s[i++];
            if (c == '"') return true;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i >= s.size()) return fail("unterminated escape");
            const char e = s[i++];
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xd800 && cp < 0xdc00 && i + 1 < s.size() && s[i] == '\\' && s[i + 1] == 'u') {
                        i += 2;
                        uint32_t lo;
                        if (!hex4(lo)) return false;
                        if (lo >= 0xdc00 && lo < 0xe000) cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                        else return fail("bad surrogate pair");
                    }
                    utf8(out, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
    }
    bool value(Json& v, int depth) {
        if (depth > 256) return fail("nesting too deep");
        skip();
        if (i >= s.size()) return fail("unexpected end");
        const char c = s[i];
        if (c == '{') {
            v.kind = Json::OBJ;
            i++;
            skip();
            if (i < s.size() && s[i] == '}') {
                i++;
                return true;
            }
            while (true) {
                skip();
                if (i >= s.size() || s[i] != '"') return fail("expected a member name");
                std::string k;
                if (!string(k)) return false;
                skip();
                if (i >= s.size() || s[i] != ':') return fail("expected ':'");
                i++;
                v.obj.emplace_back(std::move(k), Json());
                if (!value(v.obj.back().second, depth + 1)) return false;
                skip();
                if (i < s.size() && s[i] == ',') {
                    i++;
                } else if (i < s.size() && s[i] == '}') {
                    i++;
                    return true;
                } else {
                    return fail("expected ',' or '}'");
                }
            }
        }
        if (c == '[') {
            v.kind = Json::ARR;
            i++;
            skip();
            if (i < s.size() && s[i] == ']') {
                i++;
                return true;
            }
            while (true) {
                v.arr.emplace_back();
                if (!value(v.arr.back(), depth + 1)) return false;
                skip();
                if (i < s.size() && s[i] == ',') {
                    i++;
                } else if (i < s.size() && s[i] == ']') {
                    i++;
                    return true;
                } else {
                    return fail("expected ',' or ']'");
                }
            }
        }
        if (c == '"') {
            v.kind = Json::STR;
            return string(v.str);
        }
        if (s.compare(i, 4, "true") == 0) {
            v.kind = Json::BOOL;
            v.b = true;
            i += 4;
            return true;
        }
        if (s.compare(i, 5, "false") == 0) {
            v.kind = Json::BOOL;
            i += 5;
            return true;
        }
        if (s.compare(i, 4, "null") == 0) {
            v.kind = Json::NUL;
            i += 4;
            return true;
        }
        // A number: -?digits(.digits)?([eE][+-]?digits)?
        const size_t st = i;
        if (i < s.size() && s[i] == '-') i++;
        auto digits = [&]() {
            const size_t d0 = i;
            while (i < s.size() && s[i] >= '0' && s[i] <= '9') i++;
            return i > d0;
        };
        if (!digits()) return fail("unexpected input");
        if (i < s.size() && s[i] == '.') {
            i++;
            if (!digits()) return fail("bad number");
        }
        if (i < s.size() && (s[i] == 'e' || s[i] == 'E')) {
            i++;
            if (i < s.size() && (s[i] == '+' || s[i] == '-')) i++;
            if (!digits()) return fail("bad number");
        }
        v.kind = Json::NUM;
        v.num = std::strtod(s.substr(st, i - st).c_str(), nullptr);
        return true;
    }
};

bool parse_json(const std::string& text, Json& out, std::string& err) {
    JsonParser p(text);
    if (!p.value(out, 0)) {
        err = p.err;
        return false;
    }
    p.skip();
    if (p.i != text.size()) {
        err = "json: trailing data at byte " + std::to_string(p.i);
        return false;
    }
    return true;
}

bool read_file(const std::string& path, std::string& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::ostringstream ss;
    ss << f.rdbuf();
    out = ss.str();
    return true;
}

bool exists(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    return (bool)f;
}

std::string join(const std::string& dir, const std::string& name) {
    if (dir.empty() || dir.back() == '/') return dir + name;
    return dir + "/" + name;
}

// Numeric casts the way the reference's `as` casts saturate.
int64_t sat_size(double x) { return !(x > 0) ? 0 : x >= 9.2e18 ? INT64_MAX : (int64_t)x; }
int32_t sat_i32(double x) {
    if (std::isnan(x)) return 0;
    if (x >= 2147483647.0) return INT32_MAX;
    if (x <= -2147483648.0) return INT32_MIN;
    return (int32_t)x;
}

// f32 -> f16 bits, round to nearest even; NaN becomes the quiet NaN with the
// input's sign, as src/half.rs does.
u16 f16_bits(float f) {
    if (std::isnan(f)) return (u16)((std::signbit(f) ? 0x8000 : 0) | 0x7e00);
    return __builtin_bit_cast(u16, (_Float16)f);
}

// ---------------------------------------------------------------- config.json
int read_config(const std::string& dir, tsl_config& c) {
    const std::string p = join(dir, "config.json");
    std::string text, err;
    if (!read_file(p, text)) return tsl_fail(TSL_ERR_ARG, p + ": cannot read");
    Json j;
    if (!parse_json(text, j, err)) return tsl_fail(TSL_ERR_ARG, err);
    auto num = [&](const char* k, double* v) {
        const Json* x = j.get(k);
        if (!x || x->kind != Json::NUM) return false;
        *v = x->num;
        return true;
    };
    auto num_or = [&](const char* k, double d) {
        double v;
        return num(k, &v) ? v : d;
    };
    if (const Json* rs = j.get("rope_scaling"))
        if (rs->kind != Json::NUL) return tsl_fail(TSL_ERR_ARG, "config.json: rope_scaling is not supported");
    double heads, dim, layers, ffn, vocab;
    if (!num("num_attention_heads", &heads)) return tsl_fail(TSL_ERR_ARG, "config.json: no num_attention_heads");
    if (!num("hidden_size", &dim)) return tsl_fail(TSL_ERR_ARG, "config.json: no hidden_size");
    int32_t eos = -1;
    if (const Json* e = j.get("eos_token_id")) {
        if (e->kind == Json::NUM) eos = sat_i32(e->num);
        else if (e->kind == Json::ARR)
            eos = sat_i32(!e->arr.empty() && e->arr[0].kind == Json::NUM ? e->arr[0].num : -1.0);
    }
    if (!num("num_hidden_layers", &layers)) return tsl_fail(TSL_ERR_ARG, "config.json: no num_hidden_layers");
    const int64_t h = sat_size(heads), d = sat_size(dim);
    const double kvh = num_or("num_key_value_heads", (double)h);
    const double hd = num_or("head_dim", (double)(h ? d / h : 0));
    if (!num("intermediate_size", &ffn)) return tsl_fail(TSL_ERR_ARG, "config.json: no intermediate_size");
    if (!num("vocab_size", &vocab)) return tsl_fail(TSL_ERR_ARG, "config.json: no vocab_size");
    auto small = [](int64_t v) { return v <= INT32_MAX; };
    const int64_t L = sat_size(layers), KV = sat_size(kvh), HD = sat_size(hd), F = sat_size(ffn), V = sat_size(vocab);
    if (!small(h) || !small(d) || !small(L) || !small(KV) || !small(HD) || !small(F) || !small(V))
        return tsl_fail(TSL_ERR_ARG, "config.json: a size does not fit in 32 bits");
    c.dim = (int32_t)d;
    c.layers = (int32_t)L;
    c.heads = (int32_t)h;
    c.kv_heads = (int32_t)KV;
    c.head_dim = (int32_t)HD;
    c.ffn = (int32_t)F;
    c.vocab = (int32_t)V;
    c.eps = (float)num_or("rms_norm_eps", 1e-6);
    c.rope_theta = (float)num_or("rope_theta", 10000.0);
    c.max_pos = (int32_t)std::min<int64_t>(sat_size(num_or("max_position_embeddings", 2048.0)), 8192);
    c.bos = sat_i32(num_or("bos_token_id", 1.0));
    c.eos = eos;
    return 0;
}

// ---------------------------------------------------------------- safetensors
struct Entry {
    std::string file, dtype;
    std::vector<int64_t> shape;
    uint64_t start = 0, end = 0;  // absolute byte range in the file
};

std::string shape_str(const std::vector<int64_t>& s) {  // "[a, b]"
    std::string r = "[";
    for (size_t i = 0; i < s.size(); i++) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

// Every tensor of the checkpoint's safetensors files, by name (a name in
// several shards: the last shard in name order wins).
int index(const std::string& dir, std::map<std::string, Entry>& out) {
    std::vector<std::string> files;
    const std::string single = join(dir, "model.safetensors");
    if (exists(single)) {
        files.push_back(single);
    } else {
        const std::string p = join(dir, "model.safetensors.index.json");
        std::string text, err;
        if (!read_file(p, text)) return tsl_fail(TSL_ERR_ARG, p + ": cannot read");
        Json j;
        if (!parse_json(text, j, err)) return tsl_fail(TSL_ERR_ARG, err);
        const Json* wm = j.get("weight_map");
        if (!wm || wm->kind != Json::OBJ) return tsl_fail(TSL_ERR_ARG, "index: no weight_map");
        for (auto& m : wm->obj)
            if (m.second.kind == Json::STR) files.push_back(join(dir, m.second.str));
        std::sort(files.begin(), files.end());
        files.erase(std::unique(files.begin(), files.end()), files.end());
    }
    for (auto& file : files) {
        std::ifstream f(file, std::ios::binary);
        if (!f) return tsl_fail(TSL_ERR_ARG, file + ": cannot read");
        unsigned char len[8];
        if (!f.read(reinterpret_cast<char*>(len), 8)) return tsl_fail(TSL_ERR_ARG, file + ": short header");
        uint64_t n = 0;
        for (int b = 7; b >= 0; b--) n = (n << 8) | len[b];
        if (n > (1ull << 31)) return tsl_fail(TSL_ERR_ARG, file + ": header too large");
        std::string head(n, '\0');
        if (!f.read(&head[0], (std::streamsize)n)) return tsl_fail(TSL_ERR_ARG, file + ": short header");
        Json j;
        std::string err;
        if (!parse_json(head, j, err)) return tsl_fail(TSL_ERR_ARG, err);
        if (j.kind != Json::OBJ) return tsl_fail(TSL_ERR_ARG, "safetensors: bad header");
        for (auto& m : j.obj) {
            if (m.first == "__metadata__") continue;
            Entry e;
            e.file = file;
            if (const Json* d = m.second.get("dtype"))
                if (d->kind == Json::STR) e.dtype = d->str;
            if (const Json* s = m.second.get("shape"))
                if (s->kind == Json::ARR)
                    for (auto& x : s->arr) e.shape.push_back(x.kind == Json::NUM ? sat_size(x.num) : 0);
            const Json* off = m.second.get("data_offsets");
            if (!off || off->kind != Json::ARR || off->arr.size() != 2)
                return tsl_fail(TSL_ERR_ARG, m.first + ": no data_offsets");
            if (off->arr[0].kind != Json::NUM || off->arr[1].kind != Json::NUM)
                return tsl_fail(TSL_ERR_ARG, "bad offset");
            e.start = 8 + n + (uint64_t)sat_size(off->arr[0].num);
            e.end = 8 + n + (uint64_t)sat_size(off->arr[1].num);
            out[m.first] = std::move(e);
        }
    }
    return 0;
}

// Tensor `name`, checked against `shape`, as f16 bits into out.
int read_tensor(const std::map<std::string, Entry>& ix, const std::string& name, const std::vector<int64_t>& shape,
                u16* out) {
    auto it = ix.find(name);
    if (it == ix.end()) return tsl_fail(TSL_ERR_ARG, "checkpoint has no " + name);
    const Entry& e = it->second;
    if (e.shape != shape)
        return tsl_fail(TSL_ERR_ARG, name + ": shape " + shape_str(e.shape) + ", expected " + shape_str(shape));
    int64_t n = 1;
    for (auto d : shape) n *= d;
    const uint64_t bytes = e.end >= e.start ? e.end - e.start : 0;
    const int esz = e.dtype == "F32" ? 4 : (e.dtype == "F16" || e.dtype == "BF16") ? 2 : 0;
    if (esz == 0 || bytes != (uint64_t)(esz * n)) return tsl_fail(TSL_ERR_ARG, name + ": dtype " + e.dtype + " not supported");
    std::ifstream f(e.file, std::ios::binary);
    std::vector<unsigned char> b(bytes);
    if (!f || !f.seekg((std::streamoff)e.start) || !f.read(reinterpret_cast<char*>(b.data()), (std::streamsize)bytes))
        return tsl_fail(TSL_ERR_ARG, name + ": cannot read " + std::to_string(bytes) + " bytes of " + e.file);
    for (int64_t i = 0; i < n; i++) {
        if (e.dtype == "F16") {
            out[i] = (u16)(b[2 * i] | (b[2 * i + 1] << 8));
        } else if (e.dtype == "BF16") {
            const uint32_t w = (uint32_t)(b[2 * i] | (b[2 * i + 1] << 8)) << 16;
            out[i] = f16_bits(__builtin_bit_cast(float, w));
        } else {
            const uint32_t w = (uint32_t)b[4 * i] | ((uint32_t)b[4 * i + 1] << 8) | ((uint32_t)b[4 * i + 2] << 16) |
                               ((uint32_t)b[4 * i + 3] << 24);
            out[i] = f16_bits(__builtin_bit_cast(float, w));
        }
    }
    return 0;
}

bool same_config(const tsl_config& a, const tsl_config& b) {
    return a.dim == b.dim && a.layers == b.layers && a.heads == b.heads && a.kv_heads == b.kv_heads &&
           a.head_dim == b.head_dim && a.ffn == b.ffn && a.vocab == b.vocab;
}

std::string fmt_float(double x) {  // shortest round-trip decimal
    char buf[64];
    for (int p = 1; p <= 17; p++) {
        std::snprintf(buf, sizeof buf, "%.*g", p, x);
        if (std::strtod(buf, nullptr) == x) break;
    }
    std::string s = buf;
    if (s.find_first_of(".eEn") == std::string::npos) s += ".0";
    return s;
}

}  // namespace

extern "C" {

int tsl_checkpoint_config(const char* dir, tsl_config* cfg) {
    if (!dir || !cfg) return tsl_fail(TSL_ERR_ARG, "tsl_checkpoint_config: null argument");
    tsl_config c{};
    int r = read_config(dir, c);
    if (r) return r;
    *cfg = c;
    return 0;
}

int tsl_checkpoint_load(const char* dir, const tsl_config* cfg, uint16_t* embed, uint16_t* layers, uint16_t* norm,
                        uint16_t* head, int* has_head) {
    if (!dir || !cfg || !embed || !layers || !norm || !has_head)
        return tsl_fail(TSL_ERR_ARG, "tsl_checkpoint_load: null argument");
    tsl_config c{};
    int r = read_config(dir, c);
    if (r) return r;
    if (!same_config(c, *cfg))
        return tsl_fail(TSL_ERR_ARG, "tsl_checkpoint_load: cfg differs from the checkpoint's config.json");
    std::map<std::string, Entry> ix;
    if ((r = index(dir, ix))) return r;
    for (auto& kv : ix) {
        const std::string& k = kv.first;
        if (k.size() >= 5 && k.compare(k.size() - 5, 5, ".bias") == 0)
            return tsl_fail(TSL_ERR_ARG, k + ": models with biases are not supported");
    }
    const int64_t dm = c.dim, hd = c.head_dim, qd = (int64_t)c.heads * hd, kd = (int64_t)c.kv_heads * hd;
    u16* p = layers;
    for (int i = 0; i < c.layers; i++) {
        const std::string pre = "model.layers." + std::to_string(i) + ".";
        // Layer layout: attn_norm, wqkv (q; k; v rows), wo, mlp_norm, wg, wu, wd.
        u16* attn_norm = p;
        u16* wqkv = attn_norm + dm;
        u16* wo = wqkv + (qd + 2 * kd) * dm;
        u16* mlp_norm = wo + dm * qd;
        u16* wg = mlp_norm + dm;
        u16* wu = wg + (int64_t)c.ffn * dm;
        u16* wd = wu + (int64_t)c.ffn * dm;
        p = wd + dm * c.ffn;
        if ((r = read_tensor(ix, pre + "self_attn.q_proj.weight", {qd, dm}, wqkv)) ||
            (r = read_tensor(ix, pre + "self_attn.k_proj.weight", {kd, dm}, wqkv + qd * dm)) ||
            (r = read_tensor(ix, pre + "self_attn.v_proj.weight", {kd, dm}, wqkv + (qd + kd) * dm)) ||
            (r = read_tensor(ix, pre + "input_layernorm.weight", {dm}, attn_norm)) ||
            (r = read_tensor(ix, pre + "self_attn.o_proj.weight", {dm, qd}, wo)) ||
            (r = read_tensor(ix, pre + "post_attention_layernorm.weight", {dm}, mlp_norm)) ||
            (r = read_tensor(ix, pre + "mlp.gate_proj.weight", {c.ffn, dm}, wg)) ||
            (r = read_tensor(ix, pre + "mlp.up_proj.weight", {c.ffn, dm}, wu)) ||
            (r = read_tensor(ix, pre + "mlp.down_proj.weight", {dm, c.ffn}, wd)))
            return r;
    }
    *has_head = ix.count("lm_head.weight") ? 1 : 0;
    if (*has_head) {
        if (!head) return tsl_fail(TSL_ERR_ARG, "tsl_checkpoint_load: the checkpoint has lm_head.weight; head is null");
        if ((r = read_tensor(ix, "lm_head.weight", {c.vocab, dm}, head))) return r;
    }
    if ((r = read_tensor(ix, "model.embed_tokens.weight", {c.vocab, dm}, embed))) return r;
    return read_tensor(ix, "model.norm.weight", {dm}, norm);
}

int tsl_checkpoint_save(const char* dir, const tsl_config* cfg, const uint16_t* embed, const uint16_t* layers,
                        const uint16_t* norm, const uint16_t* head) {
    if (!dir || !cfg || !embed || !layers || !norm) return tsl_fail(TSL_ERR_ARG, "tsl_checkpoint_save: null argument");
    const tsl_config& c = *cfg;
    std::ostringstream js;
    js << "{\"model_type\": \"llama\", \"hidden_size\": " << c.dim << ", \"num_hidden_layers\": " << c.layers
       << ", \"num_attention_heads\": " << c.heads << ", \"num_key_value_heads\": " << c.kv_heads
       << ", \"head_dim\": " << c.head_dim << ", \"intermediate_size\": " << c.ffn << ", \"vocab_size\": " << c.vocab
       << ", \"rms_norm_eps\": " << fmt_float(c.eps) << ", \"rope_theta\": " << fmt_float(c.rope_theta)
       << ", \"max_position_embeddings\": " << c.max_pos << ", \"bos_token_id\": " << c.bos
       << ", \"eos_token_id\": " << c.eos << ", \"rope_scaling\": null, \"tie_word_embeddings\": "
       << (head ? "false" : "true") << "}";
    {
        std::ofstream f(join(dir, "config.json"), std::ios::binary);
        if (!f) return tsl_fail(TSL_ERR_ARG, join(dir, "config.json") + ": cannot write");
        f << js.str();
        if (!f) return tsl_fail(TSL_ERR_ARG, join(dir, "config.json") + ": write failed");
    }
    struct T {
        std::string name;
        std::vector<int64_t> shape;
        const u16* data;
        int64_t n;
    };
    const int64_t dm = c.dim, hd = c.head_dim, qd = (int64_t)c.heads * hd, kd = (int64_t)c.kv_heads * hd;
    std::vector<T> ts = {{"model.embed_tokens.weight", {c.vocab, dm}, embed, (int64_t)c.vocab * dm},
                         {"model.norm.weight", {dm}, norm, dm}};
    if (head) ts.push_back({"lm_head.weight", {c.vocab, dm}, head, (int64_t)c.vocab * dm});
    const u16* p = layers;
    for (int i = 0; i < c.layers; i++) {
        const std::string pre = "model.layers." + std::to_string(i) + ".";
        const u16* attn_norm = p;
        const u16* wqkv = attn_norm + dm;
        const u16* wo = wqkv + (qd + 2 * kd) * dm;
        const u16* mlp_norm = wo + dm * qd;
        const u16* wg = mlp_norm + dm;
        const u16* wu = wg + (int64_t)c.ffn * dm;
        const u16* wd = wu + (int64_t)c.ffn * dm;
        p = wd + dm * c.ffn;
        ts.push_back({pre + "input_layernorm.weight", {dm}, attn_norm, dm});
        ts.push_back({pre + "self_attn.q_proj.weight", {qd, dm}, wqkv, qd * dm});
        ts.push_back({pre + "self_attn.k_proj.weight", {kd, dm}, wqkv + qd * dm, kd * dm});
        ts.push_back({pre + "self_attn.v_proj.weight", {kd, dm}, wqkv + (qd + kd) * dm, kd * dm});
        ts.push_back({pre + "self_attn.o_proj.weight", {dm, qd}, wo, dm * qd});
        ts.push_back({pre + "post_attention_layernorm.weight", {dm}, mlp_norm, dm});
        ts.push_back({pre + "mlp.gate_proj.weight", {c.ffn, dm}, wg, (int64_t)c.ffn * dm});
        ts.push_back({pre + "mlp.up_proj.weight", {c.ffn, dm}, wu, (int64_t)c.ffn * dm});
        ts.push_back({pre + "mlp.down_proj.weight", {dm, c.ffn}, wd, dm * c.ffn});
    }
    std::string hdr = "{";
    int64_t off = 0;
    for (size_t i = 0; i < ts.size(); i++) {
        const int64_t nb = 2 * ts[i].n;
        hdr += (i ? ", \"" : "\"") + ts[i].name + "\": {\"dtype\": \"F16\", \"shape\": " + shape_str(ts[i].shape) +
               ", \"data_offsets\": [" + std::to_string(off) + ", " + std::to_string(off + nb) + "]}";
        off += nb;
    }
    hdr += "}";
    while (hdr.size() % 8) hdr += ' ';
    const std::string path = join(dir, "model.safetensors");
    std::ofstream f(path, std::ios::binary);
    if (!f) return tsl_fail(TSL_ERR_ARG, path + ": cannot write");
    unsigned char len[8];
    uint64_t n = hdr.size();
    for (int b = 0; b < 8; b++) len[b] = (unsigned char)(n >> (8 * b));
    f.write(reinterpret_cast<const char*>(len), 8);
    f.write(hdr.data(), (std::streamsize)hdr.size());
    std::vector<unsigned char> buf;
    for (auto& t : ts) {
        buf.resize(2 * t.n);
        for (int64_t i = 0; i < t.n; i++) {
            buf[2 * i] = (unsigned char)(t.data[i] & 0xff);
            buf[2 * i + 1] = (unsigned char)(t.data[i] >> 8);
        }
        f.write(reinterpret_cast<const char*>(buf.data()), (std::streamsize)buf.size());
    }
    if (!f) return tsl_fail(TSL_ERR_ARG, path + ": write failed");
    return 0;
}

// A JSON text re-emitted after parsing (strings with escapes decoded and
// re-encoded), for testing the parser: 0 and the length in *len (the text
// in out when it fits), or TSL_ERR_ARG with the parse error.
int tsl_json_roundtrip(const char* text, char* out, size_t cap, size_t* len) {
    if (!text || !len) return tsl_fail(TSL_ERR_ARG, "tsl_json_roundtrip: null argument");
    Json j;
    std::string err;
    if (!parse_json(text, j, err)) return tsl_fail(TSL_ERR_ARG, err);
    struct W {
        static void str(std::string& o, const std::string& s) {
            o += '"';
            for (unsigned char ch : s) {
                if (ch == '"') o += "\\\"";
                else if (ch == '\\') o += "\\\\";
                else if (ch < 0x20) {
                    char b[8];
                    std::snprintf(b, sizeof b, "\\u%04x", ch);
                    o += b;
                } else o += (char)ch;
            }
            o += '"';
        }
        static void val(std::string& o, const Json& v) {
            switch (v.kind) {
                case Json::NUL: o += "null"; break;
                case Json::BOOL: o += v.b ? "true" : "false"; break;
                case Json::NUM: o += fmt_float(v.num); break;
                case Json::STR: str(o, v.str); break;
                case Json::ARR:
                    o += '[';
                    for (size_t i = 0; i < v.arr.size(); i++) {
                        if (i) o += ", ";
                        val(o, v.arr[i]);
                    }
                    o += ']';
                    break;
                case Json::OBJ:
                    o += '{';
                    for (size_t i = 0; i < v.obj.size(); i++) {
                        if (i) o += ", ";
                        str(o, v.obj[i].first);
                        o += ": ";
                        val(o, v.obj[i].second);
                    }
                    o += '}';
                    break;
            }
        }
    };
    std::string o;
    W::val(o, j);
    *len = o.size();
    if (out && cap > o.size()) std::memcpy(out, o.c_str(), o.size() + 1);
    return 0;
}

}  // extern "C"
