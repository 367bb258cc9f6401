// The LLM engine on the C ABI: a Llama-family decoder whose GPU work is
// only the llm.tl kernels, with a paged KV cache and continuous batching.
//
//   Config / Weights::random / rope_tables            src/llm/mod.rs:15-129
//   (argmax, :132-140, is the GPU's fused/argmax)
//   Engine::new / mm (tuner) / step / launch_all      src/llm/engine.rs:150-529
//   sched::generate_with                              src/llm/sched.rs:52-179
//
// Host code only: every kernel is reached through tsl_kernel/tsl_launch, so
// the engine drives exactly the launch surface a Rust caller would.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/tessel.h"

int tsl_fail(int code, const std::string& msg);
int rt_event_rerecord(int id);
int rt_host_alloc(size_t n, void** p);
int rt_host_free(void* p);
int rt_upload_async(uint64_t dst, const void* pinned, size_t n);
int rt_download_pinned(void* pinned, uint64_t src, size_t n);

namespace {

typedef uint16_t u16;

// ---------------------------------------------------------------- src/llm/mod.rs

struct Rng {  // src/bench.rs:13-35
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9e3779b97f4a7c15ull | 1ull) {}
    uint64_t bits() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return s;
    }
    float uniform() { return ((float)(bits() >> 40) / (float)(1ull << 24)) * 2.0f - 1.0f; }
};

u16 to_f16(float f) { return __builtin_bit_cast(u16, (_Float16)f); }  // round to nearest even
float from_f16(u16 h) { return (float)__builtin_bit_cast(_Float16, h); }

int64_t qkv_rows(const tsl_config& c) { return (int64_t)(c.heads + 2 * c.kv_heads) * c.head_dim; }
int64_t layer_elems(const tsl_config& c) {
    int64_t d = c.dim, hd = (int64_t)c.heads * c.head_dim;
    return d + qkv_rows(c) * d + d * hd + d + 2 * (int64_t)c.ffn * d + d * c.ffn;
}

void rope_tables(const tsl_config& c, std::vector<float>& cs, std::vector<float>& sn) {
    int64_t h = c.head_dim / 2;
    cs.resize((size_t)c.max_pos * h);
    sn.resize(cs.size());
    for (int64_t p = 0; p < c.max_pos; p++)
        for (int64_t i = 0; i < h; i++) {
            double inv = std::pow((double)c.rope_theta, -((double)(2 * i)) / (double)c.head_dim);
            double a = (double)p * inv;
            cs[p * h + i] = (float)std::cos(a);
            sn[p * h + i] = (float)std::sin(a);
        }
}

// ---------------------------------------------------------------- the engine

struct Buf {
    uint64_t p = 0;
    size_t bytes = 0;
};

struct Layer {
    Buf n1, wqkv, wo, n2, wg, wu, wd, kc, vc;
};

enum Mode { PREFILL = 0, PACKED = 1, DECODE = 2 };

struct Arg {  // src/gpu.rs:22-26
    enum { BUF, F32 } kind;
    uint64_t v;
};

size_t padded(size_t n) {  // src/llm/engine.rs:96-98
    size_t t = std::max<size_t>(n, 16), p = 1;
    while (p < t) p <<= 1;
    return p;
}

typedef std::vector<std::pair<std::string, int64_t>> Meta;

// src/llm/engine.rs:106-147: the tile configurations tried for an m-row matmul.
std::vector<std::pair<Meta, int>> mm_candidates(size_t m, bool two) {
    auto c = [](int64_t bm, int64_t bn, int64_t bk, int w) {
        return std::make_pair(Meta{{"BM", bm}, {"BN", bn}, {"BK", bk}}, w);
    };
    if (m >= 64) {
        if (two) return {c(64, 64, 32, 4), c(128, 64, 32, 4), c(64, 32, 32, 4)};
        return {c(64, 128, 32, 4), c(64, 64, 32, 4), c(128, 128, 32, 4), c(128, 64, 32, 4)};
    }
    if (m >= 32) {
        std::vector<std::pair<Meta, int>> v = {c(32, 64, 64, 4),  c(32, 32, 64, 4), c(32, 32, 128, 4),
                                               c(32, 64, 128, 4), c(32, 16, 128, 2), c(16, 64, 64, 4),
                                               c(16, 32, 128, 4)};
        if (!two) v.push_back(c(32, 16, 256, 2));
        return v;
    }
    return {c(16, 64, 64, 4), c(16, 32, 64, 4), c(16, 32, 128, 4), c(16, 64, 128, 4), c(16, 16, 128, 2),
            c(16, 16, 256, 2)};
}

#define TRY(x)             \
    do {                   \
        int _r = (x);      \
        if (_r) return _r; \
    } while (0)

struct Engine {
    tsl_config cfg;
    tsl_limits lim;
    bool graphs = true, tune = true;
    // Gpu::profile (src/gpu.rs:40, :197-217): when on, every launch is timed
    // on its own and summed per (phase, "{name} -> {output shape}").
    bool profiling = false;
    const char* phase = "decode";
    std::map<std::pair<std::string, std::string>, std::pair<int64_t, double>> prof;
    std::map<int, std::string> kname;
    std::map<size_t, int> graph;
    std::map<std::string, int> tuned;
    Buf embed, head, norm, cos, sin;
    std::vector<Layer> layers;
    Buf x, h, ss, qkv, q, k, v, o, mlp, last, logits, tok, pos, slot, idx, table, lens, starts, next;
    // outw: the deferred-norm overflow flag (word 0), then at byte 16 the
    // step's token ids (next), so one download returns both.
    Buf outw, ovf;
    // Set while a step is recomputed with every rmsnorm applied before its
    // projection (after the deferred form overflowed f16).
    bool plain = false;
    int64_t prenorm_fallbacks = 0;
    // Decode-step timing (tsl_engine_step_times): the GPU span of each
    // decode step, from its input upload to the end of its last kernel, by
    // a pair of events; [0] graph replays, [1] eager launches.
    bool time_steps = false;
    int ev0 = -1, ev1 = -1;
    int64_t timed_steps[2] = {0, 0};
    double timed_ms[2] = {0.0, 0.0};
    // One device arena for a step's inputs, filled by one upload: for a step
    // of t (padded) rows, tok, pos, slot, idx, starts, lens (t ints each),
    // then table (t max_seq_pages ints). layout(t) points the buffers there;
    // the addresses depend only on t, so a graph captured for t stays valid.
    Buf in;
    // Pinned host staging: a step's inputs (enqueued without a wait: the
    // step's download synchronises before the next step rewrites them) and
    // its flag and token ids (one enqueued copy, one wait).
    int32_t* hin = nullptr;
    int32_t* hout = nullptr;
    void layout(size_t t) {
        const size_t mp = lim.max_seq_pages;
        Buf* parts[] = {&tok, &pos, &slot, &idx, &starts, &lens};
        for (int i = 0; i < 6; i++) *parts[i] = Buf{in.p + (uint64_t)i * t * 4, t * 4};
        table = Buf{in.p + 6 * t * 4, t * mp * 4};
    }

    int alloc(size_t bytes, Buf& b) {
        b.bytes = bytes;
        return tsl_alloc(bytes, &b.p);
    }
    int write(const Buf& b, size_t off, const void* data, size_t n) {
        if (off + n > b.bytes) {
            std::ostringstream e;
            e << "write of " << n << " bytes at " << off << " into a buffer of " << b.bytes;
            return tsl_fail(TSL_ERR_ARG, e.str());
        }
        return tsl_upload(b.p + off, data, n);
    }
    int up16(const u16* v, size_t n, Buf& b) {
        TRY(alloc(n * 2, b));
        return write(b, 0, v, n * 2);
    }

    int kernel(const char* name, const std::vector<std::vector<int64_t>>& shapes, const Meta& meta, int warps,
               int* handle, const char* file = "llm") {
        std::vector<int> ranks;
        std::vector<int64_t> dims;
        for (auto& s : shapes) {
            ranks.push_back((int)s.size());
            dims.insert(dims.end(), s.begin(), s.end());
        }
        std::vector<const char*> names;
        std::vector<int64_t> vals;
        for (auto& m : meta) {
            names.push_back(m.first.c_str());
            vals.push_back(m.second);
        }
        int r = tsl_kernel(file, name, (int)shapes.size(), ranks.data(), dims.data(), (int)meta.size(), names.data(),
                           vals.data(), warps, handle);
        if (r == 0 && !kname.count(*handle)) {  // src/gpu.rs:168-169
            std::ostringstream o;
            o << name << " -> [";
            const auto& last = shapes.back();
            for (size_t i = 0; i < last.size(); i++) o << (i ? ", " : "") << last[i];
            o << "]";
            kname[*handle] = o.str();
        }
        return r;
    }

    int launch(int k, const std::vector<Arg>& args) {
        std::vector<uint64_t> raw;
        for (auto& a : args) raw.push_back(a.v);
        if (!profiling) return tsl_launch(k, raw.data(), (int)raw.size());
        float ms = 0.0f;
        TRY(tsl_time_each(k, raw.data(), (int)raw.size(), 1, &ms));
        auto& e = prof[{phase, kname[k]}];
        e.first += 1;
        e.second += ms;
        return 0;
    }

    // Engine::mm (src/llm/engine.rs:233-270). The reference times each tile
    // configuration of mm_candidates and keeps the fastest. Here the llm
    // projections' launchers choose their tiles from the shape (decode-sized
    // rows: the weight-streaming skinny kernel with its K split; prompt-sized
    // rows: the 64x128 / 128x128 / 256x128 MFMA tiles and K slices), and
    // the BM/BN/BK of a candidate's meta only enters its cache key: every
    // candidate is the same code. So the default candidate is specialised
    // once, nothing is timed, and `tune` changes nothing.
    int mm(const char* name, const std::vector<std::vector<int64_t>>& shapes, bool two, const std::vector<Arg>& args,
           int* out) {
        (void)args;
        std::ostringstream key;
        key << name << " [";
        for (size_t i = 0; i < shapes.size(); i++) {
            key << (i ? ", " : "") << "[";
            for (size_t j = 0; j < shapes[i].size(); j++) key << (j ? ", " : "") << shapes[i][j];
            key << "]";
        }
        key << "]";
        auto it = tuned.find(key.str());
        if (it != tuned.end()) {
            *out = it->second;
            return 0;
        }
        auto cands = mm_candidates((size_t)shapes[0][0], two);
        int pick = -1;
        TRY(kernel(name, shapes, cands[0].first, cands[0].second, &pick));
        tuned[key.str()] = pick;
        *out = pick;
        return 0;
    }

    int init(const tsl_config& c, const tsl_limits& l, const u16* w_embed, const u16* w_layers, const u16* w_norm,
             const u16* w_head) {
        cfg = c;
        lim = l;
        if (cfg.kv_heads <= 0 || cfg.heads % cfg.kv_heads != 0 || cfg.head_dim % 2 != 0)
            return tsl_fail(TSL_ERR_ARG, "heads must be a multiple of kv_heads, head_dim even");
        size_t d = cfg.dim;
        TRY(up16(w_embed, (size_t)cfg.vocab * d, embed));
        if (w_head) TRY(up16(w_head, (size_t)cfg.vocab * d, head));
        else head = embed;
        TRY(up16(w_norm, d, norm));
        size_t slots = (size_t)lim.pages * lim.page;
        size_t kv_bytes = slots * cfg.kv_heads * cfg.head_dim * 2;
        const u16* p = w_layers;
        size_t hd = (size_t)cfg.heads * cfg.head_dim, qr = qkv_rows(cfg), ff = cfg.ffn;
        for (int i = 0; i < cfg.layers; i++) {
            Layer L;
            TRY(up16(p, d, L.n1));
            p += d;
            TRY(up16(p, qr * d, L.wqkv));
            p += qr * d;
            TRY(up16(p, d * hd, L.wo));
            p += d * hd;
            TRY(up16(p, d, L.n2));
            p += d;
            TRY(up16(p, ff * d, L.wg));
            p += ff * d;
            TRY(up16(p, ff * d, L.wu));
            p += ff * d;
            TRY(up16(p, d * ff, L.wd));
            p += d * ff;
            TRY(alloc(kv_bytes, L.kc));
            TRY(alloc(kv_bytes, L.vc));
            layers.push_back(L);
        }
        std::vector<float> cs, sn;
        rope_tables(cfg, cs, sn);
        TRY(alloc(cs.size() * 4, cos));
        TRY(write(cos, 0, cs.data(), cs.size() * 4));
        TRY(alloc(sn.size() * 4, sin));
        TRY(write(sin, 0, sn.data(), sn.size() * 4));
        size_t t = padded(lim.max_tokens);
        size_t gd = (size_t)cfg.kv_heads * cfg.head_dim;
        TRY(alloc(t * d * 4, x));
        TRY(alloc(t * d * 2, h));
        TRY(alloc(t * ((d + 7) / 8) * 4, ss));
        TRY(alloc(t * qr * 2, qkv));
        TRY(alloc(t * hd * 2, q));
        TRY(alloc(t * gd * 2, k));
        TRY(alloc(t * gd * 2, v));
        TRY(alloc(t * hd * 2, o));
        TRY(alloc(t * ff * 2, mlp));
        TRY(alloc(t * d * 2, last));
        TRY(alloc(t * (size_t)cfg.vocab * 4, logits));
        TRY(alloc(t * (6 + (size_t)lim.max_seq_pages) * 4, in));
        TRY(rt_host_alloc(t * (6 + (size_t)lim.max_seq_pages) * 4, reinterpret_cast<void**>(&hin)));
        TRY(rt_host_alloc(16 + t * 4, reinterpret_cast<void**>(&hout)));
        TRY(alloc(16 + t * 4, outw));
        ovf = Buf{outw.p, 4};
        next = Buf{outw.p + 16, t * 4};
        const int32_t zero = 0;
        TRY(write(ovf, 0, &zero, 4));
        return 0;
    }

    // Decode steps of up to 32 rows defer each rmsnorm into the projection
    // that consumes it (launch_all), unless the step is being recomputed.
    bool uses_prenorm(size_t t, bool prefill) const { return !prefill && t <= 32 && !plain; }

    // Engine::launch_all (src/llm/engine.rs:359-529).
    int launch_all(size_t t, bool prefill, size_t bw) {
        int64_t dm = cfg.dim, nh = cfg.heads, ng = cfg.kv_heads, hd = cfg.head_dim;
        int64_t w = qkv_rows(cfg), f = cfg.ffn, vv = cfg.vocab;
        int64_t ns = (int64_t)lim.pages * lim.page, mp = lim.max_seq_pages, T = (int64_t)t;
        int64_t bc = 1;
        while (bc < dm) bc <<= 1;
        float scale = 1.0f / std::sqrt((float)hd);
        uint64_t scale_bits = 0, eps_bits = 0;
        std::memcpy(&scale_bits, &scale, 4);
        std::memcpy(&eps_bits, &cfg.eps, 4);
        auto B = [](const Buf& b) { return Arg{Arg::BUF, b.p}; };
        Arg SC{Arg::F32, scale_bits}, EPS{Arg::F32, eps_bits};
        int embed_k, norm_k, qkv_k, att_k, gu_k, down_k;
        TRY(kernel("embed", {{T}, {vv, dm}, {T, dm}}, {{"BD", std::min<int64_t>(bc, 1024)}}, 4, &embed_k));
        TRY(kernel("rmsnorm", {{T, dm}, {dm}, {T, dm}}, {{"BC", bc}}, 4, &norm_k));
        const Layer& l0 = layers[0];
        int64_t npos = cfg.max_pos;
        // llm/linear (QKV), then llm/rope_q and llm/kv_write (src/llm/engine.rs
        // launch order), as one launch sequence: fused/qkv_rope_kv.
        TRY(kernel("qkv_rope_kv",
                   {{T, dm}, {w, dm}, {T, w}, {T}, {T}, {npos, hd / 2}, {npos, hd / 2}, {T, nh, hd}, {ns, ng, hd},
                    {ns, ng, hd}, {T, ng, hd}, {T, ng, hd}},
                   {}, 4, &qkv_k, "fused"));
        if (prefill) {
            TRY(kernel("prefill_attention", {{T, nh, hd}, {T, ng, hd}, {T, ng, hd}, {T}, {T, nh, hd}},
                       {{"BM", 64}, {"BN", 64}}, 4, &att_k));
        } else {
            int64_t p = lim.page;
            TRY(kernel("decode_attention",
                       {{T, nh, hd}, {lim.pages, p, ng, hd}, {lim.pages, p, ng, hd}, {T, mp}, {T}, {T, nh, hd}}, {}, 1,
                       &att_k));
        }
        TRY(mm("gate_up", {{T, dm}, {f, dm}, {f, dm}, {T, f}}, true, {B(h), B(l0.wg), B(l0.wu), B(mlp)}, &gu_k));
        TRY(mm("linear_residual", {{T, f}, {dm, f}, {T, dm}}, false, {B(mlp), B(l0.wd), B(x)}, &down_k));
        // A residual projection and the rmsnorm that follows it, as one
        // launch sequence (fused/linear_residual_rmsnorm): the o projection
        // with mlp_norm, and the down projection with the next layer's
        // attn_norm.
        int oproj_norm_k, down_norm_k;
        TRY(kernel("linear_residual_rmsnorm", {{T, nh * hd}, {dm, nh * hd}, {T, dm}, {dm}, {T, dm}}, {{"BC", bc}}, 4,
                   &oproj_norm_k, "fused"));
        TRY(kernel("linear_residual_rmsnorm", {{T, f}, {dm, f}, {T, dm}, {dm}, {T, dm}}, {{"BC", bc}}, 4,
                   &down_norm_k, "fused"));
        // Decode steps of up to 32 rows defer each rmsnorm into the projection
        // that consumes it: the residual projections leave Y = f16(R Wn) and
        // per-8-column sums of squares of R (fused/linear_residual_prenorm),
        // and gate_up / the next layer's QKV scale their rows by 1 / rms
        // (fused/gate_up_rs, fused/qkv_rs_rope_kv): no normalisation launch
        // between the two, and no second pass over R.
        const bool prenorm = uses_prenorm(t, prefill);
        const int64_t nb8 = (dm + 7) / 8;
        int o_pre_k = -1, down_pre_k = -1, gu_rs_k = -1, qkv_rs_k = -1;
        if (prenorm) {
            TRY(kernel("linear_residual_prenorm", {{T, nh * hd}, {dm, nh * hd}, {T, dm}, {dm}, {T, dm}, {nb8, T}, {1}},
                       {}, 4, &o_pre_k, "fused"));
            TRY(kernel("linear_residual_prenorm", {{T, f}, {dm, f}, {T, dm}, {dm}, {T, dm}, {nb8, T}, {1}}, {}, 4,
                       &down_pre_k, "fused"));
            TRY(kernel("gate_up_rs", {{T, dm}, {nb8, T}, {f, dm}, {f, dm}, {T, f}}, {}, 4, &gu_rs_k, "fused"));
            TRY(kernel("qkv_rs_rope_kv",
                       {{T, dm}, {w, dm}, {T, w}, {T}, {T}, {npos, hd / 2}, {npos, hd / 2}, {T, nh, hd}, {ns, ng, hd},
                        {ns, ng, hd}, {T, ng, hd}, {T, ng, hd}, {nb8, T}},
                       {}, 4, &qkv_rs_k, "fused"));
        }

        TRY(launch(embed_k, {B(tok), B(embed), B(x)}));
        TRY(launch(norm_k, {B(x), B(layers[0].n1), B(h), EPS}));
        for (size_t li = 0; li < layers.size(); li++) {
            const Layer& L = layers[li];
            if (prenorm && li > 0)
                TRY(launch(qkv_rs_k, {B(h), B(L.wqkv), B(qkv), B(pos), B(slot), B(cos), B(sin), B(q), B(L.kc), B(L.vc),
                                      B(k), B(v), B(ss), EPS}));
            else
                TRY(launch(qkv_k, {B(h), B(L.wqkv), B(qkv), B(pos), B(slot), B(cos), B(sin), B(q), B(L.kc), B(L.vc),
                                   B(k), B(v)}));
            if (prefill) TRY(launch(att_k, {B(q), B(k), B(v), B(starts), B(o), SC}));
            else TRY(launch(att_k, {B(q), B(L.kc), B(L.vc), B(table), B(lens), B(o), SC}));
            if (prenorm) {
                TRY(launch(o_pre_k, {B(o), B(L.wo), B(x), B(L.n2), B(h), B(ss), B(ovf)}));
                TRY(launch(gu_rs_k, {B(h), B(ss), B(L.wg), B(L.wu), B(mlp), EPS}));
            } else {
                TRY(launch(oproj_norm_k, {B(o), B(L.wo), B(x), B(L.n2), B(h), EPS}));
                TRY(launch(gu_k, {B(h), B(L.wg), B(L.wu), B(mlp)}));
            }
            if (li + 1 < layers.size()) {
                if (prenorm) TRY(launch(down_pre_k, {B(mlp), B(L.wd), B(x), B(layers[li + 1].n1), B(h), B(ss), B(ovf)}));
                else TRY(launch(down_norm_k, {B(mlp), B(L.wd), B(x), B(layers[li + 1].n1), B(h), EPS}));
            } else {
                TRY(launch(down_k, {B(mlp), B(L.wd), B(x)}));
            }
        }
        if (bw == 0) return 0;
        int fin_k, head_k;
        int64_t BW = (int64_t)bw;
        TRY(kernel("rmsnorm_rows", {{T, dm}, {BW}, {dm}, {BW, dm}}, {{"BC", bc}}, 4, &fin_k));
        TRY(mm("logits", {{BW, dm}, {vv, dm}, {BW, vv}}, false, {B(last), B(head), B(logits)}, &head_k));
        // The scheduler's argmax on the GPU (fused/argmax), so a step can
        // return token ids instead of logits.
        int am_k;
        TRY(kernel("argmax", {{BW, vv}, {BW}}, {}, 4, &am_k, "fused"));
        TRY(launch(fin_k, {B(x), B(idx), B(norm), B(last), EPS}));
        TRY(launch(head_k, {B(last), B(head), B(logits)}));
        TRY(launch(am_k, {B(logits), B(next)}));
        return 0;
    }

    // Engine::step (src/llm/engine.rs:275-354).
    int step(size_t n, const int32_t* tokens, const int32_t* ps_in, const int32_t* slots, int mode,
             const int32_t* st_in, size_t nseq, const int32_t* tables, const int32_t* ln_in, size_t nwant,
             const int32_t* want, float* out, int32_t* out_tok = nullptr) {
        if (n == 0 || n > (size_t)lim.max_tokens) {
            std::ostringstream e;
            e << "a step of " << n << " tokens (at most " << lim.max_tokens << ")";
            return tsl_fail(TSL_ERR_ARG, e.str());
        }
        size_t t = padded(n);
        int32_t ns = lim.pages * lim.page;
        size_t mp = lim.max_seq_pages;
        size_t bw = nwant ? padded(nwant) : 0;
        if (mode != PREFILL && mode != PACKED && mode != DECODE) return tsl_fail(TSL_ERR_ARG, "unknown attention mode");
        if (mode == PACKED && !st_in) return tsl_fail(TSL_ERR_ARG, "packed prefill: one start per token");
        if (mode == PACKED)  // each row's sequence starts at or before it, and sequences do not overlap
            for (size_t i = 0; i < n; i++)
                if (i == 0 ? st_in[0] != 0 : (st_in[i] != st_in[i - 1] && (size_t)st_in[i] != i))
                    return tsl_fail(TSL_ERR_ARG, "packed prefill: starts[0] must be 0 and each starts[i] "
                                                 "starts[i - 1] (same sequence) or i (a new one)");
        if (mode == DECODE && nseq > t) return tsl_fail(TSL_ERR_ARG, "decode: more sequences than rows");
        if (bw > t) return tsl_fail(TSL_ERR_ARG, "more logits rows than step rows");
        // Every input of the step in the arena's layout for t, one upload.
        layout(t);
        const size_t nin = 6 * t + (mode == DECODE ? t * mp : 0);
        std::memset(hin, 0, nin * 4);
        int32_t *h_tok = &hin[0], *h_pos = &hin[t], *h_slot = &hin[2 * t], *h_idx = &hin[3 * t];
        int32_t *h_st = &hin[4 * t], *h_len = &hin[5 * t];
        std::copy(tokens, tokens + n, h_tok);
        std::copy(ps_in, ps_in + n, h_pos);
        std::copy(slots, slots + n, h_slot);
        std::fill(h_slot + n, h_slot + t, ns);  // padding rows write to no slot
        if (bw) std::copy(want, want + nwant, h_idx);
        if (mode == PREFILL || mode == PACKED) {
            if (mode == PACKED) std::copy(st_in, st_in + n, h_st);
            for (size_t i = n; i < t; i++) h_st[i] = (int32_t)i;  // padding rows start at themselves
        } else {
            int32_t* h_tb = &hin[6 * t];
            for (size_t b = 0; b < nseq; b++) {
                std::memcpy(h_tb + b * mp, tables + b * mp, mp * 4);
                h_len[b] = ln_in[b];
            }
        }
        bool prefill = mode != DECODE;
        const bool timed = time_steps && !prefill && !profiling;
        if (timed) {
            if (ev0 < 0) {
                TRY(tsl_event_record(&ev0));
                TRY(tsl_event_record(&ev1));
            } else {
                TRY(rt_event_rerecord(ev0));
            }
        }
        TRY(rt_upload_async(in.p, hin, nin * 4));
        bool replayed = false;
        phase = prefill ? "prefill" : "decode";
        // Profiling times every launch on its own, so it runs without graphs.
        if (!prefill && graphs && !profiling && bw == t) {
            auto it = graph.find(t);
            if (it != graph.end()) {
                TRY(tsl_replay(it->second));
                replayed = true;
            } else {
                TRY(launch_all(t, false, bw));
                TRY(tsl_sync());
                TRY(tsl_capture_begin());
                int r = launch_all(t, false, bw);
                int g = -1;
                int r2 = tsl_capture_end(&g);
                TRY(r);
                TRY(r2);
                graph[t] = g;
            }
        } else {
            TRY(launch_all(t, prefill, bw));
        }
        if (timed) TRY(rt_event_rerecord(ev1));
        if (uses_prenorm(t, prefill)) {
            // The deferred norms leave Y = f16(R Wn), which overflows where
            // |R Wn| >= 65520 although the normalised rows need not: such a
            // step is recomputed with each norm applied first, as prefill
            // steps do (the step's KV writes are the same slots, rewritten).
            int32_t flag = 0;
            if (out_tok && nwant) {
                TRY(rt_download_pinned(hout, outw.p, 16 + nwant * 4));
                flag = hout[0];
            } else {
                TRY(tsl_download(&flag, ovf.p, 4));
            }
            if (flag) {
                prenorm_fallbacks++;
                const int32_t zero = 0;
                TRY(write(ovf, 0, &zero, 4));
                plain = true;
                const int r = launch_all(t, false, bw);
                plain = false;
                TRY(r);
            } else if (out_tok && nwant) {
                std::copy(hout + 4, hout + 4 + nwant, out_tok);
                return timed ? add_step_time(replayed) : 0;
            }
        }
        if (nwant > 0) {
            if (out_tok) {
                TRY(rt_download_pinned(hout + 4, next.p, nwant * 4));
                std::copy(hout + 4, hout + 4 + nwant, out_tok);
            } else {
                TRY(tsl_download(out, logits.p, nwant * (size_t)cfg.vocab * 4));
            }
        } else {
            TRY(tsl_sync());  // (the pinned inputs are rewritten by the next step)
        }
        return timed ? add_step_time(replayed) : 0;
    }
    int add_step_time(bool replayed) {
        float ms = 0.0f;
        TRY(tsl_event_elapsed(ev0, ev1, &ms));
        timed_steps[replayed ? 0 : 1]++;
        timed_ms[replayed ? 0 : 1] += ms;
        return 0;
    }
};

std::vector<std::unique_ptr<Engine>> g_engines;

Engine* get(int e) {
    if (e < 0 || e >= (int)g_engines.size() || !g_engines[e]) return nullptr;
    return g_engines[e].get();
}

}  // namespace

extern "C" {

int tsl_weights_sizes(const tsl_config* cfg, size_t* embed, size_t* per_layer, size_t* norm, size_t* head) {
    *embed = (size_t)cfg->vocab * cfg->dim;
    *per_layer = (size_t)layer_elems(*cfg);
    *norm = cfg->dim;
    *head = (size_t)cfg->vocab * cfg->dim;
    return 0;
}

// bench::Rng (src/bench.rs:13-35): the generator behind the benchmark
// suite's inputs, for the command line's bench.
int tsl_rng_new(uint64_t seed, uint64_t* state) {
    if (!state) return tsl_fail(TSL_ERR_ARG, "null state");
    *state = Rng(seed).s;
    return 0;
}
int tsl_rng_bits(uint64_t* state, uint64_t* out) {
    if (!state || !out) return tsl_fail(TSL_ERR_ARG, "null state");
    Rng r(0);
    r.s = *state;
    *out = r.bits();
    *state = r.s;
    return 0;
}
int tsl_rng_tensor(uint64_t* state, size_t n, float scale, int dtype, void* out) {
    if (!state || (!out && n)) return tsl_fail(TSL_ERR_ARG, "null state or output");
    if (dtype != 0 && dtype != 1) return tsl_fail(TSL_ERR_ARG, "dtype must be 0 (f32) or 1 (f16)");
    Rng r(0);
    r.s = *state;
    for (size_t i = 0; i < n; i++) {
        const float v = r.uniform() * scale;
        if (dtype == 0) static_cast<float*>(out)[i] = v;
        else static_cast<u16*>(out)[i] = to_f16(v);
    }
    *state = r.s;
    return 0;
}

// Weights::random (src/llm/mod.rs:80-108).
int tsl_weights_random(const tsl_config* cfg, uint64_t seed, uint16_t* embed, uint16_t* layers, uint16_t* norm,
                       uint16_t* head) {
    const tsl_config& c = *cfg;
    Rng r(seed);
    auto m = [&](int64_t rows, int64_t cols, u16* out) {
        float sc = 1.0f / std::sqrt((float)cols);
        for (int64_t i = 0; i < rows * cols; i++) out[i] = to_f16(r.uniform() * sc);
    };
    u16 one = to_f16(1.0f);
    int64_t d = c.dim, hd = (int64_t)c.heads * c.head_dim, qr = qkv_rows(c);
    u16* p = layers;
    for (int l = 0; l < c.layers; l++) {
        std::fill(p, p + d, one);
        p += d;
        m(qr, d, p);
        p += qr * d;
        m(d, hd, p);
        p += d * hd;
        std::fill(p, p + d, one);
        p += d;
        m(c.ffn, d, p);
        p += (int64_t)c.ffn * d;
        m(c.ffn, d, p);
        p += (int64_t)c.ffn * d;
        m(d, c.ffn, p);
        p += d * c.ffn;
    }
    m(c.vocab, d, embed);
    for (int64_t i = 0; i < (int64_t)c.vocab * d; i++) embed[i] = to_f16(from_f16(embed[i]) * 8.0f);
    std::fill(norm, norm + d, one);
    m(c.vocab, d, head);
    return 0;
}

int tsl_engine_new(const tsl_config* cfg, const tsl_limits* lim, const uint16_t* embed, const uint16_t* layers,
                   const uint16_t* norm, const uint16_t* head, int* engine) {
    auto e = std::make_unique<Engine>();
    TRY(e->init(*cfg, *lim, embed, layers, norm, head));
    g_engines.push_back(std::move(e));
    *engine = (int)g_engines.size() - 1;
    return 0;
}

int tsl_engine_free(int engine) {
    Engine* e = get(engine);
    if (!e) return tsl_fail(TSL_ERR_ARG, "no such engine");
    tsl_sync();
    // (tok, pos, slot, idx, starts, lens and table are views into `in`.)
    Buf* bufs[] = {&e->embed, &e->norm, &e->cos, &e->sin, &e->x, &e->h, &e->ss, &e->qkv, &e->q, &e->k, &e->v,
                   &e->o, &e->mlp, &e->last, &e->logits, &e->in, &e->outw};
    if (e->head.p != e->embed.p) tsl_free(e->head.p);
    for (Buf* b : bufs)
        if (b->p) tsl_free(b->p);
    for (auto& L : e->layers)
        for (Buf* b : {&L.n1, &L.wqkv, &L.wo, &L.n2, &L.wg, &L.wu, &L.wd, &L.kc, &L.vc}) tsl_free(b->p);
    rt_host_free(e->hin);
    rt_host_free(e->hout);
    g_engines[engine].reset();
    return 0;
}

// Gpu::profile on (cleared) or off, and profile_rows (src/gpu.rs:219-228):
// the rows as a JSON list of {"phase", "kernel", "launches", "ms"}, largest
// time first; *len gets its length, out the text when cap > *len.
int tsl_engine_profile(int engine, int on) {
    Engine* e = get(engine);
    if (!e) return tsl_fail(TSL_ERR_ARG, "no such engine");
    e->profiling = on != 0;
    e->prof.clear();
    return 0;
}
int tsl_engine_profile_rows(int engine, char* out, size_t cap, size_t* len) {
    Engine* e = get(engine);
    if (!e) return tsl_fail(TSL_ERR_ARG, "no such engine");
    std::vector<std::pair<std::pair<std::string, std::string>, std::pair<int64_t, double>>> rows(e->prof.begin(),
                                                                                                 e->prof.end());
    std::stable_sort(rows.begin(), rows.end(),
                     [](const auto& a, const auto& b) { return a.second.second > b.second.second; });
    std::ostringstream o;
    o << "[";
    for (size_t i = 0; i < rows.size(); i++) {
        std::string k = rows[i].first.second;
        for (auto& c : k)
            if (c == '"') c = '\'';
        char ms[32];
        std::snprintf(ms, sizeof ms, "%.6f", rows[i].second.second);
        o << (i ? ", " : "") << "{\"phase\": \"" << rows[i].first.first << "\", \"kernel\": \"" << k
          << "\", \"launches\": " << rows[i].second.first << ", \"ms\": " << ms << "}";
    }
    o << "]";
    const std::string s = o.str();
    if (len) *len = s.size();
    if (out && cap > s.size()) std::memcpy(out, s.c_str(), s.size() + 1);
    return 0;
}

int tsl_engine_graphs(int engine, int32_t* rows, int32_t* graphs, int cap, int* n) {
    Engine* e = get(engine);
    if (!e) return tsl_fail(TSL_ERR_ARG, "no such engine");
    int i = 0;
    for (auto& kv : e->graph) {
        if (i < cap) {
            rows[i] = (int32_t)kv.first;
            graphs[i] = kv.second;
        }
        i++;
    }
    *n = i;
    return 0;
}

int tsl_engine_fallbacks(int engine, int64_t* n) {
    Engine* e = get(engine);
    if (!e || !n) return tsl_fail(TSL_ERR_ARG, "no such engine, or a null count");
    *n = e->prenorm_fallbacks;
    return 0;
}

int tsl_engine_step_times(int engine, int on, int64_t* steps, double* ms) {
    Engine* e = get(engine);
    if (!e || !steps || !ms) return tsl_fail(TSL_ERR_ARG, "no such engine, or a null output");
    for (int i = 0; i < 2; i++) {
        steps[i] = e->timed_steps[i];
        ms[i] = e->timed_ms[i];
        e->timed_steps[i] = 0;
        e->timed_ms[i] = 0.0;
    }
    e->time_steps = on != 0;
    return 0;
}

int tsl_engine_set(int engine, int graphs, int tune) {
    Engine* e = get(engine);
    if (!e) return tsl_fail(TSL_ERR_ARG, "no such engine");
    e->graphs = graphs != 0;
    e->tune = tune != 0;
    return 0;
}

int tsl_engine_step(int engine, int n, const int32_t* tokens, const int32_t* pos, const int32_t* slots, int mode,
                    const int32_t* starts, int nseq, const int32_t* tables, const int32_t* lens, int nwant,
                    const int32_t* want, float* logits) {
    Engine* e = get(engine);
    if (!e) return tsl_fail(TSL_ERR_ARG, "no such engine");
    if (n < 0 || nwant < 0 || nseq < 0) return tsl_fail(TSL_ERR_ARG, "negative count");
    return e->step((size_t)n, tokens, pos, slots, mode, starts, (size_t)nseq, tables, lens, (size_t)nwant, want,
                   logits);
}

}  // extern "C"

namespace {

// One step of the scheduler's model, as sched.rs calls Engine::step: the
// rows' tokens, positions and cache slots, the attention mode with its
// starts (packed prefill) or tables and lens (decode), and the rows whose
// next token is wanted; `ids` names the request each wanted row belongs
// to. Writes one token id per wanted row into `next`.
struct StepIn {
    int mode;
    const std::vector<int32_t>& toks;
    const std::vector<int32_t>& pos;
    const std::vector<int32_t>& slots;
    const std::vector<int32_t>& starts;
    size_t nseq;
    const std::vector<int32_t>& tables;
    const std::vector<int32_t>& lens;
    const std::vector<int32_t>& want;
    const std::vector<int>& ids;
};

struct Sched {
    tsl_limits lim;
    int eos;
};

// sched::generate_with (src/llm/sched.rs:52-179): admission by token
// budget, batch size and free pages (whole sequences reserved up front),
// the LIFO page free list, one packed (or single) prefill step for what
// was admitted, else one decode step for every running sequence.
// Requests are validated before anything runs: an empty or too long
// prompt, max_new < 1, or more pages than a sequence (or the pool) can
// hold is an error (the reference panics on max_new = 0 and waits for
// ever on a request larger than the pool).
template <class Step>
int schedule(const Sched& sc, int nreq, const int32_t* prompts, const int64_t* offsets, const int32_t* max_new,
             int max_batch, int packed, int32_t* out_tokens, int32_t* out_counts, tsl_stats* stats,
             double* out_times, Step&& step) {
    using clk = std::chrono::steady_clock;
    auto start = clk::now();
    const int p = sc.lim.page;
    const size_t mp = sc.lim.max_seq_pages;
    if (nreq < 0 || max_batch < 1 || p < 1) return tsl_fail(TSL_ERR_ARG, "generate: bad request count or batch");
    if (nreq > 0 && (!prompts || !offsets || !max_new || !out_tokens || !out_counts))
        return tsl_fail(TSL_ERR_ARG, "generate: null prompts, offsets, max_new or outputs");
    for (int id = 0; id < nreq; id++) {
        int64_t plen = offsets[id + 1] - offsets[id];
        std::ostringstream m;
        if (max_new[id] < 1) {
            m << "request " << id << ": max_new must be at least 1";
            return tsl_fail(TSL_ERR_ARG, m.str());
        }
        size_t need = plen > 0 ? ((size_t)plen + (size_t)max_new[id] + p - 1) / p : 0;
        if (plen <= 0 || plen > sc.lim.max_tokens || need > mp || need > (size_t)sc.lim.pages) {
            m << "request " << id << ": prompt of " << plen << " tokens does not fit";
            return tsl_fail(TSL_ERR_ARG, m.str());
        }
    }
    std::vector<int32_t> free_pages;
    for (int i = sc.lim.pages - 1; i >= 0; i--) free_pages.push_back(i);
    std::deque<int> waiting;
    for (int i = 0; i < nreq; i++) waiting.push_back(i);
    struct Seq {
        int id;
        std::vector<int32_t> pages;
        size_t len;
        int32_t last;
        int left;
    };
    std::vector<Seq> running;
    std::vector<size_t> out_base(nreq, 0);
    for (int i = 1; i < nreq; i++) out_base[i] = out_base[i - 1] + max_new[i - 1];
    for (int i = 0; i < nreq; i++) out_counts[i] = 0;
    tsl_stats st{};
    max_batch = std::min(max_batch, sc.lim.max_tokens);
    auto since = [&]() { return std::chrono::duration<double>(clk::now() - start).count(); };
    if (out_times)
        for (int i = 0; i < 2 * nreq; i++) out_times[i] = 0.0;
    auto emit = [&](int id, int32_t t) {
        out_tokens[out_base[id] + out_counts[id]++] = t;
        if (out_times && out_counts[id] == 1) out_times[2 * id] = since();  // first_token_s
    };
    auto done = [&](int id) {
        if (out_times) out_times[2 * id + 1] = since();  // done_s
    };
    const std::vector<int32_t> none;
    while (!waiting.empty() || !running.empty()) {
        std::vector<std::pair<int, std::vector<int32_t>>> admit;
        size_t tokens = 0;
        while (!waiting.empty()) {
            int id = waiting.front();
            size_t plen = (size_t)(offsets[id + 1] - offsets[id]);
            size_t need = (plen + max_new[id] + p - 1) / p;
            bool room = (int)(running.size() + admit.size()) < max_batch && tokens + plen <= (size_t)sc.lim.max_tokens;
            if (!room || need > free_pages.size() || (!packed && !admit.empty())) break;
            waiting.pop_front();
            tokens += plen;
            std::vector<int32_t> pages;
            for (size_t i = 0; i < need; i++) {
                pages.push_back(free_pages.back());
                free_pages.pop_back();
            }
            admit.push_back({id, pages});
        }
        if (!admit.empty()) {
            std::vector<int32_t> toks, pos, slots, starts, last;
            std::vector<int> ids;
            for (auto& a : admit) {
                const int32_t* pr = prompts + offsets[a.first];
                size_t plen = (size_t)(offsets[a.first + 1] - offsets[a.first]);
                int32_t s0 = (int32_t)toks.size();
                for (size_t i = 0; i < plen; i++) {
                    toks.push_back(pr[i]);
                    pos.push_back((int32_t)i);
                    slots.push_back(a.second[i / p] * p + (int32_t)(i % p));
                    starts.push_back(s0);
                }
                last.push_back((int32_t)toks.size() - 1);
                ids.push_back(a.first);
            }
            std::vector<int32_t> next(last.size());
            int mode = admit.size() == 1 ? PREFILL : PACKED;
            TRY(step(StepIn{mode, toks, pos, slots, starts, 0, none, none, last, ids}, next.data()));
            st.prefill_steps++;
            st.prompt_tokens += toks.size();
            for (size_t i = 0; i < admit.size(); i++) {
                int id = admit[i].first;
                int32_t t = next[i];
                emit(id, t);
                size_t plen = (size_t)(offsets[id + 1] - offsets[id]);
                Seq s{id, admit[i].second, plen, t, max_new[id] - 1};
                if (s.left == 0 || t == sc.eos) {
                    done(id);
                    free_pages.insert(free_pages.end(), s.pages.begin(), s.pages.end());
                } else {
                    running.push_back(s);
                }
            }
            continue;
        }
        if (running.empty()) continue;  // unreachable: every request fits the empty pool
        auto t0 = clk::now();
        size_t nb = running.size();
        std::vector<int32_t> toks, pos, slots, tables(nb * mp, 0), lens, want;
        std::vector<int> ids;
        for (size_t b = 0; b < nb; b++) {
            const Seq& s = running[b];
            toks.push_back(s.last);
            pos.push_back((int32_t)s.len);
            slots.push_back(s.pages[s.len / p] * p + (int32_t)(s.len % p));
            std::copy(s.pages.begin(), s.pages.end(), tables.begin() + b * mp);
            lens.push_back((int32_t)s.len + 1);
            want.push_back((int32_t)b);
            ids.push_back(s.id);
        }
        std::vector<int32_t> next(nb);
        TRY(step(StepIn{DECODE, toks, pos, slots, none, nb, tables, lens, want, ids}, next.data()));
        st.decode_steps++;
        st.largest_batch = std::max<int64_t>(st.largest_batch, nb);
        st.decode_tokens += nb;
        std::vector<Seq> keep;
        for (size_t b = 0; b < nb; b++) {
            Seq s = running[b];
            int32_t t = next[b];
            s.len++;
            s.last = t;
            s.left--;
            emit(s.id, t);
            if (s.left == 0 || t == sc.eos) {
                done(s.id);
                free_pages.insert(free_pages.end(), s.pages.begin(), s.pages.end());
            } else {
                keep.push_back(s);
            }
        }
        running = keep;
        st.decode_seconds += std::chrono::duration<double>(clk::now() - t0).count();
    }
    for (int i = 0; i < nreq; i++) st.generated += out_counts[i];
    st.seconds = std::chrono::duration<double>(clk::now() - start).count();
    if (stats) *stats = st;
    return 0;
}

}  // namespace

extern "C" {

int tsl_generate(int engine, int nreq, const int32_t* prompts, const int64_t* offsets, const int32_t* max_new,
                 int max_batch, int packed, int32_t* out_tokens, int32_t* out_counts, tsl_stats* stats,
                 double* out_times) {
    Engine* e = get(engine);
    if (!e) return tsl_fail(TSL_ERR_ARG, "no such engine");
    // The next tokens come from the GPU's argmax (fused/argmax, the same
    // first-largest rule as src/llm/mod.rs:132-140), not from the logits.
    auto step = [&](const StepIn& s, int32_t* next) {
        return e->step(s.toks.size(), s.toks.data(), s.pos.data(), s.slots.data(), s.mode,
                       s.mode == PACKED ? s.starts.data() : nullptr, s.nseq, s.tables.data(), s.lens.data(),
                       s.want.size(), s.want.data(), nullptr, next);
    };
    return schedule(Sched{e->lim, e->cfg.eos}, nreq, prompts, offsets, max_new, max_batch, packed, out_tokens,
                    out_counts, stats, out_times, step);
}

int tsl_schedule_trace(const tsl_limits* lim, int eos, int nreq, const int32_t* prompts, const int64_t* offsets,
                       const int32_t* max_new, int max_batch, int packed, const int32_t* script, int32_t* out_tokens,
                       int32_t* out_counts, tsl_stats* stats, int32_t* trace, int64_t cap, int64_t* used) {
    if (!lim || !trace || !used || cap < 0) return tsl_fail(TSL_ERR_ARG, "schedule trace: null argument");
    if (nreq < 0) return tsl_fail(TSL_ERR_ARG, "schedule trace: negative request count");
    if (nreq > 0 && (!prompts || !offsets || !max_new || !script || !out_tokens || !out_counts))
        return tsl_fail(TSL_ERR_ARG, "schedule trace: null prompts, offsets, max_new, script or outputs");
    std::vector<size_t> base(nreq > 0 ? nreq : 0, 0);
    for (int i = 1; i < nreq; i++) base[i] = base[i - 1] + (max_new[i - 1] > 0 ? max_new[i - 1] : 0);
    std::vector<int> emitted(base.size(), 0);
    int64_t w = 0;
    auto put = [&](const int32_t* v, size_t n) {
        if (w + (int64_t)n <= cap) std::copy(v, v + n, trace + w);
        w += (int64_t)n;
    };
    auto step = [&](const StepIn& s, int32_t* next) {
        const int32_t head[3] = {s.mode, (int32_t)s.toks.size(), (int32_t)s.want.size()};
        put(head, 3);
        put(s.toks.data(), s.toks.size());
        put(s.pos.data(), s.pos.size());
        put(s.slots.data(), s.slots.size());
        if (s.mode == PACKED) put(s.starts.data(), s.starts.size());
        if (s.mode == DECODE) {
            put(s.tables.data(), s.tables.size());
            put(s.lens.data(), s.lens.size());
        }
        put(s.want.data(), s.want.size());
        for (size_t i = 0; i < s.want.size(); i++) {
            int id = s.ids[i];
            next[i] = script[base[id] + emitted[id]++];
        }
        return 0;
    };
    int r = schedule(Sched{*lim, eos}, nreq, prompts, offsets, max_new, max_batch, packed, out_tokens, out_counts,
                     stats, nullptr, step);
    *used = w;
    if (r == 0 && w > cap) return tsl_fail(TSL_ERR_ARG, "schedule trace: buffer too small");
    return r;
}

}  // extern "C"
