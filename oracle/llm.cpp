// TEST INFRASTRUCTURE ONLY: the CPU oracle of the LLM engine. Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
//
// Restates src/llm/mod.rs (Weights::random :80-108, rope_tables :116-129,
// argmax :132-140) and src/llm/reference.rs (the plain f32 model, one
// sequence at a time: the oracle the engine's logits are checked against).
// f32 sums are sequential in f32, as Rust's Iterator::sum over f32 is.

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

typedef uint16_t u16;
typedef int32_t i32;
typedef int64_t i64;

extern "C" {
u16 tsl_ref_f32_to_f16(float f);
float tsl_ref_f16_to_f32(u16 h);
uint64_t tsl_ref_rng_new(uint64_t seed);
float tsl_ref_rng_uniform(uint64_t* s);
}

// Mirrors the C ABI's tsl_config (include/tessel.h).
struct Cfg {
    i32 dim, layers, heads, kv_heads, head_dim, ffn, vocab;
    float eps, rope_theta;
    i32 max_pos, bos, eos;
};

static i64 qkv_rows(const Cfg& c) { return (i64)(c.heads + 2 * c.kv_heads) * c.head_dim; }
static i64 layer_elems(const Cfg& c) {
    i64 d = c.dim, hd = (i64)c.heads * c.head_dim;
    return d + qkv_rows(c) * d + d * hd + d + 2 * (i64)c.ffn * d + d * c.ffn;
}

extern "C" {

// Weights::random (src/llm/mod.rs:80-108): every matrix [rows, cols] is
// uniform * 1/sqrt(cols) rounded to f16, drawn in field order per layer,
// then the embedding (scaled by 8) and the LM head; norms are 1.
int tsl_ref_weights_random(const Cfg* cfg, uint64_t seed, u16* embed, u16* layers, u16* norm, u16* head) {
    const Cfg& c = *cfg;
    uint64_t s = tsl_ref_rng_new(seed);
    auto m = [&](i64 rows, i64 cols, u16* out) {
        float sc = 1.0f / std::sqrt((float)cols);
        for (i64 i = 0; i < rows * cols; i++) out[i] = tsl_ref_f32_to_f16(tsl_ref_rng_uniform(&s) * sc);
    };
    u16 one = tsl_ref_f32_to_f16(1.0f);
    i64 d = c.dim, hd = (i64)c.heads * c.head_dim;
    u16* p = layers;
    for (int l = 0; l < c.layers; l++) {
        for (i64 i = 0; i < d; i++) p[i] = one;
        p += d;
        m(qkv_rows(c), d, p);
        p += qkv_rows(c) * d;
        m(d, hd, p);
        p += d * hd;
        for (i64 i = 0; i < d; i++) p[i] = one;
        p += d;
        m(c.ffn, d, p);
        p += (i64)c.ffn * d;
        m(c.ffn, d, p);
        p += (i64)c.ffn * d;
        m(d, c.ffn, p);
        p += d * c.ffn;
    }
    m(c.vocab, d, embed);
    for (i64 i = 0; i < (i64)c.vocab * d; i++) embed[i] = tsl_ref_f32_to_f16(tsl_ref_f16_to_f32(embed[i]) * 8.0f);
    for (i64 i = 0; i < d; i++) norm[i] = one;
    m(c.vocab, d, head);
    return 0;
}

// rope_tables (src/llm/mod.rs:116-129): f64 angles rounded to f32.
int tsl_ref_rope_tables(const Cfg* cfg, float* cs, float* sn) {
    const Cfg& c = *cfg;
    i64 h = c.head_dim / 2;
    for (i64 p = 0; p < c.max_pos; p++)
        for (i64 i = 0; i < h; i++) {
            double inv = std::pow((double)c.rope_theta, -((double)(2 * i)) / (double)c.head_dim);
            double a = (double)p * inv;
            cs[p * h + i] = (float)std::cos(a);
            sn[p * h + i] = (float)std::sin(a);
        }
    return 0;
}

// argmax (src/llm/mod.rs:132-140): the first index of the largest value.
i64 tsl_ref_argmax(const float* xs, i64 n) {
    i64 best = 0;
    for (i64 i = 0; i < n; i++)
        if (xs[i] > xs[best]) best = i;
    return best;
}

// reference::forward (src/llm/reference.rs:38-108): logits after each of
// the n tokens, into out[n * vocab].
int tsl_ref_forward(const Cfg* cfg, const u16* embed, const u16* layers, const u16* norm, const u16* head,
                    const i32* tokens, i64 n, float* out) {
    const Cfg& c = *cfg;
    const i64 hd = c.head_dim, nh = c.heads, ng = c.kv_heads, dm = c.dim, ff = c.ffn;
    auto f = [](const u16* v, i64 n) {
        std::vector<float> r(n);
        for (i64 i = 0; i < n; i++) r[i] = tsl_ref_f16_to_f32(v[i]);
        return r;
    };
    auto matvec = [](const std::vector<float>& w, const std::vector<float>& x, i64 rows) {
        i64 cols = (i64)x.size();
        std::vector<float> y(rows);
        // Rows in parallel; each row's sum stays the sequential f32 loop.
#pragma omp parallel for schedule(static) if (rows * cols > (1 << 20))
        for (i64 r = 0; r < rows; r++) {
            float s = 0.0f;
            for (i64 k = 0; k < cols; k++) s += w[r * cols + k] * x[k];
            y[r] = s;
        }
        return y;
    };
    auto rmsnorm = [](const std::vector<float>& x, const std::vector<float>& w, float eps) {
        float ms = 0.0f;
        for (float v : x) ms += v * v;
        ms = ms / (float)x.size();
        float s = 1.0f / std::sqrt(ms + eps);
        std::vector<float> y(x.size());
        for (size_t i = 0; i < x.size(); i++) y[i] = x[i] * s * w[i];
        return y;
    };
    std::vector<float> cs((i64)c.max_pos * (hd / 2)), sn(cs.size());
    tsl_ref_rope_tables(cfg, cs.data(), sn.data());
    auto rope = [&](std::vector<float>& x, i64 pos) {
        i64 h = hd / 2;
        for (size_t base = 0; base < x.size(); base += hd)
            for (i64 i = 0; i < h; i++) {
                float cc = cs[pos * h + i], ss = sn[pos * h + i];
                float a = x[base + i], b = x[base + i + h];
                x[base + i] = a * cc - b * ss;
                x[base + i + h] = b * cc + a * ss;
            }
    };
    struct L {
        std::vector<float> n1, wqkv, wo, n2, wg, wu, wd;
    };
    std::vector<L> ls;
    const u16* p = layers;
    i64 qr = (nh + 2 * ng) * hd;
    for (int l = 0; l < c.layers; l++) {
        L x;
        x.n1 = f(p, dm);
        p += dm;
        x.wqkv = f(p, qr * dm);
        p += qr * dm;
        x.wo = f(p, dm * nh * hd);
        p += dm * nh * hd;
        x.n2 = f(p, dm);
        p += dm;
        x.wg = f(p, ff * dm);
        p += ff * dm;
        x.wu = f(p, ff * dm);
        p += ff * dm;
        x.wd = f(p, dm * ff);
        p += dm * ff;
        ls.push_back(std::move(x));
    }
    std::vector<float> emb = f(embed, (i64)c.vocab * dm), nrm = f(norm, dm), hw = f(head, (i64)c.vocab * dm);
    std::vector<std::vector<std::vector<float>>> kc(c.layers), vc(c.layers);
    for (i64 pos = 0; pos < n; pos++) {
        i64 t = tokens[pos];
        std::vector<float> x(emb.begin() + t * dm, emb.begin() + (t + 1) * dm);
        for (int li = 0; li < c.layers; li++) {
            const L& w = ls[li];
            std::vector<float> h = rmsnorm(x, w.n1, c.eps);
            std::vector<float> qkv = matvec(w.wqkv, h, qr);
            std::vector<float> q(qkv.begin(), qkv.begin() + nh * hd);
            std::vector<float> k(qkv.begin() + nh * hd, qkv.begin() + (nh + ng) * hd);
            std::vector<float> v(qkv.begin() + (nh + ng) * hd, qkv.end());
            rope(q, pos);
            rope(k, pos);
            kc[li].push_back(k);
            vc[li].push_back(v);
            std::vector<float> o(nh * hd, 0.0f);
            for (i64 hh = 0; hh < nh; hh++) {
                i64 g = hh / (nh / ng);
                std::vector<float> sc;
                for (auto& kk : kc[li]) {
                    float s = 0.0f;
                    for (i64 d = 0; d < hd; d++) s += kk[g * hd + d] * q[hh * hd + d];
                    sc.push_back(s / std::sqrt((float)hd));
                }
                float m = -INFINITY;
                for (float s : sc) m = std::fmax(m, s);
                std::vector<float> e;
                float z = 0.0f;
                for (float s : sc) e.push_back(std::exp(s - m));
                for (float v2 : e) z += v2;
                for (size_t j = 0; j < e.size(); j++)
                    for (i64 d = 0; d < hd; d++) o[hh * hd + d] += e[j] / z * vc[li][j][g * hd + d];
            }
            std::vector<float> ao = matvec(w.wo, o, dm);
            for (i64 i = 0; i < dm; i++) x[i] += ao[i];
            h = rmsnorm(x, w.n2, c.eps);
            std::vector<float> g = matvec(w.wg, h, ff), u = matvec(w.wu, h, ff), a(ff);
            for (i64 i = 0; i < ff; i++) a[i] = g[i] / (1.0f + std::exp(-g[i])) * u[i];
            std::vector<float> dn = matvec(w.wd, a, dm);
            for (i64 i = 0; i < dm; i++) x[i] += dn[i];
        }
        std::vector<float> lg = matvec(hw, rmsnorm(x, nrm, c.eps), c.vocab);
        std::memcpy(out + pos * c.vocab, lg.data(), sizeof(float) * c.vocab);
    }
    return 0;
}

}  // extern "C"
