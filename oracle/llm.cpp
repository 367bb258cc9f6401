// TEST INFRASTRUCTURE ONLY: the CPU oracle of the LLM engine. Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
//
// Restates src/llm/mod.rs (Weights::random :80-108, rope_tables :116-129,
// argmax :132-140) and src/llm/reference.rs (the plain f32 model, one
// sequence at a time: the oracle the engine's logits are checked against).
// f32 sums are sequential in f32, as Rust's Iterator::sum over f32 is.

#include <algorithm>
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

// s[j] = sum over k, in k order, of w[k] * xt[k * 16 + j], for 16 tokens j
// side by side (independent f32 chains: vector lanes, never reassociated).
// Built for AVX2 as well as the baseline, picked at load time.
__attribute__((target_clones("avx2", "default"))) static void dot_block(const float* w, const float* xt, i64 cols,
                                                                        float* s) {
    typedef float v8 __attribute__((vector_size(32)));
    v8 a0 = {}, a1 = {};
    for (i64 k = 0; k < cols; k++) {
        v8 x0, x1;
        std::memcpy(&x0, xt + k * 16, 32);
        std::memcpy(&x1, xt + k * 16 + 8, 32);
        const float wk = w[k];
        a0 += wk * x0;  // a multiply, then an add (no contraction: -ffp-contract=off)
        a1 += wk * x1;
    }
    std::memcpy(s, &a0, 32);
    std::memcpy(s + 8, &a1, 32);
}

// reference::forward (src/llm/reference.rs:38-108): logits after each of
// the n tokens, into out[n * vocab]. The reference runs token by token; this
// runs layer by layer over all n tokens (position order inside each layer),
// which performs every scalar operation of the token-by-token order in the
// same sequence per token (attention at position p reads the keys of
// positions <= p of the same layer, all present), so the bits are the same,
// while each weight row is read once per layer for all n tokens.
int tsl_ref_forward(const Cfg* cfg, const u16* embed, const u16* layers, const u16* norm, const u16* head,
                    const i32* tokens, i64 n, float* out) {
    const Cfg& c = *cfg;
    const i64 hd = c.head_dim, nh = c.heads, ng = c.kv_heads, dm = c.dim, ff = c.ffn;
    typedef std::vector<float> vf;
    // y[t][r] = sum_k w[r][k] x[t][k], the sequential f32 loop per (t, r);
    // rows in parallel, the f16 weight row converted once for all t.
    auto matmul = [n](const u16* w, const std::vector<vf>& x, i64 rows, std::vector<vf>& y) {
        const i64 cols = (i64)x[0].size();
        y.assign(n, vf(rows));
        constexpr int TB = 16;
        const i64 nb = (n + TB - 1) / TB;
        vf xT((size_t)nb * cols * TB, 0.0f);  // [token block][k][TB]
        for (i64 t = 0; t < n; t++)
            for (i64 k = 0; k < cols; k++) xT[((size_t)(t / TB) * cols + k) * TB + t % TB] = x[t][k];
#pragma omp parallel
        {
            vf wr(cols);
#pragma omp for schedule(static)
            for (i64 r = 0; r < rows; r++) {
                for (i64 k = 0; k < cols; k++) wr[k] = tsl_ref_f16_to_f32(w[r * cols + k]);
                // TB tokens' sums side by side (independent chains, each in k order).
                for (i64 t0 = 0; t0 < n; t0 += TB) {
                    const i64 nt = std::min<i64>(TB, n - t0);
                    const float* xt = &xT[(size_t)(t0 / TB) * cols * TB];
                    float s[TB];
                    dot_block(wr.data(), xt, cols, s);
                    for (i64 j = 0; j < nt; j++) y[t0 + j][r] = s[j];
                }
            }
        }
    };
    auto rmsnorm = [](const vf& x, const u16* w16, float eps) {
        float ms = 0.0f;
        for (float v : x) ms += v * v;
        ms = ms / (float)x.size();
        float s = 1.0f / std::sqrt(ms + eps);
        vf y(x.size());
        for (size_t i = 0; i < x.size(); i++) y[i] = x[i] * s * tsl_ref_f16_to_f32(w16[i]);
        return y;
    };
    vf cs((i64)c.max_pos * (hd / 2)), sn(cs.size());
    tsl_ref_rope_tables(cfg, cs.data(), sn.data());
    auto rope = [&](float* x, i64 len, i64 pos) {
        i64 h = hd / 2;
        for (i64 base = 0; base < len; base += hd)
            for (i64 i = 0; i < h; i++) {
                float cc = cs[pos * h + i], ss = sn[pos * h + i];
                float a = x[base + i], b = x[base + i + h];
                x[base + i] = a * cc - b * ss;
                x[base + i + h] = b * cc + a * ss;
            }
    };
    if (n <= 0) return 0;
    if (n > c.max_pos) return -1;  // the reference's rope table index panics past max_pos
    const i64 qr = (nh + 2 * ng) * hd;
    std::vector<vf> x(n), h(n), y, y2;
    for (i64 t = 0; t < n; t++) {
        x[t].resize(dm);
        for (i64 i = 0; i < dm; i++) x[t][i] = tsl_ref_f16_to_f32(embed[(i64)tokens[t] * dm + i]);
    }
    const u16* p = layers;
    for (int li = 0; li < c.layers; li++) {
        const u16 *n1 = p, *wqkv = n1 + dm, *wo = wqkv + qr * dm, *n2 = wo + dm * nh * hd, *wg = n2 + dm,
                  *wu = wg + ff * dm, *wd = wu + ff * dm;
        p = wd + dm * ff;
        for (i64 t = 0; t < n; t++) h[t] = rmsnorm(x[t], n1, c.eps);
        matmul(wqkv, h, qr, y);  // y[t] = qkv of token t
        for (i64 t = 0; t < n; t++) {
            rope(y[t].data(), nh * hd, t);                // q
            rope(y[t].data() + nh * hd, ng * hd, t);      // k
        }
        std::vector<vf> o(n, vf(nh * hd, 0.0f));
#pragma omp parallel for schedule(dynamic)
        for (i64 t = 0; t < n; t++) {
            const float* q = y[t].data();
            for (i64 hh = 0; hh < nh; hh++) {
                i64 g = hh / (nh / ng);
                vf sc;
                for (i64 j = 0; j <= t; j++) {
                    const float* kk = y[j].data() + nh * hd;
                    float s = 0.0f;
                    for (i64 d = 0; d < hd; d++) s += kk[g * hd + d] * q[hh * hd + d];
                    sc.push_back(s / std::sqrt((float)hd));
                }
                float m = -INFINITY;
                for (float s : sc) m = std::fmax(m, s);
                vf e;
                float z = 0.0f;
                for (float s : sc) e.push_back(std::exp(s - m));
                for (float v2 : e) z += v2;
                for (size_t j = 0; j < e.size(); j++) {
                    const float* vv = y[j].data() + (nh + ng) * hd;
                    for (i64 d = 0; d < hd; d++) o[t][hh * hd + d] += e[j] / z * vv[g * hd + d];
                }
            }
        }
        matmul(wo, o, dm, y2);
        for (i64 t = 0; t < n; t++) {
            for (i64 i = 0; i < dm; i++) x[t][i] += y2[t][i];
            h[t] = rmsnorm(x[t], n2, c.eps);
        }
        matmul(wg, h, ff, y);
        matmul(wu, h, ff, y2);
        for (i64 t = 0; t < n; t++)
            for (i64 i = 0; i < ff; i++) y[t][i] = y[t][i] / (1.0f + std::exp(-y[t][i])) * y2[t][i];
        matmul(wd, y, dm, y2);
        for (i64 t = 0; t < n; t++)
            for (i64 i = 0; i < dm; i++) x[t][i] += y2[t][i];
    }
    for (i64 t = 0; t < n; t++) h[t] = rmsnorm(x[t], norm, c.eps);
    matmul(head, h, c.vocab, y);
    for (i64 t = 0; t < n; t++) std::memcpy(out + t * c.vocab, y[t].data(), sizeof(float) * c.vocab);
    return 0;
}

}  // extern "C"
