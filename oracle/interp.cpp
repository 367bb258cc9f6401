// TEST INFRASTRUCTURE ONLY: the CPU oracle. Nothing in the product
// (tessel_amd/, include/) may link, load or call this file's library; only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as
// the checker.
//
// A restatement of tessel's reference interpreter (src/interp.rs) for each
// kernel on the hot path. The interpreter computes every op in f64 and
// rounds the result to the op's dtype (src/interp.rs:46-59, :83-86); the
// typing rules that decide those dtypes come from src/ir.rs (promote
// :310-318, f16 `sum` upcast to f32 :639-643, `dot` -> f32 :699-705, store
// casts to the array dtype :862-863, literals take the other operand's
// float dtype :209-221). Out-of-bounds loads read `other` (0, or -inf where
// the .tl says so) and out-of-bounds stores are dropped (src/interp.rs:93-117,
// :296-313). A `dot` adds this K-tile's f64 sum to the f32 accumulator and
// rounds (src/interp.rs:280-295), so tile boundaries are reproduced.
// Programs run in z -> y -> x order (src/interp.rs:360-367); every kernel
// here writes disjoint outputs per program, so the order is kept only where
// it is free.
//
// Build: g++ -O2 -ffp-contract=off -fopenmp (oracle/Makefile). No fast-math
// and no FMA contraction: every f32/f64 op must round as Rust's do.

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>
#include <algorithm>
#include <omp.h>

typedef uint16_t u16;
typedef int32_t i32;
typedef int64_t i64;

// ---------------------------------------------------------------- half.rs
// IEEE binary16, round to nearest even (src/half.rs:3-58).
static u16 f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    u16 sign = (u16)((x >> 16) & 0x8000u);
    uint32_t mant = x & 0x7fffffu;
    int e = (int)((x >> 23) & 0xff);
    if (e == 0xff) return (u16)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    int ex = e - 127 + 15;
    if (ex >= 31) return (u16)(sign | 0x7c00u);
    if (ex <= 0) {
        if (ex < -10) return sign;
        mant |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - ex);
        uint32_t h = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) h += 1;
        return (u16)(sign | h);
    }
    uint32_t h = ((uint32_t)ex << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h += 1;
    return (u16)(sign | h);
}

static float f16_to_f32(u16 h) {
    uint32_t sign = ((uint32_t)(h & 0x8000u)) << 16;
    uint32_t ex = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ffu;
    uint32_t x;
    if (ex == 0) {
        if (mant == 0) {
            x = sign;
        } else {
            int e = 1;
            while ((mant & 0x400u) == 0) {
                mant <<= 1;
                e -= 1;
            }
            x = sign | ((uint32_t)(e + 127 - 15) << 23) | ((mant & 0x3ffu) << 13);
        }
    } else if (ex == 31) {
        x = sign | 0x7f800000u | (mant << 13);
    } else {
        x = sign | ((ex + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

// round(dtype, x) of src/interp.rs:46-59.
static inline double r32(double x) { return (double)(float)x; }
static inline double r16(double x) { return (double)f16_to_f32(f32_to_f16((float)x)); }
static inline double h2d(u16 h) { return (double)f16_to_f32(h); }
// Un::Exp: (x as f32).exp(), i.e. libm expf (src/interp.rs:173).
static inline double uexp(double x) { return (double)std::exp((float)x); }
// Un::Rsqrt: 1.0 / (x as f32).sqrt() in f64 (src/interp.rs:176).
static inline double ursqrt(double x) { return 1.0 / (double)std::sqrt((float)x); }
// Bin::Max (src/interp.rs:207-213).
static inline double bmax(double x, double y) { return (x >= y || std::isnan(y)) ? x : y; }
// Red::Max folds f64::max from -inf (src/interp.rs:267).
static inline double rmax(double acc, double x) { return std::fmax(acc, x); }
static inline i64 cdiv(i64 a, i64 b) { return (a + b - 1) / b; }
static inline i64 floordiv(i64 x, i64 y) { return y == 0 ? 0 : (i64)std::floor((double)x / (double)y); }

extern "C" {

u16 tsl_ref_f32_to_f16(float f) { return f32_to_f16(f); }
float tsl_ref_f16_to_f32(u16 h) { return f16_to_f32(h); }

// ---------------------------------------------------------------- Rng
// The xorshift generator of src/bench.rs:13-35 and tests/common/mod.rs:7-23.
uint64_t tsl_ref_rng_new(uint64_t seed) { return (seed * 0x9e3779b97f4a7c15ull) | 1ull; }
uint64_t tsl_ref_rng_bits(uint64_t* s) {
    *s ^= *s << 13;
    *s ^= *s >> 7;
    *s ^= *s << 17;
    return *s;
}
float tsl_ref_rng_uniform(uint64_t* s) {
    uint64_t b = tsl_ref_rng_bits(s);
    return ((float)(b >> 40) / (float)(1ull << 24)) * 2.0f - 1.0f;
}
// Rng::tensor(dtype, shape, scale) (src/bench.rs:31-34) followed by
// Tensor::new's rounding (src/interp.rs:20-31): dtype 0 = f32 (float out),
// 1 = f16 (u16 bits out), 2 = i32 (int out, truncated).
void tsl_ref_rng_tensor(uint64_t* s, i64 n, float scale, int dtype, void* out) {
    for (i64 i = 0; i < n; i++) {
        float x = tsl_ref_rng_uniform(s) * scale;
        if (dtype == 0) ((float*)out)[i] = x;
        else if (dtype == 1) ((u16*)out)[i] = f32_to_f16(x);
        else ((i32*)out)[i] = std::isnan(x) ? 0 : (i32)(i64)std::trunc((double)x);
    }
}

// ---------------------------------------------------------------- matmul.tl

// matmul (kernels/matmul.tl:3-17): C = f16(A B), f32 accumulator updated
// once per BK-tile, programs mapped to tiles in groups of G block-rows.
// `threads` > 1 runs programs in parallel (they write disjoint tiles).
int tsl_ref_matmul(const u16* A, const u16* B, u16* C, i64 M, i64 N, i64 K, i64 BM, i64 BN, i64 BK, i64 G,
                   i64 first_pid, i64 npids, int threads) {
    i64 grid = cdiv(M, BM) * cdiv(N, BN);
    if (npids < 0 || first_pid + npids > grid) npids = grid - first_pid;
    std::vector<double> a(M * K), bt(N * K);
    for (i64 i = 0; i < M * K; i++) a[i] = h2d(A[i]);
    for (i64 k = 0; k < K; k++)
        for (i64 j = 0; j < N; j++) bt[j * K + k] = h2d(B[k * N + j]);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (i64 q = 0; q < npids; q++) {
        i64 pid = first_pid + q;
        i64 width = G * cdiv(N, BN);
        i64 first = (pid / width) * G;
        i64 rows = std::min(cdiv(M, BM) - first, G);
        i64 i = (first + (pid % width) % rows) * BM;
        i64 j = ((pid % width) / rows) * BN;
        i64 mi = std::min(BM, M - i), nj = std::min(BN, N - j);
        std::vector<double> acc(mi * nj, 0.0);
        for (i64 k = 0; k < K; k += BK) {
            i64 kl = std::min(BK, K - k);
            for (i64 ii = 0; ii < mi; ii++) {
                const double* ar = &a[(i + ii) * K + k];
                for (i64 jj = 0; jj < nj; jj++) {
                    const double* br = &bt[(j + jj) * K + k];
                    double s = 0.0;
                    for (i64 l = 0; l < kl; l++) s += ar[l] * br[l];
                    acc[ii * nj + jj] = r32(acc[ii * nj + jj] + s);
                }
            }
        }
        for (i64 ii = 0; ii < mi; ii++)
            for (i64 jj = 0; jj < nj; jj++) C[(i + ii) * N + j + jj] = f32_to_f16((float)acc[ii * nj + jj]);
    }
    return 0;
}

// matmul_f32 (kernels/matmul.tl:19-27): f32 operands, grid(cdiv(N,BN), cdiv(M,BM)).
int tsl_ref_matmul_f32(const float* A, const float* B, float* C, i64 M, i64 N, i64 K, i64 BM, i64 BN, i64 BK) {
    for (i64 i0 = 0; i0 < M; i0 += BM)
        for (i64 j0 = 0; j0 < N; j0 += BN) {
            i64 mi = std::min(BM, M - i0), nj = std::min(BN, N - j0);
            for (i64 ii = 0; ii < mi; ii++)
                for (i64 jj = 0; jj < nj; jj++) {
                    double acc = 0.0;
                    for (i64 k = 0; k < K; k += BK) {
                        double s = 0.0;
                        for (i64 l = k; l < std::min(K, k + BK); l++)
                            s += (double)A[(i0 + ii) * K + l] * (double)B[l * N + j0 + jj];
                        acc = r32(acc + s);
                    }
                    C[(i0 + ii) * N + j0 + jj] = (float)acc;
                }
        }
    return 0;
}

// The X W^T accumulation shared by matmul.tl linear and the llm.tl matmuls:
// acc[i][j] after every BK-tile of K (src/interp.rs:280-295).
static void xwt_acc(const u16* X, const u16* W, i64 M, i64 N, i64 K, i64 BK, std::vector<double>& acc) {
    acc.assign(M * N, 0.0);
    std::vector<double> x(M * K), w(N * K);
    for (i64 i = 0; i < M * K; i++) x[i] = h2d(X[i]);
    for (i64 i = 0; i < N * K; i++) w[i] = h2d(W[i]);
#pragma omp parallel for num_threads(8)
    for (i64 i = 0; i < M; i++)
        for (i64 j = 0; j < N; j++) {
            double a = 0.0;
            for (i64 k = 0; k < K; k += BK) {
                double s = 0.0;
                i64 ke = std::min(K, k + BK);
                for (i64 l = k; l < ke; l++) s += x[i * K + l] * w[j * K + l];
                a = r32(a + s);
            }
            acc[i * N + j] = a;
        }
}

// linear (kernels/matmul.tl:30-38): Y = f16(X W^T + f32(b)).
int tsl_ref_linear_bias(const u16* X, const u16* W, const u16* b, u16* Y, i64 M, i64 N, i64 K, i64 BK) {
    std::vector<double> acc;
    xwt_acc(X, W, M, N, K, BK, acc);
    for (i64 i = 0; i < M; i++)
        for (i64 j = 0; j < N; j++) Y[i * N + j] = f32_to_f16((float)r32(acc[i * N + j] + h2d(b[j])));
    return 0;
}

// ---------------------------------------------------------------- llm.tl matmuls

// linear (kernels/llm.tl:28-36): Y = f16(X W^T).
int tsl_ref_llm_linear(const u16* X, const u16* W, u16* Y, i64 M, i64 N, i64 K, i64 BK) {
    std::vector<double> acc;
    xwt_acc(X, W, M, N, K, BK, acc);
    for (i64 i = 0; i < M * N; i++) Y[i] = f32_to_f16((float)acc[i]);
    return 0;
}

// linear_residual (kernels/llm.tl:39-47): R = R + X W^T, f32.
int tsl_ref_linear_residual(const u16* X, const u16* W, float* R, i64 M, i64 N, i64 K, i64 BK) {
    std::vector<double> acc;
    xwt_acc(X, W, M, N, K, BK, acc);
    for (i64 i = 0; i < M * N; i++) R[i] = (float)r32((double)R[i] + acc[i]);
    return 0;
}

// logits (kernels/llm.tl:50-58): Y = X W^T, f32.
int tsl_ref_logits(const u16* X, const u16* W, float* Y, i64 M, i64 N, i64 K, i64 BK) {
    std::vector<double> acc;
    xwt_acc(X, W, M, N, K, BK, acc);
    for (i64 i = 0; i < M * N; i++) Y[i] = (float)acc[i];
    return 0;
}

// gate_up (kernels/llm.tl:62-73): Y = f16(g / (1.0 + exp(-g)) * u).
int tsl_ref_gate_up(const u16* X, const u16* Wg, const u16* Wu, u16* Y, i64 M, i64 F, i64 K, i64 BK) {
    std::vector<double> g, u;
    xwt_acc(X, Wg, M, F, K, BK, g);
    xwt_acc(X, Wu, M, F, K, BK, u);
    for (i64 i = 0; i < M * F; i++) {
        double e = r32(uexp(-g[i]));
        double den = r32(1.0 + e);
        double q = r32(g[i] / den);
        Y[i] = f32_to_f16((float)r32(q * u[i]));
    }
    return 0;
}

// ---------------------------------------------------------------- basic.tl

// add (kernels/basic.tl:3-7).
int tsl_ref_add(const float* X, const float* Y, float* Z, i64 N) {
    for (i64 i = 0; i < N; i++) Z[i] = (float)r32((double)X[i] + (double)Y[i]);
    return 0;
}

// softmax (kernels/basic.tl:10-17): rows of BC columns, out-of-range -inf.
int tsl_ref_softmax(const float* X, float* Y, i64 R, i64 C, i64 BC, int threads) {
#pragma omp parallel for num_threads(threads)
    for (i64 r = 0; r < R; r++) {
        std::vector<double> x(BC), e(BC);
        double m = -INFINITY;
        for (i64 c = 0; c < BC; c++) {
            x[c] = c < C ? (double)X[r * C + c] : -INFINITY;
            m = rmax(m, x[c]);
        }
        double s = 0.0;
        for (i64 c = 0; c < BC; c++) {
            e[c] = r32(uexp(r32(x[c] - m)));
            s += e[c];
        }
        s = r32(s);
        for (i64 c = 0; c < std::min(BC, C); c++) Y[r * C + c] = (float)r32(e[c] / s);
    }
    return 0;
}

// rmsnorm (kernels/basic.tl:20-26): f16 rows, f32 math.
int tsl_ref_rmsnorm_basic(const u16* X, const u16* W, u16* Y, i64 R, i64 C, float eps, i64 BC, int threads) {
#pragma omp parallel for num_threads(threads)
    for (i64 r = 0; r < R; r++) {
        double s = 0.0;
        for (i64 c = 0; c < BC; c++) {
            double x = c < C ? h2d(X[r * C + c]) : 0.0;
            s += r32(x * x);
        }
        double ms = r32(r32(s) / (double)(float)C);
        double rs = r32(ursqrt(r32(ms + (double)eps)));
        for (i64 c = 0; c < std::min(BC, C); c++)
            Y[r * C + c] = f32_to_f16((float)r32(r32(h2d(X[r * C + c]) * rs) * h2d(W[c])));
    }
    return 0;
}

// ---------------------------------------------------------------- llm.tl rows

// embed (kernels/llm.tl:10-16): X[t] = f32(E[tok[t]]); a token outside
// the vocabulary reads zeros.
int tsl_ref_embed(const i32* tok, const u16* E, float* X, i64 T, i64 V, i64 Dm) {
    for (i64 t = 0; t < T; t++)
        for (i64 c = 0; c < Dm; c++) {
            i64 row = tok[t];
            X[t * Dm + c] = (row >= 0 && row < V) ? f16_to_f32(E[row * Dm + c]) : 0.0f;
        }
    return 0;
}

// The shared body of llm.tl rmsnorm (:19-25) and rmsnorm_rows (:175-182):
// BC columns read (zeros past Dm), the mean taken over Dm.
static void rms_row(const float* x, const u16* W, u16* y, i64 Dm, i64 BC, float eps) {
    double s = 0.0;
    for (i64 c = 0; c < BC; c++) {
        double v = c < Dm ? (double)x[c] : 0.0;
        s += r32(v * v);
    }
    double ms = r32(r32(s) / (double)(float)Dm);
    double rs = r32(ursqrt(r32(ms + (double)eps)));
    for (i64 c = 0; c < std::min(BC, Dm); c++) y[c] = f32_to_f16((float)r32(r32((double)x[c] * rs) * h2d(W[c])));
}

int tsl_ref_rmsnorm(const float* X, const u16* W, u16* Y, i64 T, i64 Dm, float eps, i64 BC) {
    for (i64 t = 0; t < T; t++) rms_row(X + t * Dm, W, Y + t * Dm, Dm, BC, eps);
    return 0;
}

int tsl_ref_rmsnorm_rows(const float* X, const i32* idx, const u16* W, u16* Y, i64 T, i64 B, i64 Dm, float eps,
                         i64 BC) {
    std::vector<float> zero(Dm, 0.0f);
    for (i64 b = 0; b < B; b++) {
        i64 r = idx[b];
        const float* x = (r >= 0 && r < T) ? X + r * Dm : zero.data();
        rms_row(x, W, Y + b * Dm, Dm, BC, eps);
    }
    return 0;
}

// rope_q (kernels/llm.tl:78-88): Llama half-split rotation of each query head.
int tsl_ref_rope_q(const u16* QKV, const i32* pos, const float* Cs, const float* Sn, u16* Q, i64 T, i64 W,
                   i64 NPOS, i64 D2, i64 H, i64 D) {
    for (i64 t = 0; t < T; t++)
        for (i64 h = 0; h < H; h++) {
            i64 p = pos[t];
            bool pin = p >= 0 && p < NPOS;
            for (i64 i = 0; i < D2; i++) {
                double c = pin ? (double)Cs[p * D2 + i] : 0.0;
                double s = pin ? (double)Sn[p * D2 + i] : 0.0;
                i64 c1 = h * D + i, c2 = h * D + D2 + i;
                double x1 = c1 < W ? h2d(QKV[t * W + c1]) : 0.0;
                double x2 = c2 < W ? h2d(QKV[t * W + c2]) : 0.0;
                if (i < D) Q[(t * H + h) * D + i] = f32_to_f16((float)r32(r32(x1 * c) - r32(x2 * s)));
                if (D2 + i < D) Q[(t * H + h) * D + D2 + i] = f32_to_f16((float)r32(r32(x2 * c) + r32(x1 * s)));
            }
        }
    return 0;
}

// kv_write (kernels/llm.tl:93-112): rotated keys and values into the paged
// cache at slot[t] (dropped when out of range) and into K, V.
int tsl_ref_kv_write(const u16* QKV, const i32* pos, const i32* slot, const float* Cs, const float* Sn, u16* Kc,
                     u16* Vc, u16* K, u16* V, i64 T, i64 W, i64 NPOS, i64 D2, i64 NS, i64 G, i64 D) {
    for (i64 t = 0; t < T; t++)
        for (i64 g = 0; g < G; g++) {
            i64 p = pos[t], at = slot[t];
            bool pin = p >= 0 && p < NPOS, ain = at >= 0 && at < NS;
            i64 k0 = W - 2 * G * D + g * D;
            for (i64 i = 0; i < D2; i++) {
                double c = pin ? (double)Cs[p * D2 + i] : 0.0;
                double s = pin ? (double)Sn[p * D2 + i] : 0.0;
                i64 c1 = k0 + i, c2 = k0 + D2 + i;
                double x1 = (c1 >= 0 && c1 < W) ? h2d(QKV[t * W + c1]) : 0.0;
                double x2 = (c2 >= 0 && c2 < W) ? h2d(QKV[t * W + c2]) : 0.0;
                u16 y1 = f32_to_f16((float)r32(r32(x1 * c) - r32(x2 * s)));
                u16 y2 = f32_to_f16((float)r32(r32(x2 * c) + r32(x1 * s)));
                if (i < D) {
                    if (ain) Kc[(at * G + g) * D + i] = y1;
                    K[(t * G + g) * D + i] = y1;
                }
                if (D2 + i < D) {
                    if (ain) Kc[(at * G + g) * D + D2 + i] = y2;
                    K[(t * G + g) * D + D2 + i] = y2;
                }
            }
            for (i64 i = 0; i < D; i++) {
                i64 cv = k0 + G * D + i;
                u16 v = (cv >= 0 && cv < W) ? QKV[t * W + cv] : (u16)0;
                if (ain) Vc[(at * G + g) * D + i] = v;
                V[(t * G + g) * D + i] = v;
            }
        }
    return 0;
}

// ---------------------------------------------------------------- attention

// flash_attention (kernels/attention.tl:4-24) and prefill_attention
// (kernels/llm.tl:116-145) share one body: per block of BM query rows of
// head h, key blocks of BN from `lo`, online softmax. Strides describe
// [H,S,D] (flash) or [S,H,D]/[S,G,D] (prefill) layouts.
struct AttnView {
    const u16 *Q, *K, *V;
    u16* O;
    i64 S, D;
    i64 qrow, qhead, krow, khead;  // element strides
};

static void attn_block(const AttnView& v, i64 i, i64 hq, i64 hk, i64 BM, i64 BN, double scale, bool prefill,
                       const i32* starts) {
    const i64 D = v.D, S = v.S;
    std::vector<double> q(BM * D), m(BM), l(BM, 0.0), acc(BM * D, 0.0), s(BM * BN), p(BM * BN);
    std::vector<i64> st(BM, 0);
    for (i64 r = 0; r < BM; r++) {
        i64 row = i + r;
        for (i64 d = 0; d < D; d++) q[r * D + d] = row < S ? h2d(v.Q[row * v.qrow + hq * v.qhead + d]) : 0.0;
        m[r] = prefill ? r32(-1e30) : -INFINITY;
        if (prefill) st[r] = row < S ? starts[row] : 0;
    }
    i64 lo = prefill ? starts[i] : 0;
    i64 hi = std::min(i + BM, S);
    for (i64 j = lo; j < hi; j += BN) {
        for (i64 r = 0; r < BM; r++) {
            i64 row = i + r;
            double mx = -INFINITY;
            for (i64 c = 0; c < BN; c++) {
                i64 col = j + c;
                double dot = 0.0;
                if (col >= 0 && col < S) {
                    const u16* kr = v.K + col * v.krow + hk * v.khead;
                    for (i64 d = 0; d < D; d++) dot += q[r * D + d] * h2d(kr[d]);
                } else {
                    for (i64 d = 0; d < D; d++) dot += q[r * D + d] * 0.0;
                }
                double x = r32(r32(0.0 + dot) * scale);
                bool keep = col <= row && col < S && (!prefill || col >= st[r]);
                s[r * BN + c] = keep ? x : -INFINITY;
                mx = rmax(mx, s[r * BN + c]);
            }
            double m2 = bmax(m[r], mx);
            double psum = 0.0;
            for (i64 c = 0; c < BN; c++) {
                p[r * BN + c] = r32(uexp(r32(s[r * BN + c] - m2)));
                psum += p[r * BN + c];
            }
            double a = r32(uexp(r32(m[r] - m2)));
            l[r] = r32(r32(l[r] * a) + r32(psum));
            for (i64 d = 0; d < D; d++) {
                double pv = 0.0;
                for (i64 c = 0; c < BN; c++) {
                    i64 col = j + c;
                    double vv = (col >= 0 && col < S) ? h2d(v.V[col * v.krow + hk * v.khead + d]) : 0.0;
                    pv += r16(p[r * BN + c]) * vv;
                }
                acc[r * D + d] = r32(r32(acc[r * D + d] * a) + r32(0.0 + pv));
            }
            m[r] = m2;
        }
    }
    for (i64 r = 0; r < BM; r++) {
        i64 row = i + r;
        if (row >= S) continue;
        for (i64 d = 0; d < D; d++)
            v.O[row * v.qrow + hq * v.qhead + d] = f32_to_f16((float)r32(acc[r * D + d] / l[r]));
    }
}

int tsl_ref_flash_attention(const u16* Q, const u16* K, const u16* V, u16* O, i64 H, i64 S, i64 D, float scale,
                            i64 BM, i64 BN, int threads) {
    AttnView v{Q, K, V, O, S, D, D, S * D, D, S * D};
    i64 nb = cdiv(S, BM);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (i64 q = 0; q < H * nb; q++) attn_block(v, (q % nb) * BM, q / nb, q / nb, BM, BN, scale, false, nullptr);
    return 0;
}

int tsl_ref_prefill_attention(const u16* Q, const u16* K, const u16* V, const i32* starts, u16* O, i64 S, i64 H,
                              i64 G, i64 D, float scale, i64 BM, i64 BN, int threads) {
    AttnView v{Q, K, V, O, S, D, H * D, D, G * D, D};
    i64 nb = cdiv(S, BM);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (i64 q = 0; q < H * nb; q++) {
        i64 h = q / nb;
        i64 g = floordiv(h, H / G);
        attn_block(v, (q % nb) * BM, h, g, BM, BN, scale, true, starts);
    }
    return 0;
}

// decode_attention (kernels/llm.tl:150-172), and paged_attention
// (kernels/attention.tl:29-51) when G == H: one program per (b, h) walking
// the sequence's pages through the block table. A table read past MP reads
// page 0 and a page outside [0, NP) reads zeros (src/interp.rs:93-117).
int tsl_ref_decode_attention(const u16* Q, const u16* Kc, const u16* Vc, const i32* table, const i32* lens, u16* O,
                             i64 B, i64 H, i64 D, i64 NP, i64 P, i64 G, i64 MP, float scale, int threads) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (i64 q = 0; q < B * H; q++) {
        i64 b = q / H, h = q % H;
        i64 g = floordiv(h, H / G);
        i64 n = lens[b];
        std::vector<double> qv(D), acc(D, 0.0), sc(P), p(P), k(P * D), vv(P * D);
        for (i64 d = 0; d < D; d++) qv[d] = h2d(Q[(b * H + h) * D + d]);
        double m = -INFINITY, l = 0.0;
        for (i64 t = 0; t < n; t += P) {
            i64 ti = floordiv(t, P);
            i64 page = ti < MP ? table[b * MP + ti] : 0;
            bool pin = page >= 0 && page < NP;
            for (i64 r = 0; r < P; r++)
                for (i64 d = 0; d < D; d++) {
                    i64 o = ((page * P + r) * G + g) * D + d;
                    k[r * D + d] = pin ? h2d(Kc[o]) : 0.0;
                    vv[r * D + d] = pin ? h2d(Vc[o]) : 0.0;
                }
            double mx = -INFINITY;
            for (i64 r = 0; r < P; r++) {
                double s = 0.0;
                for (i64 d = 0; d < D; d++) s += r32(k[r * D + d] * qv[d]);
                double x = r32(r32(s) * scale);
                sc[r] = (t + r < n) ? x : -INFINITY;
                mx = rmax(mx, sc[r]);
            }
            double m2 = bmax(m, mx);
            double psum = 0.0;
            for (i64 r = 0; r < P; r++) {
                p[r] = r32(uexp(r32(sc[r] - m2)));
                psum += p[r];
            }
            double a = r32(uexp(r32(m - m2)));
            l = r32(r32(l * a) + r32(psum));
            for (i64 d = 0; d < D; d++) {
                double s = 0.0;
                for (i64 r = 0; r < P; r++) s += r32(p[r] * vv[r * D + d]);
                acc[d] = r32(r32(acc[d] * a) + r32(s));
            }
            m = m2;
        }
        for (i64 d = 0; d < D; d++) O[(b * H + h) * D + d] = f32_to_f16((float)r32(acc[d] / l));
    }
    return 0;
}

}  // extern "C"
