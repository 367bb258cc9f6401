// HBM-bound row and elementwise kernels: basic.tl softmax (:10-17),
// rmsnorm (:20-26) and add (:3-7); llm.tl embed (:10-16), rmsnorm (:19-25),
// rmsnorm_rows (:175-182), rope_q (:78-88) and kv_write (:93-112).
//
// A row is owned by one 64-lane wavefront: it is read once with 16-byte
// loads into registers, reduced across the wavefront (xor butterflies) and
// written once, so each element crosses HBM once each way. Rows longer
// than the register budget take a second, cache-resident pass.
#include "common.h"

#include <climits>
#include <type_traits>

namespace {

constexpr int ROWS_PER_WG = 4;  // one wavefront per row, 4 per workgroup

// softmax and basic.rmsnorm rows are read once and their outputs are not
// read back by the same kernel: nontemporal loads and stores (4096^2, rows
// from HBM: rmsnorm 14.0 -> 13.2 us, softmax 27.1 -> 25.6 us, with softmax's
// division as DivBy).
template <class T>
TSL_DEV T load_once(const T* p) { return __builtin_nontemporal_load(p); }
template <class T>
TSL_DEV void store_out(T v, T* p) { __builtin_nontemporal_store(v, p); }

// ---------------------------------------------------------------- softmax
// Y[r, c] = exp(x - max) / sum(exp(x - max)) over the first ncols = min(BC, C)
// columns; columns past C read -inf (kernels/basic.tl:13), so they add 0.
template <int NV, int RPW = ROWS_PER_WG>
__global__ __launch_bounds__(64 * RPW) void softmax_kernel(const float* __restrict__ X, float* __restrict__ Y, int R, int C,
                                                      int ncols) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * RPW + (threadIdx.x >> 6);
    if (row >= R) return;
    const float* x = X + (size_t)row * C;
    float* y = Y + (size_t)row * C;
    const bool vec = (C % 4) == 0;
    // FULL: every chunk of every lane lies inside the row (a uniform branch,
    // so the common shape runs without per-chunk tests).
    auto body = [&](auto full) {
        constexpr bool FULL = decltype(full)::value;
        float v[NV][4];
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int c = i * 256 + lane * 4;
            if (FULL || (vec && c + 4 <= ncols)) {
                float4v t = load_once(reinterpret_cast<const float4v*>(x + c));
                for (int e = 0; e < 4; e++) v[i][e] = t[e];
            } else {
                for (int e = 0; e < 4; e++) v[i][e] = (c + e < ncols) ? x[c + e] : -INFINITY;
            }
            for (int e = 0; e < 4; e++) m = fmaxf(m, v[i][e]);
        }
        m = wave_max(m);
        // exp(x - m) as exp2((x - m) log2(e)): one v_exp_f32 and two operations
        // per element where expf expands to ~12 (its range reduction and
        // overflow/underflow selects); x - m <= 0, so exp2's argument is in
        // range, and its rounding adds < 1e-6 relative (the f32 result is
        // within a few ulp of expf's). 4096^2 from HBM: 25.6 -> 23.8 us.
        constexpr float LOG2E_F = 1.4426950408889634f;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; i++)
            for (int e = 0; e < 4; e++) {
                v[i][e] = __builtin_amdgcn_exp2f((v[i][e] - m) * LOG2E_F);
                s += v[i][e];
            }
        const DivBy by_s(wave_sum(s));  // s >= 1: the row's max contributes exp(0)
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int c = i * 256 + lane * 4;
            if (FULL || (vec && c + 4 <= ncols)) {
                float4v t;
                for (int e = 0; e < 4; e++) t[e] = by_s(v[i][e]);
                store_out(t, reinterpret_cast<float4v*>(y + c));
            } else {
                for (int e = 0; e < 4; e++)
                    if (c + e < ncols) y[c + e] = by_s(v[i][e]);
            }
        }
    };
    if (vec && ncols == NV * 256) body(std::true_type{});
    else body(std::false_type{});
}

// Rows longer than the register tile: a max/sum pass, then the writes.
__global__ __launch_bounds__(256) void softmax_long_kernel(const float* __restrict__ X, float* __restrict__ Y, int R,
                                                           int C, int ncols) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * ROWS_PER_WG + (threadIdx.x >> 6);
    if (row >= R) return;
    const float* x = X + (size_t)row * C;
    float* y = Y + (size_t)row * C;
    float m = -INFINITY, s = 0.0f;
    for (int c = lane; c < ncols; c += 64) {
        float t = x[c];
        float m2 = fmaxf(m, t);
        s = s * expf(m - m2) + expf(t - m2);
        m = m2;
    }
    float mw = wave_max(m);
    s = wave_sum(m == -INFINITY ? 0.0f : s * expf(m - mw));
    for (int c = lane; c < ncols; c += 64) y[c] = expf(x[c] - mw) / s;
}

// ---------------------------------------------------------------- rmsnorm
// y = x * (1 / sqrt(sum(x^2 over BC columns) / n + eps)) * w, over the
// first ncols = min(BC, C) columns (columns past C read 0). XT is f16
// (basic.tl) or f32 (llm.tl); `rows` (rmsnorm_rows) gathers the input row.
// Writes y[c] = f16(v * rs * w[c]) for this lane's NV chunks of E columns
// (chunk i starts at column (64 i + lane) E), the first ncols columns only.
template <int E, int NV, bool FULL = false>
TSL_DEV void rms_store(const float (&v)[NV][E], float rs, const u16* __restrict__ W, u16* __restrict__ y, int lane,
                       int ncols, bool vec) {
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = (i * 64 + lane) * E;
        if (FULL || (vec && c + E <= ncols)) {
            // E outputs: 8 halves (16 bytes) for f16 input rows, 4 (8 bytes) for f32.
            // The weights' E halves in one load (the row's chunk is aligned alike).
            uint32_t wv[E / 2];
            if constexpr (E == 8) {
                const u32x4 t = *reinterpret_cast<const u32x4*>(W + c);
                for (int p = 0; p < 4; p++) wv[p] = t[p];
            } else {
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 t = *reinterpret_cast<const u32x2*>(W + c);
                for (int p = 0; p < 2; p++) wv[p] = t[p];
            }
            uint32_t o[E / 2];
            for (int p = 0; p < E / 2; p++) {
                u16 lo = f2h(v[i][2 * p] * rs * h2f((u16)(wv[p] & 0xffff)));
                u16 hi = f2h(v[i][2 * p + 1] * rs * h2f((u16)(wv[p] >> 16)));
                o[p] = (uint32_t)lo | ((uint32_t)hi << 16);
            }
            if constexpr (E == 8) {
                store_out(u32x4{o[0], o[1], o[2], o[3]}, reinterpret_cast<u32x4*>(y + c));
            } else {
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                store_out(u32x2{o[0], o[1]}, reinterpret_cast<u32x2*>(y + c));
            }
        } else {
            for (int e = 0; e < E; e++)
                if (c + e < ncols) y[c + e] = f2h(v[i][e] * rs * h2f(W[c + e]));
        }
    }
}

template <typename XT, int NV>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const XT* __restrict__ X, const int* __restrict__ idx,
                                                      int xrows, const u16* __restrict__ W, u16* __restrict__ Y,
                                                      int R, int C, int ncols, float n, float eps) {
    constexpr int E = 16 / sizeof(XT);  // elements per 16-byte load
    const int lane = threadIdx.x & 63, row = blockIdx.x * ROWS_PER_WG + (threadIdx.x >> 6);
    if (row >= R) return;
    int src = row;
    if (idx) src = idx[row];
    const bool rin = src >= 0 && src < xrows;
    const XT* x = X + (size_t)(rin ? src : 0) * C;
    u16* y = Y + (size_t)row * C;
    const bool vec = (C % E) == 0;
    float v[NV][E];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = (i * 64 + lane) * E;
        if (rin && vec && c + E <= ncols) {
            if constexpr (sizeof(XT) == 2) {
                u32x4 t = load_once(reinterpret_cast<const u32x4*>(x + c));
                for (int e = 0; e < E; e++) v[i][e] = h2f((u16)(t[e >> 1] >> (16 * (e & 1))));
            } else {
                float4v t = load_once(reinterpret_cast<const float4v*>(x + c));
                for (int e = 0; e < E; e++) v[i][e] = t[e];
            }
        } else {
            for (int e = 0; e < E; e++) {
                float t = 0.0f;
                if (rin && c + e < ncols) {
                    if constexpr (sizeof(XT) == 2) t = h2f(x[c + e]);
                    else t = x[c + e];
                }
                v[i][e] = t;
            }
        }
        for (int e = 0; e < E; e++) ss += v[i][e] * v[i][e];
    }
    ss = wave_sum(ss);
    const float rs = 1.0f / sqrtf(ss / n + eps);
    rms_store<E, NV>(v, rs, W, y, lane, ncols, vec);
}

// basic.rmsnorm over f16 rows whose every 16-byte chunk is present (ncols ==
// C == 512 NV): the row and its NV weight chunks stay packed (4 registers a
// chunk each, not 8 floats), so the weight loads are issued with the row's,
// before the reduction, and the wavefront waits on one memory round trip
// instead of two with all 4096 wavefronts of a 4096^2 call resident. The
// weights come once per workgroup through LDS (each wavefront reading all
// of them from L2 doubled the L2 traffic of a 4096^2 call): 4096^2 from HBM
// 11.23 -> 10.86 us. Same arithmetic, in the same order, as rmsnorm_kernel.
// Wavefronts past R load row R - 1 and leave after the barrier.
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_f16_full_kernel(const u16* __restrict__ X, const u16* __restrict__ W,
                                                               u16* __restrict__ Y, int R, int C, float n, float eps) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * ROWS_PER_WG + (threadIdx.x >> 6);
    __shared__ u32x4 wl[NV * 64];
    u32x4 xv[NV], wv[NV];
    const u16* x = X + (size_t)min(row, R - 1) * C;
    u16* y = Y + (size_t)row * C;
#pragma unroll
    for (int i = 0; i < NV; i++) xv[i] = load_once(reinterpret_cast<const u32x4*>(x + (i * 64 + lane) * 8));
    for (int c = threadIdx.x; c < NV * 64; c += 256) wl[c] = *reinterpret_cast<const u32x4*>(W + c * 8);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NV; i++) wv[i] = wl[i * 64 + lane];
    if (row >= R) return;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++)
        for (int e = 0; e < 8; e++) {
            const float v = h2f((u16)(xv[i][e >> 1] >> (16 * (e & 1))));
            ss += v * v;
        }
    ss = wave_sum(ss);
    const float rs = 1.0f / sqrtf(ss / n + eps);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        u32x4 o;
        for (int p = 0; p < 4; p++) {
            const u16 lo = f2h(h2f((u16)(xv[i][p] & 0xffff)) * rs * h2f((u16)(wv[i][p] & 0xffff)));
            const u16 hi = f2h(h2f((u16)(xv[i][p] >> 16)) * rs * h2f((u16)(wv[i][p] >> 16)));
            o[p] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        store_out(o, reinterpret_cast<u32x4*>(y + (i * 64 + lane) * 8));
    }
}

// ---- one workgroup per row (llm.tl rmsnorm over f32 rows, and the fused
// residual projection): thread t owns the float4 chunks t, t + 256, ... of
// the row, so a decode-sized batch (a few dozen rows) still spreads its
// loads over 256 lanes per row, all issued before the reduction.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Loads this thread's chunks of W (zeros past ncols).
template <int NC>
TSL_DEV void rms_wg_weights(const u16* __restrict__ W, int t, int ncols, u32x2 (&w)[NC]) {
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int c = (i * 256 + t) * 4;
        if (c + 4 <= ncols) {
            w[i] = *reinterpret_cast<const u32x2*>(W + c);
        } else {
            uint32_t h[4];
            for (int e = 0; e < 4; e++) h[e] = c + e < ncols ? W[c + e] : 0;
            w[i] = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        }
    }
}

// Given this thread's values v (zero past ncols) and weights, writes
// y[c] = f16(v * rs * w[c]) for the first ncols columns, rs = 1 / sqrt(sum
// of squares of the row / n + eps): per-thread sums in chunk order, then
// the wavefront butterfly, then the 4 wavefronts in order.
template <int NC>
TSL_DEV void rms_wg_finish(const float4v (&v)[NC], const u32x2 (&w)[NC], int t, int ncols, float n, float eps,
                           u16* __restrict__ y, float* red) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; i++)
        for (int e = 0; e < 4; e++) ss += v[i][e] * v[i][e];
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const float rs = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / n + eps);
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int c = (i * 256 + t) * 4;
        u16 o[4];
        for (int e = 0; e < 4; e++) o[e] = f2h(v[i][e] * rs * h2f((u16)(w[i][e >> 1] >> (16 * (e & 1)))));
        if (c + 4 <= ncols) {
            *reinterpret_cast<u32x2*>(y + c) = u32x2{o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16)};
        } else {
            for (int e = 0; e < 4; e++)
                if (c + e < ncols) y[c + e] = o[e];
        }
    }
}

// llm.tl rmsnorm / rmsnorm_rows over f32 rows with C % 4 == 0 and
// ncols <= 1024 NC; idx (rmsnorm_rows) gathers the input row.
template <int NC>
__global__ __launch_bounds__(256) void rmsnorm_wg_kernel(const float* __restrict__ X, const int* __restrict__ idx,
                                                         int xrows, const u16* __restrict__ W, u16* __restrict__ Y,
                                                         int C, int ncols, float n, float eps) {
    __shared__ float red[4];
    TSL_POISON(red);
    const int t = threadIdx.x, row = blockIdx.x;
    const int src = idx ? idx[row] : row;
    const bool rin = src >= 0 && src < xrows;
    const float* x = X + (size_t)(rin ? src : 0) * C;
    float4v v[NC];
    u32x2 w[NC];
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int c = (i * 256 + t) * 4;
        if (rin && c + 4 <= ncols) {
            v[i] = *reinterpret_cast<const float4v*>(x + c);
        } else {
            for (int e = 0; e < 4; e++) v[i][e] = rin && c + e < ncols ? x[c + e] : 0.0f;
        }
    }
    rms_wg_weights<NC>(W, t, ncols, w);
    rms_wg_finish<NC>(v, w, t, ncols, n, eps, Y + (size_t)row * C, red);
}

// The engine's fused step after a K-split residual projection: R[m] += the
// S slices of part[ks][m], added in slice order as skinny_reduce adds them,
// then Y[m] = rmsnorm(R[m]) W as rmsnorm_wg_kernel computes it, over all C
// columns (C % 4 == 0, C <= 1024 NC): the bits of llm/linear_residual (same
// split) followed by llm/rmsnorm. SU > 0: S == SU, every load of the row
// issued at once; 0: any S.
template <int NC, int SU>
__global__ __launch_bounds__(256) void reduce_rmsnorm_kernel(const float* __restrict__ part, int S,
                                                             float* __restrict__ R, const u16* __restrict__ W,
                                                             u16* __restrict__ Y, int M, int C, float n, float eps) {
    __shared__ float red[4];
    TSL_POISON(red);
    const int t = threadIdx.x, row = blockIdx.x;
    const size_t mc = (size_t)M * C;
    float* r = R + (size_t)row * C;
    const float* pr = part + (size_t)row * C;
    const float4v z = {0.0f, 0.0f, 0.0f, 0.0f};
    float4v old[NC], acc[NC];
    u32x2 w[NC];
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int c = (i * 256 + t) * 4;
        old[i] = c < C ? *reinterpret_cast<const float4v*>(r + c) : z;
        acc[i] = z;
    }
    rms_wg_weights<NC>(W, t, C, w);
    auto slice = [&](int ks) {
#pragma unroll
        for (int i = 0; i < NC; i++) {
            const int c = (i * 256 + t) * 4;
            if (c < C) acc[i] += *reinterpret_cast<const float4v*>(pr + ks * mc + c);
        }
    };
    if constexpr (SU > 0) {
#pragma unroll
        for (int ks = 0; ks < SU; ks++) slice(ks);
    } else {
        for (int ks = 0; ks < S; ks++) slice(ks);
    }
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int c = (i * 256 + t) * 4;
        if (c < C) {
            old[i] += acc[i];
            *reinterpret_cast<float4v*>(r + c) = old[i];
        }
    }
    rms_wg_finish<NC>(old, w, t, C, n, eps, Y + (size_t)row * C, red);
}

template <typename XT>
__global__ __launch_bounds__(256) void rmsnorm_long_kernel(const XT* __restrict__ X, const int* __restrict__ idx,
                                                           int xrows, const u16* __restrict__ W, u16* __restrict__ Y,
                                                           int R, int C, int ncols, float n, float eps) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * ROWS_PER_WG + (threadIdx.x >> 6);
    if (row >= R) return;
    int src = idx ? idx[row] : row;
    const bool rin = src >= 0 && src < xrows;
    const XT* x = X + (size_t)(rin ? src : 0) * C;
    auto ld = [&](int c) -> float {
        if (!rin) return 0.0f;
        if constexpr (sizeof(XT) == 2) return h2f(x[c]);
        else return x[c];
    };
    float ss = 0.0f;
    for (int c = lane; c < ncols; c += 64) {
        float t = ld(c);
        ss += t * t;
    }
    const float rs = 1.0f / sqrtf(wave_sum(ss) / n + eps);
    for (int c = lane; c < ncols; c += 64) Y[(size_t)row * C + c] = f2h(ld(c) * rs * h2f(W[c]));
}

template <typename XT>
int run_rmsnorm(const XT* X, const int* idx, int xrows, const u16* W, u16* Y, int R, int C, int ncols, float eps,
                hipStream_t s, const char* what) {
    if (R == 0) return 0;
    const float n = (float)C;
    if constexpr (sizeof(XT) == 4) {
        if (C % 4 == 0 && ncols <= 4096) {
            if (ncols <= 1024)
                hipLaunchKernelGGL(rmsnorm_wg_kernel<1>, dim3(R), dim3(256), 0, s, X, idx, xrows, W, Y, C, ncols, n, eps);
            else if (ncols <= 2048)
                hipLaunchKernelGGL(rmsnorm_wg_kernel<2>, dim3(R), dim3(256), 0, s, X, idx, xrows, W, Y, C, ncols, n, eps);
            else
                hipLaunchKernelGGL(rmsnorm_wg_kernel<4>, dim3(R), dim3(256), 0, s, X, idx, xrows, W, Y, C, ncols, n, eps);
            return TSL_LAUNCHED(what);
        }
    }
    dim3 grid((R + ROWS_PER_WG - 1) / ROWS_PER_WG);
    if constexpr (sizeof(XT) == 2) {
        if (!idx && ncols == C && (C == 2048 || C == 4096)) {
            if (C == 2048)
                hipLaunchKernelGGL(rmsnorm_f16_full_kernel<4>, grid, dim3(256), 0, s, X, W, Y, R, C, n, eps);
            else
                hipLaunchKernelGGL(rmsnorm_f16_full_kernel<8>, grid, dim3(256), 0, s, X, W, Y, R, C, n, eps);
            return TSL_LAUNCHED(what);
        }
    }
    constexpr int E = 16 / sizeof(XT);
    if (ncols <= 64 * E * 4)
        hipLaunchKernelGGL((rmsnorm_kernel<XT, 4>), grid, dim3(256), 0, s, X, idx, xrows, W, Y, R, C, ncols, n, eps);
    else if (ncols <= 64 * E * 8)
        hipLaunchKernelGGL((rmsnorm_kernel<XT, 8>), grid, dim3(256), 0, s, X, idx, xrows, W, Y, R, C, ncols, n, eps);
    else
        hipLaunchKernelGGL((rmsnorm_long_kernel<XT>), grid, dim3(256), 0, s, X, idx, xrows, W, Y, R, C, ncols, n, eps);
    return TSL_LAUNCHED(what);
}

// ---------------------------------------------------------------- add, embed

__global__ __launch_bounds__(256) void add_kernel(const float* __restrict__ X, const float* __restrict__ Y,
                                                  float* __restrict__ Z, long n) {
    long i = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i + 4 <= n) {
        float4v a = *reinterpret_cast<const float4v*>(X + i), b = *reinterpret_cast<const float4v*>(Y + i);
        *reinterpret_cast<float4v*>(Z + i) = a + b;
    } else {
        for (; i < n; i++) Z[i] = X[i] + Y[i];
    }
}

// X[t, :] = f32(E[tok[t], :]); a token outside [0, V) reads zeros.
__global__ __launch_bounds__(256) void embed_kernel(const int* __restrict__ tok, const u16* __restrict__ E,
                                                    float* __restrict__ X, int T, int V, int Dm) {
    const int t = blockIdx.y;
    const int row = tok[t];
    const bool in = row >= 0 && row < V;
    for (int c = (blockIdx.x * 256 + threadIdx.x) * 8; c < Dm; c += gridDim.x * 256 * 8) {
        float* x = X + (size_t)t * Dm + c;
        if (c + 8 <= Dm && (Dm % 8) == 0) {
            float4v a, b;
            if (in) {
                u32x4 h = *reinterpret_cast<const u32x4*>(E + (size_t)row * Dm + c);
                for (int e = 0; e < 4; e++) a[e] = h2f((u16)(h[e >> 1] >> (16 * (e & 1))));
                for (int e = 0; e < 4; e++) b[e] = h2f((u16)(h[2 + (e >> 1)] >> (16 * (e & 1))));
            } else {
                a = float4v{0, 0, 0, 0};
                b = a;
            }
            *reinterpret_cast<float4v*>(x) = a;
            *reinterpret_cast<float4v*>(x + 4) = b;
        } else {
            for (int e = 0; e < 8 && c + e < Dm; e++) x[e] = in ? h2f(E[(size_t)row * Dm + c + e]) : 0.0f;
        }
    }
}

// ---------------------------------------------------------------- rotary
// rope_q: Q[t, h, i] = x1 c - x2 s and Q[t, h, D2 + i] = x2 c + x1 s with
// x1 = QKV[t, h D + i], x2 = QKV[t, h D + D2 + i], (c, s) at pos[t].
struct RopeArgs {
    const u16* QKV;
    const int *pos, *slot;
    const float *Cs, *Sn;
    u16* Q;
    u16 *Kc, *Vc, *K, *V;
    int T, W, NPOS, D2, H, NS, G, D;
};

// Element e of rope_q's T x H x D2 index space.
TSL_DEV void rope_q_elem(const RopeArgs& a, long e) {
    const int i = e % a.D2, h = (e / a.D2) % a.H, t = e / ((long)a.D2 * a.H);
    const int p = a.pos[t];
    const bool pin = p >= 0 && p < a.NPOS;
    const float c = pin ? a.Cs[(size_t)p * a.D2 + i] : 0.0f, s = pin ? a.Sn[(size_t)p * a.D2 + i] : 0.0f;
    const int c1 = h * a.D + i, c2 = h * a.D + a.D2 + i;
    const float x1 = c1 < a.W ? h2f(a.QKV[(size_t)t * a.W + c1]) : 0.0f;
    const float x2 = c2 < a.W ? h2f(a.QKV[(size_t)t * a.W + c2]) : 0.0f;
    u16* q = a.Q + ((size_t)t * a.H + h) * a.D;
    u16 y1, y2;
    rope_rotate(x1, x2, c, s, y1, y2);
    if (i < a.D) q[i] = y1;
    if (a.D2 + i < a.D) q[a.D2 + i] = y2;
}

// kv_write: the rotated keys and the values of kv head g into the paged
// cache at slot[t] (dropped when outside [0, NS)) and into K, V [T, G, D].
// Element e of its T x G x max(D2, D) index space.
TSL_DEV void kv_write_elem(const RopeArgs& a, long e) {
    const int nd = a.D2 > a.D ? a.D2 : a.D;
    const int i = e % nd, g = (e / nd) % a.G, t = e / ((long)nd * a.G);
    const int p = a.pos[t], at = a.slot[t];
    const bool pin = p >= 0 && p < a.NPOS, ain = at >= 0 && at < a.NS;
    const long k0 = (long)a.W - 2L * a.G * a.D + (long)g * a.D;
    u16* kc = a.Kc + ((size_t)(ain ? at : 0) * a.G + g) * a.D;
    u16* vc = a.Vc + ((size_t)(ain ? at : 0) * a.G + g) * a.D;
    u16* kk = a.K + ((size_t)t * a.G + g) * a.D;
    u16* vv = a.V + ((size_t)t * a.G + g) * a.D;
    if (i < a.D2) {
        const float c = pin ? a.Cs[(size_t)p * a.D2 + i] : 0.0f, s = pin ? a.Sn[(size_t)p * a.D2 + i] : 0.0f;
        const long c1 = k0 + i, c2 = k0 + a.D2 + i;
        const float x1 = (c1 >= 0 && c1 < a.W) ? h2f(a.QKV[(size_t)t * a.W + c1]) : 0.0f;
        const float x2 = (c2 >= 0 && c2 < a.W) ? h2f(a.QKV[(size_t)t * a.W + c2]) : 0.0f;
        u16 y1, y2;
        rope_rotate(x1, x2, c, s, y1, y2);
        if (i < a.D) {
            if (ain) kc[i] = y1;
            kk[i] = y1;
        }
        if (a.D2 + i < a.D) {
            if (ain) kc[a.D2 + i] = y2;
            kk[a.D2 + i] = y2;
        }
    }
    if (i < a.D) {
        const long cv = k0 + (long)a.G * a.D + i;
        const u16 v = (cv >= 0 && cv < a.W) ? a.QKV[(size_t)t * a.W + cv] : (u16)0;
        if (ain) vc[i] = v;
        vv[i] = v;
    }
}

// rope_q and kv_write together, 8 columns per thread: item e = (t, head
// slot hh of the H query, G key and G value heads of QKV's row, chunk c of
// D2 / 8). Query and key slots rotate columns 8c .. 8c+7 with their D2
// partners (16-byte loads and stores, the same rope_rotate arithmetic as
// the element kernels, so the same bits); value slots copy both chunks. For
// D = 2 D2, D2 % 8 == 0, W = (H + 2 G) D and 32-bit indices.
__global__ __launch_bounds__(256) void rope_kv_vec(RopeArgs a, int n) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    const int nc = a.D2 / 8, slots = a.H + 2 * a.G;
    const int c = e % nc, hh = (e / nc) % slots, t = e / (nc * slots);
    const int i0 = 8 * c;
    const u16* row = a.QKV + (size_t)t * a.W + hh * a.D;
    const u32x4 v1 = *reinterpret_cast<const u32x4*>(row + i0), v2 = *reinterpret_cast<const u32x4*>(row + a.D2 + i0);
    const int at = a.slot ? a.slot[t] : -1;
    const bool ain = at >= 0 && at < a.NS;
    if (hh >= a.H + a.G) {  // a value head: copied
        const int g = hh - a.H - a.G;
        u16* vv = a.V + ((size_t)t * a.G + g) * a.D;
        *reinterpret_cast<u32x4*>(vv + i0) = v1;
        *reinterpret_cast<u32x4*>(vv + a.D2 + i0) = v2;
        if (ain) {
            u16* vc = a.Vc + ((size_t)at * a.G + g) * a.D;
            *reinterpret_cast<u32x4*>(vc + i0) = v1;
            *reinterpret_cast<u32x4*>(vc + a.D2 + i0) = v2;
        }
        return;
    }
    const int p = a.pos[t];
    const bool pin = p >= 0 && p < a.NPOS;
    float cs[8], sn[8];
    if (pin) {
        const float4v* cp = reinterpret_cast<const float4v*>(a.Cs + (size_t)p * a.D2 + i0);
        const float4v* sp = reinterpret_cast<const float4v*>(a.Sn + (size_t)p * a.D2 + i0);
        const float4v c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            cs[j] = c0[j], cs[4 + j] = c1[j];
            sn[j] = s0[j], sn[4 + j] = s1[j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) cs[j] = sn[j] = 0.0f;
    }
    u32x4 y1, y2;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        u16 a1, a2, b1, b2;
        rope_rotate(h2f((u16)(v1[j] & 0xffff)), h2f((u16)(v2[j] & 0xffff)), cs[2 * j], sn[2 * j], a1, a2);
        rope_rotate(h2f((u16)(v1[j] >> 16)), h2f((u16)(v2[j] >> 16)), cs[2 * j + 1], sn[2 * j + 1], b1, b2);
        y1[j] = (uint32_t)a1 | ((uint32_t)b1 << 16);
        y2[j] = (uint32_t)a2 | ((uint32_t)b2 << 16);
    }
    if (hh < a.H) {
        u16* q = a.Q + ((size_t)t * a.H + hh) * a.D;
        *reinterpret_cast<u32x4*>(q + i0) = y1;
        *reinterpret_cast<u32x4*>(q + a.D2 + i0) = y2;
        return;
    }
    const int g = hh - a.H;
    u16* kk = a.K + ((size_t)t * a.G + g) * a.D;
    *reinterpret_cast<u32x4*>(kk + i0) = y1;
    *reinterpret_cast<u32x4*>(kk + a.D2 + i0) = y2;
    if (ain) {
        u16* kc = a.Kc + ((size_t)at * a.G + g) * a.D;
        *reinterpret_cast<u32x4*>(kc + i0) = y1;
        *reinterpret_cast<u32x4*>(kc + a.D2 + i0) = y2;
    }
}

// KIND 0: rope_q, 1: kv_write, 2: both (the engine's fused step; the index
// space of rope_q first, then kv_write's).
template <int KIND>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a, long nq, long nkv) {
    const long n = nq + nkv;
    for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < n; e += (long)gridDim.x * 256) {
        if (KIND == 0 || (KIND == 2 && e < nq)) rope_q_elem(a, e);
        else kv_write_elem(a, e - nq);
    }
}

// ---------------------------------------------------------------- argmax
// out[r] = argmax (src/llm/mod.rs:132-140) of row r of X [B, V]: the index
// the sequential scan `if x[i] > x[best] { best = i }` ends on. So a NaN at
// index 0 is the answer (nothing compares greater), later NaNs never are,
// and otherwise it is the first index of the largest value (+0 and -0 tie).
// A workgroup per row (1024 threads, 8 loads in flight each): each thread
// scans its float4 chunks in ascending order, then (value, index) pairs
// meet in a tree that keeps the larger value, the lower index on ties.

// Keeps the better of (bv, bi) and (v, i): i == INT_MAX is no candidate;
// candidates are never NaN.
TSL_DEV void am_pick(float& bv, int& bi, float v, int i) {
    if (i == INT_MAX) return;
    if (bi == INT_MAX || v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

constexpr int AM_THREADS = 1024, AM_UNROLL = 8;  // a 32000-float row in one round of loads
__global__ __launch_bounds__(AM_THREADS) void argmax_kernel(const float* __restrict__ X, int V, int* __restrict__ out) {
    constexpr int NW = AM_THREADS / 64;
    __shared__ float rv[NW];
    __shared__ int ri[NW];
    TSL_POISON(rv); TSL_POISON(ri);
    const int tid = threadIdx.x;
    const float* x = X + (size_t)blockIdx.x * V;
    float bv = 0.0f;
    int bi = INT_MAX;  // no candidate yet
    auto see = [&](float v, int i) {
        if (v == v && (bi == INT_MAX || v > bv)) {  // ascending i: strict > keeps the first
            bv = v;
            bi = i;
        }
    };
    if ((V & 3) == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0) {
        const int nc = V / 4;
        for (int c0 = tid; c0 < nc; c0 += AM_THREADS * AM_UNROLL) {
            float4v q[AM_UNROLL];
#pragma unroll
            for (int u = 0; u < AM_UNROLL; u++) {
                const int c = c0 + u * AM_THREADS;
                q[u] = c < nc ? *reinterpret_cast<const float4v*>(x + 4 * c) : float4v{};
            }
#pragma unroll
            for (int u = 0; u < AM_UNROLL; u++) {
                const int c = c0 + u * AM_THREADS;
                if (c < nc)
                    for (int e = 0; e < 4; e++) see(q[u][e], 4 * c + e);
            }
        }
    } else {
        for (int c = tid; c < V; c += AM_THREADS) see(x[c], c);
    }
    // Within each 16-lane row by DPP (value and index moved together), then
    // the four rows by readlane: registers only.
    auto step = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        const float ov = dpp<C>(bv);
        const int oi = __builtin_amdgcn_mov_dpp(bi, C, 0xf, 0xf, false);
        am_pick(bv, bi, ov, oi);
    };
    step(std::integral_constant<int, DPP_XOR1>{});
    step(std::integral_constant<int, DPP_XOR2>{});
    step(std::integral_constant<int, DPP_HALF_MIRROR>{});
    step(std::integral_constant<int, DPP_MIRROR>{});
    for (int r = 16; r < 64; r += 16)
        am_pick(bv, bi, lane_value(bv, r), __builtin_amdgcn_readlane(bi, r));
    bv = lane_value(bv, 0);  // rows 1..3 were folded into lane 0's pair; every lane takes it
    bi = __builtin_amdgcn_readlane(bi, 0);
    if ((tid & 63) == 0) {
        rv[tid >> 6] = bv;
        ri[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NW; w++) am_pick(bv, bi, rv[w], ri[w]);
        const float x0 = x[0];
        out[blockIdx.x] = (x0 != x0 || bi == INT_MAX) ? 0 : bi;
    }
}

int grid1(long n) {
    long g = (n + 255) / 256;
    return (int)(g < 1 ? 1 : (g > 65535 * 4 ? 65535 * 4 : g));
}

}  // namespace

// ---------------------------------------------------------------- launchers

int launch_softmax(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int R = k.dim("R"), C = k.dim("C");
    int ncols = (int)std::min<int64_t>(k.metav("BC"), C);
    if (R == 0) return 0;
    dim3 grid((R + ROWS_PER_WG - 1) / ROWS_PER_WG);
    const float* X = P<float>(a[0]);
    float* Y = P<float>(a[1]);
    if (ncols <= 1024)
        hipLaunchKernelGGL((softmax_kernel<4>), grid, dim3(256), 0, s, X, Y, R, C, ncols);
    else if (ncols <= 4096)
        // Two rows per workgroup (4096^2 from HBM: 1 / 2 / 4 / 8 rows per
        // workgroup 23.3 / 22.9 / 23.3 / 23.5 us).
        hipLaunchKernelGGL((softmax_kernel<16, 2>), dim3((R + 1) / 2), dim3(128), 0, s, X, Y, R, C, ncols);
    else
        hipLaunchKernelGGL(softmax_long_kernel, grid, dim3(256), 0, s, X, Y, R, C, ncols);
    return TSL_LAUNCHED("softmax");
}

int launch_rmsnorm_basic(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int R = k.dim("R"), C = k.dim("C");
    int ncols = (int)std::min<int64_t>(k.metav("BC"), C);
    return run_rmsnorm<u16>(P<u16>(a[0]), nullptr, R, P<u16>(a[1]), P<u16>(a[2]), R, C, ncols, arg_f32(a[3]), s,
                            "rmsnorm");
}

int launch_add(TslKernel& k, const uint64_t* a, hipStream_t s) {
    long N = k.dim("N");
    if (N == 0) return 0;
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)((N + 1023) / 1024)), dim3(256), 0, s, P<float>(a[0]),
                       P<float>(a[1]), P<float>(a[2]), N);
    return TSL_LAUNCHED("add");
}

int launch_embed(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int T = k.dim("T"), V = k.dim("V"), Dm = k.dim("Dm");
    if (T == 0) return 0;
    dim3 grid((Dm + 2047) / 2048, T);
    hipLaunchKernelGGL(embed_kernel, grid, dim3(256), 0, s, P<int>(a[0]), P<u16>(a[1]), P<float>(a[2]), T, V, Dm);
    return TSL_LAUNCHED("embed");
}

// For the fused residual projection (gemm.hip): R += the S slices of part,
// then Y = rmsnorm(R) W (C % 4 == 0, C <= 4096; reduce_rmsnorm_kernel).
bool reduce_rmsnorm_fits(int C) { return C > 0 && C % 4 == 0 && C <= 4096; }
int run_reduce_rmsnorm(const float* part, int S, float* R, const u16* W, u16* Y, int M, int C, float eps,
                       hipStream_t s) {
    if (M == 0) return 0;
    auto go = [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
        auto k = [&](auto su) {
            hipLaunchKernelGGL((reduce_rmsnorm_kernel<NC, decltype(su)::value>), dim3(M), dim3(256), 0, s, part, S, R,
                               W, Y, M, C, (float)C, eps);
        };
        switch (S) {
            case 2: k(std::integral_constant<int, 2>{}); break;
            case 3: k(std::integral_constant<int, 3>{}); break;
            case 4: k(std::integral_constant<int, 4>{}); break;
            default: k(std::integral_constant<int, 0>{}); break;
        }
    };
    if (C <= 1024) go(std::integral_constant<int, 1>{});
    else if (C <= 2048) go(std::integral_constant<int, 2>{});
    else go(std::integral_constant<int, 4>{});
    return TSL_LAUNCHED("linear_residual_rmsnorm");
}
// llm/rmsnorm over f32 rows, for the fused projection's unsplit path.
int run_rmsnorm_f32(const float* X, const u16* W, u16* Y, int M, int C, int ncols, float eps, hipStream_t s) {
    return run_rmsnorm<float>(X, nullptr, M, W, Y, M, C, ncols, eps, s, "linear_residual_rmsnorm");
}

int launch_llm_rmsnorm(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int T = k.dim("T"), Dm = k.dim("Dm");
    int ncols = (int)std::min<int64_t>(k.metav("BC"), Dm);
    return run_rmsnorm<float>(P<float>(a[0]), nullptr, T, P<u16>(a[1]), P<u16>(a[2]), T, Dm, ncols, arg_f32(a[3]), s,
                              "rmsnorm");
}

int launch_rmsnorm_rows(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int T = k.dim("T"), B = k.dim("B"), Dm = k.dim("Dm");
    int ncols = (int)std::min<int64_t>(k.metav("BC"), Dm);
    return run_rmsnorm<float>(P<float>(a[0]), P<int>(a[1]), T, P<u16>(a[2]), P<u16>(a[3]), B, Dm, ncols,
                              arg_f32(a[4]), s, "rmsnorm_rows");
}

// fused/argmax (the engine's scheduler, not a .tl kernel): X [B, V] -> T [B].
int launch_argmax(TslKernel& k, const uint64_t* a, hipStream_t s) {
    const int B = k.dim("B"), V = k.dim("V");
    if (B == 0) return 0;
    if (V == 0) return tsl_fail(-2, "argmax: rows of 0 values");
    hipLaunchKernelGGL(argmax_kernel, dim3(B), dim3(AM_THREADS), 0, s, P<float>(a[0]), V, P<int>(a[1]));
    return TSL_LAUNCHED("argmax");
}

int launch_rope_q(TslKernel& k, const uint64_t* a, hipStream_t s) {
    RopeArgs r{};
    r.T = k.dim("T"), r.W = k.dim("W"), r.NPOS = k.dim("NPOS"), r.D2 = k.dim("D2"), r.H = k.dim("H"), r.D = k.dim("D");
    r.QKV = P<u16>(a[0]), r.pos = P<int>(a[1]), r.Cs = P<float>(a[2]), r.Sn = P<float>(a[3]), r.Q = P<u16>(a[4]);
    const long nq = (long)r.T * r.H * r.D2;
    if (nq == 0) return 0;
    hipLaunchKernelGGL(rope_kernel<0>, dim3(grid1(nq)), dim3(256), 0, s, r, nq, 0L);
    return TSL_LAUNCHED("rope_q");
}

int launch_kv_write(TslKernel& k, const uint64_t* a, hipStream_t s) {
    RopeArgs r{};
    r.T = k.dim("T"), r.W = k.dim("W"), r.NPOS = k.dim("NPOS"), r.D2 = k.dim("D2"), r.NS = k.dim("NS");
    r.G = k.dim("G"), r.D = k.dim("D");
    r.QKV = P<u16>(a[0]), r.pos = P<int>(a[1]), r.slot = P<int>(a[2]), r.Cs = P<float>(a[3]), r.Sn = P<float>(a[4]);
    r.Kc = P<u16>(a[5]), r.Vc = P<u16>(a[6]), r.K = P<u16>(a[7]), r.V = P<u16>(a[8]);
    const long nkv = (long)r.T * r.G * std::max(r.D2, r.D);
    if (nkv == 0) return 0;
    hipLaunchKernelGGL(rope_kernel<1>, dim3(grid1(nkv)), dim3(256), 0, s, r, 0L, nkv);
    return TSL_LAUNCHED("kv_write");
}

// fused/rope_kv: rope_q and kv_write of the same step in one launch (the
// engine's decode and prefill steps; not a .tl kernel). Arguments: QKV, pos,
// slot, C, S, Q, Kc, Vc, K, V.
int launch_rope_kv(TslKernel& k, const uint64_t* a, hipStream_t s) {
    RopeArgs r{};
    r.T = k.dim("T"), r.W = k.dim("W"), r.NPOS = k.dim("NPOS"), r.D2 = k.dim("D2"), r.H = k.dim("H");
    r.NS = k.dim("NS"), r.G = k.dim("G"), r.D = k.dim("D");
    r.QKV = P<u16>(a[0]), r.pos = P<int>(a[1]), r.slot = P<int>(a[2]), r.Cs = P<float>(a[3]), r.Sn = P<float>(a[4]);
    r.Q = P<u16>(a[5]), r.Kc = P<u16>(a[6]), r.Vc = P<u16>(a[7]), r.K = P<u16>(a[8]), r.V = P<u16>(a[9]);
    const long nq = (long)r.T * r.H * r.D2, nkv = (long)r.T * r.G * std::max(r.D2, r.D);
    if (nq + nkv == 0) return 0;
    const long nvec = (long)r.T * (r.H + 2 * r.G) * (r.D2 / 8);
    const bool aligned = ((reinterpret_cast<uintptr_t>(r.QKV) | reinterpret_cast<uintptr_t>(r.Q) |
                           reinterpret_cast<uintptr_t>(r.Kc) | reinterpret_cast<uintptr_t>(r.Vc) |
                           reinterpret_cast<uintptr_t>(r.K) | reinterpret_cast<uintptr_t>(r.V) |
                           reinterpret_cast<uintptr_t>(r.Cs) | reinterpret_cast<uintptr_t>(r.Sn)) & 15) == 0;
    if (aligned && r.D == 2 * r.D2 && r.D2 % 8 == 0 && r.W == (r.H + 2 * r.G) * r.D && (long)r.T * r.W < (1L << 31) &&
        (long)r.NS * r.G * r.D < (1L << 31) && (long)r.NPOS * r.D2 < (1L << 31)) {
        hipLaunchKernelGGL(rope_kv_vec, dim3((unsigned)((nvec + 255) / 256)), dim3(256), 0, s, r, (int)nvec);
        return TSL_LAUNCHED("rope_kv");
    }
    hipLaunchKernelGGL(rope_kernel<2>, dim3(grid1(nq + nkv)), dim3(256), 0, s, r, nq, nkv);
    return TSL_LAUNCHED("rope_kv");
}
