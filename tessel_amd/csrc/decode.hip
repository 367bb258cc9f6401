// Decode attention over the paged KV cache: decode_attention
// (kernels/llm.tl:150-172, grouped-query) and paged_attention
// (kernels/attention.tl:29-51, the same with G == H). HBM-bound.
//
// The .tl runs one program per (sequence b, query head h) and so reads each
// KV page H/G times; here one workgroup owns (b, kv head g, chunk of CH
// pages) and reads each page once for all QPG = H/G query heads sharing it.
// A token's D halves are spread over D/8 lanes (16-byte loads, 256
// contiguous bytes per token at D = 128); every lane keeps its own online
// softmax over the tokens it reads (log2 domain), and the states are merged
// across lanes, wavefronts and then chunks (a second, tiny kernel) in a
// fixed order. Page lookups follow the interpreter exactly: the table entry
// of token t is table[b, t / P], reading page 0 when t / P >= MP, and a page
// outside [0, NP) reads as zeros (scores 0, values 0) (src/interp.rs:93-117).
// lens[b] == 0 gives 0/0 = NaN, as in the .tl.
#include "common.h"

namespace {

constexpr float LOG2E = 1.4426950408889634f;
constexpr int DEC_CHUNK = 16;  // pages per workgroup

struct DecArgs {
    const u16* Q;
    const u16 *Kc, *Vc;
    const int *table, *lens;
    u16* O;
    float* part;  // [B][G][NCH][QPG][2 + D]: m, l, acc
    int B, H, G, NP, P, MP, NCH;
    float c2;  // scale * log2(e)
};

template <int LPT>
TSL_DEV float group_sum(float x) {  // sum over aligned groups of LPT lanes (within a 16-lane DPP row)
    if constexpr (LPT >= 2) x += dpp<DPP_XOR1>(x);
    if constexpr (LPT >= 4) x += dpp<DPP_XOR2>(x);
    if constexpr (LPT >= 8) x += dpp<DPP_HALF_MIRROR>(x);
    if constexpr (LPT >= 16) x += dpp<DPP_MIRROR>(x);
    return x;
}

TSL_DEV float h2f_lo(uint32_t w) { return h2f((u16)(w & 0xffff)); }
TSL_DEV float h2f_hi(uint32_t w) { return h2f((u16)(w >> 16)); }

template <int D, int QPG>
__global__ __launch_bounds__(256) void decode_partial(DecArgs a) {
    constexpr int LPT = D / 8;       // lanes per token
    constexpr int TPI = 64 / LPT;    // tokens per wavefront per step
    constexpr int TPS = 4 * TPI;     // tokens per workgroup per step
    constexpr int U = 4;             // steps per softmax update
    __shared__ float red[4][QPG][2 + D];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = blockIdx.x % a.NCH, bg = blockIdx.x / a.NCH;
    const int g = bg % a.G, b = bg / a.G;
    const int n = a.lens[b];
    const int npages = n > 0 ? (n + a.P - 1) / a.P : 0;
    const int page_lo = c * DEC_CHUNK;
    if (page_lo >= npages && !(a.NCH == 1)) return;  // nothing here (the combine skips this chunk)
    // The last chunk also takes tokens past MP * P (their table reads give page 0).
    const int t_lo = page_lo * a.P;
    const int t_hi = c == a.NCH - 1 ? n : min(n, (page_lo + DEC_CHUNK) * a.P);
    const int dl = lane % LPT, tg = lane / LPT;

    // q of the QPG heads of group g, this lane's 8 d values, as f16 pairs.
    uint32_t q[QPG][4];
#pragma unroll
    for (int i = 0; i < QPG; i++) {
        u32x4 t = *reinterpret_cast<const u32x4*>(a.Q + ((long)b * a.H + g * QPG + i) * D + dl * 8);
        for (int e = 0; e < 4; e++) q[i][e] = t[e];
    }
    float m[QPG], l[QPG], acc[QPG][8];
#pragma unroll
    for (int i = 0; i < QPG; i++) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
        for (int e = 0; e < 8; e++) acc[i][e] = 0.0f;
    }
    const long tok_stride = (long)a.G * D;  // elements between tokens of a page
    for (int t0 = t_lo; t0 < t_hi; t0 += TPS * U) {
        float s[U][QPG], vv[U][8];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = t0 + u * TPS + wave * TPI + tg;
            const bool valid = t < t_hi;
            u32x4 kw = {0, 0, 0, 0}, vw = {0, 0, 0, 0};
            if (valid) {
                const int pi = t / a.P;
                const int page = pi < a.MP ? a.table[(long)b * a.MP + pi] : 0;
                if (page >= 0 && page < a.NP) {
                    const long off = ((long)page * a.P + (t % a.P)) * tok_stride + (long)g * D + dl * 8;
                    kw = *reinterpret_cast<const u32x4*>(a.Kc + off);
                    vw = *reinterpret_cast<const u32x4*>(a.Vc + off);
                }
            }
#pragma unroll
            for (int i = 0; i < QPG; i++) {
                float p = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    p = __builtin_amdgcn_fdot2(as_half2(q[i][e]), as_half2(kw[e]), p, false);
                p = group_sum<LPT>(p);
                s[u][i] = valid ? p * a.c2 : -INFINITY;
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                vv[u][2 * e] = h2f_lo(vw[e]);
                vv[u][2 * e + 1] = h2f_hi(vw[e]);
            }
        }
#pragma unroll
        for (int i = 0; i < QPG; i++) {
            float mx = m[i];
#pragma unroll
            for (int u = 0; u < U; u++) mx = fmaxf(mx, s[u][i]);
            const float ms = mx == -INFINITY ? 0.0f : mx;
            const float corr = __builtin_amdgcn_exp2f(m[i] - ms);
            float ps = 0.0f, pu[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                pu[u] = __builtin_amdgcn_exp2f(s[u][i] - ms);
                ps += pu[u];
            }
            l[i] = l[i] * corr + ps;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float x = acc[i][e] * corr;
#pragma unroll
                for (int u = 0; u < U; u++) x += pu[u] * vv[u][e];
                acc[i][e] = x;
            }
            m[i] = mx;
        }
    }
    // Merge the TPI token groups of the wavefront (lanes differing above LPT).
#pragma unroll
    for (int i = 0; i < QPG; i++) {
        float M = m[i];
#pragma unroll
        for (int o = LPT; o < 64; o <<= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        const float f = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[i] - M);
        float L = l[i] * f;
#pragma unroll
        for (int o = LPT; o < 64; o <<= 1) L += __shfl_xor(L, o, 64);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float x = acc[i][e] * f;
#pragma unroll
            for (int o = LPT; o < 64; o <<= 1) x += __shfl_xor(x, o, 64);
            acc[i][e] = x;
        }
        if (tg == 0) {
            if (dl == 0) {
                red[wave][i][0] = M;
                red[wave][i][1] = L;
            }
            for (int e = 0; e < 8; e++) red[wave][i][2 + dl * 8 + e] = acc[i][e];
        }
    }
    __syncthreads();
    // Merge the 4 wavefronts: thread (i, d).
    for (int x = threadIdx.x; x < QPG * D; x += 256) {
        const int i = x / D, d = x % D;
        float M = -INFINITY;
        for (int w = 0; w < 4; w++) M = fmaxf(M, red[w][i][0]);
        float L = 0.0f, A = 0.0f;
        for (int w = 0; w < 4; w++) {
            const float f = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red[w][i][0] - M);
            L += red[w][i][1] * f;
            A += red[w][i][2 + d] * f;
        }
        if (a.NCH == 1) {
            a.O[((long)b * a.H + g * QPG + i) * D + d] = f2h(A / L);
        } else {
            float* pe = a.part + ((((long)b * a.G + g) * a.NCH + c) * QPG + i) * (2 + D);
            if (d == 0) {
                pe[0] = M;
                pe[1] = L;
            }
            pe[2 + d] = A;
        }
    }
}

// Merges the chunks of (b, h) in chunk order: one wavefront per (b, h).
template <int D, int QPG>
__global__ __launch_bounds__(64) void decode_combine(DecArgs a) {
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int g = h / QPG, i = h % QPG;
    const int n = a.lens[b];
    const int npages = n > 0 ? (n + a.P - 1) / a.P : 0;
    const int nch = min((npages + DEC_CHUNK - 1) / DEC_CHUNK, a.NCH);
    const float* base = a.part + (((long)b * a.G + g) * a.NCH * QPG + i) * (2 + D);
    const long cs = (long)QPG * (2 + D);
    float M = -INFINITY;
    for (int c = 0; c < nch; c++) M = fmaxf(M, base[c * cs]);
    for (int d = threadIdx.x; d < D; d += 64) {
        float L = 0.0f, A = 0.0f;
        for (int c = 0; c < nch; c++) {
            const float f = __builtin_amdgcn_exp2f(base[c * cs] - M);
            L += base[c * cs + 1] * f;
            A += base[c * cs + 2 + d] * f;
        }
        a.O[((long)b * a.H + h) * D + d] = f2h(A / L);
    }
}

template <int D, int QPG>
int run_decode(DecArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((decode_partial<D, QPG>), dim3(a.B * a.G * a.NCH), dim3(256), 0, s, a);
    int r = TSL_LAUNCHED("decode_attention");
    if (r || a.NCH == 1) return r;
    hipLaunchKernelGGL((decode_combine<D, QPG>), dim3(a.B * a.H), dim3(64), 0, s, a);
    return TSL_LAUNCHED("decode_attention combine");
}

template <int D>
int run_decode_d(DecArgs& a, int qpg, hipStream_t s) {
    switch (qpg) {
        case 1: return run_decode<D, 1>(a, s);
        case 2: return run_decode<D, 2>(a, s);
        case 4: return run_decode<D, 4>(a, s);
        case 8: return run_decode<D, 8>(a, s);
        case 16: return run_decode<D, 16>(a, s);
    }
    return tsl_fail(-2, "decode_attention: H / G must be 1, 2, 4, 8 or 16");
}

int nchunks(const TslKernel& k) { return (int)((k.dim("MP") + DEC_CHUNK - 1) / DEC_CHUNK); }

}  // namespace

// Sizes the per-chunk partial buffer once, when the kernel is specialised.
int prepare_decode(TslKernel& k) {
    int64_t D = k.dim("D"), H = k.dim("H");
    int64_t G = k.name == "paged_attention" ? H : k.dim("G");
    if (D != 16 && D != 32 && D != 64 && D != 128)
        return tsl_fail(-2, k.name + ": head dimension " + std::to_string(D) + " unsupported (16, 32, 64 or 128)");
    if (G <= 0 || H % G != 0) return tsl_fail(-2, k.name + ": H must be a multiple of G");
    int64_t qpg = H / G;
    if (qpg != 1 && qpg != 2 && qpg != 4 && qpg != 8 && qpg != 16)
        return tsl_fail(-2, k.name + ": H / G must be 1, 2, 4, 8 or 16");
    int nch = nchunks(k);
    if (nch > 1) {
        size_t bytes = (size_t)k.dim("B") * G * nch * qpg * (2 + D) * sizeof(float);
        if (tsl_hip_check(hipMalloc(&k.scratch, bytes), "decode_attention scratch")) return -1;
        k.scratch_bytes = bytes;
    }
    return 0;
}

static int launch_decode_common(TslKernel& k, const uint64_t* args, hipStream_t s, bool gqa) {
    DecArgs a{};
    a.Q = P<u16>(args[0]);
    a.Kc = P<u16>(args[1]);
    a.Vc = P<u16>(args[2]);
    a.table = P<int>(args[3]);
    a.lens = P<int>(args[4]);
    a.O = P<u16>(args[5]);
    a.c2 = arg_f32(args[6]) * LOG2E;
    a.B = k.dim("B");
    a.H = k.dim("H");
    a.G = gqa ? k.dim("G") : a.H;
    a.NP = k.dim("NP");
    a.P = k.dim("P");
    a.MP = k.dim("MP");
    a.NCH = nchunks(k);
    a.part = reinterpret_cast<float*>(k.scratch);
    if (a.B == 0) return 0;
    const int D = k.dim("D"), qpg = a.H / a.G;
    switch (D) {
        case 16: return run_decode_d<16>(a, qpg, s);
        case 32: return run_decode_d<32>(a, qpg, s);
        case 64: return run_decode_d<64>(a, qpg, s);
        case 128: return run_decode_d<128>(a, qpg, s);
    }
    return tsl_fail(-2, "decode_attention: unsupported head dimension");
}

int launch_decode_attention(TslKernel& k, const uint64_t* args, hipStream_t s) {
    return launch_decode_common(k, args, s, true);
}

int launch_paged_attention(TslKernel& k, const uint64_t* args, hipStream_t s) {
    return launch_decode_common(k, args, s, false);
}
