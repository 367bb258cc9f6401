// Causal attention prefill on CDNA4 matrix cores: flash_attention
// (kernels/attention.tl:4-24, Q/K/V/O [H, S, D]) and the engine's
// grouped-query, packed-prompt prefill_attention (kernels/llm.tl:116-145,
// Q/O [S, H, D], K/V [S, G, D], row r attending keys starts[r] .. r, running
// maximum starting at -1e30).
//
// A workgroup of 4 wavefronts owns 128 query rows of one head; each
// wavefront owns 32. Per block of 64 keys, staged in LDS (double-buffered
// through registers):
//   S^T = K Q^T     (v_mfma_f32_32x32x16_f16; lane l holds query l % 32,
//                    so the online-softmax state is per lane)
//   O^T += V^T P^T  (P^T taken straight from the S^T accumulators, rounded
//                    to f16 as the .tl's f16(p) does)
// K is staged row-major ([key][d], 16-byte chunks XOR-swizzled); V is
// staged transposed ([d][key]) by 4x4 register transposes so that the V^T
// operand reads 4 consecutive keys per 8-byte LDS read. The key order
// inside a 16-key MFMA step is permuted identically for P^T and V^T (the
// reduction does not depend on it). exp is exp2 with log2(e) folded into
// the scale. Query blocks are issued longest (most keys) first.
#include "common.h"

namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr float LOG2E = 1.4426950408889634f;
constexpr int BQ = 128;  // queries per workgroup
constexpr int BKEY = 64;  // keys per block

struct AttnArgs {
    const u16 *Q, *K, *V;
    u16* O;
    const int* starts;  // prefill only
    int S, H, G;
    long q_row, q_head, k_row, k_head;  // element strides
    float scale;
};

template <int D, bool PREFILL>
__global__ __launch_bounds__(256, 2) void attn_fwd(AttnArgs a) {
    constexpr int DP = D < 32 ? 32 : D;   // V^T rows, padded to one MFMA tile
    constexpr int KCH = D / 8;            // 16-byte chunks per K row
    constexpr int NVB = (BKEY / 4) * (D / 4);  // 4x4 blocks of a V tile
    constexpr int VPT = (NVB + 255) / 256;
    constexpr int KPT = (BKEY * KCH + 255) / 256;

    __shared__ u32x4 lds_k[2][BKEY * KCH];
    __shared__ u32x2 lds_v[2][DP * (BKEY / 4)];  // [d][key/4] 8-byte chunks

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g4 = lane >> 5;
    const int nqb = (a.S + BQ - 1) / BQ;
    const int qb = nqb - 1 - (int)(blockIdx.x / a.H);
    const int h = blockIdx.x % a.H;
    const int hk = PREFILL ? h / (a.H / a.G) : h;
    const int q0 = qb * BQ, qw = q0 + wave * 32;
    const int myq = qw + (lane & 31);

    const u16* Qh = a.Q + (long)h * a.q_head;
    const u16* Kh = a.K + (long)hk * a.k_head;
    const u16* Vh = a.V + (long)hk * a.k_head;

    // Q^T operand, kept in registers: lane l holds d = 16 s + 8 (l/32) .. +8 of its query.
    half8 qop[D / 16];
#pragma unroll
    for (int s = 0; s < D / 16; s++) {
        u32x4 t = {0, 0, 0, 0};
        if (myq < a.S) t = *reinterpret_cast<const u32x4*>(Qh + (long)myq * a.q_row + 16 * s + 8 * g4);
        qop[s] = __builtin_bit_cast(half8, t);
    }
    const int my_start = PREFILL ? (myq < a.S ? a.starts[myq] : 0) : 0;
    const float c2 = a.scale * LOG2E;

    float m = PREFILL ? -1e30f * LOG2E : -INFINITY;  // running max, log2 domain
    float lsum = 0.0f;
    float16v acc[DP / 32];
#pragma unroll
    for (int i = 0; i < DP / 32; i++) acc[i] = float16v{};

    const int kend = min(q0 + BQ, a.S);
    int kbeg = 0;
    if (PREFILL) kbeg = (a.starts[q0] / BKEY) * BKEY;

    u32x4 rk[KPT > 0 ? KPT : 1];
    u32x2 rv[VPT][4];
    auto gload = [&](int j) {
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            int c = tid + i * 256;
            int key = c / KCH, ch = c % KCH;
            u32x4 t = {0, 0, 0, 0};
            if (c < BKEY * KCH && j + key < a.S)
                t = *reinterpret_cast<const u32x4*>(Kh + (long)(j + key) * a.k_row + ch * 8);
            rk[i] = t;
        }
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            int b = tid + i * 256;
            int kg = b / (D / 4), dg = b % (D / 4);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int key = j + kg * 4 + r;
                u32x2 t = {0, 0};
                if (b < NVB && key < a.S) t = *reinterpret_cast<const u32x2*>(Vh + (long)key * a.k_row + dg * 4);
                rv[i][r] = t;
            }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            int c = tid + i * 256;
            if (c >= BKEY * KCH) break;
            int key = c / KCH, ch = c % KCH;
            lds_k[buf][key * KCH + (ch ^ ((key ^ (key >> 3)) & (KCH - 1)))] = rk[i];
        }
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            int b = tid + i * 256;
            if (b >= NVB) break;
            int kg = b / (D / 4), dg = b % (D / 4);
#pragma unroll
            for (int c = 0; c < 4; c++) {  // d = 4 dg + c: keys 4 kg .. 4 kg + 3
                uint32_t w0 = c < 2 ? rv[i][0][0] : rv[i][0][1], w1 = c < 2 ? rv[i][1][0] : rv[i][1][1];
                uint32_t w2 = c < 2 ? rv[i][2][0] : rv[i][2][1], w3 = c < 2 ? rv[i][3][0] : rv[i][3][1];
                uint32_t lo, hi;
                if (c & 1) {
                    lo = (w0 >> 16) | (w1 & 0xffff0000u);
                    hi = (w2 >> 16) | (w3 & 0xffff0000u);
                } else {
                    lo = (w0 & 0xffffu) | (w1 << 16);
                    hi = (w2 & 0xffffu) | (w3 << 16);
                }
                int d = dg * 4 + c;
                lds_v[buf][d * (BKEY / 4) + (kg ^ (d & 15))] = u32x2{lo, hi};
            }
        }
        if constexpr (D < 32) {  // zero V^T rows D .. 31 (read by the padded tile)
            for (int e = tid; e < (DP - D) * (BKEY / 4); e += 256) lds_v[buf][D * (BKEY / 4) + e] = u32x2{0, 0};
        }
    };

    if (kbeg < kend) {
        gload(kbeg);
        sstore(0);
    }
    __syncthreads();
    int it = 0;
    for (int j = kbeg; j < kend; j += BKEY, it++) {
        const int buf = it & 1;
        if (j + BKEY < kend) gload(j + BKEY);
        const bool active = j <= qw + 31 && qw < a.S;  // some key of this block <= some query of the wave
        if (active) {
            float16v st[2];
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                st[kt] = float16v{};
                const int key = kt * 32 + (lane & 31);
#pragma unroll
                for (int s = 0; s < D / 16; s++) {
                    const int ch = 2 * s + g4;
                    half8 kop = __builtin_bit_cast(half8, lds_k[buf][key * KCH + (ch ^ ((key ^ (key >> 3)) & (KCH - 1)))]);
                    st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop, qop[s], st[kt], 0, 0, 0);
                }
            }
            const bool need_mask = PREFILL || j + BKEY - 1 > qw || j + BKEY > a.S;
            float mb = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    float v = st[kt][r] * c2;
                    if (need_mask) {
                        const int key = j + kt * 32 + 8 * (r >> 2) + 4 * g4 + (r & 3);
                        bool keep = key <= myq && key < a.S;
                        if (PREFILL) keep = keep && key >= my_start;
                        v = keep ? v : -INFINITY;
                    }
                    st[kt][r] = v;
                    mb = fmaxf(mb, v);
                }
            mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
            const float mn = fmaxf(m, mb);
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
            float ps = 0.0f;
            half8 pk[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
#pragma unroll
                for (int hh = 0; hh < 8; hh++) {
                    float p = __builtin_amdgcn_exp2f(st[t >> 1][8 * (t & 1) + hh] - mn);
                    ps += p;
                    pk[t][hh] = (half_t)p;
                }
            }
            lsum = lsum * alpha + ps;
            m = mn;
#pragma unroll
            for (int dt = 0; dt < DP / 32; dt++) {
                acc[dt] *= alpha;
                const int d = dt * 32 + (lane & 31);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    u32x2 lo = lds_v[buf][d * (BKEY / 4) + ((4 * t + g4) ^ (d & 15))];
                    u32x2 hi = lds_v[buf][d * (BKEY / 4) + ((4 * t + 2 + g4) ^ (d & 15))];
                    half8 vop = __builtin_bit_cast(half8, u32x4{lo[0], lo[1], hi[0], hi[1]});
                    acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, pk[t], acc[dt], 0, 0, 0);
                }
            }
        }
        if (j + BKEY < kend) sstore(buf ^ 1);
        __syncthreads();
    }

    const float l = lsum + __shfl_xor(lsum, 32, 64);
    if (myq < a.S) {
        u16* o = a.O + (long)myq * a.q_row + (long)h * a.q_head;
        const float inv = 1.0f / l;
#pragma unroll
        for (int dt = 0; dt < DP / 32; dt++)
#pragma unroll
            for (int rg = 0; rg < 4; rg++) {
                const int d = dt * 32 + 8 * rg + 4 * g4;
                if (d >= D) continue;
                u32x2 w;
                w[0] = (uint32_t)f2h(acc[dt][4 * rg] / l) | ((uint32_t)f2h(acc[dt][4 * rg + 1] / l) << 16);
                w[1] = (uint32_t)f2h(acc[dt][4 * rg + 2] / l) | ((uint32_t)f2h(acc[dt][4 * rg + 3] / l) << 16);
                *reinterpret_cast<u32x2*>(o + d) = w;
            }
        (void)inv;
    }
}

template <bool PREFILL>
int run_attn(const AttnArgs& a, int D, hipStream_t s, const char* what) {
    if (a.S == 0 || a.H == 0) return 0;
    dim3 grid(((a.S + BQ - 1) / BQ) * a.H);
    switch (D) {
        case 16: hipLaunchKernelGGL((attn_fwd<16, PREFILL>), grid, dim3(256), 0, s, a); break;
        case 32: hipLaunchKernelGGL((attn_fwd<32, PREFILL>), grid, dim3(256), 0, s, a); break;
        case 64: hipLaunchKernelGGL((attn_fwd<64, PREFILL>), grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL((attn_fwd<128, PREFILL>), grid, dim3(256), 0, s, a); break;
        default: return tsl_fail(-2, std::string(what) + ": head dimension " + std::to_string(D) +
                                         " unsupported (16, 32, 64 or 128)");
    }
    return TSL_LAUNCHED(what);
}

}  // namespace

int prepare_attention(TslKernel& k) {
    int64_t D = k.dim("D");
    if (D != 16 && D != 32 && D != 64 && D != 128)
        return tsl_fail(-2, k.name + ": head dimension " + std::to_string(D) + " unsupported (16, 32, 64 or 128)");
    if (k.name == "prefill_attention" && k.dim("H") % k.dim("G") != 0)
        return tsl_fail(-2, "prefill_attention: H must be a multiple of G");
    return 0;
}

// flash_attention(Q, K, V, O: f16[H, S, D], scale: f32)
int launch_flash_attention(TslKernel& k, const uint64_t* args, hipStream_t s) {
    AttnArgs a{};
    int H = k.dim("H"), S = k.dim("S"), D = k.dim("D");
    a.Q = P<u16>(args[0]);
    a.K = P<u16>(args[1]);
    a.V = P<u16>(args[2]);
    a.O = P<u16>(args[3]);
    a.scale = arg_f32(args[4]);
    a.S = S;
    a.H = H;
    a.G = H;
    a.q_row = D;
    a.q_head = (long)S * D;
    a.k_row = D;
    a.k_head = (long)S * D;
    return run_attn<false>(a, D, s, "flash_attention");
}

// prefill_attention(Q: f16[S, H, D], K, V: f16[S, G, D], starts: i32[S], O: f16[S, H, D], scale: f32)
int launch_prefill_attention(TslKernel& k, const uint64_t* args, hipStream_t s) {
    AttnArgs a{};
    int S = k.dim("S"), H = k.dim("H"), G = k.dim("G"), D = k.dim("D");
    a.Q = P<u16>(args[0]);
    a.K = P<u16>(args[1]);
    a.V = P<u16>(args[2]);
    a.starts = P<int>(args[3]);
    a.O = P<u16>(args[4]);
    a.scale = arg_f32(args[5]);
    a.S = S;
    a.H = H;
    a.G = G;
    a.q_row = (long)H * D;
    a.q_head = D;
    a.k_row = (long)G * D;
    a.k_head = D;
    return run_attn<true>(a, D, s, "prefill_attention");
}
