// Decode attention over the paged KV cache: decode_attention
// (kernels/llm.tl:150-172, grouped-query) and paged_attention
// (kernels/attention.tl:29-51, the same with G == H). HBM-bound.
//
// The .tl runs one program per (sequence b, query head h) and so reads each
// KV page H/G times; here each page is read once for all QPG = H/G query
// heads sharing it. Three forms: decode_stream (tables longer than 64 pages,
// 4 or 8 kv heads: persistent workgroups over equal shares of all the
// sequences' tiles), decode_tiles (matrix-core form; one workgroup per
// (b, kv head g, chunk of CH pages)) and decode_partial (any D and P).
// A token's D halves are spread over D/8 lanes (16-byte loads, 256
// contiguous bytes per token at D = 128); every lane keeps its own online
// softmax over the tokens it reads (log2 domain), and the states are merged
// across lanes, wavefronts and then chunks (a second, tiny kernel) in a
// fixed order. Page lookups follow the interpreter exactly: the table entry
// of token t is table[b, t / P], reading page 0 when t / P >= MP, and a page
// outside [0, NP) reads as zeros (scores 0, values 0) (src/interp.rs:93-117).
// lens[b] == 0 gives 0/0 = NaN, as in the .tl.
#include "common.h"

#include <mutex>

#include "../../include/tessel.h"

#include <algorithm>

namespace {

constexpr float LOG2E = 1.4426950408889634f;
constexpr int DEC_MAX_CHUNK = 24;  // pages per chunk of a long table, at most
constexpr int DEC_WIDE_MAX_PAGES = 64;  // tables up to this many pages: one chunk per sequence

struct DecArgs {
    const u16* Q;
    const u16 *Kc, *Vc;
    const int *table, *lens;
    u16* O;
    float* part;  // [B][G][NCH][QPG][2 + D]: m, l, acc (stream path: range states, see DsGeom)
    int* pre;     // stream path: first unit of each (virtual) sequence, [B NG + 1]
    int NG;       // stream path: head groups of NWV kv heads per sequence
    int B, H, G, NP, P, MP, NCH;
    int CH;  // pages per chunk
    int pshift;  // log2(P) (P is a power of two)
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
    TSL_POISON(red);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = blockIdx.x % a.NCH, bg = blockIdx.x / a.NCH;
    const int g = bg % a.G, b = bg / a.G;
    const int n = a.lens[b];
    const int npages = n > 0 ? (n + a.P - 1) / a.P : 0;
    const int page_lo = c * a.CH;
    const int nact = min((npages + a.CH - 1) / a.CH, a.NCH);  // chunks holding tokens
    if (c >= nact) {
        if (c == 0)  // lens 0: 0 / 0, as the .tl computes
            for (int x = threadIdx.x; x < QPG * D; x += 256) a.O[((long)b * a.H + g * QPG) * D + x] = f2h(0.0f / 0.0f);
        return;
    }
    // The last chunk also takes tokens past MP * P (their table reads give page 0).
    const int t_lo = page_lo * a.P;
    const int t_hi = c == a.NCH - 1 ? n : min(n, (page_lo + a.CH) * a.P);
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
        if (nact == 1) {  // the only chunk: O directly
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
// Sequences of at most one chunk were written by the chunk kernel.
template <int D, int QPG>
__global__ __launch_bounds__(64) void decode_combine(DecArgs a) {
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int g = h / QPG, i = h % QPG;
    const int n = a.lens[b];
    const int npages = n > 0 ? (n + a.P - 1) / a.P : 0;
    const int nch = min((npages + a.CH - 1) / a.CH, a.NCH);
    if (nch <= 1) return;  // written by the chunk kernel
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

// ---------------------------------------------------------------------------
// Matrix-core path (D = 64 or 128, P a multiple of 16). A workgroup owns
// (b, kv head g, chunk of CH pages): one wavefront for the chunks of a long
// table, NWV of them (tiles w, w + NWV, ...; states merged in LDS) when the
// whole table is one chunk. A wavefront walks its
// 16-token tiles through a DEC_STAGES-deep ring of LDS stages, each filled by
// direct buffer->LDS loads (K rows then V rows, 16 x 2D bytes each), so that
// DEC_STAGES - 1 tiles are in flight while one is computed. Per tile:
//   S^T = K Q^T      v_mfma_f32_16x16x32_f16, A = K rows (token l%16), B =
//                    the QPG query heads (columns >= QPG are zero); lane l
//                    then holds tokens 4(l/16)+r of head l%16
//   O^T += V^T P^T   v_mfma_f32_16x16x16_f16 per 16 d; P^T is the S^T
//                    accumulator layout, V^T comes from transposed LDS reads.
// p stays f32 as in the .tl: it enters the MFMA as two f16 terms (hi + lo),
// which carries 22 bits of it. Softmax runs in the log2 domain on scaled
// scores with the running maximum moved lazily (by > 2^8 only). Tiles run to
// the end of the sequence's last page (masked), as the .tl's per-page loop
// does. A sequence of one chunk writes O directly; longer ones leave one
// state per chunk for decode_merge.
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 fp16x4_t;
constexpr int TT = 16;  // tokens per tile
constexpr int DEC_STAGES = 3;  // LDS stages per wavefront: 2 tiles in flight

TSL_DEV i32x4 buf_rsrc(const void* p, uint32_t bytes) {
    const uint64_t x = reinterpret_cast<uint64_t>(p);
    return i32x4{(int)(uint32_t)x, (int)(uint32_t)((x >> 32) & 0xffff), (int)bytes, 0x00020000};
}

// 16-byte-chunk XOR swizzles of a tile row (2D bytes). K: the 16 lanes of a
// 16-byte read hit 16 rows at one logical chunk. V: the 32 lanes of an 8-byte
// transposed read hit 8 rows at one 32-byte granule.
template <int D>
TSL_DEV int tswz_k(int row) { return D == 128 ? (row & 15) : ((row >> 1) & 7); }
template <int D>
TSL_DEV int tswz_v(int row) { return D == 128 ? 2 * (row & 7) : 2 * ((row >> 1) & 3); }

// s_waitcnt immediate for vmcnt(n) alone (6-bit vmcnt: bits 3:0 and 15:14).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0f70; }

// Waits until at most `tiles` tiles (2 NLD loads each) are still loading.
template <int NLD>
TSL_DEV void wait_tiles(int tiles) {
    switch (tiles) {  // s_waitcnt takes an immediate
        case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
        case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * NLD)); break;
        case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * NLD)); break;
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(6 * NLD)); break;
    }
}

template <int D, int QPG, int NWV>
__global__ __launch_bounds__(64 * NWV) void decode_tiles(DecArgs a) {
    constexpr int ROWB = 2 * D, KCH = D / 8;
    constexpr int TILE = TT * ROWB;   // bytes of K (or V) per tile
    constexpr int NLD = TILE / 1024;  // 1 KB loads per matrix per tile
    constexpr int RPL = 1024 / ROWB;  // rows per 1 KB load
    constexpr int WSTAGE = 2 * TILE;  // K then V
    constexpr float LAZY = 8.0f;
    static_assert(DEC_STAGES >= 2 && DEC_STAGES <= 4, "wait_tiles covers up to 3 tiles in flight");
    __shared__ __attribute__((aligned(16))) char lds[NWV * DEC_STAGES * WSTAGE];  // a ring per wavefront
    TSL_POISON(lds);

    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, col = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // The kv heads of one (b, chunk) are adjacent in launch order, so the
    // pages' token rows (all G heads' 2D-byte slices) are read at one time.
    const int g = blockIdx.x % a.G, c = (blockIdx.x / a.G) % a.NCH, b = blockIdx.x / (a.G * a.NCH);
    // The length, the query rows and the chunk's table entries (one per lane;
    // tiles past the table read page 0) in one round trip: none of these
    // loads depends on another.
    const int n = a.lens[b];
    half8 qop[D / 32];  // Q^T operand: lane l holds head l%16, d = 32 s + 8 (l/16) .. +8.
#pragma unroll
    for (int s = 0; s < D / 32; s++) {
        u32x4 t = {0, 0, 0, 0};
        if (col < QPG) t = *reinterpret_cast<const u32x4*>(a.Q + ((long)b * a.H + g * QPG + col) * D + 32 * s + 8 * grp);
        qop[s] = __builtin_bit_cast(half8, t);
    }
    const int page_lo = c * a.CH;
    const int tab = lane < a.CH && page_lo + lane < a.MP ? a.table[(long)b * a.MP + page_lo + lane] : 0;
    const int npages = n > 0 ? (n + a.P - 1) / a.P : 0;
    const int nact = min((npages + a.CH - 1) / a.CH, a.NCH);
    if (c >= nact) {
        if (c == 0)  // lens 0: 0 / 0, as the .tl computes
            for (int x = tid; x < QPG * D; x += 64 * NWV) a.O[((long)b * a.H + g * QPG) * D + x] = f2h(0.0f / 0.0f);
        return;
    }
    const int t_lo = c * a.CH * a.P;
    const int t_hi = c == a.NCH - 1 ? n : min(n, (c + 1) * a.CH * a.P);
    const int t_end = (t_hi + a.P - 1) / a.P * a.P;  // through the last page
    const int ntile = (t_end - t_lo) / TT;
    const int nt = wave < ntile ? (ntile - wave + NWV - 1) / NWV : 0;  // tiles wave, wave + NWV, ...


    // Load offsets (bytes from the tile's first row): load q, lane i fills
    // LDS chunk i % KCH of row q RPL + i / KCH with the logical chunk that
    // the swizzle puts there.
    const long tok_bytes = (long)a.G * D * 2;
    uint32_t offk[NLD], offv[NLD];
#pragma unroll
    for (int q = 0; q < NLD; q++) {
        const int row = q * RPL + lane / KCH, pc = lane % KCH;
        offk[q] = (uint32_t)(row * tok_bytes + ((pc ^ tswz_k<D>(row)) * 16));
        offv[q] = (uint32_t)(row * tok_bytes + ((pc ^ tswz_v<D>(row)) * 16));
    }
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t*)lds) + wave * DEC_STAGES * WSTAGE;
    const char* Kg = reinterpret_cast<const char*>(a.Kc) + (long)g * D * 2;
    const char* Vg = reinterpret_cast<const char*>(a.Vc) + (long)g * D * 2;
    auto issue = [&](int i, int st) {  // this wave's i-th tile
        const int t0 = t_lo + (wave + NWV * i) * TT;
        const int pi = t0 >> a.pshift;
        const int page = pi < a.MP ? __builtin_amdgcn_readlane(tab, pi - page_lo) : 0;
        const bool ok = page >= 0 && page < a.NP;  // outside the pool: zeros
        const long shift = ((long)(ok ? page : 0) * a.P + (t0 & (a.P - 1))) * tok_bytes;
        const uint32_t range = ok ? (uint32_t)(TT * tok_bytes) : 0u;
        const i32x4 rk = buf_rsrc(Kg + shift, range), rv = buf_rsrc(Vg + shift, range);
        const uint32_t sk = lds0 + st * WSTAGE, sv = sk + TILE;
#pragma unroll
        for (int q = 0; q < NLD; q++) {
            // K and V are read once: nontemporal (streamed past the caches).
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(sk + q * 1024),
                         "v"(offk[q]), "s"(rk));
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(sv + q * 1024),
                         "v"(offv[q]), "s"(rv));
        }
    };

    // Operand addresses within a stage. K: row l%16, logical chunk 4 s + l/16.
    // V^T by transposed reads: provider lane p of group G points at token row
    // 4 G + p/4 and d = 16 dt + 4 (p%4) .. +3, so lane l receives d = 16 dt + l%16
    // for tokens 4 G + 0..3.
    uint32_t kaddr[D / 32], vaddr[D / 16];
#pragma unroll
    for (int s = 0; s < D / 32; s++) kaddr[s] = (uint32_t)(col * ROWB + (((4 * s + grp) ^ tswz_k<D>(col)) * 16));
    const int vrow = 4 * grp + (col >> 2);
#pragma unroll
    for (int dt = 0; dt < D / 16; dt++) {
        const int lc = 2 * dt + ((col & 3) >> 1);
        vaddr[dt] = (uint32_t)(TILE + vrow * ROWB + ((lc ^ tswz_v<D>(vrow)) * 16) + 8 * (col & 1));
    }

    float m = -1e30f, lsum = 0.0f;  // running max of the scaled scores; this lane's share of l
    float4v acc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; dt++) acc[dt] = float4v{};

    // Q and the table entries have arrived before the tile loads are issued
    // (the loop waits on those loads by count).
#pragma unroll
    for (int s = 0; s < D / 32; s++) asm volatile("" ::"v"(qop[s]));
    asm volatile("" ::"v"(tab));
    const int pre = min(nt, DEC_STAGES - 1);
    for (int i = 0; i < pre; i++) issue(i, i);
    int st = 0;
    for (int i = 0; i < nt; i++) {
        if (i + DEC_STAGES - 1 < nt) {
            int sn = st + DEC_STAGES - 1;
            issue(i + DEC_STAGES - 1, sn >= DEC_STAGES ? sn - DEC_STAGES : sn);
        }
        wait_tiles<NLD>(min(nt - 1 - i, DEC_STAGES - 1));  // tile i has landed
        const char* sb = lds + (wave * DEC_STAGES + st) * WSTAGE;
        st = st + 1 == DEC_STAGES ? 0 : st + 1;
        float4v sc = float4v{};
#pragma unroll
        for (int s = 0; s < D / 32; s++) {
            const half8 kop = *reinterpret_cast<const half8*>(sb + kaddr[s]);
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[s], sc, 0, 0, 0);
        }
        const int t0 = t_lo + (wave + NWV * i) * TT + 4 * grp;  // token of register 0
        float x[4], mb = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            x[r] = t0 + r < n ? sc[r] * a.c2 : -INFINITY;
            mb = fmaxf(mb, x[r]);
        }
        mb = fmaxf(mb, xor16(mb));
        mb = fmaxf(mb, xor32(mb));
        if (__builtin_amdgcn_ballot_w64(mb > m + LAZY) != 0) {
            const float mn = fmaxf(m, mb);
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < D / 16; dt++) acc[dt] *= alpha;
            m = mn;
        }
        half4 phi, plo;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = __builtin_amdgcn_exp2f(x[r] - m);
            lsum += p;
            phi[r] = (half_t)p;
            plo[r] = (half_t)(p - (float)phi[r]);
        }
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
            const fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                (__attribute__((address_space(3))) fp16x4_t*)(sb + vaddr[dt]));
            const half4 vop = __builtin_bit_cast(half4, v);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vop, phi, acc[dt], 0, 0, 0);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vop, plo, acc[dt], 0, 0, 0);
        }
    }

    // Lane l holds head l%16, d = 16 dt + 4 (l/16) + r.
    lsum += xor16(lsum);
    lsum += xor32(lsum);
    // Merge the wavefronts' states in LDS (the rings are idle), in wave order.
    static_assert(NWV * QPG * (2 + D) * 4 <= NWV * DEC_STAGES * WSTAGE, "merge area exceeds the rings");
    float* red = reinterpret_cast<float*>(lds);  // [NWV][QPG][2 + D]
    __syncthreads();
    if (col < QPG) {
        float* rw = red + (wave * QPG + col) * (2 + D);
        if (grp == 0) {
            rw[0] = m;
            rw[1] = lsum;
        }
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++) rw[2 + 16 * dt + 4 * grp + r] = acc[dt][r];
    }
    __syncthreads();
    for (int x = tid; x < QPG * D; x += 64 * NWV) {
        const int i = x / D, d = x % D;
        float M = red[i * (2 + D)];
        for (int w = 1; w < NWV; w++) M = fmaxf(M, red[(w * QPG + i) * (2 + D)]);
        float L = 0.0f, A = 0.0f;
        for (int w = 0; w < NWV; w++) {
            const float* rw = red + (w * QPG + i) * (2 + D);
            const float f = __builtin_amdgcn_exp2f(rw[0] - M);
            L += rw[1] * f;
            A += rw[2 + d] * f;
        }
        if (nact == 1) {
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

// Merges the chunk states of (b, g) in chunk order: one workgroup per (b, g).
// All partial states are fetched at once into LDS (one memory latency), then
// each thread merges one (head, d).
template <int D, int QPG>
__global__ __launch_bounds__(256) void decode_merge(DecArgs a) {
    constexpr int ST = QPG * (2 + D);  // floats per chunk state
    extern __shared__ float sm[];      // [nact][QPG][2 + D]
    TSL_POISON_BYTES(sm, (unsigned)(a.NCH * ST * sizeof(float)));  // the launch's dynamic LDS
    const int bg = blockIdx.x, b = bg / a.G, g = bg % a.G;
    const int n = a.lens[b];
    const int npages = n > 0 ? (n + a.P - 1) / a.P : 0;
    const int nact = min((npages + a.CH - 1) / a.CH, a.NCH);
    if (nact <= 1) return;  // written by the chunk kernel
    const float4v* src = reinterpret_cast<const float4v*>(a.part + (long)bg * a.NCH * ST);
    float4v* dst = reinterpret_cast<float4v*>(sm);
    const int nv = nact * ST / 4;
    for (int x0 = 0; x0 < nv; x0 += 256 * 8) {
        float4v v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int x = x0 + u * 256 + (int)threadIdx.x;
            if (x < nv) v[u] = src[x];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int x = x0 + u * 256 + (int)threadIdx.x;
            if (x < nv) dst[x] = v[u];
        }
    }
    __syncthreads();
    for (int x = threadIdx.x; x < QPG * D; x += 256) {
        const int i = x / D, d = x % D;
        const float* pe = sm + i * (2 + D);
        float M = pe[0];
        for (int cc = 1; cc < nact; cc++) M = fmaxf(M, pe[cc * ST]);
        float L = 0.0f, A = 0.0f;
        for (int cc = 0; cc < nact; cc++) {
            const float f = __builtin_amdgcn_exp2f(pe[cc * ST] - M);
            L += pe[cc * ST + 1] * f;
            A += pe[cc * ST + 2 + d] * f;
        }
        a.O[((long)b * a.H + g * QPG + i) * D + d] = f2h(A / L);
    }
}

// ---- Balanced decode of long tables (decode_stream) ----
// The work is the list of units (sequence b, 16-token tile j) over all kv
// heads, j running through b's last page: U = sum_b ceil(lens_b / P) P / 16,
// sequence-major. W persistent workgroups (one per CU) take equal contiguous
// ranges [w U / W, (w + 1) U / W) of it, so every CU streams the same number
// of bytes whatever the lengths, and no workgroup waits on a startup or a
// tail of its own. Wavefront g of a workgroup computes kv head g, so the
// workgroup reads whole K and V token rows (all G heads' 2D-byte slices) of
// every page at one time. A sequence whose units lie in one range is
// finished there; one that straddles ranges leaves one state per range
// (ds_state), merged in range order by decode_stream_merge, so the result
// does not depend on timing. A range's first sequence, when it began in an
// earlier range, keeps its state in registers until the range's end: a
// store in mid-stream would hold up the next tile's wait.
// Per tile a wavefront moves K, V and its QPG query rows into an LDS stage
// by direct buffer->LDS loads; the table entries of 64 tiles at a time come
// the same way, a window ahead. Tile arithmetic is decode_tiles'.
constexpr int DS_MAX_B = 1024;  // sequences per call on this path (LDS prefix table)

// Integer division has no instruction; the 32-bit routine is a few times
// shorter than the 64-bit one, and the products fit it at usual sizes.
TSL_DEV int ds_div(uint64_t num, uint32_t den) {
    return (int)((num >> 32) == 0 ? (uint32_t)num / den : num / den);
}
TSL_DEV int ds_start(int w, int U, int W) { return ds_div((uint64_t)w * U, W); }
// The range holding unit u: the largest w with ds_start(w) <= u.
TSL_DEV int ds_owner(int u, int U, int W) { return min(ds_div((uint64_t)(u + 1) * W - 1, U), W - 1); }
// The range after w that holds units (every range does when U >= W); W
// after the last range, so that a walk over ranges always ends.
TSL_DEV int ds_next(int w, int U, int W) {
    return w >= W - 1 ? W : U >= W ? w + 1 : ds_owner(ds_start(w + 1, U, W), U, W);
}

#define DS_WAIT_CASE(n) \
    case n: asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory"); break;
// Waits until at most n vector-memory loads of this wavefront are in flight.
TSL_DEV void ds_wait(int n) {
    switch (n) {
        DS_WAIT_CASE(0) DS_WAIT_CASE(1) DS_WAIT_CASE(2) DS_WAIT_CASE(3) DS_WAIT_CASE(4) DS_WAIT_CASE(5)
        DS_WAIT_CASE(6) DS_WAIT_CASE(7) DS_WAIT_CASE(8) DS_WAIT_CASE(9) DS_WAIT_CASE(10) DS_WAIT_CASE(11)
        DS_WAIT_CASE(12) DS_WAIT_CASE(13) DS_WAIT_CASE(14) DS_WAIT_CASE(15) DS_WAIT_CASE(16) DS_WAIT_CASE(17)
        DS_WAIT_CASE(18) DS_WAIT_CASE(19) DS_WAIT_CASE(20) DS_WAIT_CASE(21) DS_WAIT_CASE(22) DS_WAIT_CASE(23)
        DS_WAIT_CASE(24) DS_WAIT_CASE(25) DS_WAIT_CASE(26) DS_WAIT_CASE(27) DS_WAIT_CASE(28) DS_WAIT_CASE(29)
        DS_WAIT_CASE(30)
        default: asm volatile("s_waitcnt vmcnt(31)" ::: "memory"); break;
    }
}
#undef DS_WAIT_CASE

template <int D, int QPG>
struct DsGeom {
    static constexpr int ROWB = 2 * D, TILE = TT * ROWB, NLD = TILE / 1024;
    static constexpr int QB = QPG * D * 2, NQ = (QB + 1023) / 1024;
    static constexpr int WSTAGE = 2 * TILE + NQ * 1024;  // K, V, Q
    static constexpr int LPT = 2 * NLD + NQ;             // loads per tile
    static constexpr int ST = QPG * (4 + D);             // floats per state: [QPG][m, l, pad, pad, acc[D]]
};
// Range states: piece p < DS_PM of sequence b (its p-th range) at
// [b][g][p] (so the merge reads them without first finding the ranges),
// later pieces at [DS_PM B G + (w 2 + slot) G + g], slot 1 for a range's
// last sequence when it is not also its first.
constexpr int DS_PM = 8;
TSL_DEV long ds_state(int b, int g, int p, int w, int slot, int B, int G) {
    return p < DS_PM ? ((long)b * G + g) * DS_PM + p : (long)DS_PM * B * G + ((long)w * 2 + slot) * G + g;
}
// LDS bytes of a decode_stream workgroup: the rings, the table windows, the
// unit prefix and lens.
constexpr int ds_lds(int D, int QPG, int NWV, int STG) {
    return NWV * STG * (2 * TT * 2 * D + (QPG * D * 2 + 1023) / 1024 * 1024) + NWV * 512 + (2 * DS_MAX_B + 1) * 4;
}
// LDS stages per wavefront: 3 (2 tiles in flight) where they fit, else 2
// (0: the shape does not fit).
constexpr int ds_stages(int D, int QPG, int NWV) {
    return ds_lds(D, QPG, NWV, 3) <= 163840 ? 3 : ds_lds(D, QPG, NWV, 2) <= 163840 ? 2 : 0;
}

template <int D, int QPG, int NWV, int STG>
__global__ __launch_bounds__(64 * NWV) void decode_stream(DecArgs a) {
    using Gm = DsGeom<D, QPG>;
    constexpr int ROWB = Gm::ROWB, KCH = D / 8, TILE = Gm::TILE, NLD = Gm::NLD, RPL = 1024 / ROWB;
    constexpr int NQ = Gm::NQ, WSTAGE = Gm::WSTAGE, LPT = Gm::LPT;
    constexpr float LAZY = 8.0f;
    constexpr int LDS = ds_lds(D, QPG, NWV, STG);
    static_assert(LDS == NWV * STG * WSTAGE + NWV * 512 + (2 * DS_MAX_B + 1) * 4 && LDS <= 163840, "LDS");
    static_assert(2 * LPT + 2 <= 30, "ds_wait covers the loads in flight");
    __shared__ __attribute__((aligned(16))) char lds[LDS];
    TSL_POISON(lds);
    int* wsl = reinterpret_cast<int*>(lds + NWV * STG * WSTAGE);  // [NWV][2][64] table windows
    int* pre = wsl + NWV * 128;                                   // [B + 1] first unit of b
    int* ln = pre + DS_MAX_B + 1;                                 // [B] lens

    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, col = lane & 15;
    const int g = __builtin_amdgcn_readfirstlane(tid >> 6);  // the wavefront's kv head
    const int W = gridDim.x, w = blockIdx.x;
    const int tpp = a.P / TT;

    // Virtual sequences vb = b NG + hg: sequence b's kv heads hg NWV ..
    // hg NWV + NWV - 1 (NG = G / NWV head groups; 1 when the wavefronts
    // cover all G heads), each its own run of units.
    const int NG = a.NG, VB = a.B * NG;
    if (g == 0) {  // prefix of the units per virtual sequence
        int run = 0;
        for (int b0 = 0; b0 < VB; b0 += 64) {
            const int b = b0 + lane;
            const int n = b < VB ? a.lens[b / NG] : 0;
            const int t = n > 0 ? ((n + a.P - 1) >> a.pshift) * tpp : 0;
            int x = t;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(x, o);
                if (lane >= o) x += y;
            }
            if (b < VB) {
                pre[b] = run + x - t;
                ln[b] = n;
            }
            run += __shfl(x, 63);
        }
        if (lane == 0) pre[VB] = run;
    }
    __syncthreads();
    const int U = pre[VB];
    if (w == 0)
        for (int x = tid; x <= VB; x += 64 * NWV) a.pre[x] = pre[x];
    for (int vb = w; vb < VB; vb += W)  // lens 0: 0 / 0, as the .tl computes (the group's heads)
        if (pre[vb + 1] == pre[vb])
            for (int x = tid; x < NWV * QPG * D; x += 64 * NWV)
                a.O[((long)(vb / NG) * a.H + (vb % NG) * NWV * QPG) * D + x] = f2h(0.0f / 0.0f);
    const int u0 = ds_start(w, U, W), u1 = ds_start(w + 1, U, W), nt = u1 - u0;
    if (nt <= 0) return;

    // Window k: lane l describes unit u0 + 64 k + l (clamped to the range):
    // its sequence, first token and length, and the flat table index of its page.
    auto window = [&](int k, int& wb, int& wt, int& wn, int& widx) {
        const int u = min(u0 + 64 * k + lane, u1 - 1);
        int lo = 0, hi = VB - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (pre[mid] <= u) lo = mid;
            else hi = mid - 1;
        }
        wb = lo;
        wt = (u - pre[lo]) * TT;
        wn = ln[lo];
        const int pi = wt >> a.pshift;
        widx = pi < a.MP ? (lo / NG) * a.MP + pi : 0;  // (past the table: any in-range entry; issue reads page 0)
    };

    const long tok_bytes = (long)a.G * D * 2;
    uint32_t offk[NLD], offv[NLD];
#pragma unroll
    for (int q = 0; q < NLD; q++) {
        const int row = q * RPL + lane / KCH, pc = lane % KCH;
        offk[q] = (uint32_t)(row * tok_bytes + ((pc ^ tswz_k<D>(row)) * 16));
        offv[q] = (uint32_t)(row * tok_bytes + ((pc ^ tswz_v<D>(row)) * 16));
    }
    const uint32_t lbase = (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t*)lds);
    const uint32_t ring0 = lbase + g * STG * WSTAGE;
    const uint32_t wsl0 = lbase + NWV * STG * WSTAGE + g * 512;
    const i32x4 rtab = buf_rsrc(a.table, (uint32_t)((long)a.B * a.MP * 4));

    int ib, it, in, ipg;       // the issuing side's window
    int nb = 0, nx = 0, nn = 0;  // the next window's (its pages land in LDS)
    {
        int idx;
        window(0, ib, it, in, idx);
        ipg = a.table[idx];
    }
    asm volatile("" ::"v"(ipg));  // window 0 has arrived before the first asynchronous load

    auto issue = [&](int j) {  // tile j of the range into stage j % STG
        if ((j & 63) == 0) {
            if (j > 0) {
                ib = nb;
                it = nx;
                in = nn;
                ipg = wsl[(g * 2 + ((j >> 6) & 1)) * 64 + lane];
            }
            if (j + 64 < nt) {  // the next window's table entries, one load
                int idx;
                window((j >> 6) + 1, nb, nx, nn, idx);
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(
                                 wsl0 + (((j >> 6) + 1) & 1) * 256),
                             "v"((uint32_t)idx * 4u), "s"(rtab)
                             : "memory");
            }
        }
        const int jl = j & 63;
        const int vb = __builtin_amdgcn_readlane(ib, jl), t0 = __builtin_amdgcn_readlane(it, jl);
        const int b = vb / NG, gh = (vb % NG) * NWV + g;  // sequence, kv head
        const char* Kg = reinterpret_cast<const char*>(a.Kc) + (long)gh * D * 2;
        const char* Vg = reinterpret_cast<const char*>(a.Vc) + (long)gh * D * 2;
        // Tiles past the table read pool page 0 (their window entry is a stand-in).
        const int page = (t0 >> a.pshift) < a.MP ? __builtin_amdgcn_readlane(ipg, jl) : 0;
        const bool ok = page >= 0 && page < a.NP;  // outside the pool: zeros
        const long shift = ((long)(ok ? page : 0) * a.P + (t0 & (a.P - 1))) * tok_bytes;
        const uint32_t range = ok ? (uint32_t)(TT * tok_bytes) : 0u;
        const i32x4 rk = buf_rsrc(Kg + shift, range), rv = buf_rsrc(Vg + shift, range);
        const i32x4 rq = buf_rsrc(a.Q + ((long)b * a.H + gh * QPG) * D, (uint32_t)Gm::QB);
        const uint32_t sk = ring0 + (j % STG) * WSTAGE, sv = sk + TILE, sq = sv + TILE;
#pragma unroll
        for (int q = 0; q < NLD; q++) {
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(sk + q * 1024),
                         "v"(offk[q]), "s"(rk)
                         : "memory");
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(sv + q * 1024),
                         "v"(offv[q]), "s"(rv)
                         : "memory");
        }
#pragma unroll
        for (int q = 0; q < NQ; q++)
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(sq + q * 1024),
                         "v"((uint32_t)(lane * 16 + q * 1024)), "s"(rq)
                         : "memory");
    };
    // Loads issued with tile j: its own and, every 64 tiles, the next window's.
    auto loads_with = [&](int j) { return LPT + (((j & 63) == 0 && j + 64 < nt) ? 1 : 0); };

    uint32_t kaddr[D / 32], vaddr[D / 16];
#pragma unroll
    for (int s = 0; s < D / 32; s++) kaddr[s] = (uint32_t)(col * ROWB + (((4 * s + grp) ^ tswz_k<D>(col)) * 16));
    const int vrow = 4 * grp + (col >> 2);
#pragma unroll
    for (int dt = 0; dt < D / 16; dt++) {
        const int lc = 2 * dt + ((col & 3) >> 1);
        vaddr[dt] = (uint32_t)(TILE + vrow * ROWB + ((lc ^ tswz_v<D>(vrow)) * 16) + 8 * (col & 1));
    }
    const uint32_t qaddr = (uint32_t)(2 * TILE + (col & (QPG - 1)) * D * 2 + grp * 16);

    float m = -1e30f, lsum = 0.0f;
    float4v acc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; dt++) acc[dt] = float4v{};

    // Ends sequence b's part of this range: O directly when the whole
    // sequence lies here, else this range's state for it.
    // This range's state of sequence b (m, l, acc of its part), stored by
    // the lanes that hold it.
    auto store_state = [&](int b, float sm, float sl, const float4v* sa) {
        const int lo = pre[b], wlo = ds_owner(lo, U, W);
        int p = 0;  // which piece of b this range is
        if (U >= W) p = w - wlo;
        else
            for (int x = wlo; x < w; x = ds_next(x, U, W)) p++;
        const int slot = lo <= u0 ? 0 : 1;
        float* pe = a.part + ds_state(b, g, p, w, slot, VB, NWV) * Gm::ST + col * (4 + D);
        if (col < QPG) {
            if (grp == 0) *reinterpret_cast<float4v*>(pe) = float4v{sm, sl, 0.0f, 0.0f};
#pragma unroll
            for (int dt = 0; dt < D / 16; dt++) *reinterpret_cast<float4v*>(pe + 4 + 16 * dt + 4 * grp) = sa[dt];
        }
    };
    // Ends sequence b's part of this range before the range's end: O directly
    // when the whole sequence lies here; else it is the range's first
    // sequence, begun in an earlier range, and its state is held in
    // registers until the end (a store now would stall the next tile's wait).
    bool held = false;
    float hm = 0.0f, hl = 0.0f;
    float4v hacc[D / 16];
    auto flush = [&](int b) {
        float l = lsum + xor16(lsum);
        l += xor32(l);
        if (pre[b] >= u0) {
            if (col < QPG) {
                u16* o = a.O + ((long)(b / NG) * a.H + ((b % NG) * NWV + g) * QPG + col) * D + 4 * grp;
#pragma unroll
                for (int dt = 0; dt < D / 16; dt++) {
                    half4 h;
#pragma unroll
                    for (int q = 0; q < 4; q++) h[q] = (half_t)(acc[dt][q] / l);
                    *reinterpret_cast<half4*>(o + 16 * dt) = h;
                }
            }
        } else {
            held = true;
            hm = m;
            hl = l;
#pragma unroll
            for (int dt = 0; dt < D / 16; dt++) hacc[dt] = acc[dt];
        }
    };

    const int npre = min(nt, STG - 1);
    for (int j = 0; j < npre; j++) issue(j);
    int cwb = 0, cwt = 0, cwn = 0;  // the computing side's window
    int cb = -1;                    // sequence being accumulated
    for (int i = 0; i < nt; i++) {
        const int ja = i + STG - 1;
        if (ja < nt) issue(ja);
        int after = 0;  // loads issued after tile i's
        for (int j = i + 1; j <= min(ja, nt - 1); j++) after += loads_with(j);
        ds_wait(after);
        if ((i & 63) == 0) {
            cwb = ib;
            cwt = it;
            cwn = in;
        }
        const int il = i & 63;
        const int b = __builtin_amdgcn_readlane(cwb, il);
        const int n = __builtin_amdgcn_readlane(cwn, il);
        const int t0 = __builtin_amdgcn_readlane(cwt, il) + 4 * grp;  // token of register 0
        if (b != cb) {
            if (cb >= 0) flush(cb);
            cb = b;
            m = -1e30f;
            lsum = 0.0f;
#pragma unroll
            for (int dt = 0; dt < D / 16; dt++) acc[dt] = float4v{};
        }
        const char* sb = lds + (g * STG + i % STG) * WSTAGE;
        float4v sc = float4v{};
#pragma unroll
        for (int s = 0; s < D / 32; s++) {
            const half8 kop = *reinterpret_cast<const half8*>(sb + kaddr[s]);
            half8 qop = *reinterpret_cast<const half8*>(sb + qaddr + s * 64);
            if (col >= QPG) qop = half8{};
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop, sc, 0, 0, 0);
        }
        float x[4], mb = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            x[r] = t0 + r < n ? sc[r] * a.c2 : -INFINITY;
            mb = fmaxf(mb, x[r]);
        }
        mb = fmaxf(mb, xor16(mb));
        mb = fmaxf(mb, xor32(mb));
        if (__builtin_amdgcn_ballot_w64(mb > m + LAZY) != 0) {
            const float mn = fmaxf(m, mb);
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < D / 16; dt++) acc[dt] *= alpha;
            m = mn;
        }
        half4 phi, plo;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = __builtin_amdgcn_exp2f(x[r] - m);
            lsum += p;
            phi[r] = (half_t)p;
            plo[r] = (half_t)(p - (float)phi[r]);
        }
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
            const fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                (__attribute__((address_space(3))) fp16x4_t*)(sb + vaddr[dt]));
            const half4 vop = __builtin_bit_cast(half4, v);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vop, phi, acc[dt], 0, 0, 0);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vop, plo, acc[dt], 0, 0, 0);
        }
    }
    // The last sequence: finished here when it began in this range and ends
    // with it, else a state.
    if (held) {  // the range's first sequence (it holds unit u0)
        int bl = 0, bh = VB - 1;
        while (bl < bh) {
            const int mid = (bl + bh + 1) >> 1;
            if (pre[mid] <= u0) bl = mid;
            else bh = mid - 1;
        }
        store_state(bl, hm, hl, hacc);
    }
    if (pre[cb] >= u0 && pre[cb + 1] <= u1) {
        flush(cb);
    } else {
        float l = lsum + xor16(lsum);
        l += xor32(l);
        store_state(cb, m, l, acc);
    }
}

// Merges the range states of each straddling (b, g), in range order (so the
// bits do not depend on timing): one wavefront per (b, g). Lane e of a pass
// owns 8 consecutive d of one query head. The first DS_PM pieces' states are
// read together with the unit prefix (one memory round trip); more pieces
// follow in batches of 8 ranges.
template <int D, int QPG, int NWV>
__global__ __launch_bounds__(64) void decode_stream_merge(DecArgs a, int W) {
    constexpr int ST = DsGeom<D, QPG>::ST, NE = QPG * D / 8;
    const int b = blockIdx.x / NWV, g = blockIdx.x % NWV, lane = threadIdx.x;  // virtual sequence, its head
    const int VB = a.B * a.NG;
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(a.part, 0, 0x7fffffff, 0x00020000);
    for (int e0 = 0; e0 < NE; e0 += 64) {
        const int e = min(e0 + lane, NE - 1), h = e / (D / 8), d0 = (e % (D / 8)) * 8;
        auto load = [&](long st, float2v& ml, float4v& x0, float4v& x1) {
            const uint32_t pe = (uint32_t)((st * ST + h * (4 + D)) * 4);
            ml = __builtin_amdgcn_raw_buffer_load_b64(rp, pe, 0, 0);
            x0 = __builtin_amdgcn_raw_buffer_load_b128(rp, pe + (4 + d0) * 4, 0, 0);
            x1 = __builtin_amdgcn_raw_buffer_load_b128(rp, pe + (8 + d0) * 4, 0, 0);
        };
        float2v ml[DS_PM];
        float4v x0[DS_PM], x1[DS_PM];
#pragma unroll
        for (int p = 0; p < DS_PM; p++) load(ds_state(b, g, p, 0, 0, VB, NWV), ml[p], x0[p], x1[p]);
        const int U = a.pre[VB], lo = a.pre[b], hi = a.pre[b + 1];
        if (hi <= lo) return;  // lens 0: written by decode_stream
        const int wlo = ds_owner(lo, U, W), whi = ds_owner(hi - 1, U, W);
        if (wlo == whi) return;  // finished by its range
        int np = 1, wn = wlo;    // pieces, and the range after the first DS_PM
        for (int x = wlo; x < whi; x = ds_next(x, U, W)) {
            if (np == DS_PM) wn = x;
            np++;
        }
        float M = -INFINITY, L = 0.0f, A[8];
#pragma unroll
        for (int q = 0; q < 8; q++) A[q] = 0.0f;
        // Folds a batch of n states into (M, L, A): the batch maximum first.
        auto fold = [&](int n) {
            float Mb = M;
#pragma unroll
            for (int p = 0; p < DS_PM; p++)
                if (p < n) Mb = fmaxf(Mb, ml[p][0]);
            const float sc = __builtin_amdgcn_exp2f(M - Mb);
            L *= sc;
#pragma unroll
            for (int q = 0; q < 8; q++) A[q] *= sc;
#pragma unroll
            for (int p = 0; p < DS_PM; p++) {
                if (p < n) {
                    const float f = __builtin_amdgcn_exp2f(ml[p][0] - Mb);
                    L += ml[p][1] * f;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        A[q] += x0[p][q] * f;
                        A[4 + q] += x1[p][q] * f;
                    }
                }
            }
            M = Mb;
        };
        fold(min(np, DS_PM));
        if (np > DS_PM) {
            // Every piece past the first is its range's first sequence: slot 0.
            wn = ds_next(wn, U, W);  // the range of piece DS_PM
            for (int p0 = DS_PM; p0 < np; p0 += DS_PM) {
#pragma unroll
                for (int p = 0; p < DS_PM; p++) {
                    const int wq = min(wn, whi);
                    load(ds_state(b, g, DS_PM, wq, 0, VB, NWV), ml[p], x0[p], x1[p]);
                    if (p0 + p + 1 < np) wn = ds_next(wn, U, W);
                }
                fold(min(np - p0, DS_PM));
            }
        }
        if (e0 + lane < NE) {
            half8 o;
#pragma unroll
            for (int q = 0; q < 8; q++) o[q] = (half_t)(A[q] / L);
            *reinterpret_cast<half8*>(a.O + ((long)(b / a.NG) * a.H + ((b % a.NG) * NWV + g) * QPG + h) * D + d0) = o;
        }
    }
}

// Persistent workgroups of the stream path: one per CU.
int stream_groups() { return num_cus(); }

// Wavefronts (kv heads) per workgroup of the balanced path: 4 kv heads, or
// 8 at a time of a multiple of 8 (0: not this path).
int64_t stream_nwv(int64_t G) { return G == 4 ? 4 : G > 0 && G % 8 == 0 ? 8 : 0; }

// Bytes of the stream path's range states: DS_PM per (virtual sequence,
// wavefront), then two per (range, wavefront) (ds_state).
size_t stream_state_bytes(const TslKernel& k) {
    const int64_t H = k.dim("H"), G = k.name == "paged_attention" ? H : k.dim("G");
    const int64_t st = (H / G) * (4 + k.dim("D")) * 4, nwv = stream_nwv(G);
    return (size_t)((DS_PM * k.dim("B") * G + (int64_t)stream_groups() * 2 * nwv) * st);
}

template <int D, int QPG, int NWV>
int run_decode_stream(DecArgs& a, hipStream_t s) {
    constexpr int STG = ds_stages(D, QPG, NWV);
    if constexpr (STG == 0) {
        return tsl_fail(-2, "decode_attention: no stream variant");
    } else {
    const int W = stream_groups();
    hipLaunchKernelGGL((decode_stream<D, QPG, NWV, STG>), dim3(W), dim3(64 * NWV), 0, s, a);
    int r = TSL_LAUNCHED("decode_attention");
    if (r) return r;
    hipLaunchKernelGGL((decode_stream_merge<D, QPG, NWV>), dim3(a.B * a.NG * NWV), dim3(64), 0, s, a, W);
    return TSL_LAUNCHED("decode_attention merge");
    }
}

template <int D>
int run_stream_d(DecArgs& a, int qpg, hipStream_t s) {
    if (a.G % 8 == 0) {
        a.NG = a.G / 8;
        switch (qpg) {
            case 1: return run_decode_stream<D, 1, 8>(a, s);
            case 2: return run_decode_stream<D, 2, 8>(a, s);
            case 4: return run_decode_stream<D, 4, 8>(a, s);
            case 8: return run_decode_stream<D, 8, 8>(a, s);
        }
    } else {
        a.NG = 1;
        switch (qpg) {
            case 1: return run_decode_stream<D, 1, 4>(a, s);
            case 2: return run_decode_stream<D, 2, 4>(a, s);
            case 4: return run_decode_stream<D, 4, 4>(a, s);
            case 8: return run_decode_stream<D, 8, 4>(a, s);
        }
    }
    return tsl_fail(-2, "decode_attention: no stream variant");
}

template <int D, int QPG>
int run_decode_tiles(DecArgs& a, hipStream_t s) {
    constexpr int WIDE = D == 64 ? 8 : 4;  // wavefronts per workgroup of a one-chunk table (rings fit LDS)
    if (a.NCH == 1)
        hipLaunchKernelGGL((decode_tiles<D, QPG, WIDE>), dim3(a.B * a.G), dim3(64 * WIDE), 0, s, a);
    else
        // Chunks of a long table: two wavefronts per chunk, merged in LDS
        // (108.5 against 110.7 us for one, bench config).
        hipLaunchKernelGGL((decode_tiles<D, QPG, 2>), dim3(a.B * a.G * a.NCH), dim3(128), 0, s, a);
    int r = TSL_LAUNCHED("decode_attention");
    if (r || a.NCH == 1) return r;
    const size_t lds = (size_t)a.NCH * QPG * (2 + D) * sizeof(float);
    if (lds > 65536) {  // too many states for one workgroup's LDS: the serial merge
        hipLaunchKernelGGL((decode_combine<D, QPG>), dim3(a.B * a.H), dim3(64), 0, s, a);
        return TSL_LAUNCHED("decode_attention combine");
    }
    hipLaunchKernelGGL((decode_merge<D, QPG>), dim3(a.B * a.G), dim3(256), lds, s, a);
    return TSL_LAUNCHED("decode_attention merge");
}

template <int D>
int run_tiles_d(DecArgs& a, int qpg, hipStream_t s) {
    switch (qpg) {
        case 1: return run_decode_tiles<D, 1>(a, s);
        case 2: return run_decode_tiles<D, 2>(a, s);
        case 4: return run_decode_tiles<D, 4>(a, s);
        case 8: return run_decode_tiles<D, 8>(a, s);
        case 16: return run_decode_tiles<D, 16>(a, s);
    }
    return tsl_fail(-2, "decode_attention: H / G must be 1, 2, 4, 8 or 16");
}

bool tiles_path(int64_t D, int64_t P) { return (D == 64 || D == 128) && P % TT == 0; }

// The balanced path: matrix-core shapes with 4 or a multiple of 8 kv heads
// (a wavefront each, 8 at a time), 1-8 query heads per kv head, tables
// longer than one chunk, at most DS_MAX_B (sequence, head group) pairs and
// 32-bit flat table offsets.
bool stream_path(const TslKernel& k) {
    const int64_t H = k.dim("H"), G = k.name == "paged_attention" ? H : k.dim("G");
    const int64_t qpg = G > 0 ? H / G : 0, nwv = stream_nwv(G);
    return tiles_path(k.dim("D"), k.dim("P")) && nwv > 0 && (qpg == 1 || qpg == 2 || qpg == 4 || qpg == 8) &&
           ds_stages((int)k.dim("D"), (int)qpg, (int)nwv) > 0 && k.dim("MP") > DEC_WIDE_MAX_PAGES &&
           k.dim("B") * (G / nwv) <= DS_MAX_B && k.dim("B") * k.dim("MP") * 4 < (1LL << 32);
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

// Pages per chunk: enough chunks for about 2048 workgroups over B x G at the
// table's full length (short contexts get short chunks, so the cache is
// still read by the whole chip), few enough that one (b, g)'s chunk states
// fit the merge's 64 KB of LDS; between 2 and 24 pages.
int chunk_pages(const TslKernel& k) {
    const int64_t H = k.dim("H"), G = k.name == "paged_attention" ? H : k.dim("G");
    const int64_t bg = std::max<int64_t>(1, k.dim("B") * G), mp = k.dim("MP");
    const int64_t state = (H / std::max<int64_t>(1, G)) * (2 + k.dim("D")) * 4;  // bytes per chunk
    const int64_t ch = std::max((mp * bg + 2047) / 2048, (mp * state + 65535) / 65536);
    // Short tables on the matrix-core path: one chunk, read by a workgroup of
    // several wavefronts that merge in LDS (no second kernel).
    if (tiles_path(k.dim("D"), k.dim("P")) && mp <= DEC_WIDE_MAX_PAGES) return (int)std::max<int64_t>(1, mp);
    return (int)std::min<int64_t>(DEC_MAX_CHUNK, std::max<int64_t>(2, ch));
}
int nchunks(const TslKernel& k) {
    const int ch = chunk_pages(k);
    return (int)((k.dim("MP") + ch - 1) / ch);
}

}  // namespace

// Checks a decode specialisation and gives the scratch bytes its launch
// needs (0: none): the stream path's range states then its [B + 1] unit
// prefix, or the chunked path's [B][G][NCH][QPG][2 + D] per-chunk states.
static int decode_scratch_bytes(const TslKernel& k, size_t* bytes) {
    int64_t D = k.dim("D"), H = k.dim("H");
    int64_t G = k.name == "paged_attention" ? H : k.dim("G");
    *bytes = 0;
    if (D != 16 && D != 32 && D != 64 && D != 128)
        return tsl_fail(-2, k.name + ": head dimension " + std::to_string(D) + " unsupported (16, 32, 64 or 128)");
    if (G <= 0 || H % G != 0) return tsl_fail(-2, k.name + ": H must be a multiple of G");
    int64_t qpg = H / G;
    if (qpg != 1 && qpg != 2 && qpg != 4 && qpg != 8 && qpg != 16)
        return tsl_fail(-2, k.name + ": H / G must be 1, 2, 4, 8 or 16");
    if (stream_path(k)) {
        *bytes = stream_state_bytes(k) + (size_t)(k.dim("B") * (G / stream_nwv(G)) + 1) * 4;
        return 0;
    }
    int nch = nchunks(k);
    if (nch > 1) *bytes = (size_t)k.dim("B") * G * nch * qpg * (2 + D) * sizeof(float);
    return 0;
}

// Sizes the partial-state buffer once, when the kernel is specialised.
int prepare_decode(TslKernel& k) {
    size_t bytes = 0;
    if (int r = decode_scratch_bytes(k, &bytes)) return r;
    if (bytes) {
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
    a.pshift = __builtin_ctz((unsigned)a.P);
    a.MP = k.dim("MP");
    a.NCH = nchunks(k);
    a.CH = chunk_pages(k);
    a.part = reinterpret_cast<float*>(k.scratch);
    if (a.B == 0) return 0;
    const int D = k.dim("D"), qpg = a.H / a.G;
    if (stream_path(k)) {
        a.pre = reinterpret_cast<int*>(reinterpret_cast<char*>(k.scratch) + stream_state_bytes(k));
        return D == 128 ? run_stream_d<128>(a, qpg, s) : run_stream_d<64>(a, qpg, s);
    }
    if (tiles_path(D, a.P)) return D == 128 ? run_tiles_d<128>(a, qpg, s) : run_tiles_d<64>(a, qpg, s);
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

// ---------------------------------------------------------------- no-alloc entry

// The scratch of tsl_decode_attention_noalloc: one array per GPU, resident
// until the process ends, shared by every call on that GPU. Host code uses
// only the address hipGetSymbolAddress gives for the current device, never
// the array's name (a host-side stand-in, not a device address).
static __device__ __align__(256) char scratch[TSL_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[NOALLOC_MAX_DEVICES];

// The current device's scratch address, looked up once per device.
int noalloc_scratch(void** out) {
    int dev = 0;
    if (tsl_hip_check(hipGetDevice(&dev), "hipGetDevice")) return -1;
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return tsl_fail(-2, "decode_attention_noalloc: device index too large");
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void* p = nullptr;
        if (tsl_hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return -1;
        g_noalloc_ptr[dev] = p;
    }
    *out = g_noalloc_ptr[dev];
    return 0;
}
}  // namespace

extern "C" int tsl_decode_attention_noalloc(uint64_t q, uint64_t kc, uint64_t vc, uint64_t table, uint64_t lens,
                                            uint64_t o, float scale, int B, int H, int G, int D, int NP, int P,
                                            int MP) {
    if (B < 0 || H <= 0 || G <= 0 || D <= 0 || NP <= 0 || P <= 0 || MP <= 0 || (P & (P - 1)))
        return tsl_fail(-2, "decode_attention_noalloc: sizes must be positive (B >= 0) and P a power of two");
    if (tsl_open()) return -1;
    TslKernel k;
    k.file = "llm";
    k.name = "decode_attention";
    k.nparams = 7;
    k.dims = {{"B", B}, {"H", H}, {"D", D}, {"NP", NP}, {"P", P}, {"G", G}, {"MP", MP}};
    size_t bytes = 0;
    if (int r = decode_scratch_bytes(k, &bytes)) return r;
    if (bytes > sizeof(scratch))
        return tsl_fail(-2, "decode_attention_noalloc: this shape needs " + std::to_string(bytes) +
                                " bytes of scratch; at most " + std::to_string(sizeof(scratch)));
    void* ptr = nullptr;
    if (int r = noalloc_scratch(&ptr)) return r;
    k.scratch = ptr;
    k.scratch_bytes = sizeof(scratch);
    uint32_t sb;
    __builtin_memcpy(&sb, &scale, 4);
    const uint64_t args[7] = {q, kc, vc, table, lens, o, (uint64_t)sb};
    return launch_decode_common(k, args, (hipStream_t)tsl_stream(), true);
}
