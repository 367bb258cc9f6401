// Causal attention prefill on CDNA4 matrix cores: flash_attention
// (kernels/attention.tl:4-24, Q/K/V/O [H, S, D]) and the engine's
// grouped-query, packed-prompt prefill_attention (kernels/llm.tl:116-145,
// Q/O [S, H, D], K/V [S, G, D], row r attending keys starts[r] .. r, running
// maximum starting at -1e30).
//
// A workgroup of 4 wavefronts owns 128 query rows of one head; each
// wavefront owns 32. Per block of 64 keys, staged in LDS (double-buffered
// by direct loads that overlap the previous block's compute):
//   S^T = K Q^T     (v_mfma_f32_32x32x16_f16; lane l holds query l % 32,
//                    so the online-softmax state is per lane)
//   O^T += V^T P^T  (P^T taken straight from the S^T accumulators, rounded
//                    to f16 as the .tl's f16(p) does)
// K and V are staged row-major ([key][d], 16-byte chunks XOR-swizzled) by
// direct buffer->LDS loads; the V^T operand comes from transposed LDS reads
// (ds_read_b64_tr_b16), 4 keys of one d column per lane. The key order
// inside a 16-key MFMA step is permuted identically for P^T and V^T (the
// reduction does not depend on it). exp is exp2 with log2(e) folded into
// the scale. Query blocks are issued longest (most keys) first.
#include "common.h"

namespace {

constexpr float LOG2E = 1.4426950408889634f;
constexpr int BQ = 128;  // queries per workgroup
constexpr int BKEY = 64;  // keys per block

struct AttnArgs {
    const u16 *Q, *K, *V;
    u16* O;
    const int* starts;  // prefill only
    int S, H, G;
    int ncu;  // compute units (workgroups dispatched round-robin over them)
    long q_row, q_head, k_row, k_head;  // element strides
    float scale;
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 fp16x4_t;
typedef int i32x4 __attribute__((ext_vector_type(4)));

TSL_DEV i32x4 make_rsrc(const void* p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    return i32x4{(int)(uint32_t)a, (int)(uint32_t)((a >> 32) & 0xffff), (int)bytes, 0x00020000};
}

TSL_DEV half4 lds_read_tr(const void* p) {
    fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) fp16x4_t*)(p));
    return __builtin_bit_cast(half4, v);
}

// LDS layouts of a 64-key block (K then V, each [64][D] row-major, 2D bytes
// a row) with 16-byte-chunk XOR swizzles chosen so that the lane groups LDS
// serves together (16 lanes of a 16-byte read, 32 of an 8-byte transposed
// read) fall on distinct banks of the 256-byte bank window:
//   K: 16 consecutive keys read the same logical chunk -> chunk ^ ((key / (128/D)) % (D/8))
//   V: 4 key rows x 32 d of a transposed read -> 32-byte granule ^ 2*((row>>1)&1)
//      (D = 64) or 2*(row&3) (D = 128); D <= 32 needs none.
template <int D>
TSL_DEV int swz_k(int key) {
    constexpr int KCH = D / 8, RPW = D >= 128 ? 1 : 128 / D;
    return (key / RPW) & (KCH - 1);
}
template <int D>
TSL_DEV int swz_v(int key) {  // in 16-byte chunks
    if constexpr (D == 64) return 4 * ((key >> 1) & 1);
    else if constexpr (D == 128) return 4 * (key & 3);
    else return 0;
}

// KS = 2 (short sequences): the 4 wavefronts form 2 query groups of 32 rows,
// and the 2 wavefronts of a group take alternate key blocks (block b to
// wavefront b % 2, each block with its own LDS stages), so a workgroup's
// critical path is half its keys; the two states of each row are merged
// through LDS at the end (max, then the rescaled sums, in wavefront order).
// D = 128 with the key split holds 4 stages of 32 KB: one workgroup per CU,
// so its launch bounds ask for one (and the registers that allows).
//
// FOLD (KS = 1): Q is scaled by c2 = scale log2(e) on its way into
// registers (rounded to f16) and the score MFMAs start from -mc (a
// 16-register tile of this lane's running max) instead of 0, so the
// accumulators are the exponents and the per-score multiply-add goes. A
// block's two 32-key tiles are then computed and exponentiated one after the
// other (the second tile's MFMAs can run under the first's exponentials), so
// only one tile of scores is live and the -mc tile fits the 128 registers
// that keep 4 workgroups per CU. Same box, H32 D64: S = 2048 502 -> 546,
// S = 4096 781 -> 841 TFLOP/s. With the key split (KS = 2) the fold lost
// (packed prefill 214 -> 170, S = 512 142 -> 137): that form stays unfolded.
template <int D, bool PREFILL, int KS, bool FOLD>
__global__ __launch_bounds__(256, (D == 128 && KS == 2) ? 1 : 2) void attn_fwd(AttnArgs a) {
    constexpr int DP = D < 32 ? 32 : D;     // V^T rows, padded to one MFMA tile
    constexpr int KCH = D / 8;              // 16-byte chunks per row
    constexpr int ROWB = 2 * D;             // bytes per K or V row
    constexpr int KPL = 1024 / ROWB;        // rows per 1 KB load
    constexpr int NL = BKEY / KPL;          // 1 KB loads per matrix per block
    constexpr int LPW = NL >= 4 ? NL / 4 : 1;  // loads per wave per matrix (waves >= NL idle when NL < 4)
    constexpr int STAGE = 2 * BKEY * ROWB;  // K then V
    constexpr float LAZY = 8.0f;            // rescale only when the max grows by more than 2^8
    constexpr int BQW = BQ / KS;            // queries per workgroup
    static_assert(KS == 1 || KS == 2, "key split");
    constexpr int NF = 2 + 16 * (DP / 32);  // floats per lane of a merged state: mc, lsum, acc
    constexpr int LDSB = KS * 2 * STAGE > 4 * NF * 64 * 4 || KS == 1 ? KS * 2 * STAGE : 4 * NF * 64 * 4;
    __shared__ __attribute__((aligned(16))) char lds[LDSB];  // [ks][stage]; at the end, the merge
    TSL_POISON(lds);

    const int tid = threadIdx.x, lane = tid & 63, g4 = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qg = wave / KS, ks = wave % KS;  // query group, key split
    const int nqb = (a.S + BQW - 1) / BQW;
    // Work rank (0 = most keys): longest first, and within every full round of
    // NCU workgroups (one per CU) alternately reversed, so the workgroups
    // sharing a CU add up to about the same work. The reversal moves whole
    // groups of 8 ranks (workgroup i runs on XCD i % 8), so with H a multiple
    // of 8 a head's query blocks all run on one XCD and its K and V are
    // fetched into one L2 (H32 S4096: 78.6 -> 50.4 MiB read per call).
    int rank = blockIdx.x;
    {
        const int r = rank / a.ncu, j = rank % a.ncu;
        if ((r & 1) && (r + 1) * a.ncu <= (int)gridDim.x)
            rank = r * a.ncu + (a.ncu % 8 == 0 ? a.ncu - 8 - (j & ~7) + (j & 7) : a.ncu - 1 - j);
    }
    const int qb = nqb - 1 - rank / a.H;
    const int h = rank % a.H;
    const int hk = PREFILL ? h / (a.H / a.G) : h;
    const int q0 = qb * BQW, qw = q0 + qg * 32;
    const int myq = qw + (lane & 31);

    const u16* Qh = a.Q + (long)h * a.q_head;
    const char* Kh = reinterpret_cast<const char*>(a.K + (long)hk * a.k_head);
    const char* Vh = reinterpret_cast<const char*>(a.V + (long)hk * a.k_head);
    const uint32_t lds_base = (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t*)lds);

    // Q^T operand, kept in registers: lane l holds d = 16 s + 8 (l/32) .. +8
    // of its query (FOLD: times c2, rounded to f16).
    const float c2 = a.scale * LOG2E;
    half8 qop[D / 16];
#pragma unroll
    for (int s = 0; s < D / 16; s++) {
        u32x4 t = {0, 0, 0, 0};
        if (myq < a.S) t = *reinterpret_cast<const u32x4*>(Qh + (long)myq * a.q_row + 16 * s + 8 * g4);
        qop[s] = __builtin_bit_cast(half8, t);
        if constexpr (FOLD)
#pragma unroll
            for (int e = 0; e < 8; e++) qop[s][e] = (half_t)((float)qop[s][e] * c2);
    }
    const int my_start = PREFILL ? (myq < a.S ? a.starts[myq] : 0) : 0;

    // This lane's byte offsets (relative to the block's first key row) for the
    // wave's K and V loads; the buffer base advances with the block.
    uint32_t offk[LPW], offv[LPW];
    bool ldk[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const int q = wave * LPW + i;
        const int key = q * KPL + lane / KCH, p = lane % KCH;
        ldk[i] = q < NL;
        offk[i] = (uint32_t)(key * a.k_row * 2 + ((p ^ swz_k<D>(key)) * 16));
        offv[i] = (uint32_t)(key * a.k_row * 2 + ((p ^ swz_v<D>(key)) * 16));
    }
    // Iteration it's key blocks it KS .. it KS + KS - 1 (those below nblk)
    // into [ks][stage]; every wavefront loads its share of each.
    auto issue = [&](int it, int stage, int kbeg, int nblk) {
#pragma unroll
        for (int kk = 0; kk < KS; kk++) {
            const int bi = it * KS + kk;
            if (bi >= nblk) break;
            const int j = kbeg + bi * BKEY;
            const long shift = (long)j * a.k_row * 2;
            const uint32_t range = (uint32_t)(((long)a.S - j) * a.k_row * 2);
            const i32x4 rk = make_rsrc(Kh + shift, range), rv = make_rsrc(Vh + shift, range);
            const uint32_t sk = lds_base + (kk * 2 + stage) * STAGE + wave * LPW * 1024, sv = sk + BKEY * ROWB;
#pragma unroll
            for (int i = 0; i < LPW; i++) {
                if (!ldk[i]) continue;  // wave-uniform
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(sk + i * 1024),
                             "v"(offk[i]), "s"(rk));
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(sv + i * 1024),
                             "v"(offv[i]), "s"(rv));
            }
        }
    };

    // Operand addresses within a stage. K (A operand of S^T): key kt*32 + l%32,
    // logical chunk 2 s + g. V^T (A operand of O^T) by transposed reads:
    // provider (grp, jj) points at key row 16 t + 8 h + 4 g + jj/4 and
    // columns dt*32 + 16 (grp&1) + 4 (jj&3) .. +3, so lane l receives column
    // dt*32 + l%32 for keys 16 t + 8 h + 4 g + 0..3, the key order the P^T
    // operand (the S^T accumulator) has.
    const int grp = lane >> 4, jj = lane & 15;
    uint32_t kaddr[2][D / 16];
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int s = 0; s < D / 16; s++) {
            const int key = kt * 32 + (lane & 31);
            kaddr[kt][s] = (uint32_t)(key * ROWB + (((2 * s + g4) ^ swz_k<D>(key)) * 16));
        }
    uint32_t vaddr[DP / 32];
    const int vrow0 = 4 * g4 + (jj >> 2);  // + 16 t + 8 h
#pragma unroll
    for (int dt = 0; dt < DP / 32; dt++) {
        const int d = dt * 32 + 16 * (grp & 1) + 4 * (jj & 3);
        const int dd = d < D ? d : 0;
        vaddr[dt] = (uint32_t)(BKEY * ROWB + vrow0 * ROWB + ((((dd >> 3) ^ swz_v<D>(vrow0)) << 4) + (dd & 7) * 2));
    }

    float m = PREFILL ? -1e30f : -INFINITY;  // running max of raw scores
    float mc = PREFILL ? -1e30f * c2 : -INFINITY;  // the same, times c2
    // FOLD: p = exp2(c2 s - mc) with mc the running max of the scaled scores
    // (0 until a block sets it), and the score MFMAs start from nm = -mc.
    if constexpr (FOLD) mc = 0.0f;
    float16v nm = float16v{};
    float lsum = 0.0f;
    bool have_m = false;  // a block's max has set m
    float16v acc[DP / 32];
#pragma unroll
    for (int i = 0; i < DP / 32; i++) acc[i] = float16v{};
    const half2v ones = {(half_t)1.0f, (half_t)1.0f};

    const int kend = min(q0 + BQW, a.S);
    const int kbeg = PREFILL ? (max(a.starts[q0], 0) / BKEY) * BKEY : 0;  // a negative start reads no memory before K/V
    const int nblk = kbeg < kend ? (kend - kbeg + BKEY - 1) / BKEY : 0;
    const int nit = (nblk + KS - 1) / KS;
    if (nit > 0) issue(0, 0, kbeg, nblk);
    for (int it = 0; it < nit; it++) {
        const int b = it * KS + ks, j = kbeg + b * BKEY;  // this wavefront's block
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's loads of the iteration are in LDS
        __syncthreads();                     // everyone's; and the last iteration's reads of the other stage are done
        if (it + 1 < nit) issue(it + 1, (it + 1) & 1, kbeg, nblk);
        const char* st_base = lds + (ks * 2 + (it & 1)) * STAGE;
        // O^T += V^T P^T over the block's 4 k-steps.
        auto pv = [&](const half8 (&pk)[4]) {
#pragma unroll
            for (int dt = 0; dt < DP / 32; dt++) {
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    half8 vop;
                    if (D < 32 && (grp & 1)) {
                        vop = half8{};  // V^T rows D .. 31 of the padded tile
                    } else {
                        const char* pvp = st_base + vaddr[dt] + 16 * t * ROWB;
                        const half4 lo = lds_read_tr(pvp), hi = lds_read_tr(pvp + 8 * ROWB);
                        vop = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                    }
                    acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, pk[t], acc[dt], 0, 0, 0);
                }
            }
        };
        const bool active = b < nblk && j <= qw + 31 && qw < a.S;  // some key of this block <= some query of the wave
        if (!active) continue;
        // Keys masked off: above the diagonal, past S and (prefill) before the
        // row's own start. Key = j + 4 g + off_r with off_r a constant of the
        // register, so each test is one compare against a per-lane limit.
        const bool edge = PREFILL || j + BKEY - 1 > qw || j + BKEY > a.S;
        const int hi_lim = min(myq, a.S - 1) - j - 4 * g4;                 // keep off_r <= hi_lim
        const int lo_lim = PREFILL ? my_start - j - 4 * g4 : -(1 << 30);  // keep off_r >= lo_lim
        auto mask = [&](float16v& t, int kt) {
            if (!edge) return;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int off = kt * 32 + 8 * (r >> 2) + (r & 3);
                bool keep = off <= hi_lim;
                if (PREFILL) keep = keep && off >= lo_lim;
                t[r] = keep ? t[r] : -INFINITY;
            }
        };
        if constexpr (FOLD) {
            // One 32-key tile at a time: S^T - mc (its MFMAs start from nm),
            // masked, exponentiated; the second tile's MFMAs can run under
            // the first's exponentials, and only one tile of scores is live.
            auto tile = [&](int kt) {
                float16v t = nm;
#pragma unroll
                for (int s2 = 0; s2 < D / 16; s2++) {
                    const half8 kop = *reinterpret_cast<const half8*>(st_base + kaddr[kt][s2]);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop, qop[s2], t, 0, 0, 0);
                }
                mask(t, kt);
                return t;
            };
            half8 pk[4];
            auto exps2 = [&](const float16v& t, int kt) {
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int tt = 2 * kt + u;
#pragma unroll
                    for (int hh = 0; hh < 8; hh++) pk[tt][hh] = (half_t)__builtin_amdgcn_exp2f(t[8 * u + hh]);
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        lsum = __builtin_amdgcn_fdot2(half2v{pk[tt][2 * e], pk[tt][2 * e + 1]}, ones, lsum, false);
                }
            };
            bool redo = !have_m;
            if (have_m) {
                const float l0 = lsum;
                exps2(tile(0), 0);
                exps2(tile(1), 1);
                if (__builtin_amdgcn_ballot_w64(__builtin_isinf(lsum)) != 0) {
                    lsum = l0;
                    redo = true;
                }
            }
            if (redo) {
                // Both tiles again, the block's largest exponent relative to
                // mc (-inf where every key of the row is masked); lazy
                // rescaling: mc moves only when it would grow by more than
                // 2^LAZY (the first block sets it where it has a key).
                float16v t0 = tile(0), t1 = tile(1);
                float mb = -INFINITY;
#pragma unroll
                for (int r = 0; r < 16; r++) mb = fmaxf(mb, fmaxf(t0[r], t1[r]));
                mb = fmaxf(mb, xor32(mb));
                const bool grow = have_m ? mb > LAZY : mb > -INFINITY;
                if (__builtin_amdgcn_ballot_w64(grow) != 0) {
                    const float dm = have_m ? fmaxf(mb, 0.0f) : (mb > -INFINITY ? mb : 0.0f);
                    if (have_m) {
                        const float alpha = __builtin_amdgcn_exp2f(-dm);
                        lsum *= alpha;
#pragma unroll
                        for (int dt = 0; dt < DP / 32; dt++) acc[dt] *= alpha;
                    }
                    t0 -= dm;
                    t1 -= dm;
                    mc += dm;
#pragma unroll
                    for (int r = 0; r < 16; r++) nm[r] = -mc;
                }
                have_m = true;
                exps2(t0, 0);
                exps2(t1, 1);
            }
            pv(pk);
            continue;
        }
        // S^T = K Q^T for the 64 keys x this wave's 32 queries (two 32-key tiles).
        float16v st[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            st[kt] = float16v{};
#pragma unroll
            for (int s = 0; s < D / 16; s++) {
                const half8 kop = *reinterpret_cast<const half8*>(st_base + kaddr[kt][s]);
                st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop, qop[s], st[kt], 0, 0, 0);
            }
        }
#pragma unroll
        for (int kt = 0; kt < 2; kt++) mask(st[kt], kt);
        // P = exp2(s c2 - m c2), rounded to f16 as the .tl's f16(p); row sums
        // from the f16 pairs. Then O^T += V^T P^T over the block's 4 k-steps.
        half8 pk[4];
        auto exps = [&]() {
#pragma unroll
            for (int t = 0; t < 4; t++) {
#pragma unroll
                for (int hh = 0; hh < 8; hh++)
                    pk[t][hh] = (half_t)__builtin_amdgcn_exp2f(__builtin_fmaf(st[t >> 1][8 * (t & 1) + hh], c2, -mc));
#pragma unroll
                for (int e = 0; e < 4; e++)
                    lsum = __builtin_amdgcn_fdot2(half2v{pk[t][2 * e], pk[t][2 * e + 1]}, ones, lsum, false);
            }
        };
        // The running max is taken from the scores only when it must move:
        // p is exponentiated against the current one, and only a score that
        // outgrew it by 2^16 (an f16 p, and so the row sum, infinite) sends
        // the block back through the max below. The first block always goes
        // there. acc / l does not depend on which max was used.
        bool redo = !have_m;
        if (have_m) {
            const float l0 = lsum;
            exps();
            if (__builtin_amdgcn_ballot_w64(__builtin_isinf(lsum)) != 0) {
                lsum = l0;
                redo = true;
            }
        }
        if (redo) {
            float mb = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) mb = fmaxf(mb, st[kt][r]);
            mb = fmaxf(mb, xor32(mb));
            // Lazy rescaling: the running max moves only when it would grow
            // by more than 2^LAZY.
            const bool grow = mb * c2 > mc + LAZY;
            if (__builtin_amdgcn_ballot_w64(grow) != 0) {
                const float mn = fmaxf(m, mb);
                const float mcn = mn * c2;
                if (have_m) {  // before the first block acc and lsum are zero
                    const float alpha = __builtin_amdgcn_exp2f(mc - mcn);
                    lsum *= alpha;
#pragma unroll
                    for (int dt = 0; dt < DP / 32; dt++) acc[dt] *= alpha;
                }
                m = mn;
                mc = mcn;
            }
            have_m = true;
            exps();
        }
        pv(pk);
    }

    if constexpr (KS > 1) {
        // Merge the KS states of each query group through LDS (the stages are
        // idle): the max of the scaled running maxima, then the sums rescaled
        // to it, in wavefront order. Lane layouts agree, so lane by lane.
        float* st = reinterpret_cast<float*>(lds);  // [4 waves][NF][64]
        static_assert(4 * NF * 64 * 4 <= LDSB, "merge area");
        __syncthreads();
        {
            float* me = st + wave * NF * 64 + lane;
            me[0] = FOLD && !have_m ? -INFINITY : mc;  // (FOLD: no block, no weight in the merge)
            me[64] = lsum;
#pragma unroll
            for (int dt = 0; dt < DP / 32; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) me[(2 + 16 * dt + r) * 64] = acc[dt][r];
        }
        __syncthreads();
        if (ks != 0) return;
        float M = mc;
#pragma unroll
        for (int k = 1; k < KS; k++) M = fmaxf(M, st[(wave + k) * NF * 64 + lane]);
        if (M == -INFINITY) M = 0.0f;  // no key anywhere (rows past S): every factor below is 0
        float L = 0.0f;
#pragma unroll
        for (int dt = 0; dt < DP / 32; dt++) acc[dt] = float16v{};
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const float* o = st + (wave + k) * NF * 64 + lane;
            const float f = __builtin_amdgcn_exp2f(o[0] - M);
            L += o[64] * f;
#pragma unroll
            for (int dt = 0; dt < DP / 32; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[dt][r] += o[(2 + 16 * dt + r) * 64] * f;
        }
        lsum = L;
    }
    const DivBy by_l(lsum + xor32(lsum));  // l >= 1: the row's largest p is 1 or more
    if (myq < a.S) {
        u16* o = a.O + (long)myq * a.q_row + (long)h * a.q_head;
#pragma unroll
        for (int dt = 0; dt < DP / 32; dt++)
#pragma unroll
            for (int rg = 0; rg < 4; rg++) {
                const int d = dt * 32 + 8 * rg + 4 * g4;
                if (d >= D) continue;
                const half4 y = {(half_t)by_l(acc[dt][4 * rg]), (half_t)by_l(acc[dt][4 * rg + 1]),
                                 (half_t)by_l(acc[dt][4 * rg + 2]), (half_t)by_l(acc[dt][4 * rg + 3])};
                *reinterpret_cast<half4*>(o + d) = y;
            }
    }
}


template <bool PREFILL, int KS, bool FOLD>
int run_attn_ks(AttnArgs a, int D, hipStream_t s, const char* what) {
    dim3 grid(((a.S + BQ / KS - 1) / (BQ / KS)) * a.H);
    switch (D) {
        case 16: hipLaunchKernelGGL((attn_fwd<16, PREFILL, KS, FOLD>), grid, dim3(256), 0, s, a); break;
        case 32: hipLaunchKernelGGL((attn_fwd<32, PREFILL, KS, FOLD>), grid, dim3(256), 0, s, a); break;
        case 64: hipLaunchKernelGGL((attn_fwd<64, PREFILL, KS, FOLD>), grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL((attn_fwd<128, PREFILL, KS, FOLD>), grid, dim3(256), 0, s, a); break;
        default: return tsl_fail(-2, std::string(what) + ": head dimension " + std::to_string(D) +
                                         " unsupported (16, 32, 64 or 128)");
    }
    return TSL_LAUNCHED(what);
}

template <bool PREFILL>
int run_attn(AttnArgs a, int D, hipStream_t s, const char* what) {
    if (a.S == 0 || a.H == 0) return 0;
    a.ncu = num_cus();
    // Key split 2 when 128-query workgroups would not give every CU a second
    // one (H32 D64: S <= 1024 139 / 335 against 108 / 266 TFLOP/s at S 512 /
    // 1024; the packed 2 x 512 prefill 201 against 165). Beyond that the
    // split's halved K/V reuse costs more than the shorter critical path
    // gains (S=4096: 659 against 779), and a split of 4 (its stages fill the
    // LDS, one workgroup per CU) loses everywhere.
    const long wgs = (long)((a.S + BQ - 1) / BQ) * a.H;
    if (wgs <= a.ncu) return run_attn_ks<PREFILL, 2, false>(a, D, s, what);
    return run_attn_ks<PREFILL, 1, true>(a, D, s, what);
}

}  // namespace

int prepare_attention(TslKernel& k) {
    int64_t D = k.dim("D");
    if (D != 16 && D != 32 && D != 64 && D != 128)
        return tsl_fail(-2, k.name + ": head dimension " + std::to_string(D) + " unsupported (16, 32, 64 or 128)");
    if (k.name == "prefill_attention" && k.dim("H") % k.dim("G") != 0)
        return tsl_fail(-2, "prefill_attention: H must be a multiple of G");
    // K and V are read through 32-bit buffer ranges: a head's rows must span
    // less than 4 GiB.
    const int64_t row = k.name == "prefill_attention" ? k.dim("G") * D : D;
    if (k.dim("S") * row * 2 >= (int64_t(1) << 32))
        return tsl_fail(-2, k.name + ": K/V rows span 4 GiB or more (S x row too large)");
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
