// fp16 GEMMs on CDNA4 matrix cores (f32 accumulation): matmul
// (kernels/matmul.tl:3-17, C = A B with B [K, N]), the llm.tl projections
// X W^T (linear :28-36, linear_residual :39-47, logits :50-58, gate_up
// :62-73) and matmul.tl's biased linear (:30-38).
//
// One workgroup computes a BM x BN tile of C. Each K step of BK stages the
// A tile and the B tile in LDS as rows of BK contiguous k values (the
// layout both MFMA operands read: 8 consecutive k per lane), XOR-swizzled
// by 16-byte chunk so that the rows an MFMA operand read touches fall in
// distinct banks, and double-buffered: the next tile's global loads are in
// flight while the current one feeds the MFMAs. The tiled kernels
// (gemm_pp16, gemm_big, the skinny forms) issue v_mfma_f32_16x16x32_f16,
// which the matrix cores sustain at a higher clock on random data than
// v_mfma_f32_32x32x16_f16; gemm_f16 (any shape and alignment) keeps the
// 32x32x16 form and stages through registers. Out-of-range rows and k read
// as zero and out-of-range outputs are dropped, which is the interpreter's
// rule (src/interp.rs:93-117, :296-313).
#include "common.h"

#include <algorithm>
#include <type_traits>

bool reduce_rmsnorm_fits(int C);
int run_reduce_rmsnorm(const float* part, int S, float* R, const u16* W, u16* Y, int M, int C, float eps,
                       hipStream_t s);
int run_rmsnorm_f32(const float* X, const u16* W, u16* Y, int M, int C, int ncols, float eps, hipStream_t s);

namespace {

constexpr int NUM_XCD = 8;

TSL_DEV u32x4 ldg16(const u16* p) { return *reinterpret_cast<const u32x4*>(p); }

// 8 consecutive elements of a row starting at column c (zeros past n).
TSL_DEV u32x4 load_chunk(const u16* row, int c, int n, bool vec) {
    if (vec && c + 8 <= n) return ldg16(row + c);
    u32x4 r = {0, 0, 0, 0};
    for (int e = 0; e < 8; e++) {
        uint32_t v = (c + e < n) ? row[c + e] : 0;
        r[e >> 1] |= v << (16 * (e & 1));
    }
    return r;
}

template <int KC>
TSL_DEV int swz(int row, int c) {
    constexpr int LG = KC == 8 ? 3 : (KC == 4 ? 2 : 1);
    return c ^ ((row ^ (row >> LG)) & (KC - 1));
}

enum Epi { EPI_F16 = 0, EPI_F32 = 1, EPI_RESID = 2, EPI_BIAS = 3, EPI_SWIGLU = 4, EPI_ROPE = 5 };

// gate_up's SwiGLU, silu(g) u = g / (1 + exp(-g)) u, for an output rounded
// to f16: exp as one v_exp_f32 of -g log2(e) and the division as a
// reciprocal (each within a few f32 ulp of expf / IEEE division, far below
// the f16 rounding that follows; expf and the division expand to ~20
// instructions). g -> -inf gives exp2 = inf, a reciprocal of 0 and -0, as
// the division does.
TSL_DEV float silu_mul(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// The fused QKV projection's epilogue (EPI_ROPE): llm.tl rope_q and kv_write
// applied to the projection's f16-rounded outputs (column layout of QKV:
// H query heads, G key heads, G value heads of D columns each).
struct RopeEpi {
    const int *pos = nullptr, *slot = nullptr;
    const float *Cs = nullptr, *Sn = nullptr;
    u16 *Q = nullptr, *Kc = nullptr, *Vc = nullptr, *K = nullptr, *V = nullptr;
    int H = 0, G = 0, D = 0, D2 = 0, NS = 0, NPOS = 0;
};

// C tile mapping: workgroups are dispatched round-robin over the 8 XCDs, so
// the id is first regrouped to give each XCD a contiguous run of tiles, and
// the run is walked G tile-rows at a time (kernels/matmul.tl:8-13) so tiles
// resident together share A rows and B columns in that XCD's L2.
TSL_DEV void tile_of(int bid, int nwg, int tiles_m, int tiles_n, int G, int& tm, int& tn) {
    int pid = bid;
    if (nwg % NUM_XCD == 0) pid = (bid % NUM_XCD) * (nwg / NUM_XCD) + bid / NUM_XCD;
    int width = G * tiles_n;
    int first = (pid / width) * G;
    int rows = min(tiles_m - first, G);
    tm = first + (pid % width) % rows;
    tn = (pid % width) / rows;
}

template <int BM, int BN, int BK, int WGM, int WGN, bool BT, int EPI>
__global__ __launch_bounds__(WGM* WGN * 64, 1) void gemm_f16(const u16* __restrict__ A, const u16* __restrict__ B,
                                                             const u16* __restrict__ B2, void* __restrict__ C,
                                                             const u16* __restrict__ bias, int M, int N, int K,
                                                             int G) {
    constexpr int NT = WGM * WGN * 64;
    constexpr int KC = BK / 8;            // 16-byte chunks per LDS row
    constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
    constexpr int TM = WM / 32, TN = WN / 32;    // MFMA tiles per wave
    constexpr bool DUAL = EPI == EPI_SWIGLU;
    constexpr int CA = BM * KC / NT;      // A chunks per thread
    static_assert(CA * NT == BM * KC, "A tile must split evenly");
    constexpr int NBLK = (BK / 8) * (BN / 8);  // 8x8 blocks of a [K, N] B tile
    constexpr int CB = BT ? BN * KC / NT : (NBLK + NT - 1) / NT;  // B chunks (or blocks) per thread
    static_assert(!BT || CB * NT == BN * KC, "B tile must split evenly");
    static_assert(!DUAL || BT, "gate_up reads W [F, K]");

    __shared__ u32x4 lds_a[2][BM * KC];
    __shared__ u32x4 lds_b[2][BN * KC];
    __shared__ u32x4 lds_b2[DUAL ? 2 : 1][DUAL ? BN * KC : 1];
    TSL_POISON(lds_a); TSL_POISON(lds_b); TSL_POISON(lds_b2);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, G, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const bool veck = (K % 8) == 0, vecn = (N % 8) == 0;

    u32x4 ra[CA], rb[BT ? CB : CB * 8], rb2[DUAL ? CB : 1];

    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; i++) {
            int c = tid + i * NT, row = c / KC, kc = c % KC;
            int gr = m0 + row;
            ra[i] = gr < M ? load_chunk(A + (size_t)gr * K, k0 + kc * 8, K, veck) : u32x4{0, 0, 0, 0};
        }
        if constexpr (BT) {
#pragma unroll
            for (int i = 0; i < CB; i++) {
                int c = tid + i * NT, row = c / KC, kc = c % KC;
                int gr = n0 + row;
                rb[i] = gr < N ? load_chunk(B + (size_t)gr * K, k0 + kc * 8, K, veck) : u32x4{0, 0, 0, 0};
                if constexpr (DUAL)
                    rb2[i] = gr < N ? load_chunk(B2 + (size_t)gr * K, k0 + kc * 8, K, veck) : u32x4{0, 0, 0, 0};
            }
        } else {
#pragma unroll
            for (int i = 0; i < CB; i++) {
                int blk = tid + i * NT, nc = blk % (BN / 8), kg = blk / (BN / 8);
#pragma unroll
                for (int r = 0; r < 8; r++) {
                    int k = k0 + kg * 8 + r;
                    rb[i * 8 + r] = (blk < NBLK && k < K) ? load_chunk(B + (size_t)k * N, n0 + nc * 8, N, vecn)
                                                          : u32x4{0, 0, 0, 0};
                }
            }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CA; i++) {
            int c = tid + i * NT, row = c / KC, kc = c % KC;
            lds_a[buf][row * KC + swz<KC>(row, kc)] = ra[i];
        }
        if constexpr (BT) {
#pragma unroll
            for (int i = 0; i < CB; i++) {
                int c = tid + i * NT, row = c / KC, kc = c % KC;
                lds_b[buf][row * KC + swz<KC>(row, kc)] = rb[i];
                if constexpr (DUAL) lds_b2[buf][row * KC + swz<KC>(row, kc)] = rb2[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < CB; i++) {
                int blk = tid + i * NT, nc = blk % (BN / 8), kg = blk / (BN / 8);
                if (blk >= NBLK) continue;
#pragma unroll
                for (int j = 0; j < 8; j++) {  // column n0 + nc*8 + j: its 8 k values
                    u32x4 o;
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        uint32_t lo = rb[i * 8 + 2 * p][j >> 1], hi = rb[i * 8 + 2 * p + 1][j >> 1];
                        o[p] = (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
                    }
                    int row = nc * 8 + j;
                    lds_b[buf][row * KC + swz<KC>(row, kg)] = o;
                }
            }
        }
    };

    float16v acc[TM][TN], acc2[DUAL ? TM : 1][DUAL ? TN : 1];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            acc[i][j] = float16v{};
            if constexpr (DUAL) acc2[i][j] = float16v{};
        }

    const int nk = (K + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
        for (int s = 0; s < BK / 16; s++) {
            const int c = s * 2 + (lane >> 5);
            half8 av[TM], bv[TN], bv2[DUAL ? TN : 1];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                int row = wm0 + i * 32 + (lane & 31);
                av[i] = __builtin_bit_cast(half8, lds_a[buf][row * KC + swz<KC>(row, c)]);
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                int row = wn0 + j * 32 + (lane & 31);
                bv[j] = __builtin_bit_cast(half8, lds_b[buf][row * KC + swz<KC>(row, c)]);
                if constexpr (DUAL) bv2[j] = __builtin_bit_cast(half8, lds_b2[buf][row * KC + swz<KC>(row, c)]);
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
                    if constexpr (DUAL)
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv2[j], acc2[i][j], 0, 0, 0);
                }
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // D layout of a 32x32 MFMA: lane l, register r holds row
    // 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int col = n0 + wn0 + j * 32 + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= M) continue;
                const size_t o = (size_t)row * N + col;
                const float v = acc[i][j][r];
                if constexpr (EPI == EPI_F16) {
                    reinterpret_cast<u16*>(C)[o] = f2h(v);
                } else if constexpr (EPI == EPI_F32) {
                    reinterpret_cast<float*>(C)[o] = v;
                } else if constexpr (EPI == EPI_RESID) {
                    float* R = reinterpret_cast<float*>(C);
                    R[o] = R[o] + v;
                } else if constexpr (EPI == EPI_BIAS) {
                    reinterpret_cast<u16*>(C)[o] = f2h(v + h2f(bias[col]));
                } else {
                    const float u = acc2[i][j][r];
                    reinterpret_cast<u16*>(C)[o] = f2h(silu_mul(v, u));
                }
            }
        }
}

// ---------------------------------------------------------------- the large-tile path
// For K % 8 == 0 (and N % 8 == 0 when B is [K, N]): 256 x 256 x 64 tiles,
// 8 wavefronts of 128 x 64. Tiles move global -> LDS with 16-byte buffer
// loads that write LDS directly (no VGPR staging; lane i of a load lands at
// the load's LDS base + 16 i, so the XOR swizzle is applied by choosing which
// global chunk each lane fetches). Rows past M/N and k past K read as zero
// (buffer range checking; a chunk past K is sent out of range explicitly).
// A (and W [N, K]) is read as MFMA operands with ds_read_b128; B [K, N] stays
// row-major in LDS and is read with ds_read_b64_tr_b16, which hands lane i
// of each 16-lane group column n0 + i of 4 consecutive k rows: the B
// operand's 8 k values per lane come from two such reads, no transpose pass.
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 fp16x4_t;

constexpr uint32_t RSRC_FLAGS = 0x00020000;  // gfx9 buffer resource word 3
constexpr int OOB = 0x7fffffff;              // a byte offset past any range

typedef int i32x4 __attribute__((ext_vector_type(4)));

// s_waitcnt immediate for vmcnt(n) alone (6-bit vmcnt: bits 3:0 and 15:14).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0f70; }

// A buffer resource (base, byte range, gfx9 flags) for buffer loads.
TSL_DEV i32x4 make_rsrc(const void* p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    return i32x4{(int)(uint32_t)a, (int)(uint32_t)((a >> 32) & 0xffff), (int)bytes, (int)RSRC_FLAGS};
}

TSL_DEV half4 lds_read_tr(const u16* p) {
    fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) fp16x4_t*)(p));
    return __builtin_bit_cast(half4, v);
}

// The epilogue of one 16x16 accumulator tile (lane l: column col = .. + l % 16,
// register r: row row0 + 4 (l / 16) + r) for the plain epilogues.
template <int EPI>
TSL_DEV void store_acc16(void* C, const u16* bias, int M, int N, int row0, int col, int g, const float4v& acc) {
    if (col >= N) return;
    float old[EPI == EPI_RESID ? 4 : 1];
    if constexpr (EPI == EPI_RESID) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = row0 + 4 * g + r;
            old[r] = row < M ? reinterpret_cast<const float*>(C)[(size_t)row * N + col] : 0.0f;
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int row = row0 + 4 * g + r;
        if (row >= M) continue;
        const size_t o = (size_t)row * N + col;
        const float v = acc[r];
        if constexpr (EPI == EPI_F16) {
            reinterpret_cast<u16*>(C)[o] = f2h(v);
        } else if constexpr (EPI == EPI_F32) {
            reinterpret_cast<float*>(C)[o] = v;
        } else if constexpr (EPI == EPI_RESID) {
            reinterpret_cast<float*>(C)[o] = old[r] + v;
        } else if constexpr (EPI == EPI_BIAS) {
            reinterpret_cast<u16*>(C)[o] = f2h(v + h2f(bias[col]));
        }
    }
}

// The compute of a K step is software pipelined: the MFMA operands of
// 32-k substep s+1 are read from LDS while the MFMAs of substep s run.
//
// LDS is served 16 lanes per cycle for 16-byte reads and 32 lanes for 8-byte
// ones, so the swizzles keep every such lane group on distinct banks: A row r
// holds logical chunk c at chunk c ^ ((r >> 1) & 7) (16 consecutive rows of an
// operand read cover all 16 slots of the 256-byte bank window); B row k (NN)
// holds logical chunk c at c ^ (4 (k & 3) + 2 ((k >> 3) & 1)), so the two
// 16-lane groups a transposed read serves together (4 k rows each, 8 apart,
// over the same 16 columns) touch 16 distinct 16-byte slots.
//
// With SPLIT, gridDim.y = S slices of K: workgroup (t, ks) runs the ks-th of S
// slices of the K steps and leaves its f32 sums in part[ks][p][m][n] (p: gate,
// up) for skinny_reduce, which adds the slices in order and applies the
// epilogue.
template <bool BT, int EPI, int BM, int BN, int WGM, int WGN, int BK, int NS, bool SPLIT = false>
__global__ __launch_bounds__(WGM* WGN * 64, 1) void gemm_big(const u16* __restrict__ A, const u16* __restrict__ B,
                                                             const u16* __restrict__ B2, void* __restrict__ C,
                                                             const u16* __restrict__ bias, int M, int N, int K,
                                                             int G, float* __restrict__ part = nullptr) {
    constexpr int KC = BK / 8;                    // 16-byte chunks per LDS row of A (and W)
    static_assert((BK == 64 || BK == 32) && NS >= 2 && NS <= 4, "k step and stages");
    constexpr int NW = WGM * WGN;                 // wavefronts: WGM x WGN, each (BM/WGM) x (BN/WGN)
    constexpr int WM = BM / WGM, WN = BN / WGN;
    // v_mfma_f32_16x16x32_f16 on 16 x 16 tiles (lane l: row / column l % 16,
    // k 8 (l / 16) .. +7 of a 32-k substep; gemm_pp16's layout and B swizzle),
    // which the matrix cores sustain at a higher clock on random data than the
    // v_mfma_f32_32x32x16_f16 form this kernel had (prefill-sized products:
    // down 1024x2048x5632 41.8 -> 39.7 us, gate_up 1024x5632x2048 50.7 -> 48.6,
    // qkv 21.6 -> 21.1).
    constexpr int MT = 16;                        // MFMA tile edge
    constexpr int TM = WM / MT, TN = WN / MT;     // MFMA tiles per wave
    constexpr int KSUB = 32, NSUB = BK / KSUB;    // k per substep, substeps per K step
    typedef float4v AccT;
    constexpr int LPA = BM * BK / 512 / NW, LPB = BN * BK / 512 / NW;  // 1 KB loads per wave per K step
    constexpr int RPL = 512 / BN;                 // B [K, N] rows per 1 KB load
    constexpr int RPA = 512 / BK;                 // A (W) rows per 1 KB load
    constexpr bool DUAL = EPI == EPI_SWIGLU;      // gate_up: B and B2 share A
    static_assert(TM >= 1 && TN >= 1 && LPA >= 1 && LPB >= 1 && (BT || BN >= 128) && (BT || !DUAL), "tile shape");
    constexpr int BB = BN * BK * 2;               // bytes of one B tile
    constexpr int STAGE = BM * BK * 2 + (DUAL ? 2 : 1) * BB;  // bytes per stage: A [BM][BK], then B (, B2)
    constexpr int LPS = LPA + (DUAL ? 2 : 1) * LPB;          // loads per wave per stage
    __shared__ __attribute__((aligned(16))) u16 lds[NS * STAGE / 2];
    TSL_POISON(lds);
    // Row r of an A (W) tile holds logical 16-byte chunk c at c ^ sw(r).
    auto sw = [](int r) { return KC == 8 ? (r >> 1) & 7 : (r >> 2) & 3; };
    auto bsw = [](int k) { return ((k & 3) << 2) | (((k >> 3) & 1) << 1); };  // B [K, N] rows

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, (M + BM - 1) / BM, (N + BN - 1) / BN, G, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const uint32_t lds_base = (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t*)lds);

    // This wave's LPA + LPB loads per K step (for A, then B), each filling 1 KB of
    // a stage. Per-lane byte offsets are relative to the K step's first
    // column (A, W) or row (B): the buffer base advances with k instead, in
    // scalar registers. OOB marks a row or column outside the matrix.
    uint32_t offa[LPA], offb[LPB];
    int ka[LPA], kb[LPB];  // the k this lane's chunk starts at, within the step (for a partial last step)
#pragma unroll
    for (int i = 0; i < LPA; i++) {
        const int q = wave * LPA + i;
        const int r = RPA * q + lane / KC;
        const int c = (lane % KC) ^ sw(r);
        ka[i] = 8 * c;
        offa[i] = m0 + r < M ? (uint32_t)(((m0 + r) * K + 8 * c) * 2) : (uint32_t)OOB;
    }
#pragma unroll
    for (int i = 0; i < LPB; i++) {
        const int q = wave * LPB + i;
        if constexpr (BT) {
            const int r = RPA * q + lane / KC;
            const int c = (lane % KC) ^ sw(r);
            kb[i] = 8 * c;
            offb[i] = n0 + r < N ? (uint32_t)(((n0 + r) * K + 8 * c) * 2) : (uint32_t)OOB;
        } else {
            const int rk = RPL * q + lane / (BN / 8);  // k row of the step
            const int cb = (lane % (BN / 8)) ^ bsw(rk);
            const int n = n0 + 8 * cb;
            kb[i] = rk;
            offb[i] = n < N ? (uint32_t)((rk * N + n) * 2) : (uint32_t)OOB;
        }
    }
    auto issue = [&](int k0, int stage) {
        // Resources whose base is the step's first column (A) / row (B).
        const long a_shift = (long)k0 * 2, b_shift = BT ? (long)k0 * 2 : (long)k0 * N * 2;
        const i32x4 ra = make_rsrc(reinterpret_cast<const char*>(A) + a_shift, (uint32_t)((long)M * K * 2 - a_shift));
        const uint32_t b_range = (uint32_t)((BT ? (long)N * K : (long)K * N) * 2 - b_shift);
        const i32x4 rb = make_rsrc(reinterpret_cast<const char*>(B) + b_shift, b_range);
        const i32x4 rb2 = make_rsrc(reinterpret_cast<const char*>(DUAL ? B2 : B) + b_shift, b_range);
        const uint32_t sa = lds_base + stage * STAGE + wave * LPA * 1024;
        const uint32_t sb = lds_base + stage * STAGE + BM * BK * 2 + wave * LPB * 1024;
        if (k0 + BK <= K) {  // every k of the step exists (uniform)
#pragma unroll
            for (int i = 0; i < LPA; i++)
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(sa + i * 1024),
                             "v"(offa[i]), "s"(ra));
#pragma unroll
            for (int i = 0; i < LPB; i++)
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(sb + i * 1024),
                             "v"(offb[i]), "s"(rb));
            if constexpr (DUAL)
#pragma unroll
                for (int i = 0; i < LPB; i++)
                    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(sb + BB + i * 1024),
                                 "v"(offb[i]), "s"(rb2));
        } else {
#pragma unroll
            for (int i = 0; i < LPA; i++) {
                const uint32_t v = k0 + ka[i] < K ? offa[i] : (uint32_t)OOB;
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(sa + i * 1024),
                             "v"(v), "s"(ra));
            }
#pragma unroll
            for (int i = 0; i < LPB; i++) {
                const uint32_t v = k0 + kb[i] < K ? offb[i] : (uint32_t)OOB;
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(sb + i * 1024),
                             "v"(v), "s"(rb));
                if constexpr (DUAL)
                    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(sb + BB + i * 1024),
                                 "v"(v), "s"(rb2));
            }
        }
    };

    // LDS byte addresses of this lane's operands in stage 0: A at k-step s,
    // tile i: a_addr[s] + 4096 i; B (NN) tile j: b_addr[j] + (16 s + 4 h) 512.
    const int l16 = lane & 15, g16 = lane >> 4;
    const int lr = l16, kg = g16;  // operand row / column in the tile, k group
    uint32_t a_addr[NSUB], b_addr[TN];
#pragma unroll
    for (int st = 0; st < NSUB; st++) {
        const int r = wm0 + lr;
        a_addr[st] = (uint32_t)((r * KC + ((4 * st + kg) ^ sw(r))) * 16);
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
        if constexpr (BT) {
            const int r = wn0 + j * MT + lr;
            b_addr[j] = (uint32_t)(BM * BK * 2 + r * KC * 16);
        } else {
            const int jj = lane & 15;
            const int n = wn0 + j * 16 + 4 * (jj & 3);
            const int k = 8 * g16 + (jj >> 2);
            b_addr[j] = (uint32_t)(BM * BK * 2 + k * BN * 2 + ((((n >> 3) ^ bsw(k)) << 3) + (n & 7)) * 2);
        }
    }
    const char* ldsc = reinterpret_cast<const char*>(lds);
    auto read_ops = [&](int so, int st, half8* av, half8* bv, half8* bv2) {
#pragma unroll
        for (int i = 0; i < TM; i++) av[i] = *reinterpret_cast<const half8*>(ldsc + so + a_addr[st] + i * MT * BK * 2);
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if constexpr (BT) {
                const int r = wn0 + j * MT + lr;
                const int cb = so + b_addr[j] + (((4 * st + kg) ^ sw(r)) * 16);
                bv[j] = *reinterpret_cast<const half8*>(ldsc + cb);
                if constexpr (DUAL) bv2[j] = *reinterpret_cast<const half8*>(ldsc + cb + BB);
            } else {
                const half4 h0 = lds_read_tr(reinterpret_cast<const u16*>(ldsc + so + b_addr[j] + (KSUB * st) * BN * 2));
                const half4 h1 = lds_read_tr(reinterpret_cast<const u16*>(ldsc + so + b_addr[j] + (KSUB * st + 4) * BN * 2));
                bv[j] = __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        }
    };

    AccT acc[TM][TN], acc2[DUAL ? TM : 1][DUAL ? TN : 1];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = AccT{};
    if constexpr (DUAL)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc2[i][j] = AccT{};
    auto mfma = [](const half8& x, const half8& y, const AccT& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(x, y, c, 0, 0, 0);
    };

    // NS stages in a ring, NS - 1 k steps in flight: iteration kt waits for
    // step kt (this wave's loads of later steps may still run), syncs (every
    // wave's loads have landed, and step kt-1's reads of its stage are done),
    // then refills that stage with step kt + NS - 1.
    const int nsteps = (K + BK - 1) / BK, S = SPLIT ? gridDim.y : 1, ks = SPLIT ? blockIdx.y : 0;
    const int kbeg = (int)((long)ks * nsteps / S), nk = (int)((long)(ks + 1) * nsteps / S) - kbeg;
    for (int p = 0; p < NS - 1 && p < nk; p++) issue((kbeg + p) * BK, p);
    half8 a0[TM], b0[TN], a1[TM], b1[TN], c0[DUAL ? TN : 1], c1[DUAL ? TN : 1];
    int stage = 0;
    for (int kt = 0; kt < nk; kt++) {
        const int ahead = min(NS - 2, nk - 1 - kt);  // steps after kt already issued
        if (ahead <= 0) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
        else if (ahead == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(LPS));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * LPS));
        __syncthreads();
        if (kt + NS - 1 < nk) issue((kbeg + kt + NS - 1) * BK, stage == 0 ? NS - 1 : stage - 1);
        const int so = stage * STAGE;
        stage = stage + 1 == NS ? 0 : stage + 1;
        read_ops(so, 0, a0, b0, c0);
#pragma unroll
        for (int st = 0; st < NSUB; st++) {
            half8* av = (st & 1) ? a1 : a0;
            half8* bv = (st & 1) ? b1 : b0;
            half8* cv = (st & 1) ? c1 : c0;
            if (st + 1 < NSUB) read_ops(so, st + 1, (st & 1) ? a0 : a1, (st & 1) ? b0 : b1, (st & 1) ? c0 : c1);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    acc[i][j] = mfma(av[i], bv[j], acc[i][j]);
                    if constexpr (DUAL) acc2[i][j] = mfma(av[i], cv[j], acc2[i][j]);
                }
        }
        // Pin the schedule: step 0's operand reads, then per k-step the next
        // step's reads spread over its first MFMAs, the rest back to back.
        constexpr int NRD = BT ? TM + (DUAL ? 2 : 1) * TN : TM + 2 * TN;  // LDS reads per k-step
        constexpr int NMF = (DUAL ? 2 : 1) * TM * TN;                    // MFMAs per k-step
        __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);
#pragma unroll
        for (int st = 0; st < NSUB; st++) {
            if (st + 1 < NSUB) {
#pragma unroll
                for (int t = 0; t < NRD / 2; t++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, NMF - NRD / 2, 0);
            } else {
                __builtin_amdgcn_sched_group_barrier(0x008, NMF, 0);
            }
        }
    }

#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int row0 = m0 + wm0 + i * MT, col = n0 + wn0 + j * MT + lr;
            if constexpr (!SPLIT && !DUAL) {
                store_acc16<EPI>(C, bias, M, N, row0, col, g16, acc[i][j]);
                continue;
            }
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = row0 + 4 * g16 + r;
                if (row >= M) continue;
                const size_t o = (size_t)row * N + col;
                const float v = acc[i][j][r];
                if constexpr (SPLIT) {
                    const size_t mn = (size_t)M * N;
                    float* pp = part + (size_t)ks * (DUAL ? 2 : 1) * mn + o;
                    pp[0] = v;
                    if constexpr (DUAL) pp[mn] = acc2[DUAL ? i : 0][DUAL ? j : 0][r];
                } else {
                    const float u = acc2[DUAL ? i : 0][DUAL ? j : 0][r];
                    reinterpret_cast<u16*>(C)[o] = f2h(silu_mul(v, u));
                }
            }
        }
}

// Large products as a ping-pong of two wavefront groups (K % (64 NH) == 0).
// 8 wavefronts of (BM/2) x (BN/4) (256 x 256: 128 x 64); group
// 0 (waves 0-3) and group 1 (waves 4-7) put one wavefront on each SIMD and
// take turns, separated by workgroup barriers: while one group runs a
// phase's MFMAs back to back from registers, the other reads its next
// phase's operands from LDS into registers. A phase covers NH steps of 64 k
// (each stage holds NH halves laid out as gemm_big's 64-k stages, same
// swizzles), so a phase keeps the matrix cores busy long enough for the
// other group's reads. Group 0 also loads the A tile of the next phase and
// group 1 the B tile of the phase after that, so the direct-to-LDS writes
// are spread over both groups' read phases. Two stages.
//
// Phase p (between barriers p and p + 1): group 0 reads step p/2 (p even)
// or computes step (p-1)/2 (p odd); group 1 is one phase behind. A stage's
// A (B) tile is rewritten only after both groups' reads of its previous step,
// and every load has landed (its issuing wave's vmcnt, then a barrier) before
// the phase that reads it: A of step s + 1 is issued at the start of group
// 0's read of step s and waited for at the end of its compute of step s; B
// of step s + 2 is issued by group 1 right after its read of step s and
// waited for at the end of its read of step s + 1.
//
// The MFMAs are v_mfma_f32_16x16x32_f16: on random f16 operands the matrix
// cores sustain ~1.85 PFLOP/s in this form against ~1.62 in the 32x32x16
// form (a quarter of the accumulator registers read and written per MFMA;
// the clock falls less). Each wavefront holds (WM/16) x (WN/16) tiles of
// 16 x 16; a 64-k half is two 32-k substeps. Operands: lane l holds row (A)
// or column (B) l % 16 and k 8 (l / 16) .. +7 of the substep. B [K, N] rows
// carry the swizzle chunk ^ bsw(k), bsw(k) = 4 (k & 3) + 2 ((k >> 3) & 1):
// the two 16-lane groups a transposed read serves together (k rows 8 apart,
// the same 16 columns) land on distinct banks. 4096^3: 1254-1262 -> 1355-1358
// TFLOP/s, 2048^3 (128 x 128, NH = 2): 737-742 -> 773-775 against the same
// ping-pong on 32x32x16 MFMAs, same box.
template <bool BT, int EPI, int BM = 256, int BN = 256, int NH = 1>
__global__ __launch_bounds__(512, 1) void gemm_pp16(const u16* __restrict__ A, const u16* __restrict__ B,
                                                    void* __restrict__ C, const u16* __restrict__ bias, int M, int N,
                                                    int K, int G) {
    constexpr int BK = 64, WGN = 4, KC = BK / 8;
    constexpr int WM = BM / 2, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
    constexpr int LP = BM * BK / 512 / 4;
    static_assert(BM == BN && TM >= 1 && TN >= 1 && (BT || BN >= 128), "tile shape");
    constexpr int RPL = 512 / BN, RPA = 512 / BK;
    constexpr int HALF = (BM + BN) * BK * 2;  // bytes of one 64-k half: A [BM][64], then B
    constexpr int STAGE = NH * HALF;
    constexpr int SUB = 2 * NH;  // 32-k substeps per phase
    __shared__ __attribute__((aligned(16))) u16 lds[2 * STAGE / 2];
    TSL_POISON(lds);
    auto sw = [](int r) { return (r >> 1) & 7; };
    auto bsw = [](int k) { return ((k & 3) << 2) | (((k >> 3) & 1) << 1); };

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wave >> 2, w4 = wave & 3;
    const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, (M + BM - 1) / BM, (N + BN - 1) / BN, G, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int l16 = lane & 15, g16 = lane >> 4;
    const uint32_t lds_base = (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t*)lds);

    uint32_t off[LP];
#pragma unroll
    for (int i = 0; i < LP; i++) {
        const int q = w4 * LP + i;
        if (grp == 0 || BT) {
            const int r = RPA * q + lane / KC, c = (lane % KC) ^ sw(r);
            const int lim = grp == 0 ? M - m0 : N - n0, base = grp == 0 ? m0 : n0;
            off[i] = r < lim ? (uint32_t)(((base + r) * K + 8 * c) * 2) : (uint32_t)OOB;
        } else {
            const int rk = RPL * q + lane / (BN / 8), cb = (lane % (BN / 8)) ^ bsw(rk), n = n0 + 8 * cb;
            off[i] = n < N ? (uint32_t)((rk * N + n) * 2) : (uint32_t)OOB;
        }
    }
    auto issue = [&](int k0, int stage) {
        const bool a = grp == 0;
#pragma unroll
        for (int h = 0; h < NH; h++) {
            const int k = k0 + BK * h;
            const long shift = a || BT ? (long)k * 2 : (long)k * N * 2;
            const char* base = reinterpret_cast<const char*>(a ? A : B) + shift;
            i32x4 rs = make_rsrc(base, (uint32_t)((a ? (long)M * K : (long)N * K) * 2 - shift));
#pragma unroll
            for (int c = 0; c < 4; c++) rs[c] = __builtin_amdgcn_readfirstlane(rs[c]);
            const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_base + stage * STAGE + h * HALF +
                                                                (a ? 0 : BM * BK * 2) + w4 * LP * 1024);
#pragma unroll
            for (int i = 0; i < LP; i++)
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(dst + i * 1024),
                             "v"(off[i]), "s"(rs));
        }
    };

    // LDS byte addresses (stage 0) of this lane's operands: A tile i at
    // a_addr[st] + i 16 rows; B tile j at b_addr[j] (+ the substep's k).
    uint32_t a_addr[2], b_addr[TN];
#pragma unroll
    for (int st = 0; st < 2; st++) {
        const int r = wm0 + l16;
        a_addr[st] = (uint32_t)((r * KC + ((4 * st + g16) ^ sw(r))) * 16);
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
        if constexpr (BT) {
            b_addr[j] = (uint32_t)(BM * BK * 2 + (wn0 + j * 16 + l16) * KC * 16);
        } else {
            const int n = wn0 + j * 16 + 4 * (l16 & 3), k = 8 * g16 + (l16 >> 2);
            b_addr[j] = (uint32_t)(BM * BK * 2 + k * BN * 2 + ((((n >> 3) ^ bsw(k)) << 3) + (n & 7)) * 2);
        }
    }
    const char* ldsc = reinterpret_cast<const char*>(lds);
    half8 av[SUB][TM], bv[SUB][TN];
    auto read_step = [&](int stage) {
#pragma unroll
        for (int u = 0; u < SUB; u++) {
            const int so = stage * STAGE + (u >> 1) * HALF, st = u & 1;
#pragma unroll
            for (int i = 0; i < TM; i++)
                av[u][i] = *reinterpret_cast<const half8*>(ldsc + so + a_addr[st] + i * 16 * BK * 2);
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if constexpr (BT) {
                    const int r = wn0 + j * 16 + l16;
                    bv[u][j] = *reinterpret_cast<const half8*>(ldsc + so + b_addr[j] + (((4 * st + g16) ^ sw(r)) * 16));
                } else {
                    const u16* p = reinterpret_cast<const u16*>(ldsc + so + b_addr[j] + 32 * st * BN * 2);
                    bv[u][j] = __builtin_shufflevector(lds_read_tr(p), lds_read_tr(p + 4 * BN), 0, 1, 2, 3, 4, 5, 6, 7);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        __builtin_amdgcn_sched_barrier(0);
    };
    float4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = float4v{};
    auto compute = [&]() {
#pragma unroll
        for (int u = 0; u < SUB; u++)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u][i], bv[u][j], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto bar = [] {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };

    constexpr int PK = BK * NH;  // k per phase
    const int nk = K / PK;
    issue(0, 0);
    __builtin_amdgcn_s_waitcnt(0x0f70);
    bar();
    if (grp == 0) {
        for (int s = 0; s < nk; s++) {
            if (s + 1 < nk) issue((s + 1) * PK, (s + 1) & 1);
            read_step(s & 1);
            bar();
            compute();
            __builtin_amdgcn_s_waitcnt(0x0f70);
            bar();
        }
    } else {
        if (nk > 1) issue(PK, 1);
        bar();
        for (int s = 0; s < nk; s++) {
            read_step(s & 1);
            if (s + 2 < nk) {
                issue((s + 2) * PK, s & 1);
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(LP * NH));
            } else {
                __builtin_amdgcn_s_waitcnt(0x0f70);
            }
            bar();
            compute();
            if (s + 1 < nk) bar();
        }
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            store_acc16<EPI>(C, bias, M, N, m0 + wm0 + i * 16, n0 + wn0 + j * 16 + l16, g16, acc[i][j]);
}

// matmul_f32 (kernels/matmul.tl:19-27): f32 operands through LDS, f32 FMA.
__global__ __launch_bounds__(256) void matmul_f32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                         float* __restrict__ C, int M, int N, int K) {
    __shared__ float As[16][64 + 1], Bs[16][64 + 1];
    TSL_POISON(As); TSL_POISON(Bs);
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += 16) {
        for (int e = threadIdx.x; e < 16 * 64; e += 256) {
            int kk = e / 64, mm = e % 64;
            As[kk][mm] = (m0 + mm < M && k0 + kk < K) ? A[(size_t)(m0 + mm) * K + k0 + kk] : 0.0f;
            Bs[kk][mm] = (n0 + mm < N && k0 + kk < K) ? B[(size_t)(k0 + kk) * N + n0 + mm] : 0.0f;
        }
        __syncthreads();
        for (int kk = 0; kk < 16; kk++)
            for (int i = 0; i < 4; i++)
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(As[kk][ty * 4 + i], Bs[kk][tx * 4 + j], acc[i][j]);
        __syncthreads();
    }
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) {
            int r = m0 + ty * 4 + i, c = n0 + tx * 4 + j;
            if (r < M && c < N) C[(size_t)r * N + c] = acc[i][j];
        }
}

// ---------------------------------------------------------------- the skinny path
// Y = X W^T with few rows (M <= 64: the engine's decode steps) is a stream of
// W, N x K x 2 bytes, so it is laid out for bandwidth: a workgroup of 8
// wavefronts owns 16 rows of W and the wavefronts take interleaved 64-wide
// steps of K, so a workgroup reads neighbouring 128-byte segments of the same
// rows together. An MFMA operand load is 16 rows x 64 contiguous bytes (4
// lanes a row), the two halves of a row's 128-byte segment in consecutive
// loads, and
//   Y^T (16 n x 16 m) += W (16 n x 32 k) X^T (32 k x 16 m)
// runs on v_mfma_f32_16x16x32_f16, one 16-row tile of X per MT. The 8
// partial tiles are summed in LDS in wavefront order (deterministic), then
// the epilogue writes Y. Needs K % 64 == 0; rows past M or N read as zero and
// their outputs are dropped. This register-operand form serves K % 128 != 0;
// otherwise gemm_skinny_lds (below) stages both operands in LDS with whole
// 128-byte lines per load, which streams W about 1.5x faster.
constexpr int SK_WAVES = 8;

// The epilogue of one output (m, n): v = (X W^T)[m, n], u its SwiGLU partner.
template <int EPI>
TSL_DEV void sk_store(void* C, const u16* bias, int N, int m, int n, float v, float u) {
    const size_t o = (size_t)m * N + n;
    if constexpr (EPI == EPI_F16) {
        reinterpret_cast<u16*>(C)[o] = f2h(v);
    } else if constexpr (EPI == EPI_F32) {
        reinterpret_cast<float*>(C)[o] = v;
    } else if constexpr (EPI == EPI_RESID) {
        float* R = reinterpret_cast<float*>(C);
        R[o] = R[o] + v;
    } else if constexpr (EPI == EPI_BIAS) {
        reinterpret_cast<u16*>(C)[o] = f2h(v + h2f(bias[n]));
    } else {
        reinterpret_cast<u16*>(C)[o] = f2h(silu_mul(v, u));
    }
}

// RT 16-row tiles of W per workgroup (one X load feeds all of them); with
// SPLIT, workgroup (b, ks) covers the ks-th of gridDim.y slices of the K
// steps and leaves its sums in part[ks][p][m][n] (p: gate, up) for
// skinny_reduce.
template <int EPI, int MT, int RT, bool SPLIT>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_skinny(const u16* __restrict__ X, const u16* __restrict__ W,
                                                               const u16* __restrict__ W2, void* C,
                                                               const u16* __restrict__ bias, int M, int N, int K,
                                                               float* __restrict__ part) {
    constexpr bool DUAL = EPI == EPI_SWIGLU;
    constexpr int NW = DUAL ? 2 * RT : RT;  // W tiles per step (gate rows then up rows)
    constexpr int NACC = NW * MT;
    __shared__ float red[SK_WAVES][4][64];
    TSL_POISON(red);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * 16 * RT;
    const int row = lane & 15, g = lane >> 4;
    const u16* wp[NW];
    bool nok[NW];
#pragma unroll
    for (int r = 0; r < NW; r++) {
        const int n = n0 + 16 * (r % RT) + row;
        nok[r] = n < N;
        wp[r] = (DUAL && r >= RT ? W2 : W) + (size_t)(nok[r] ? n : 0) * K + 8 * g;
    }
    const u16* xp[MT];
    bool mok[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        mok[t] = 16 * t + row < M;
        xp[t] = X + (size_t)(mok[t] ? 16 * t + row : 0) * K + 8 * g;
    }
    float4v acc[NACC];  // [W tile][m tile]
#pragma unroll
    for (int i = 0; i < NACC; i++) acc[i] = float4v{};
    const u32x4 z = {0, 0, 0, 0};
    const int nst = K / 64, S = SPLIT ? gridDim.y : 1, ks = SPLIT ? blockIdx.y : 0;
    const int st_hi = (int)((long)(ks + 1) * nst / S);
    constexpr int U = 2;  // steps in flight per wavefront
    auto step = [&](const u32x4 (&w)[NW][2], const u32x4 (&x)[MT][2]) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < NW; r++)
#pragma unroll
                for (int t = 0; t < MT; t++)
                    acc[r * MT + t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(half8, w[r][i]), __builtin_bit_cast(half8, x[t][i]), acc[r * MT + t], 0, 0,
                        0);
    };
    auto load = [&](int kb, u32x4 (&w)[NW][2], u32x4 (&x)[MT][2]) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int r = 0; r < NW; r++) w[r][i] = nok[r] ? ldg16(wp[r] + kb + 32 * i) : z;
#pragma unroll
            for (int t = 0; t < MT; t++) x[t][i] = mok[t] ? ldg16(xp[t] + kb + 32 * i) : z;
        }
    };
    int st = (int)((long)ks * nst / S) + wave;
    for (; st + SK_WAVES * (U - 1) < st_hi; st += SK_WAVES * U) {
        u32x4 w[U][NW][2], x[U][MT][2];
#pragma unroll
        for (int u = 0; u < U; u++) load(64 * (st + SK_WAVES * u), w[u], x[u]);
#pragma unroll
        for (int u = 0; u < U; u++) step(w[u], x[u]);
    }
    for (; st < st_hi; st += SK_WAVES) {  // the remaining steps, one at a time
        u32x4 w[NW][2], x[MT][2];
        load(64 * st, w, x);
        step(w, x);
    }
    // Sum the 8 partial tiles, one accumulator at a time through LDS; thread
    // tid < 256 keeps element tid (register tid/64 of lane tid%64) of each.
    float sum[NACC];
#pragma unroll
    for (int i = 0; i < NACC; i++) {
        if (i) __syncthreads();
#pragma unroll
        for (int r = 0; r < 4; r++) red[wave][r][lane] = acc[i][r];
        __syncthreads();
        float v = 0.0f;
        if (tid < 256)
#pragma unroll
            for (int w = 0; w < SK_WAVES; w++) v += red[w][tid >> 6][tid & 63];
        sum[i] = v;
    }
    if (tid >= 256) return;
    // Element (r, l) of tile (rt, t): output n = n0 + 16 rt + 4 (l/16) + r, m = 16 t + l%16.
    const int r = tid >> 6, l = tid & 63;
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int n = n0 + 16 * rt + 4 * (l >> 4) + r, m = 16 * t + (l & 15);
            if (m >= M || n >= N) continue;
            const float v = sum[rt * MT + t], u = DUAL ? sum[(RT + rt) * MT + t] : 0.0f;
            if constexpr (SPLIT) {
                constexpr int NP = DUAL ? 2 : 1;
                float* pp = part + (size_t)ks * NP * M * N + (size_t)m * N + n;
                pp[0] = v;
                if constexpr (DUAL) pp[(size_t)M * N] = u;
            } else {
                sk_store<EPI>(C, bias, N, m, n, v, u);
            }
        }
}

// The skinny product with both operands staged in LDS (K % 128 == 0). A
// workgroup owns a block of 16 rows of W (gate_up: 8 rows of Wg and the same
// 8 rows of Wu) over a slice of at most SL_KS k values:
// - each wavefront takes interleaved 64-wide k steps;
// - W: at the start, every step of the block at once, each wavefront loading
//   its own steps' rows (8 rows x 128 bytes, whole lines, per direct-to-LDS
//   load), so a wavefront starts as soon as its first step has landed;
// - X: a step's X rows (16 MT x 128 bytes, 8 whole lines per load) into the
//   wavefront's own LDS ring of XD stages;
// - in both, chunk c (16 bytes) of row r sits at position c ^ ((r >> 1) & 7),
//   so the 16 rows an operand read touches fall in distinct bank groups.
// Y^T (16 n x 16 m) += W (16 n x 32 k) X^T (32 k x 16 m) on
// v_mfma_f32_16x16x32_f16; the 8 partial tiles are summed in LDS in
// wavefront order, then the epilogue (or the split layout of gemm_skinny).
// EPI_ROPE pairs rows the same way inside W: block b holds rotary pairs
// 8 b .. 8 b + 7 (pair p: column h D + i and its partner h D + D2 + i, with
// h = p / D2, i = p % D2), so N counts pairs and the epilogue rotates them.
constexpr int SL_KS = 2816;  // 22 x 128: K = 5632 in two slices (256 workgroups at N = 2048, one round)

// Rotary pair n of token m from its two projection sums: QKV's f16 rounding,
// then llm.tl rope_q (query heads) or kv_write (key heads rotated, value
// heads copied), with the arithmetic of rope_q_elem / kv_write_elem (c, s
// from rope_cs); y1 goes to column n % D2 of its head, y2 to column
// D2 + n % D2.
// The rotation's cos and sin for pair n at position p (zeros outside the
// tables; value heads are not rotated).
TSL_DEV void rope_cs(const RopeEpi& ep, int p, int n, float& c, float& s) {
    const bool use = n / ep.D2 < ep.H + ep.G && p >= 0 && p < ep.NPOS;
    const int i = n % ep.D2;
    c = use ? ep.Cs[(size_t)p * ep.D2 + i] : 0.0f;
    s = use ? ep.Sn[(size_t)p * ep.D2 + i] : 0.0f;
}
TSL_DEV void rope_pair(const RopeEpi& ep, int n, float v1, float v2, float c, float s, u16& y1, u16& y2) {
    const int h = n / ep.D2;
    const u16 b1 = f2h(v1), b2 = f2h(v2);
    if (h < ep.H + ep.G) {
        rope_rotate(h2f(b1), h2f(b2), c, s, y1, y2);
    } else {
        y1 = b1;
        y2 = b2;
    }
}

// The 16 rotated halves of a block (8 pairs of head h from column i0) for
// token m, as two 16-byte runs: Q rows, or K / V rows and the paged cache at
// slot[m] when it is in [0, NS).
TSL_DEV void rope_row_store(const RopeEpi& ep, int m, int h, int i0, int half, int at, u32x4 v) {
    const int c = half * ep.D2 + i0;
    if (h < ep.H) {
        *reinterpret_cast<u32x4*>(ep.Q + ((size_t)m * ep.H + h) * ep.D + c) = v;
        return;
    }
    const bool key = h < ep.H + ep.G;
    const int g = key ? h - ep.H : h - ep.H - ep.G;
    u16* row = key ? ep.K : ep.V;
    u16* cache = key ? ep.Kc : ep.Vc;
    *reinterpret_cast<u32x4*>(row + ((size_t)m * ep.G + g) * ep.D + c) = v;
    if (at >= 0 && at < ep.NS) *reinterpret_cast<u32x4*>(cache + ((size_t)at * ep.G + g) * ep.D + c) = v;
}

template <int MT>
constexpr int sl_xdepth() { return MT <= 2 ? 2 : 1; }
// The rows' deferred RMS normalisation (fused/linear_residual_prenorm and its
// consumers): the producer leaves Y = f16(R Wn) with R the updated residual
// and ss[b][m] = the sum of R[m][n]^2 over its 8-column block b (column
// order); a consumer takes rs[m] = 1 / sqrt(sum_b ss[b][m] / K + eps) (the
// partial sums added in a fixed order) and scales its products of row m by
// rs[m] before its epilogue: rmsnorm(R) Wn W^T = rs (R Wn) W^T.
struct NormPre {
    const u16* w = nullptr;  // producer: Wn [N]
    u16* y = nullptr;        // producer: Y [M, N]
    int* ovf = nullptr;      // producer: set to 1 when some Y overflows f16
    const float* ss = nullptr;  // consumer: [nr, M]
    int nr = 0;
    float eps = 0.0f;
};

// Thread t of a 512-thread workgroup: rs[m] into lds_rs[m] for m < M <= 32.
// Thread (q = t / 32, m = t % 32) adds partials q, q + 16, .. in order
// (loaded before the call, ssv), then m adds its 16 sums in q order.
TSL_DEV void rs_from_partials(const float (&ssv)[16], int nr, int M, int K, float eps, float* lds_sum,
                              float* lds_rs) {
    const int t = threadIdx.x, q = t >> 5;
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) a += q + 16 * i < nr ? ssv[i] : 0.0f;
    lds_sum[t] = a;
    __syncthreads();
    if (t < M) {
        float tot = 0.0f;
#pragma unroll
        for (int qq = 0; qq < 16; qq++) tot += lds_sum[qq * 32 + t];
        lds_rs[t] = 1.0f / sqrtf(tot / (float)K + eps);
    }
    __syncthreads();
}
// The partial sums thread t adds (nr <= 256), written out as loads the
// compiler does not count (issued before the caller's W loads; the caller
// waits for them with an explicit vmcnt, then fences them with
// ssv_fence).
TSL_DEV void ssv_load(const float* ss, int nr, int M, float (&ssv)[16]) {
    const int t = threadIdx.x, m = min(t & 31, M - 1), q = t >> 5;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int b = min(q + 16 * i, nr - 1);
        asm volatile("global_load_dword %0, %1, off" : "=v"(ssv[i]) : "v"(ss + (size_t)b * M + m));
    }
}
TSL_DEV void ssv_fence(float (&ssv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; i++) asm volatile("" : "+v"(ssv[i]));
}

// s_waitcnt vmcnt(n) for a run-time n (the instruction takes an immediate).
TSL_DEV void sk_vm_wait(int n) {
    switch (n) {
#define SK_VM_CASE(k) case k: __builtin_amdgcn_s_waitcnt(vmcnt_imm(k)); break;
        SK_VM_CASE(1) SK_VM_CASE(2) SK_VM_CASE(3) SK_VM_CASE(4) SK_VM_CASE(5) SK_VM_CASE(6) SK_VM_CASE(7)
        SK_VM_CASE(8) SK_VM_CASE(9) SK_VM_CASE(10) SK_VM_CASE(11) SK_VM_CASE(12) SK_VM_CASE(13) SK_VM_CASE(14)
        SK_VM_CASE(15) SK_VM_CASE(16) SK_VM_CASE(17) SK_VM_CASE(18) SK_VM_CASE(19) SK_VM_CASE(20)
#undef SK_VM_CASE
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;  // (0, or more than listed: wait for all)
    }
}

// R8 (linear_residual_prenorm, EPI_RESID): blocks of 8 rows of W over the
// whole K (up to 2 SL_KS, the same LDS); after R += Y the block writes
// np.y = f16(R np.w) for its 8 columns and the per-row sums of squares of
// the new R to part[block][m] (column order). RS (a consumer, ROPE): the
// sums of row m are scaled by rs[m] from np.ss first.
template <int EPI, int MT, bool SPLIT, bool R8 = false, bool RS = false>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_skinny_lds(const u16* __restrict__ X, const u16* __restrict__ W,
                                                                   const u16* __restrict__ W2, void* C,
                                                                   const u16* __restrict__ bias, int M, int N, int K,
                                                                   float* __restrict__ part, RopeEpi ep,
                                                                   NormPre np = {}) {
    constexpr bool ROPE = EPI == EPI_ROPE;
    constexpr bool DUAL = EPI == EPI_SWIGLU || ROPE;  // paired rows: 8 + 8 per block
    static_assert(!(ROPE && SPLIT), "the rotary epilogue needs whole sums");
    static_assert(!R8 || (EPI == EPI_RESID && !SPLIT), "8-row blocks: the residual epilogue over the whole K");
    static_assert(!RS || (ROPE && MT <= 2), "row scaling: the rotary consumer, M <= 32");
    constexpr int KSL = R8 ? 2 * SL_KS : SL_KS;  // k values per block (slice), at most
    constexpr int WB = (R8 ? 8 : 16) * KSL * 2;  // LDS bytes of the W block
    constexpr int XS = 16 * MT * 128;            // LDS bytes of one X step
    constexpr int XD = sl_xdepth<MT>();          // X stages per wavefront
    constexpr int MAXU = (KSL / 64 + SK_WAVES - 1) / SK_WAVES;  // k steps per wavefront, at most
    constexpr int XL = 2 * MT;                   // X loads per step (8 rows each)
    __shared__ __attribute__((aligned(16))) u16 lds[(WB + SK_WAVES * XD * XS) / 2];
    __shared__ __attribute__((aligned(16))) float red[SK_WAVES][4][64];
    TSL_POISON(lds); TSL_POISON(red);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row = lane & 15, g = lane >> 4;
    // Rows of this block: n0 .. n0 + 15 of W, or n0 .. n0 + 7 of Wg and of Wu.
    const int n0 = blockIdx.x * (DUAL || R8 ? 8 : 16);
    const int nb = K / 128, S = SPLIT ? gridDim.y : 1, ks = SPLIT ? blockIdx.y : 0;
    const int b0 = ks * nb / S, b1 = (ks + 1) * nb / S;
    const int k0 = 128 * b0, KS = 128 * (b1 - b0), nst = KS / 64;
    const uint32_t lds_w = (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t*)lds);
    const uint32_t lds_x = lds_w + WB + wave * XD * XS;
    // The rotary epilogue's positions and cache slots, loaded before the
    // stream; its cos and sin follow after the k loop, behind the
    // reduction's barriers.
    int rpos[ROPE ? MT : 1], rslot = -1;
    if constexpr (ROPE) {
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int m = 16 * t + (lane & 15);
            rpos[t] = m < M ? ep.pos[m] : -1;
        }
        if (tid < 2 * M) rslot = ep.slot[tid >> 1];  // the write-out's row
    }

    // The consumer's partial sums of squares, before any W load.
    float ssv[RS ? 16 : 1];
    if constexpr (RS) ssv_load(np.ss, np.nr, M, ssv);
    // R8: the epilogue's residual values and norm weights, loaded first (so
    // every wait of the stream covers them) instead of behind the reduction:
    // thread tid < 128 MT owns one output, (r, l) = ((tid % 128) / 32, tid % 32)
    // of row tile t = tid / 128: column n0 + 4 (l / 16) + r, row 16 t + l % 16.
    // Written out like the stream's loads; threads without an element read
    // column n0 of row 0.
    const int et = tid >> 7, er = (tid & 127) >> 5, el = tid & 31;  // (R8; the rotary epilogue too)
    const int ej = 4 * (el >> 4) + er, em = 16 * et + (el & 15);
    float rv = 0.0f;
    uint32_t wnv = 0;
    if constexpr (R8) {
        if (wave < 2 * MT) {  // (uniform)
            const bool ok = em < M && n0 + ej < N;
            const float* o = reinterpret_cast<const float*>(C) + (ok ? (size_t)em * N + n0 + ej : (size_t)n0);
            asm volatile("global_load_dword %0, %1, off" : "=v"(rv) : "v"(o));
            const u16* wp = np.w + (n0 + ej < N ? n0 + ej : n0);
            asm volatile("global_load_ushort %0, %1, off" : "=v"(wnv) : "v"(wp));
        }
    }
    // W block, by k step: step st (of this slice) holds the block's WR rows x
    // 64 k at lds_w + st WSB, row r at r 128 with chunk c at c ^ ((r >> 1) & 7)
    // (the X stages' layout). Each wavefront loads the steps it multiplies
    // (st = wave + 8 u), 8 rows per 1 KB load, so it waits for nobody else's
    // loads. Rows past N read as zero.
    constexpr int WR = R8 ? 8 : 16, WSB = WR * 128, WL = WR / 8;
    const int rows_n = min(DUAL || R8 ? 8 : 16, N - n0);
    const uint32_t wrange = (uint32_t)(((long)(rows_n - 1) * K + KS) * 2);
    // First rows of the block's two halves (rotary pairs: within one head of W).
    const long ra = ROPE ? (long)(n0 / ep.D2) * ep.D + n0 % ep.D2 : n0;
    const i32x4 rw = make_rsrc(W + ra * K + k0, wrange);
    const i32x4 rw2 = make_rsrc(ROPE ? W + (ra + ep.D2) * K + k0 : (DUAL ? W2 : W) + (size_t)n0 * K + k0, wrange);
    auto load_w = [&](int st) {
#pragma unroll
        for (int h = 0; h < WL; h++) {
            const int r = 8 * h + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
            const int rr = DUAL ? r & 7 : r;  // row within its matrix
            const uint32_t off = (uint32_t)((rr * K + 64 * st + 8 * c) * 2);
            if (DUAL && h == 1)  // rows 8..15: Wu (or the rotary partners)
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(lds_w + st * WSB + h * 1024),
                             "v"(off), "s"(rw2)
                             : "memory");
            else
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(lds_w + st * WSB + h * 1024),
                             "v"(off), "s"(rw)
                             : "memory");
        }
    };
    // X step st into stage slot: load j covers rows 8 j .. 8 j + 7, lane l
    // row 8 j + l / 8 at position l % 8. Rows past M read as zero.
    const i32x4 rx = make_rsrc(X, (uint32_t)((long)M * K * 2));
    auto load_x = [&](int st, int slot) {
        const int xr = lane >> 3, pos = lane & 7;
#pragma unroll
        for (int j = 0; j < XL; j++) {
            const int r = 8 * j + xr;
            const int c = pos ^ ((r >> 1) & 7);
            const uint32_t off = (uint32_t)((r * K + k0 + 64 * st + 8 * c) * 2);
            // (the clobber keeps the stage's earlier operand reads before it)
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds_x + slot * XS + j * 1024),
                         "v"(off), "s"(rx)
                         : "memory");
        }
    };
    const int mysteps = nst > wave ? (nst - wave + SK_WAVES - 1) / SK_WAVES : 0;
    // Issue order: W(0) X(0) .. W(XD-1) X(XD-1), then W(XD) .. W(mysteps-1);
    // X(u + XD) after step u's MFMAs.
#pragma unroll
    for (int u = 0; u < XD; u++)
        if (u < mysteps) {
            load_w(wave + SK_WAVES * u);
            load_x(wave + SK_WAVES * u, u);
        }
    for (int u = XD; u < mysteps; u++) load_w(wave + SK_WAVES * u);
    // Loads issued after X(u) by the time step u waits for it.
    auto after_x = [&](int u) {
        int n = 0;
        if (u < XD) {
            for (int v = u + 1; v < min(XD, mysteps); v++) n += WL + XL;
            n += WL * max(0, mysteps - XD);
        }
        for (int v = max(0, u - XD + 1); v < u; v++)
            if (v + XD < mysteps) n += XL;
        return n;
    };

    float4v acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = float4v{};
    const char* ldsc = reinterpret_cast<const char*>(lds);
    const int wr = R8 ? row & 7 : row;  // (R8: rows 8..15 repeat 0..7, sums dropped)
    const char* wrow = ldsc + wr * 128;
    const char* xbase = ldsc + WB + wave * XD * XS;
    for (int u = 0; u < MAXU; u++) {  // (a run-time trip count: not unrolled)
        if (u >= mysteps) break;
        // Wait for step u's W and X (issued before X(u)); later loads may fly.
        sk_vm_wait(after_x(u));
        asm volatile("" ::: "memory");  // no LDS read moves above the wait
        const int st = wave + SK_WAVES * u, slot = u % XD;
        const char* xs = xbase + slot * XS;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int c = 4 * i + g;
            const half8 w = *reinterpret_cast<const half8*>(wrow + st * WSB + 16 * (c ^ ((wr >> 1) & 7)));
            const int xc = 4 * i + g;
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const int r = 16 * t + row;
                const half8 x = *reinterpret_cast<const half8*>(xs + r * 128 + 16 * (xc ^ ((r >> 1) & 7)));
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, x, acc[t], 0, 0, 0);
            }
        }
        if (u + XD < mysteps) load_x(st + SK_WAVES * XD, slot);
    }
    // Sum the 8 partial tiles through LDS in wavefront order; thread tid < 256
    // keeps element tid (register tid/64 of lane tid%64) of each. All MT
    // tiles go at once into the W block's LDS, free once every wavefront's
    // MFMAs are done: [MT][wave][4][64] partials, then [MT][4][64] for the
    // partner exchange.
    static_assert(MT * (SK_WAVES + 1) * 256 * 4 <= WB, "the reduction fits the W block");
    float* rd = reinterpret_cast<float*>(lds);
    float* xc = rd + MT * SK_WAVES * 256;
    __syncthreads();  // every wavefront's W and X reads are done
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) rd[((t * SK_WAVES + wave) * 4 + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    float sum[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) {
        float v = 0.0f;
        if (!R8 && !ROPE && tid < 256)  // (R8 and the rotary epilogue sum their own elements below)
#pragma unroll
            for (int w = 0; w < SK_WAVES; w++) v += rd[(t * SK_WAVES + w) * 256 + tid];
        sum[t] = v;
    }
    // Element (r, l): block row 4 (l / 16) + r, m = 16 t + l % 16. For
    // gate_up, rows 0..7 are gate rows and 8..15 their up partners, which
    // sit 32 lanes on: exchanged through LDS.
    const int r = tid >> 6, l = tid & 63;
    float up[MT];
    if constexpr (DUAL && !ROPE) {
#pragma unroll
        for (int t = 0; t < MT; t++)
            if (tid < 256) xc[t * 256 + tid] = sum[t];
        __syncthreads();
#pragma unroll
        for (int t = 0; t < MT; t++) up[t] = tid < 256 && l < 32 ? xc[t * 256 + r * 64 + l + 32] : 0.0f;
    }
    if constexpr (ROPE) {
        // One pair per thread tid < 128 MT (the R8 epilogue's element
        // mapping: pair ej of row em), both halves summed from the reduction
        // buffer (the partner sits 32 lanes on), scaled by rs[em] (RS; the
        // ring is free: every wavefront is past the reduction's barriers).
        // The block's 8 pairs lie in one head (D2 % 8 == 0): the rotated
        // halves go through LDS, then each token row leaves as two 16-byte
        // stores (per element 2-byte stores would scatter over 16 rows).
        float f = 1.0f;
        if constexpr (RS) {
            ssv_fence(ssv);
            float* rsb = reinterpret_cast<float*>(lds + WB / 2);  // [512] sums, then [32] rs
            rs_from_partials(ssv, np.nr, M, K, np.eps, rsb, rsb + 512);
            f = em < M ? rsb[512 + em] : 0.0f;
        }
        static_assert(16 * MT * 16 * 2 <= (int)sizeof(red), "staging fits the reduction buffer");
        u16 (*yb)[16] = reinterpret_cast<u16 (*)[16]>(&red[0][0][0]);  // [16 MT][16] (red is not the reduction's)
        if (tid < 128 * MT && em < M && n0 + ej < N) {
            float v1 = 0.0f, v2 = 0.0f;
#pragma unroll
            for (int w = 0; w < SK_WAVES; w++) {
                const float* e = rd + ((et * SK_WAVES + w) * 4 + er) * 64 + el;
                v1 += e[0];
                v2 += e[32];
            }
            int p = rpos[0];
#pragma unroll
            for (int t = 1; t < MT; t++) p = et == t ? rpos[t] : p;
            float c, sn;
            rope_cs(ep, p, n0 + ej, c, sn);
            u16 y1, y2;
            rope_pair(ep, n0 + ej, v1 * f, v2 * f, c, sn, y1, y2);
            yb[em][ej] = y1;
            yb[em][8 + ej] = y2;
        }
        __syncthreads();
        const int h = n0 / ep.D2, i0 = n0 % ep.D2;
        if (tid < 2 * M)  // M <= 64: one row half per thread
            rope_row_store(ep, tid >> 1, h, i0, tid & 1, rslot, *reinterpret_cast<const u32x4*>(&yb[tid >> 1][8 * (tid & 1)]));
        return;
    }
    if constexpr (R8) {
        // R += Y for the block's 8 columns; np.y = f16(R np.w); then the
        // squares of the new values summed per row in column order (through
        // red).
        float* sq = &red[0][0][0];  // [MT][8 columns][16 rows] (red is not the reduction's)
        static_assert(MT * 8 * 16 <= SK_WAVES * 4 * 64, "squares fit the staging buffer");
        __builtin_amdgcn_s_waitcnt(0x0f70);  // (the prefetched values: landed long ago)
        asm volatile("" : "+v"(rv), "+v"(wnv));
        if (tid < 128 * MT) {
            float se = 0.0f;
#pragma unroll
            for (int w = 0; w < SK_WAVES; w++) se += rd[((et * SK_WAVES + w) * 4 + er) * 64 + el];
            const int n = n0 + ej;
            float nv = 0.0f;
            if (em < M && n < N) {
                nv = rv + se;
                reinterpret_cast<float*>(C)[(size_t)em * N + n] = nv;
                float yv = nv * h2f((u16)wnv);
                asm volatile("" : "+v"(yv));  // rounded to f32, then to f16 (no fused multiply-convert)
                const u16 yh = f2h(yv);
                np.y[(size_t)em * N + n] = yh;
                // An infinite Y from a finite R (an R that is NaN already, as
                // in the padding rows of a decode step, whose attention over
                // no keys is 0/0, is not flagged): the caller normalises first.
                if ((yh & 0x7fff) == 0x7c00) *np.ovf = 1;
            }
            sq[(et * 8 + ej) * 16 + (el & 15)] = nv * nv;
        }
        __syncthreads();
        if (tid < 16 * MT) {
            const int t = tid >> 4, mm = tid & 15, m = 16 * t + mm;
            if (m < M) {
                float a = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) a += sq[(t * 8 + j) * 16 + mm];
                part[(size_t)blockIdx.x * M + m] = a;
            }
        }
        return;
    }
    if constexpr (DUAL) {
        if (l >= 32) return;
    }
    if (tid >= 256) return;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int n = n0 + 4 * (l >> 4) + r, m = 16 * t + (l & 15);
        if (m >= M || n >= N) continue;
        const float v = sum[t], uu = DUAL ? up[t] : 0.0f;
        if constexpr (SPLIT) {
            float* pp = part + (size_t)ks * (DUAL ? 2 : 1) * M * N + (size_t)m * N + n;
            pp[0] = v;
            if constexpr (DUAL) pp[(size_t)M * N] = uu;
        } else {
            sk_store<EPI>(C, bias, N, m, n, v, uu);
        }
    }
}

// The skinny product for many row blocks (more than the CUs: gate_up,
// logits), persistent: one workgroup per CU walks blocks b, b + gridDim.x,
// ... Wavefront w always owns the same contiguous K steps (K / 512 of them,
// K = 1024 or 2048), so its X operands are loaded once into registers; per
// block it streams its 512-byte segment of each of the 16 W rows (whole
// lines, 2 rows per 1 KB direct-to-LDS load) into its own 2-slot LDS ring,
// the next block's loads in flight while it computes. Block layout, MFMA,
// reduction and epilogue are gemm_skinny_lds's (M <= 32).
//
// RS (a consumer of linear_residual_prenorm): the sums of row m are scaled by
// rs[m] from np.ss before the epilogue.
template <int EPI, int MT, bool RS = false>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_skinny_pst(const u16* __restrict__ X, const u16* __restrict__ W,
                                                                   const u16* __restrict__ W2, void* C,
                                                                   const u16* __restrict__ bias, int M, int N, int K,
                                                                   NormPre np = {}) {
    constexpr bool DUAL = EPI == EPI_SWIGLU;
    constexpr int SPW = 4;                   // most k steps per wavefront (K <= 2048)
    constexpr int SLOT = 16 * SPW * 128;     // LDS bytes of one block's segments
    static_assert(MT <= 2, "X stays in registers");
    __shared__ __attribute__((aligned(16))) u16 lds[SK_WAVES * 2 * SLOT / 2];
    // Every wavefront's partial tiles of both row tiles at once, gate_up's
    // partner exchange beside them, and the row scales' scratch: two
    // barriers per block.
    __shared__ float red[MT][SK_WAVES][4][64];
    __shared__ float xch[DUAL ? MT : 1][4][64];
    __shared__ float rsl[RS ? 512 + 32 : 1];
    TSL_POISON(lds); TSL_POISON(red); TSL_POISON(xch); TSL_POISON(rsl);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row = lane & 15, g = lane >> 4;
    const int nsw = K / 512;                 // k steps of this wavefront: nsw * wave ..
    const int kw = 64 * nsw * wave;          // its first k
    const int cpr = 8 * nsw;                 // 16-byte chunks per row segment (16 or 32)
    const int nl = 2 * nsw;                  // 1 KB loads per block
    const int rpb = DUAL ? 8 : 16;
    const int nblk = (N + rpb - 1) / rpb;
    const uint32_t ring = (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t*)lds) + wave * 2 * SLOT;

    // X operands of this wavefront's steps (rows past M are zero), loaded
    // before the W blocks. The loads are written out: the compiler counts
    // only its own loads, so its wait before the first use would also wait
    // for every W load issued after them; an explicit vmcnt below leaves the
    // W loads in flight, and each operand passes through an empty asm after
    // it, so nothing reads it earlier.
    const u32x4 z = {0, 0, 0, 0};
    float ssv[RS ? 16 : 1];
    if constexpr (RS) ssv_load(np.ss, np.nr, M, ssv);
    u32x4 xv[SPW][MT][2];
#pragma unroll
    for (int j = 0; j < SPW; j++)
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const bool ok = j < nsw && 16 * t + row < M;
            const u16* xp = X + (size_t)(ok ? 16 * t + row : 0) * K + kw + 64 * (ok ? j : 0) + 8 * g;
#pragma unroll
            for (int i = 0; i < 2; i++) asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(xv[j][t][i]) : "v"(xp + 32 * i));
        }
    // W segments of block b into ring slot: load q covers chunks 64 q ..
    // 64 q + 63 (row p / cpr, position p % cpr, holding chunk pos ^ (row & 15)).
    auto load_w = [&](int b, int slot) {
        const int n0 = b * rpb, rows = min(rpb, N - n0);
        const uint32_t range = (uint32_t)(((long)(rows - 1) * K + K - kw) * 2);
        const i32x4 rw = make_rsrc(W + (size_t)n0 * K + kw, range);
        const i32x4 rw2 = make_rsrc((DUAL ? W2 : W) + (size_t)n0 * K + kw, range);
        for (int q = 0; q < nl; q++) {
            const int p = 64 * q + lane, r = p / cpr, pos = p - r * cpr;
            const int rr = DUAL ? r & 7 : r;
            const uint32_t off = (uint32_t)((rr * K + 8 * (pos ^ (r & 15))) * 2);
            if (DUAL && q >= nl / 2)  // rows 8..15: Wu
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(ring + slot * SLOT + q * 1024),
                             "v"(off), "s"(rw2)
                             : "memory");
            else
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(ring + slot * SLOT + q * 1024),
                             "v"(off), "s"(rw)
                             : "memory");
        }
    };
    const int b0 = blockIdx.x, bs = gridDim.x;
    if (b0 < nblk) load_w(b0, 0);
    if (b0 + bs < nblk) load_w(b0 + bs, 1);
    {
        const int wl = (b0 < nblk ? nl : 0) + (b0 + bs < nblk ? nl : 0);  // W loads in flight
        if (wl == 16) __builtin_amdgcn_s_waitcnt(vmcnt_imm(16));
        else if (wl == 8) __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
        else if (wl == 4) __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
        else __builtin_amdgcn_s_waitcnt(0x0f70);
#pragma unroll
        for (int j = 0; j < SPW; j++)
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    asm volatile("" : "+v"(xv[j][t][i]));
                    if (j >= nsw || 16 * t + row >= M) xv[j][t][i] = z;
                }
    }
    float rsv[MT];  // rs of rows 16 t + row (RS; formed after the first block's MFMAs)
    if constexpr (RS) ssv_fence(ssv);
    const char* ldsc = reinterpret_cast<const char*>(lds) + wave * 2 * SLOT;
    int slot = 0;
    for (int b = b0; b < nblk; b += bs, slot ^= 1) {
        // Wait for this block's segments (the next block's may still fly).
        if (b + bs < nblk) {
            if (nl == 8) __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(4));
        } else {
            __builtin_amdgcn_s_waitcnt(0x0f70);
        }
        asm volatile("" ::: "memory");
        float4v acc[MT];
#pragma unroll
        for (int t = 0; t < MT; t++) acc[t] = float4v{};
        const char* wrow = ldsc + slot * SLOT + row * cpr * 16;
#pragma unroll
        for (int j = 0; j < SPW; j++) {
            if (j >= nsw) break;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = 8 * j + 4 * i + g;
                const half8 w = *reinterpret_cast<const half8*>(wrow + 16 * (c ^ row));
#pragma unroll
                for (int t = 0; t < MT; t++)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, __builtin_bit_cast(half8, xv[j][t][i]), acc[t], 0,
                                                                  0, 0);
            }
        }
        if constexpr (RS) {
            if (b == b0) {  // (uniform) behind the first block's MFMAs
                rs_from_partials(ssv, np.nr, M, K, np.eps, rsl, rsl + 512);
#pragma unroll
                for (int t = 0; t < MT; t++) rsv[t] = 16 * t + row < M ? rsl[512 + 16 * t + row] : 0.0f;
            }
        }
        // Sum the 8 partial tiles in wavefront order, thread tid element
        // tid % 256 of row tile tid / 256 (MT = 2: every thread one), then
        // gate_up's partner exchange and the epilogue, one output per thread.
        // The previous block's reads of red and xch are behind barriers every
        // wavefront has passed: red's behind this block's exchange barrier
        // (gate_up) or the barrier after the sums; xch's behind this block's
        // first.
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[t][wave][r][lane] = acc[t][r];
        __syncthreads();
        const int te = tid >> 8, ie = tid & 255;  // element (r, l) = (ie / 64, ie % 64) of row tile te
        const bool has = te < MT;
        float se = 0.0f;
        if (has)
#pragma unroll
            for (int w = 0; w < SK_WAVES; w++) se += red[te < MT ? te : 0][w][ie >> 6][ie & 63];
        // Element (r, l): block row 4 (l / 16) + r, m = 16 te + l % 16 (so l % 16
        // is this thread's row: rsv applies). gate_up: rows 0..7 are gate rows
        // and 8..15 their up partners, 32 lanes on.
        const int n0 = b * rpb;
        const float rs_t = [&](int t) { return RS ? (MT == 2 && t ? rsv[MT - 1] : rsv[0]) : 1.0f; }(DUAL ? tid >> 7 : te);
        if constexpr (DUAL) {
            if (has) xch[te < MT ? te : 0][ie >> 6][ie & 63] = se;
            __syncthreads();
            if (tid < 128 * MT) {  // output tid: gate element (q / 32, q % 32) of row tile tid / 128, q = tid % 128
                const int t = tid >> 7, q = tid & 127, r = q >> 5, l = q & 31;
                const int n = n0 + 4 * (l >> 4) + r, m = 16 * t + (l & 15);
                if (m < M && n < N) sk_store<EPI>(C, bias, N, m, n, xch[t][r][l] * rs_t, xch[t][r][l + 32] * rs_t);
            }
        } else {
            __syncthreads();
            if (has) {
                const int r = ie >> 6, l = ie & 63;
                const int n = n0 + 4 * (l >> 4) + r, m = 16 * te + (l & 15);
                if (m < M && n < N) sk_store<EPI>(C, bias, N, m, n, se * rs_t, 0.0f);
            }
        }
        // The block after next into the slot just read. Issued after the
        // epilogue's stores (which also count in vmcnt), so the next wait
        // leaves exactly these loads in flight.
        if (b + 2 * bs < nblk) load_w(b + 2 * bs, slot);
    }
}

// Sums the S slices of a split skinny product in slice order, then the epilogue.
template <int EPI>
__global__ __launch_bounds__(256) void skinny_reduce(const float* __restrict__ part, int S, int M, int N, void* C,
                                                     const u16* __restrict__ bias) {
    constexpr int NP = EPI == EPI_SWIGLU ? 2 : 1;
    const long e = (long)blockIdx.x * 256 + threadIdx.x, mn = (long)M * N;
    if (e >= mn) return;
    float v = 0.0f, u = 0.0f;
    for (int ks = 0; ks < S; ks++) {
        v += part[(size_t)ks * NP * mn + e];
        if constexpr (NP == 2) u += part[(size_t)ks * NP * mn + mn + e];
    }
    sk_store<EPI>(C, bias, N, (int)(e / N), (int)(e % N), v, u);
}

// The skinny path's shape plan: 16-row tiles per workgroup and K slices.
struct SkPlan {
    bool use = false;
    bool lds = false;  // gemm_skinny_lds (K % 128 == 0): slices of at most SL_KS
    int rt = 1, split = 1;
};
SkPlan sk_plan(bool bt, int M, int N, int K) {
    SkPlan p;
    if (!bt || M <= 0 || M > 64 || N <= 0 || K <= 0 || K % 64) return p;
    p.use = true;
    if (K % 128 == 0) {
        p.lds = true;
        p.split = (K / 128 + SL_KS / 128 - 1) / (SL_KS / 128);
        return p;
    }
    p.rt = N >= 4096 ? 2 : 1;
    const int blocks = (N + 16 * p.rt - 1) / (16 * p.rt), nst = K / 64;
    // K slices only pay for their extra reduce launch when K is long and the
    // row tiles alone leave most CUs idle.
    if (blocks < 256 && nst >= 64) p.split = std::max(1, std::min(512 / blocks, nst / (2 * SK_WAVES)));
    return p;
}

// K slices for the 128 x 128 tiled path when its tiles alone leave CUs idle
// (prefill-sized M): enough slices to give every CU a workgroup, each at
// least 32 K steps long (shorter slices lose more to the extra partial
// traffic and reduce launch than the idle CUs cost). 1 = no split.
int big_split(int M, int N, int K) {
    if (M <= 64 || K % 8) return 1;
    const long tiles = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (tiles >= 256 || tiles == 0) return 1;
    if ((long)((M + 63) / 64) * ((N + 63) / 64) >= 256) return 1;  // 64 x 64 tiles fill the CUs (gemm_dispatch)
    const int nst = (K + 63) / 64;
    return std::max(1, std::min((int)((256 + tiles - 1) / tiles), nst / 32));
}

// reduce = false leaves a split product's slices in part (the caller sums them).
template <int EPI, int MT, int RT>
void launch_skinny_rt(const u16* X, const u16* W, const u16* W2, void* C, const u16* bias, int M, int N, int K,
                      int split, float* part, hipStream_t s, bool reduce) {
    const unsigned blocks = (N + 16 * RT - 1) / (16 * RT);
    if (split > 1) {
        hipLaunchKernelGGL((gemm_skinny<EPI, MT, RT, true>), dim3(blocks, split), dim3(64 * SK_WAVES), 0, s, X, W, W2, C,
                           bias, M, N, K, part);
        if (!reduce) return;
        const long mn = (long)M * N;
        hipLaunchKernelGGL(skinny_reduce<EPI>, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, part, split, M, N,
                           C, bias);
    } else {
        hipLaunchKernelGGL((gemm_skinny<EPI, MT, RT, false>), dim3(blocks), dim3(64 * SK_WAVES), 0, s, X, W, W2, C,
                           bias, M, N, K, part);
    }
}

template <int EPI, int MT>
void launch_skinny(const u16* X, const u16* W, const u16* W2, void* C, const u16* bias, int M, int N, int K,
                   const SkPlan& p, float* part, hipStream_t s, bool reduce = true) {
    if (p.lds) {
        const unsigned blocks = EPI == EPI_SWIGLU ? (N + 7) / 8 : (N + 15) / 16;
        if constexpr (MT <= 2) {
            if (p.split == 1 && blocks > (unsigned)num_cus() && (K == 1024 || K == 2048)) {
                hipLaunchKernelGGL((gemm_skinny_pst<EPI, MT>), dim3(num_cus()), dim3(64 * SK_WAVES), 0, s, X, W, W2, C,
                                   bias, M, N, K);
                return;
            }
        }
        if (p.split > 1) {
            hipLaunchKernelGGL((gemm_skinny_lds<EPI, MT, true>), dim3(blocks, p.split), dim3(64 * SK_WAVES), 0, s, X, W,
                               W2, C, bias, M, N, K, part, RopeEpi{});
            if (!reduce) return;
            const long mn = (long)M * N;
            hipLaunchKernelGGL(skinny_reduce<EPI>, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, part, p.split,
                               M, N, C, bias);
        } else {
            hipLaunchKernelGGL((gemm_skinny_lds<EPI, MT, false>), dim3(blocks), dim3(64 * SK_WAVES), 0, s, X, W, W2, C,
                               bias, M, N, K, part, RopeEpi{});
        }
        return;
    }
    if (p.rt == 2) launch_skinny_rt<EPI, MT, 2>(X, W, W2, C, bias, M, N, K, p.split, part, s, reduce);
    else launch_skinny_rt<EPI, MT, 1>(X, W, W2, C, bias, M, N, K, p.split, part, s, reduce);
}

template <int EPI>
void launch_skinny_m(const u16* X, const u16* W, const u16* W2, void* C, const u16* bias, int M, int N, int K,
                     const SkPlan& p, float* part, hipStream_t s, bool reduce = true) {
    switch ((M + 15) / 16) {
        case 1: launch_skinny<EPI, 1>(X, W, W2, C, bias, M, N, K, p, part, s, reduce); break;
        case 2: launch_skinny<EPI, 2>(X, W, W2, C, bias, M, N, K, p, part, s, reduce); break;
        case 3: launch_skinny<EPI, 3>(X, W, W2, C, bias, M, N, K, p, part, s, reduce); break;
        default: launch_skinny<EPI, 4>(X, W, W2, C, bias, M, N, K, p, part, s, reduce); break;
    }
}

template <int BM, int BN, int BK, int WGM, int WGN, bool BT, int EPI>
int run_gemm(const u16* A, const u16* B, const u16* B2, void* C, const u16* bias, int M, int N, int K,
             hipStream_t s, const char* what) {
    int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (tiles == 0) return 0;
    hipLaunchKernelGGL((gemm_f16<BM, BN, BK, WGM, WGN, BT, EPI>), dim3(tiles), dim3(WGM * WGN * 64), 0, s, A, B, B2, C,
                       bias, M, N, K, 4);
    return TSL_LAUNCHED(what);
}

// Tile choice: the largest tile that still gives every CU (256 on MI355X)
// a workgroup, else the smallest.
template <bool BT, int EPI>
int gemm_dispatch(const u16* A, const u16* B, const u16* B2, void* C, const u16* bias, int M, int N, int K,
                  hipStream_t s, const char* what, float* part = nullptr) {
    auto tiles = [&](int bm, int bn) { return (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    constexpr bool DUAL = EPI == EPI_SWIGLU;
    if constexpr (BT) {
        const SkPlan p = sk_plan(true, M, N, K);
        if (p.use && (p.split == 1 || part)) {  // a weight stream: the skinny path
            launch_skinny_m<EPI>(A, B, B2, C, bias, M, N, K, p, part, s);
            return TSL_LAUNCHED(what);
        }
    }
    const bool aligned = (K % 8) == 0 && (BT || (N % 8) == 0) && (long)M * K < (1L << 30) && (long)N * K < (1L << 30);
    if constexpr (!DUAL) {
        if (tiles(256, 256) >= 224 && aligned) {
            // 8 wavefronts of 128 x 64 (2 per SIMD, 128 accumulator registers
            // each): the ping-pong form when K is whole steps, else one
            // wave's MFMAs cover the other's loads and barrier.
            if (K % 64 == 0)
                hipLaunchKernelGGL((gemm_pp16<BT, EPI>), dim3(tiles(256, 256)), dim3(512), 0, s, A, B, C, bias, M, N, K, 4);
            else
                hipLaunchKernelGGL((gemm_big<BT, EPI, 256, 256, 2, 4, 64, 2, false>), dim3(tiles(256, 256)), dim3(512), 0, s, A,
                                   B, B2, C, bias, M, N, K, 4);
            return TSL_LAUNCHED(what);
        }
    }
    if constexpr (DUAL) {
        if (aligned && M > 64 && tiles(256, 128) >= 128) {
            // 8 wavefronts of 64 x 64 x (gate, up): the 256 x 256 tile's
            // register budget, and half the workgroups of 128 x 128 tiles, so
            // prefill-sized products (M ~ 1024) fill the CUs in one round.
            hipLaunchKernelGGL((gemm_big<BT, EPI, 256, 128, 4, 2, 64, 2, false>), dim3(tiles(256, 128)), dim3(512), 0, s, A, B, B2,
                               C, bias, M, N, K, 4);
            return TSL_LAUNCHED(what);
        }
    }
    if constexpr (BT && !DUAL) {
        if (aligned && M > 64 && tiles(128, 128) < 256 && tiles(64, 64) >= 256) {
            // X W^T at prefill sizes (the engine's 1024-row qkv, o and down):
            // 128 x 64 tiles, 8 wavefronts when they make one round of
            // workgroups (one per CU), else 4 (two fit on a CU). On 16x16x32
            // MFMAs, against the 64 x 64 tiles of 4 wavefronts chosen on
            // 32x32x16 (same box): down 1024 x 2048 x 5632 39.3 -> 36.2 us,
            // o 1024 x 2048 x 2048 17.9 -> 17.5, qkv 1024 x 2560 x 2048 (320
            // tiles, 4 wavefronts) 20.9 -> 18.7; 128 x 128 and 64 x 128 were
            // slower.
            if (tiles(128, 64) <= num_cus())
                hipLaunchKernelGGL((gemm_big<BT, EPI, 128, 64, 4, 2, 64, 3, false>), dim3(tiles(128, 64)), dim3(512), 0, s, A,
                                   B, B2, C, bias, M, N, K, 4);
            else
                hipLaunchKernelGGL((gemm_big<BT, EPI, 128, 64, 2, 2, 64, 3, false>), dim3(tiles(128, 64)), dim3(256), 0, s, A,
                                   B, B2, C, bias, M, N, K, 4);
            return TSL_LAUNCHED(what);
        }
    }
    if (aligned && M > 64 && (BT || !DUAL)) {
        const int split = part ? big_split(M, N, K) : 1;
        if (split > 1) {  // 128 x 128 tiles over K slices, then the ordered sum
            hipLaunchKernelGGL((gemm_big<BT, EPI, 128, 128, 2, 2, 64, 2, true>), dim3(tiles(128, 128), split), dim3(256), 0, s, A,
                               B, B2, C, bias, M, N, K, 4, part);
            const long mn = (long)M * N;
            hipLaunchKernelGGL(skinny_reduce<EPI>, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, part, split, M,
                               N, C, bias);
        } else if (tiles(128, 128) >= 256 && !BT) {
            // matmul (B [K, N]) at 128 x 128: 8 wavefronts of 64 x 32, the
            // ping-pong form with phases of 128 k when K allows (2048^3:
            // 25.7 -> 24.8 us), else 3 stages (30.0 -> 26.5 us against 4
            // wavefronts, 2 stages).
            if (K % 128 == 0)
                hipLaunchKernelGGL((gemm_pp16<BT, EPI, 128, 128, 2>), dim3(tiles(128, 128)), dim3(512), 0, s, A, B, C, bias,
                                   M, N, K, 4);
            else
                hipLaunchKernelGGL((gemm_big<BT, EPI, 128, 128, 2, 4, 64, 3, false>), dim3(tiles(128, 128)), dim3(512), 0, s, A,
                                   B, B2, C, bias, M, N, K, 4);
        } else if (tiles(128, 128) >= 256) {
            hipLaunchKernelGGL((gemm_big<BT, EPI, 128, 128, 2, 2, 64, 2, false>), dim3(tiles(128, 128)), dim3(256), 0, s, A, B, B2,
                               C, bias, M, N, K, 4);
        } else if (!BT && tiles(64, 128) < 256 && tiles(32, 128) >= 256) {
            // matmul with too few 64 x 128 tiles to fill the CUs (1024^3):
            // 32 x 128 tiles, 4 wavefronts of 32 x 32 (9.05 -> 7.95 us).
            hipLaunchKernelGGL((gemm_big<BT, EPI, 32, 128, 1, 4, 64, 2, false>), dim3(tiles(32, 128)), dim3(256), 0, s, A, B, B2,
                               C, bias, M, N, K, 4);
        } else {  // 64 x 128 tiles (4 wavefronts of 64 x 32): twice the workgroups;
                  // X W^T keeps two K steps in flight (matmul's in-register B
                  // transpose does better with one)
            hipLaunchKernelGGL((gemm_big<BT, EPI, 64, 128, 1, 4, 64, BT ? 3 : 2, false>), dim3(tiles(64, 128)), dim3(256), 0, s, A,
                               B, B2, C, bias, M, N, K, 4);
        }
        return TSL_LAUNCHED(what);
    }
    if constexpr (!DUAL)
        if (tiles(256, 256) >= 224) return run_gemm<256, 256, 64, 2, 2, BT, EPI>(A, B, B2, C, bias, M, N, K, s, what);
    if (tiles(128, 128) >= 224 || M > 64) return run_gemm<128, 128, 64, 2, 2, BT, EPI>(A, B, B2, C, bias, M, N, K, s, what);
    if (M > 32) return run_gemm<64, 64, 64, 2, 2, BT, EPI>(A, B, B2, C, bias, M, N, K, s, what);
    return run_gemm<32, 64, 64, 1, 2, BT, EPI>(A, B, B2, C, bias, M, N, K, s, what);
}

}  // namespace

// ---------------------------------------------------------------- launchers
// Arguments arrive in .tl parameter order (src/gpu.rs:179-195).

int launch_matmul(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    return gemm_dispatch<false, EPI_F16>(P<u16>(a[0]), P<u16>(a[1]), nullptr, P<void>(a[2]), nullptr, M, N, K, s,
                                         "matmul");
}

int launch_matmul_f32(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    dim3 grid((N + 63) / 64, (M + 63) / 64);
    if (M == 0 || N == 0) return 0;
    hipLaunchKernelGGL(matmul_f32_kernel, grid, dim3(256), 0, s, P<float>(a[0]), P<float>(a[1]), P<float>(a[2]), M, N,
                       K);
    return TSL_LAUNCHED("matmul_f32");
}

// matmul.tl linear: X [M, K], W [N, K], b [N], Y [M, N].
int launch_linear_bias(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    return gemm_dispatch<true, EPI_BIAS>(P<u16>(a[0]), P<u16>(a[1]), nullptr, P<void>(a[3]), P<u16>(a[2]), M, N, K, s,
                                         "linear", reinterpret_cast<float*>(k.scratch));
}

int launch_llm_linear(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    return gemm_dispatch<true, EPI_F16>(P<u16>(a[0]), P<u16>(a[1]), nullptr, P<void>(a[2]), nullptr, M, N, K, s,
                                        "linear", reinterpret_cast<float*>(k.scratch));
}

int launch_linear_residual(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    return gemm_dispatch<true, EPI_RESID>(P<u16>(a[0]), P<u16>(a[1]), nullptr, P<void>(a[2]), nullptr, M, N, K, s,
                                          "linear_residual", reinterpret_cast<float*>(k.scratch));
}

int launch_logits(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    return gemm_dispatch<true, EPI_F32>(P<u16>(a[0]), P<u16>(a[1]), nullptr, P<void>(a[2]), nullptr, M, N, K, s,
                                        "logits", reinterpret_cast<float*>(k.scratch));
}

int launch_gate_up(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), F = k.dim("F"), K = k.dim("K");
    return gemm_dispatch<true, EPI_SWIGLU>(P<u16>(a[0]), P<u16>(a[1]), P<u16>(a[2]), P<void>(a[3]), nullptr, M, F, K,
                                           s, "gate_up", reinterpret_cast<float*>(k.scratch));
}

// fused/linear_residual_rmsnorm (the engine's fusion, not a .tl kernel):
// llm/linear_residual then llm/rmsnorm of the updated residual, arguments
// X [M, K], W [N, K], R [M, N], Wn [N], Y [M, N], eps. Few-row products run
// K-split (at least 2 slices) and one kernel adds the slices to R and
// normalises each row; with the slice count linear_residual would use, the
// bits are that pair's. Prefill-sized products that linear_residual
// splits over K (128 x 128 tiles) end in the same kernel, with the pair's
// bits too; other shapes launch the pair.
SkPlan fused_plan(int M, int N, int K, int ncols) {
    SkPlan p = sk_plan(true, M, N, K);
    if (!p.use || ncols != N || !reduce_rmsnorm_fits(N)) return SkPlan{};
    if (p.split == 1 && K / 64 >= 2 * SK_WAVES) p.split = 2;
    if (p.split == 1) return SkPlan{};
    return p;
}

int launch_linear_residual_rmsnorm(TslKernel& k, const uint64_t* a, hipStream_t s) {
    const int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    const int ncols = (int)std::min<int64_t>(k.metav("BC"), N);
    const float eps = arg_f32(a[5]);
    float* R = P<float>(a[2]);
    const SkPlan p = fused_plan(M, N, K, ncols);
    if (p.use && k.scratch) {
        float* part = reinterpret_cast<float*>(k.scratch);
        launch_skinny_m<EPI_RESID>(P<u16>(a[0]), P<u16>(a[1]), nullptr, R, nullptr, M, N, K, p, part, s, false);
        return run_reduce_rmsnorm(part, p.split, R, P<u16>(a[3]), P<u16>(a[4]), M, N, eps, s);
    }
    // Prefill-sized products that linear_residual splits over K (128 x 128
    // tiles, big_split) feed the same reduce-and-normalise kernel.
    const bool aligned = K % 8 == 0 && (long)M * K < (1L << 30) && (long)N * K < (1L << 30);
    const long tiles256 = (long)((M + 255) / 256) * ((N + 255) / 256);
    const int bsplit = k.scratch && aligned && M > 64 && tiles256 < 224 ? big_split(M, N, K) : 1;
    if (bsplit > 1 && ncols == N && reduce_rmsnorm_fits(N)) {
        const long tiles = (long)((M + 127) / 128) * ((N + 127) / 128);
        hipLaunchKernelGGL((gemm_big<true, EPI_RESID, 128, 128, 2, 2, 64, 2, true>), dim3(tiles, bsplit), dim3(256), 0, s,
                           P<u16>(a[0]), P<u16>(a[1]), nullptr, R, nullptr, M, N, K, 4,
                           reinterpret_cast<float*>(k.scratch));
        if (int e = TSL_LAUNCHED("linear_residual_rmsnorm")) return e;
        return run_reduce_rmsnorm(reinterpret_cast<float*>(k.scratch), bsplit, R, P<u16>(a[3]), P<u16>(a[4]), M, N, eps,
                                  s);
    }
    if (int e = gemm_dispatch<true, EPI_RESID>(P<u16>(a[0]), P<u16>(a[1]), nullptr, R, nullptr, M, N, K, s,
                                               "linear_residual_rmsnorm", reinterpret_cast<float*>(k.scratch)))
        return e;
    return run_rmsnorm_f32(R, P<u16>(a[3]), P<u16>(a[4]), M, N, ncols, eps, s);
}

// fused/qkv_rope_kv (the engine's fusion, not a .tl kernel): llm/linear
// QKV = X Wqkv^T, then llm/rope_q and llm/kv_write of that QKV, arguments X
// [T, Dm], Wqkv [W, Dm], QKV [T, W], pos, slot, C, S, Q, Kc, Vc, K, V (the
// kernels' own). Decode-sized batches (T <= 64, Dm % 128 == 0, Dm <= 2048,
// D = 2 D2, D2 % 8 == 0, W = (H + 2 G) D) run one skinny product whose
// epilogue rotates and stores (QKV is then left unwritten); the outputs are
// the bits the three launches give. Other shapes launch the three.
int launch_rope_kv(TslKernel& k, const uint64_t* a, hipStream_t s);
namespace {
// fused/qkv_rope_kv with X given (a[0] is not read), and with np.ss set the
// rows of X scaled by rs (fused/qkv_rs_rope_kv; T <= 32 on the fused path).
int qkv_rope_kv_run(TslKernel& k, const uint64_t* a, hipStream_t s, const u16* X, float* part, const NormPre& np) {
    const int T = k.dim("T"), W = k.dim("W"), Dm = k.dim("Dm");
    RopeEpi ep;
    ep.H = k.dim("H"), ep.G = k.dim("G"), ep.D = k.dim("D"), ep.D2 = k.dim("D2"), ep.NS = k.dim("NS");
    ep.NPOS = k.dim("NPOS");
    const SkPlan p = sk_plan(true, T, W, Dm);
    const bool fused = p.use && p.lds && p.split == 1 && ep.D == 2 * ep.D2 && ep.D2 % 8 == 0 &&
                       W == (ep.H + 2 * ep.G) * ep.D;
    if (!fused) {
        if (int e = gemm_dispatch<true, EPI_F16>(X, P<u16>(a[1]), nullptr, P<void>(a[2]), nullptr, T, W, Dm, s,
                                                 "qkv_rope_kv", part))
            return e;
        return launch_rope_kv(k, a + 2, s);
    }
    ep.pos = P<int>(a[3]), ep.slot = P<int>(a[4]), ep.Cs = P<float>(a[5]), ep.Sn = P<float>(a[6]);
    ep.Q = P<u16>(a[7]), ep.Kc = P<u16>(a[8]), ep.Vc = P<u16>(a[9]), ep.K = P<u16>(a[10]), ep.V = P<u16>(a[11]);
    const int pairs = W / 2;
    const unsigned blocks = (pairs + 7) / 8;
    const u16* Wq = P<u16>(a[1]);
    if (np.ss) {  // T <= 32
        if (T <= 16)
            hipLaunchKernelGGL((gemm_skinny_lds<EPI_ROPE, 1, false, false, true>), dim3(blocks), dim3(64 * SK_WAVES), 0,
                               s, X, Wq, nullptr, nullptr, nullptr, T, pairs, Dm, nullptr, ep, np);
        else
            hipLaunchKernelGGL((gemm_skinny_lds<EPI_ROPE, 2, false, false, true>), dim3(blocks), dim3(64 * SK_WAVES), 0,
                               s, X, Wq, nullptr, nullptr, nullptr, T, pairs, Dm, nullptr, ep, np);
        return TSL_LAUNCHED("qkv_rs_rope_kv");
    }
    auto go = [&](auto mt) {
        hipLaunchKernelGGL((gemm_skinny_lds<EPI_ROPE, decltype(mt)::value, false>), dim3(blocks), dim3(64 * SK_WAVES), 0,
                           s, X, Wq, nullptr, nullptr, nullptr, T, pairs, Dm, nullptr, ep);
    };
    switch ((T + 15) / 16) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 3: go(std::integral_constant<int, 3>{}); break;
        default: go(std::integral_constant<int, 4>{}); break;
    }
    return TSL_LAUNCHED("qkv_rope_kv");
}

// Whether the qkv product takes the fused skinny path (as qkv_rope_kv_run decides).
bool qkv_fused(TslKernel& k) {
    const int T = k.dim("T"), W = k.dim("W"), Dm = k.dim("Dm"), D = k.dim("D"), D2 = k.dim("D2");
    const SkPlan p = sk_plan(true, T, W, Dm);
    return p.use && p.lds && p.split == 1 && D == 2 * D2 && D2 % 8 == 0 && W == (k.dim("H") + 2 * k.dim("G")) * D;
}

// The fallback of the rs consumers: H[m] = f16(Y[m] rs[m]), rs from the
// partial sums in the consumers' order (16 strided sums, then those in order).
__global__ __launch_bounds__(256) void rows_rs_kernel(const u16* __restrict__ Y, const float* __restrict__ SS,
                                                      u16* __restrict__ H, int M, int K, int NB, float eps) {
    __shared__ float pr[16];
    TSL_POISON(pr);
    const int m = blockIdx.x, t = threadIdx.x;
    if (t < 16) {
        float a = 0.0f;
        for (int b = t; b < NB; b += 16) a += SS[(size_t)b * M + m];
        pr[t] = a;
    }
    __syncthreads();
    float a = 0.0f;
    for (int q = 0; q < 16; q++) a += pr[q];
    const float rs = 1.0f / sqrtf(a / (float)K + eps);
    for (int k = t; k < K; k += 256) H[(size_t)m * K + k] = f2h(h2f(Y[(size_t)m * K + k]) * rs);
}

// The prenorm producer's fallback: Y = f16(R Wn) and the per-8-column sums
// of squares, as the fused kernel computes them.
__global__ __launch_bounds__(256) void prenorm_kernel(const float* __restrict__ R, const u16* __restrict__ Wn,
                                                      u16* __restrict__ Y, float* __restrict__ SS, int* ovf, int M,
                                                      int N, int NB) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)NB * M) return;
    const int b = (int)(i / M), m = (int)(i % M);
    float a = 0.0f;
    for (int j = 0; j < 8; j++) {
        const int n = 8 * b + j;
        if (n >= N) break;
        const float v = R[(size_t)m * N + n];
        float yv = v * h2f(Wn[n]);
        asm volatile("" : "+v"(yv));  // rounded to f32, then to f16 (as the fused kernel)
        const u16 yh = f2h(yv);
        Y[(size_t)m * N + n] = yh;
        if ((yh & 0x7fff) == 0x7c00) *ovf = 1;  // infinite (not NaN), as the fused kernel
        float q = v * v;
        asm volatile("" : "+v"(q));  // the product rounded, not contracted into an fma (as in the fused kernel)
        a += q;
    }
    SS[i] = a;
}
}  // namespace

int launch_qkv_rope_kv(TslKernel& k, const uint64_t* a, hipStream_t s) {
    return qkv_rope_kv_run(k, a, s, P<u16>(a[0]), reinterpret_cast<float*>(k.scratch), NormPre{});
}

// fused/linear_residual_prenorm (the engine's fusion, not a .tl kernel):
// llm/linear_residual, R += X W^T, leaving for the next projection's rmsnorm
// Y = f16(R Wn) and SS[b][m], the sum over the 8 columns n = 8 b .. 8 b + 7
// (column order) of the new R[m][n]^2. Arguments X [M, K], W [N, K], R [M, N],
// Wn [N], Y [M, N], SS [NB, M], NB = ceil(N / 8), OVF [1]. Y overflows f16
// where |R Wn| >= 65520 although rmsnorm(R) Wn may not: then (Y infinite)
// the kernel sets OVF[0] = 1 (it never clears it) and the caller should
// normalise first
// (fused/linear_residual_rmsnorm), as the engine does.
int launch_linear_residual_prenorm(TslKernel& k, const uint64_t* a, hipStream_t s) {
    const int M = k.dim("M"), N = k.dim("N"), K = k.dim("K"), NB = k.dim("NB");
    if (NB != (N + 7) / 8) return tsl_fail(-2, "linear_residual_prenorm: NB must be ceil(N / 8)");
    if (M == 0 || N == 0) return 0;
    const u16 *X = P<u16>(a[0]), *W = P<u16>(a[1]);
    float* R = P<float>(a[2]);
    NormPre np;
    np.w = P<u16>(a[3]), np.y = P<u16>(a[4]);
    float* SS = P<float>(a[5]);
    np.ovf = P<int>(a[6]);
    if (M <= 64 && K % 128 == 0 && K > 0 && K <= 2 * SL_KS) {
        auto go = [&](auto mt) {
            hipLaunchKernelGGL((gemm_skinny_lds<EPI_RESID, decltype(mt)::value, false, true>), dim3(NB),
                               dim3(64 * SK_WAVES), 0, s, X, W, nullptr, R, nullptr, M, N, K, SS, RopeEpi{}, np);
        };
        switch ((M + 15) / 16) {
            case 1: go(std::integral_constant<int, 1>{}); break;
            case 2: go(std::integral_constant<int, 2>{}); break;
            case 3: go(std::integral_constant<int, 3>{}); break;
            default: go(std::integral_constant<int, 4>{}); break;
        }
        return TSL_LAUNCHED("linear_residual_prenorm");
    }
    if (int e = gemm_dispatch<true, EPI_RESID>(X, W, nullptr, R, nullptr, M, N, K, s, "linear_residual_prenorm", nullptr))
        return e;
    const long n = (long)NB * M;
    hipLaunchKernelGGL(prenorm_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, R, np.w, np.y, SS, np.ovf, M, N, NB);
    return TSL_LAUNCHED("linear_residual_prenorm");
}

// fused/gate_up_rs (the engine's fusion, not a .tl kernel): llm/gate_up of
// rmsnorm(R) Wn given as Y = f16(R Wn) and SS (linear_residual_prenorm):
// each row's products are scaled by rs = 1 / sqrt(sum SS / K + eps).
// Arguments Y [M, K], SS [NB, M], Wg [F, K], Wu [F, K], O [M, F], eps.
bool rs_pst_fits(int M, int F, int K, int NB) {
    return M <= 32 && (K == 1024 || K == 2048) && NB <= 256 && (F + 7) / 8 > num_cus();
}
int launch_gate_up_rs(TslKernel& k, const uint64_t* a, hipStream_t s) {
    const int M = k.dim("M"), F = k.dim("F"), K = k.dim("K"), NB = k.dim("NB");
    if (M == 0 || F == 0) return 0;
    NormPre np;
    np.ss = P<float>(a[1]), np.nr = NB, np.eps = arg_f32(a[5]);
    const u16 *Y = P<u16>(a[0]), *Wg = P<u16>(a[2]), *Wu = P<u16>(a[3]);
    u16* O = P<u16>(a[4]);
    if (rs_pst_fits(M, F, K, NB)) {
        if (M <= 16)
            hipLaunchKernelGGL((gemm_skinny_pst<EPI_SWIGLU, 1, true>), dim3(num_cus()), dim3(64 * SK_WAVES), 0, s, Y, Wg,
                               Wu, O, nullptr, M, F, K, np);
        else
            hipLaunchKernelGGL((gemm_skinny_pst<EPI_SWIGLU, 2, true>), dim3(num_cus()), dim3(64 * SK_WAVES), 0, s, Y, Wg,
                               Wu, O, nullptr, M, F, K, np);
        return TSL_LAUNCHED("gate_up_rs");
    }
    if (!k.scratch) return tsl_fail(-1, "gate_up_rs: no scratch for the scaled rows");
    u16* H = reinterpret_cast<u16*>(k.scratch);
    hipLaunchKernelGGL(rows_rs_kernel, dim3(M), dim3(256), 0, s, Y, np.ss, H, M, K, NB, np.eps);
    if (int e = TSL_LAUNCHED("gate_up_rs")) return e;
    return gemm_dispatch<true, EPI_SWIGLU>(H, Wg, Wu, O, nullptr, M, F, K, s, "gate_up_rs", nullptr);
}
int prepare_gate_up_rs(TslKernel& k) {
    const int64_t M = k.dim("M"), F = k.dim("F"), K = k.dim("K"), NB = k.dim("NB");
    if (NB != (K + 7) / 8) return tsl_fail(-2, "gate_up_rs: NB must be ceil(K / 8)");
    if (M > (1 << 20) || K > (1 << 20) || rs_pst_fits((int)M, (int)F, (int)K, (int)NB)) return 0;
    const size_t bytes = (size_t)M * K * 2;
    if (bytes == 0) return 0;
    if (tsl_hip_check(hipMalloc(&k.scratch, bytes), "gate_up_rs scratch")) return -1;
    k.scratch_bytes = bytes;
    return 0;
}

// fused/qkv_rs_rope_kv (the engine's fusion, not a .tl kernel):
// fused/qkv_rope_kv of rmsnorm(R) Wn given as Y = f16(R Wn) and SS
// (linear_residual_prenorm), its arguments then SS [NB, T], eps.
bool qkv_rs_fits(TslKernel& k) { return k.dim("T") <= 32 && k.dim("NB") <= 256 && qkv_fused(k); }
int launch_qkv_rs_rope_kv(TslKernel& k, const uint64_t* a, hipStream_t s) {
    const int T = k.dim("T"), Dm = k.dim("Dm"), NB = k.dim("NB");
    if (T == 0) return 0;
    NormPre np;
    np.ss = P<float>(a[12]), np.nr = NB, np.eps = arg_f32(a[13]);
    if (qkv_rs_fits(k)) return qkv_rope_kv_run(k, a, s, P<u16>(a[0]), nullptr, np);
    if (!k.scratch) return tsl_fail(-1, "qkv_rs_rope_kv: no scratch for the scaled rows");
    u16* H = reinterpret_cast<u16*>(k.scratch);
    hipLaunchKernelGGL(rows_rs_kernel, dim3(T), dim3(256), 0, s, P<u16>(a[0]), np.ss, H, T, Dm, NB, np.eps);
    if (int e = TSL_LAUNCHED("qkv_rs_rope_kv")) return e;
    return qkv_rope_kv_run(k, a, s, H, nullptr, NormPre{});
}
int prepare_qkv_rs_rope_kv(TslKernel& k) {
    if (k.dim("NB") != (k.dim("Dm") + 7) / 8) return tsl_fail(-2, "qkv_rs_rope_kv: NB must be ceil(Dm / 8)");
    if (qkv_rs_fits(k)) return 0;
    const size_t bytes = (size_t)k.dim("T") * k.dim("Dm") * 2;
    if (bytes == 0) return 0;
    if (tsl_hip_check(hipMalloc(&k.scratch, bytes), "qkv_rs_rope_kv scratch")) return -1;
    k.scratch_bytes = bytes;
    return 0;
}

// Sizes the split-K partials (the skinny path at decode-sized M, the 128 x 128
// path at prefill-sized M) once, when the kernel is specialised: split x (2
// for gate_up) x M x N floats.
int prepare_projection(TslKernel& k) {
    const bool dual = k.name == "gate_up", qkv = k.name == "qkv_rope_kv";
    const int64_t M = qkv ? k.dim("T") : k.dim("M"), K = qkv ? k.dim("Dm") : k.dim("K");
    const int64_t N = dual ? k.dim("F") : qkv ? k.dim("W") : k.dim("N");
    if (M > (1 << 20) || N > (1 << 30)) return 0;
    SkPlan p = sk_plan(true, (int)M, (int)N, (int)K);
    if (k.name == "linear_residual_rmsnorm") {
        const SkPlan f = fused_plan((int)M, (int)N, (int)K, (int)std::min<int64_t>(k.metav("BC"), N));
        if (f.use) p = f;
    }
    const int split = p.use ? p.split : big_split((int)M, (int)N, (int)K);
    if (split == 1) return 0;
    const size_t bytes = (size_t)split * (dual ? 2 : 1) * M * N * sizeof(float);
    if (tsl_hip_check(hipMalloc(&k.scratch, bytes), "projection split-K scratch")) return -1;
    k.scratch_bytes = bytes;
    return 0;
}
