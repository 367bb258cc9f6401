// fp16 GEMMs on CDNA4 matrix cores (v_mfma_f32_32x32x16_f16, f32
// accumulation): matmul (kernels/matmul.tl:3-17, C = A B with B [K, N]),
// the llm.tl projections X W^T (linear :28-36, linear_residual :39-47,
// logits :50-58, gate_up :62-73) and matmul.tl's biased linear (:30-38).
//
// One workgroup computes a BM x BN tile of C. Each K step of BK stages the
// A tile and the B tile in LDS as rows of BK contiguous k values (the
// layout both MFMA operands read: 8 consecutive k per lane), XOR-swizzled
// by 16-byte chunk so that the 32 rows an MFMA operand read touches fall in
// distinct banks, and double-buffered: the next tile's global loads are in
// flight while the current one feeds the MFMAs. B given [K, N] (matmul) is
// transposed 8x8 in registers on its way to LDS; W given [N, K] is copied.
// Out-of-range rows and k read as zero and out-of-range outputs are
// dropped, which is the interpreter's rule (src/interp.rs:93-117, :296-313).
#include "common.h"

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

enum Epi { EPI_F16 = 0, EPI_F32 = 1, EPI_RESID = 2, EPI_BIAS = 3, EPI_SWIGLU = 4 };

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
                    reinterpret_cast<u16*>(C)[o] = f2h(v / (1.0f + expf(-v)) * u);
                }
            }
        }
}

// matmul_f32 (kernels/matmul.tl:19-27): f32 operands through LDS, f32 FMA.
__global__ __launch_bounds__(256) void matmul_f32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                         float* __restrict__ C, int M, int N, int K) {
    __shared__ float As[16][64 + 1], Bs[16][64 + 1];
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
                  hipStream_t s, const char* what) {
    auto tiles = [&](int bm, int bn) { return (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    constexpr bool DUAL = EPI == EPI_SWIGLU;
    if constexpr (!DUAL) {
        if (tiles(256, 256) >= 224) return run_gemm<256, 256, 64, 2, 2, BT, EPI>(A, B, B2, C, bias, M, N, K, s, what);
    }
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
                                         "linear");
}

int launch_llm_linear(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    return gemm_dispatch<true, EPI_F16>(P<u16>(a[0]), P<u16>(a[1]), nullptr, P<void>(a[2]), nullptr, M, N, K, s,
                                        "linear");
}

int launch_linear_residual(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    return gemm_dispatch<true, EPI_RESID>(P<u16>(a[0]), P<u16>(a[1]), nullptr, P<void>(a[2]), nullptr, M, N, K, s,
                                          "linear_residual");
}

int launch_logits(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), N = k.dim("N"), K = k.dim("K");
    return gemm_dispatch<true, EPI_F32>(P<u16>(a[0]), P<u16>(a[1]), nullptr, P<void>(a[2]), nullptr, M, N, K, s,
                                        "logits");
}

int launch_gate_up(TslKernel& k, const uint64_t* a, hipStream_t s) {
    int M = k.dim("M"), F = k.dim("F"), K = k.dim("K");
    return gemm_dispatch<true, EPI_SWIGLU>(P<u16>(a[0]), P<u16>(a[1]), P<u16>(a[2]), P<void>(a[3]), nullptr, M, F, K,
                                           s, "gate_up");
}
