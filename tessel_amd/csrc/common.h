// Shared device helpers for the gfx950 kernels: vector types, f16
// conversions, 64-lane wavefront reductions and the kernel-handle type the
// launchers receive.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

typedef _Float16 half_t;
typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef half_t half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16;

#define TSL_DEV __device__ __forceinline__

// LDS poisoning for a debug build (hipcc -DTSL_POISON_LDS; build.py --poison):
// at the start of a kernel every thread of the workgroup fills its LDS arrays
// with all-ones words (NaN as f32 and as each f16 half), then a barrier, so a
// read of LDS that nothing wrote shows up as NaN in the outputs (what the
// reference's emulator does with its shared memory). Off in normal builds.
#ifdef TSL_POISON_LDS
#define TSL_POISON(arr) tsl_poison_lds(&(arr), sizeof(arr))
#define TSL_POISON_BYTES(ptr, bytes) tsl_poison_lds((ptr), (bytes))
__device__ inline void tsl_poison_lds(void* p, unsigned bytes) {
    uint32_t* w = static_cast<uint32_t*>(p);
    const unsigned nt = blockDim.x * blockDim.y * blockDim.z;
    const unsigned t = threadIdx.x + blockDim.x * (threadIdx.y + blockDim.y * threadIdx.z);
    for (unsigned i = t; i < bytes / 4; i += nt) w[i] = 0xffffffffu;
    __syncthreads();
}
#else
#define TSL_POISON(arr) ((void)0)
#define TSL_POISON_BYTES(ptr, bytes) ((void)0)
#endif

// Reinterpreting one element of an ext_vector in place,
// __builtin_bit_cast(T, v[i]), reads element 0 whatever i is with this
// clang (checked on the host: {1, 2, 3, 4}[i] as float gives 1 for every i).
// Elements are therefore always passed by value through these helpers.
TSL_DEV half2v as_half2(uint32_t x) { return __builtin_bit_cast(half2v, x); }
TSL_DEV float as_float(uint32_t x) { return __builtin_bit_cast(float, x); }

// f16 bits <-> f32 (hardware conversions: round to nearest even).
TSL_DEV float h2f(u16 h) { return (float)__builtin_bit_cast(half_t, h); }
TSL_DEV u16 f2h(float f) { return __builtin_bit_cast(u16, (half_t)f); }

// The rotary pair (x1 c - x2 s, x2 c + x1 s) rounded to f16, with its
// multiply-adds spelled out, so every kernel that rotates (rope_q, kv_write,
// the fused QKV epilogue) produces the same bits.
TSL_DEV void rope_rotate(float x1, float x2, float c, float s, u16& y1, u16& y2) {
    y1 = f2h(__builtin_fmaf(x1, c, -(x2 * s)));
    y2 = f2h(__builtin_fmaf(x2, c, x1 * s));
}

// x / d for many x and one d (Markstein's method: a reciprocal refined by one
// Newton step, then one residual correction of each quotient). Three
// operations per quotient instead of a full IEEE division's ~11; the result is
// the correctly rounded f32 quotient except in rare near-halfway cases, where it
// is one ulp off. For d finite, positive and normal.
struct DivBy {
    float d, r;
    TSL_DEV explicit DivBy(float den) : d(den) {
        const float r0 = __builtin_amdgcn_rcpf(den);
        r = __builtin_fmaf(__builtin_fmaf(-den, r0, 1.0f), r0, r0);
    }
    TSL_DEV float operator()(float x) const {
        const float q = x * r;
        return __builtin_fmaf(__builtin_fmaf(-q, d, x), r, q);
    }
};

// DPP row operations within 16-lane rows (gfx9 DPP controls).
template <int CTRL>
TSL_DEV float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
// quad_perm [1,0,3,2] (xor 1), quad_perm [2,3,0,1] (xor 2), row_half_mirror, row_mirror.
#define DPP_XOR1 0xb1
#define DPP_XOR2 0x4e
#define DPP_HALF_MIRROR 0x141
#define DPP_MIRROR 0x140

// x of lane l ^ 32 / l ^ 16, by v_permlane32_swap / v_permlane16_swap
// (registers only; a __shfl_xor would round-trip through LDS with
// ds_bpermute). Swapping a copy of x with itself leaves the partner's value
// in the source for the lower lanes of each pair and in the destination
// for the upper ones.
TSL_DEV float xor32(float x) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}
TSL_DEV float xor16(float x) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}

TSL_DEV float lane_value(float x, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

// Largest / sum over the 64 lanes of a (fully active) wavefront, every lane
// receiving it: four DPP steps within each 16-lane row (all of a row's lanes
// then hold its result), then the four rows read out by readlane. Registers
// only: a __shfl_xor butterfly would make six ds_bpermute round trips.
TSL_DEV float wave_max(float x) {
    x = fmaxf(x, dpp<DPP_XOR1>(x));
    x = fmaxf(x, dpp<DPP_XOR2>(x));
    x = fmaxf(x, dpp<DPP_HALF_MIRROR>(x));
    x = fmaxf(x, dpp<DPP_MIRROR>(x));
    return fmaxf(fmaxf(lane_value(x, 0), lane_value(x, 16)), fmaxf(lane_value(x, 32), lane_value(x, 48)));
}
TSL_DEV float wave_sum(float x) {
    x += dpp<DPP_XOR1>(x);
    x += dpp<DPP_XOR2>(x);
    x += dpp<DPP_HALF_MIRROR>(x);
    x += dpp<DPP_MIRROR>(x);
    return (lane_value(x, 0) + lane_value(x, 16)) + (lane_value(x, 32) + lane_value(x, 48));
}

// A kernel specialised by tsl_kernel: its resolved dimensions and meta
// values, in the order the .tl signature names them.
struct TslKernel {
    std::string file, name, key;
    std::vector<std::vector<int64_t>> shapes;          // array params, in order
    std::vector<std::pair<std::string, int64_t>> meta;  // declared order, overrides applied
    std::vector<std::pair<std::string, int64_t>> dims;  // symbolic dims -> values
    int warps = 4;
    int nparams = 0;
    // Library-owned device scratch (allocated once per handle, outside any
    // graph capture): decode attention's per-chunk states, the split-K
    // partials of few-row projections.
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    int64_t dim(const char* n) const;
    int64_t metav(const char* n) const;
};

typedef int (*tsl_launcher)(TslKernel& k, const uint64_t* args, hipStream_t s);
typedef int (*tsl_preparer)(TslKernel& k);  // optional: scratch sizing at tsl_kernel time

// Compute units of the current device (runtime.hip; cached).
int num_cus();

// Records an argument/launch error (the C ABI's last error).
int tsl_fail(int code, const std::string& msg);
int tsl_hip_check(hipError_t e, const char* what);

template <class T>
inline T* P(uint64_t a) { return reinterpret_cast<T*>(a); }
inline float arg_f32(uint64_t a) {
    uint32_t b = (uint32_t)a;
    float f;
    __builtin_memcpy(&f, &b, 4);
    return f;
}
inline int32_t arg_i32(uint64_t a) { return (int32_t)(uint32_t)a; }

// The launch check after a kernel launch (a bad configuration fails here).
#define TSL_LAUNCHED(what) tsl_hip_check(hipGetLastError(), what)
