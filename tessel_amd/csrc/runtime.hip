// The C ABI (include/tessel.h): one device, one stream, the kernel registry
// and launches. It keeps the launch surface of tessel's GPU layer
// (src/gpu.rs Gpu::{alloc,write,read,kernel,launch,capture_*,replay,sync},
// src/runtime.rs Compiled::launch_raw, src/driver.rs Cuda::*) with HIP
// underneath and hand-written gfx950 kernels behind the .tl names.
//
// tsl_kernel specialises a kernel for its shapes the way src/ir.rs:970-1081
// does (each array's rank checked, symbolic dimensions bound and checked
// for consistency, meta defaults from the .tl overridden by name, unknown
// meta names refused), and caches the result under the reference's key
// "{file}/{name} {shapes:?} {meta:?} {warps}" (src/gpu.rs:156). Shapes are
// then runtime arguments of the kernels; meta values matter only where
// they change results (softmax/rmsnorm BC, the columns a row kernel reads).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <sstream>
#include <array>
#include <string>
#include <vector>

#include "../../include/tessel.h"
#include "common.h"

// Launchers (gemm.hip, rows.hip, attention.hip, decode.hip).
int launch_matmul(TslKernel&, const uint64_t*, hipStream_t);
int launch_matmul_f32(TslKernel&, const uint64_t*, hipStream_t);
int launch_linear_bias(TslKernel&, const uint64_t*, hipStream_t);
int launch_llm_linear(TslKernel&, const uint64_t*, hipStream_t);
int launch_linear_residual(TslKernel&, const uint64_t*, hipStream_t);
int launch_logits(TslKernel&, const uint64_t*, hipStream_t);
int launch_gate_up(TslKernel&, const uint64_t*, hipStream_t);
int launch_softmax(TslKernel&, const uint64_t*, hipStream_t);
int launch_rmsnorm_basic(TslKernel&, const uint64_t*, hipStream_t);
int launch_add(TslKernel&, const uint64_t*, hipStream_t);
int launch_embed(TslKernel&, const uint64_t*, hipStream_t);
int launch_llm_rmsnorm(TslKernel&, const uint64_t*, hipStream_t);
int launch_rmsnorm_rows(TslKernel&, const uint64_t*, hipStream_t);
int launch_rope_q(TslKernel&, const uint64_t*, hipStream_t);
int launch_kv_write(TslKernel&, const uint64_t*, hipStream_t);
int launch_rope_kv(TslKernel&, const uint64_t*, hipStream_t);
int launch_linear_residual_rmsnorm(TslKernel&, const uint64_t*, hipStream_t);
int launch_qkv_rope_kv(TslKernel&, const uint64_t*, hipStream_t);
int launch_linear_residual_prenorm(TslKernel&, const uint64_t*, hipStream_t);
int launch_gate_up_rs(TslKernel&, const uint64_t*, hipStream_t);
int launch_qkv_rs_rope_kv(TslKernel&, const uint64_t*, hipStream_t);
int prepare_gate_up_rs(TslKernel&);
int prepare_qkv_rs_rope_kv(TslKernel&);
int launch_argmax(TslKernel&, const uint64_t*, hipStream_t);
int launch_flash_attention(TslKernel&, const uint64_t*, hipStream_t);
int launch_prefill_attention(TslKernel&, const uint64_t*, hipStream_t);
int launch_decode_attention(TslKernel&, const uint64_t*, hipStream_t);
int launch_paged_attention(TslKernel&, const uint64_t*, hipStream_t);
int prepare_attention(TslKernel&);
int prepare_decode(TslKernel&);
int prepare_projection(TslKernel&);

// Compute units of the current device (cached; 256 if the query fails).
int num_cus() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = v;
        else
            n = 256;
    }
    return n;
}

namespace {

thread_local std::string g_err;

// ---------------------------------------------------------------- the .tl signatures

struct Param {
    std::string name;
    bool array;
    std::string dtype;
    std::vector<std::string> dims;  // names or integer literals
};

struct KernelDef {
    const char* file;
    const char* name;
    const char* sig;   // the .tl parameter list
    const char* meta;  // the .tl meta line ("" if none)
    const char* pow2;  // dimensions the body slices in full (tile sizes: powers of two)
    tsl_launcher launch;
    tsl_preparer prepare;
    std::vector<Param> params;
    std::vector<std::pair<std::string, int64_t>> meta_defaults;
};

// The kernels of kernels/{basic,matmul,attention,llm}.tl, signatures as written there.
std::vector<KernelDef> g_defs = {
    {"basic", "add", "X: f32[N], Y: f32[N], Z: f32[N]", "B = 1024", "", launch_add, nullptr},
    {"basic", "softmax", "X: f32[R, C], Y: f32[R, C]", "BR = 4, BC = 1024", "", launch_softmax, nullptr},
    {"basic", "rmsnorm", "X: f16[R, C], W: f16[C], Y: f16[R, C], eps: f32", "BR = 4, BC = 1024", "",
     launch_rmsnorm_basic, nullptr},
    {"matmul", "matmul", "A: f16[M, K], B: f16[K, N], C: f16[M, N]", "BM = 128, BN = 128, BK = 32, G = 8", "",
     launch_matmul, nullptr},
    {"matmul", "matmul_f32", "A: f32[M, K], B: f32[K, N], C: f32[M, N]", "BM = 64, BN = 64, BK = 16", "",
     launch_matmul_f32, nullptr},
    {"matmul", "linear", "X: f16[M, K], W: f16[N, K], b: f16[N], Y: f16[M, N]", "BM = 64, BN = 128, BK = 32", "",
     launch_linear_bias, prepare_projection},
    {"attention", "flash_attention", "Q: f16[H, S, D], K: f16[H, S, D], V: f16[H, S, D], O: f16[H, S, D], scale: f32",
     "BM = 64, BN = 64", "D", launch_flash_attention, prepare_attention},
    {"attention", "paged_attention",
     "q: f16[B, H, D], Kc: f16[NP, P, H, D], Vc: f16[NP, P, H, D], table: i32[B, MP], lens: i32[B], "
     "out: f16[B, H, D], scale: f32",
     "BQ = 16", "P D", launch_paged_attention, prepare_decode},
    {"llm", "embed", "tok: i32[T], E: f16[V, Dm], X: f32[T, Dm]", "BD = 1024", "", launch_embed, nullptr},
    {"llm", "rmsnorm", "X: f32[T, Dm], W: f16[Dm], Y: f16[T, Dm], eps: f32", "BR = 1, BC = 2048", "",
     launch_llm_rmsnorm, nullptr},
    {"llm", "linear", "X: f16[M, K], W: f16[N, K], Y: f16[M, N]", "BM = 16, BN = 64, BK = 64", "", launch_llm_linear,
     prepare_projection},
    {"llm", "linear_residual", "X: f16[M, K], W: f16[N, K], R: f32[M, N]", "BM = 16, BN = 64, BK = 64", "",
     launch_linear_residual, prepare_projection},
    {"llm", "logits", "X: f16[M, K], W: f16[N, K], Y: f32[M, N]", "BM = 16, BN = 64, BK = 64", "", launch_logits,
     prepare_projection},
    {"llm", "gate_up", "X: f16[M, K], Wg: f16[F, K], Wu: f16[F, K], Y: f16[M, F]", "BM = 16, BN = 64, BK = 64", "",
     launch_gate_up, prepare_projection},
    {"llm", "rope_q", "QKV: f16[T, W], pos: i32[T], C: f32[NPOS, D2], S: f32[NPOS, D2], Q: f16[T, H, D]", "", "D2",
     launch_rope_q, nullptr},
    {"llm", "kv_write",
     "QKV: f16[T, W], pos: i32[T], slot: i32[T], C: f32[NPOS, D2], S: f32[NPOS, D2], Kc: f16[NS, G, D], "
     "Vc: f16[NS, G, D], K: f16[T, G, D], V: f16[T, G, D]",
     "", "D2 D", launch_kv_write, nullptr},
    // Not a .tl kernel: llm/rope_q and llm/kv_write of one step in one launch
    // (the engine's fusion; same arguments, Q after slot/C/S).
    {"fused", "rope_kv",
     "QKV: f16[T, W], pos: i32[T], slot: i32[T], C: f32[NPOS, D2], S: f32[NPOS, D2], Q: f16[T, H, D], "
     "Kc: f16[NS, G, D], Vc: f16[NS, G, D], K: f16[T, G, D], V: f16[T, G, D]",
     "", "D2 D", launch_rope_kv, nullptr},
    // Not a .tl kernel: llm/linear_residual then llm/rmsnorm of the updated
    // residual (the engine's fusion; Wn, Y and eps are rmsnorm's W, Y, eps).
    {"fused", "linear_residual_rmsnorm",
     "X: f16[M, K], W: f16[N, K], R: f32[M, N], Wn: f16[N], Y: f16[M, N], eps: f32", "BC = 2048", "",
     launch_linear_residual_rmsnorm, prepare_projection},
    // Not a .tl kernel: llm/linear (QKV = X Wqkv^T), then llm/rope_q and
    // llm/kv_write of that QKV (the engine's fusion; their arguments after X, Wqkv).
    {"fused", "qkv_rope_kv",
     "X: f16[T, Dm], Wqkv: f16[W, Dm], QKV: f16[T, W], pos: i32[T], slot: i32[T], C: f32[NPOS, D2], "
     "S: f32[NPOS, D2], Q: f16[T, H, D], Kc: f16[NS, G, D], Vc: f16[NS, G, D], K: f16[T, G, D], V: f16[T, G, D]",
     "", "D2 D", launch_qkv_rope_kv, prepare_projection},
    // Not a .tl kernel: argmax of each row (src/llm/mod.rs:132-140), so the
    // scheduler reads back token ids instead of logits.
    {"fused", "argmax", "X: f32[B, V], T: i32[B]", "", "", launch_argmax, nullptr},
    // Not a .tl kernel: llm/linear_residual that leaves the next rmsnorm
    // deferred, as Y = f16(R Wn) and per-8-column sums of squares of R (the
    // engine's fusion; its consumers are gate_up_rs and qkv_rs_rope_kv).
    {"fused", "linear_residual_prenorm",
     "X: f16[M, K], W: f16[N, K], R: f32[M, N], Wn: f16[N], Y: f16[M, N], SS: f32[NB, M], OVF: i32[1]", "", "",
     launch_linear_residual_prenorm, nullptr},
    // Not a .tl kernel: llm/gate_up of rmsnorm(R) Wn given as Y and SS (the
    // engine's fusion).
    {"fused", "gate_up_rs",
     "Y: f16[M, K], SS: f32[NB, M], Wg: f16[F, K], Wu: f16[F, K], O: f16[M, F], eps: f32", "", "",
     launch_gate_up_rs, prepare_gate_up_rs},
    // Not a .tl kernel: fused/qkv_rope_kv of rmsnorm(R) Wn given as X = Y and
    // SS (the engine's fusion; qkv_rope_kv's arguments, then SS and eps).
    {"fused", "qkv_rs_rope_kv",
     "X: f16[T, Dm], Wqkv: f16[W, Dm], QKV: f16[T, W], pos: i32[T], slot: i32[T], C: f32[NPOS, D2], "
     "S: f32[NPOS, D2], Q: f16[T, H, D], Kc: f16[NS, G, D], Vc: f16[NS, G, D], K: f16[T, G, D], V: f16[T, G, D], "
     "SS: f32[NB, T], eps: f32",
     "", "D2 D", launch_qkv_rs_rope_kv, prepare_qkv_rs_rope_kv},
    {"llm", "prefill_attention",
     "Q: f16[S, H, D], K: f16[S, G, D], V: f16[S, G, D], starts: i32[S], O: f16[S, H, D], scale: f32",
     "BM = 64, BN = 64", "D", launch_prefill_attention, prepare_attention},
    {"llm", "decode_attention",
     "Q: f16[B, H, D], Kc: f16[NP, P, G, D], Vc: f16[NP, P, G, D], table: i32[B, MP], lens: i32[B], "
     "O: f16[B, H, D], scale: f32",
     "", "P D", launch_decode_attention, prepare_decode},
    {"llm", "rmsnorm_rows", "X: f32[T, Dm], idx: i32[B], W: f16[Dm], Y: f16[B, Dm], eps: f32", "BC = 2048", "",
     launch_rmsnorm_rows, nullptr},
};

std::string trim(const std::string& s) {
    size_t a = s.find_first_not_of(" \t"), b = s.find_last_not_of(" \t");
    return a == std::string::npos ? "" : s.substr(a, b - a + 1);
}

std::vector<std::string> split_top(const std::string& s, char sep) {  // split outside brackets
    std::vector<std::string> out;
    int depth = 0;
    std::string cur;
    for (char c : s) {
        if (c == '[') depth++;
        if (c == ']') depth--;
        if (c == sep && depth == 0) {
            out.push_back(trim(cur));
            cur.clear();
        } else {
            cur += c;
        }
    }
    if (!trim(cur).empty()) out.push_back(trim(cur));
    return out;
}

void parse_defs() {
    static bool done = false;
    if (done) return;
    done = true;
    for (auto& d : g_defs) {
        for (auto& p : split_top(d.sig, ',')) {
            Param q;
            size_t colon = p.find(':');
            q.name = trim(p.substr(0, colon));
            std::string ty = trim(p.substr(colon + 1));
            size_t br = ty.find('[');
            q.array = br != std::string::npos;
            q.dtype = trim(q.array ? ty.substr(0, br) : ty);
            if (q.array) {
                std::string in = ty.substr(br + 1, ty.rfind(']') - br - 1);
                for (auto& dim : split_top(in, ',')) q.dims.push_back(dim);
            }
            d.params.push_back(q);
        }
        for (auto& m : split_top(d.meta, ',')) {
            size_t eq = m.find('=');
            d.meta_defaults.push_back({trim(m.substr(0, eq)), std::stoll(trim(m.substr(eq + 1)))});
        }
    }
}

bool is_int(const std::string& s) { return !s.empty() && s.find_first_not_of("0123456789") == std::string::npos; }

// ---------------------------------------------------------------- device state

struct State {
    bool open = false;
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<TslKernel*> kernels;
    std::vector<tsl_launcher> launchers;
    std::map<std::string, int> by_key;
    std::vector<hipGraphExec_t> graphs;
    std::vector<std::array<int64_t, 4>> graph_nodes;  // per graph: kernel, memset, memcpy, other nodes
    std::vector<hipEvent_t> events;
    std::string name;
    int cus = 0, mhz = 0;
};
State g;
std::mutex g_mu;

}  // namespace

int64_t TslKernel::dim(const char* n) const {
    for (auto& d : dims)
        if (d.first == n) return d.second;
    return 0;
}

int64_t TslKernel::metav(const char* n) const {
    for (auto& m : meta)
        if (m.first == n) return m.second;
    return 0;
}

int tsl_fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int tsl_hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return 0;
    // Reported here, so clear HIP's last-error state: a later, unrelated
    // launch check (hipGetLastError) must not report this call again.
    (void)hipGetLastError();
    std::ostringstream o;
    o << what << ": HIP error " << (int)e << " " << hipGetErrorName(e) << " (" << hipGetErrorString(e) << ")";
    return tsl_fail(TSL_ERR_HIP, o.str());
}

#define CHECK(call, what)                                  \
    do {                                                   \
        int _r = tsl_hip_check((call), what);              \
        if (_r) return _r;                                 \
    } while (0)

#define NEED_OPEN()                         \
    do {                                    \
        int _r = tsl_open();                \
        if (_r) return _r;                  \
    } while (0)

extern "C" {

const char* tsl_last_error(void) { return g_err.c_str(); }

int tsl_open(void) {
    if (g.open) {
        (void)hipSetDevice(g.device);  // per-thread binding, as Cuda::bind (src/driver.rs:174-179)
        return 0;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (g.open) return 0;
    parse_defs();
    int n = 0;
    CHECK(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (n < 1) return tsl_fail(TSL_ERR_HIP, "no HIP device");
    CHECK(hipSetDevice(0), "hipSetDevice");
    hipDeviceProp_t p;
    CHECK(hipGetDeviceProperties(&p, 0), "hipGetDeviceProperties");
    g.name = std::string(p.gcnArchName) + " " + p.name;
    g.cus = p.multiProcessorCount;
    g.mhz = p.clockRate / 1000;
    CHECK(hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking), "hipStreamCreate");
    g.open = true;
    return 0;
}

int tsl_device_name(char* buf, size_t len) {
    NEED_OPEN();
    snprintf(buf, len, "%s", g.name.c_str());
    return 0;
}

int tsl_device_info(int* cus, int* mhz) {
    NEED_OPEN();
    *cus = g.cus;
    *mhz = g.mhz;
    return 0;
}

int tsl_sync(void) {
    NEED_OPEN();
    CHECK(hipStreamSynchronize(g.stream), "sync");
    return 0;
}

void* tsl_stream(void) { return tsl_open() ? nullptr : (void*)g.stream; }

int tsl_alloc(size_t bytes, uint64_t* dptr) {
    NEED_OPEN();
    void* p = nullptr;
    size_t n = bytes < 4 ? 4 : bytes;
    CHECK(hipMalloc(&p, n), "hipMalloc");
    CHECK(hipMemsetAsync(p, 0, n, g.stream), "zero fill");
    CHECK(hipStreamSynchronize(g.stream), "zero fill");
    *dptr = (uint64_t)p;
    return 0;
}

int tsl_free(uint64_t dptr) {
    NEED_OPEN();
    CHECK(hipStreamSynchronize(g.stream), "free");
    CHECK(hipFree((void*)dptr), "hipFree");
    return 0;
}

int tsl_upload(uint64_t dst, const void* src, size_t n) {
    NEED_OPEN();
    if (n == 0) return 0;
    CHECK(hipMemcpyAsync((void*)dst, src, n, hipMemcpyHostToDevice, g.stream), "upload");
    CHECK(hipStreamSynchronize(g.stream), "upload");
    return 0;
}

int tsl_download(void* dst, uint64_t src, size_t n) {
    NEED_OPEN();
    CHECK(hipStreamSynchronize(g.stream), "sync");
    if (n == 0) return 0;
    CHECK(hipMemcpyAsync(dst, (const void*)src, n, hipMemcpyDeviceToHost, g.stream), "download");
    CHECK(hipStreamSynchronize(g.stream), "download");
    return 0;
}

int tsl_fill_nan(uint64_t dst, size_t n) {
    NEED_OPEN();
    CHECK(hipMemsetD32Async((hipDeviceptr_t)dst, 0x7fc00000, n, g.stream), "memset");
    return 0;
}

int tsl_kernel(const char* file, const char* name, int nshapes, const int* ranks, const int64_t* dims, int nmeta,
               const char* const* meta_names, const int64_t* meta_values, int warps, int* handle) {
    parse_defs();
    KernelDef* def = nullptr;
    bool file_known = false;
    for (auto& d : g_defs) {
        if (std::string(d.file) == file) file_known = true;
        if (std::string(d.file) == file && std::string(d.name) == name) def = &d;
    }
    if (!file_known) return tsl_fail(TSL_ERR_NOKERNEL, std::string("no kernel file ") + file);
    if (!def) return tsl_fail(TSL_ERR_NOKERNEL, std::string("no kernel ") + name);

    // The key, formatted as Rust's Debug prints the shapes and meta.
    std::ostringstream key;
    key << file << "/" << name << " [";
    std::vector<std::vector<int64_t>> shapes;
    const int64_t* dp = dims;
    for (int i = 0; i < nshapes; i++) {
        std::vector<int64_t> s(dp, dp + ranks[i]);
        dp += ranks[i];
        key << (i ? ", " : "") << "[";
        for (size_t j = 0; j < s.size(); j++) key << (j ? ", " : "") << s[j];
        key << "]";
        shapes.push_back(s);
    }
    key << "] [";
    for (int i = 0; i < nmeta; i++) key << (i ? ", " : "") << "(\"" << meta_names[i] << "\", " << meta_values[i] << ")";
    key << "] " << warps;
    auto it = g.by_key.find(key.str());
    if (it != g.by_key.end()) {
        *handle = it->second;
        return 0;
    }

    // Specialise (src/ir.rs:970-1043).
    TslKernel* k = new TslKernel();
    k->file = file;
    k->name = name;
    k->key = key.str();
    k->warps = warps;
    k->nparams = (int)def->params.size();
    size_t si = 0;
    auto bad = [&](const std::string& m) {
        delete k;
        return tsl_fail(TSL_ERR_ARG, std::string(name) + ": " + m);
    };
    for (auto& p : def->params) {
        if (!p.array) continue;
        if (si >= shapes.size()) return bad("no shape given for array " + p.name);
        const auto& s = shapes[si++];
        if (s.size() != p.dims.size()) {
            std::ostringstream o;
            o << p.name << " has " << p.dims.size() << " dimensions, shape of " << s.size() << " given";
            return bad(o.str());
        }
        for (size_t j = 0; j < s.size(); j++) {
            if (s[j] < 0) return bad("negative dimension");
            const std::string& dn = p.dims[j];
            if (is_int(dn)) {
                if (std::stoll(dn) != s[j]) return bad(p.name + " dimension must be " + dn);
                continue;
            }
            bool found = false;
            for (auto& d : k->dims)
                if (d.first == dn) {
                    found = true;
                    if (d.second != s[j]) {
                        std::ostringstream o;
                        o << "dimension " << dn << " is " << d.second << " and " << s[j];
                        return bad(o.str());
                    }
                }
            if (!found) k->dims.push_back({dn, s[j]});
        }
        k->shapes.push_back(s);
    }
    k->meta = def->meta_defaults;
    for (int i = 0; i < nmeta; i++) {
        bool found = false;
        for (auto& m : k->meta)
            if (m.first == meta_names[i]) {
                m.second = meta_values[i];
                found = true;
            }
        if (!found) return bad(std::string("no meta constant ") + meta_names[i]);
    }
    // Tile sizes must be powers of two (src/ir.rs:399-409): the meta tile
    // constants (all but matmul's group count G) and the dimensions a body
    // slices whole.
    auto pow2 = [](int64_t x) { return x > 0 && (x & (x - 1)) == 0; };
    for (auto& m : k->meta)
        if (!(std::string(def->file) == "matmul" && m.first == "G") && !pow2(m.second))
            return bad("tile dimensions must be powers of two, got " + m.first + " = " + std::to_string(m.second));
    {
        std::istringstream ps(def->pow2);
        std::string dn;
        while (ps >> dn)
            if (!pow2(k->dim(dn.c_str())))
                return bad("tile dimensions must be powers of two, got " + dn + " = " + std::to_string(k->dim(dn.c_str())));
    }
    if (def->prepare) {
        int o = tsl_open();
        if (o) {
            delete k;
            return o;
        }
        int r = def->prepare(*k);
        if (r) {
            delete k;
            return r;
        }
    }
    g.kernels.push_back(k);
    g.launchers.push_back(def->launch);
    *handle = (int)g.kernels.size() - 1;
    g.by_key[k->key] = *handle;
    return 0;
}

int tsl_kernel_key(int handle, char* buf, size_t len) {
    if (handle < 0 || handle >= (int)g.kernels.size()) return tsl_fail(TSL_ERR_ARG, "no such kernel handle");
    snprintf(buf, len, "%s", g.kernels[handle]->key.c_str());
    return 0;
}

int tsl_launch(int handle, const uint64_t* args, int nargs) {
    if (handle < 0 || handle >= (int)g.kernels.size()) return tsl_fail(TSL_ERR_ARG, "no such kernel handle");
    TslKernel& k = *g.kernels[handle];
    if (nargs != k.nparams) {
        std::ostringstream o;
        o << k.name << ": " << nargs << " arguments for " << k.nparams << " parameters";
        return tsl_fail(TSL_ERR_ARG, o.str());
    }
    return g.launchers[handle](k, args, g.stream);
}

int tsl_time_launches(int handle, const uint64_t* args, int nargs, int iters, float* ms) {
    NEED_OPEN();
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a), "event");
    CHECK(hipEventCreate(&b), "event");
    CHECK(hipStreamSynchronize(g.stream), "sync");
    CHECK(hipEventRecord(a, g.stream), "record");
    int r = 0;
    for (int i = 0; i < iters && !r; i++) r = tsl_launch(handle, args, nargs);
    if (!r) r = tsl_hip_check(hipEventRecord(b, g.stream), "record");
    if (!r) r = tsl_hip_check(hipEventSynchronize(b), "event sync");
    if (!r) r = tsl_hip_check(hipEventElapsedTime(ms, a, b), "elapsed");
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return r;
}

// Cuda::time around one launch, `iters` times (src/driver.rs:365-380, as
// Compiled::time uses it, src/runtime.rs:294-316): ms[i] is launch i's time.
int tsl_time_each(int handle, const uint64_t* args, int nargs, int iters, float* ms) {
    NEED_OPEN();
    if (iters > 0 && !ms) return tsl_fail(TSL_ERR_ARG, "null ms");
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a), "event");
    CHECK(hipEventCreate(&b), "event");
    int r = 0;
    for (int i = 0; i < iters && !r; i++) {
        r = tsl_hip_check(hipEventRecord(a, g.stream), "record");
        if (!r) r = tsl_launch(handle, args, nargs);
        if (!r) r = tsl_hip_check(hipEventRecord(b, g.stream), "record");
        if (!r) r = tsl_hip_check(hipEventSynchronize(b), "event sync");
        if (!r) r = tsl_hip_check(hipEventElapsedTime(&ms[i], a, b), "elapsed");
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return r;
}

int tsl_capture_begin(void) {
    NEED_OPEN();
    CHECK(hipStreamBeginCapture(g.stream, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
    return 0;
}

int tsl_capture_end(int* graph) {
    NEED_OPEN();
    hipGraph_t gr;
    hipGraphExec_t ex;
    CHECK(hipStreamEndCapture(g.stream, &gr), "hipStreamEndCapture");
    // What the recording holds, by node type, before it is instantiated.
    std::array<int64_t, 4> kinds{};
    size_t nn = 0;
    CHECK(hipGraphGetNodes(gr, nullptr, &nn), "hipGraphGetNodes");
    std::vector<hipGraphNode_t> nodes(nn);
    if (nn) CHECK(hipGraphGetNodes(gr, nodes.data(), &nn), "hipGraphGetNodes");
    for (size_t i = 0; i < nn; i++) {
        hipGraphNodeType t;
        CHECK(hipGraphNodeGetType(nodes[i], &t), "hipGraphNodeGetType");
        kinds[t == hipGraphNodeTypeKernel ? 0 : t == hipGraphNodeTypeMemset ? 1 : t == hipGraphNodeTypeMemcpy ? 2 : 3]++;
    }
    CHECK(hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0), "hipGraphInstantiate");
    g.graph_nodes.push_back(kinds);
    (void)hipGraphDestroy(gr);
    g.graphs.push_back(ex);
    *graph = (int)g.graphs.size() - 1;
    return 0;
}

int tsl_graph_nodes(int graph, int64_t* counts) {
    if (graph < 0 || graph >= (int)g.graph_nodes.size()) return tsl_fail(TSL_ERR_ARG, "no such graph");
    for (int i = 0; i < 4; i++) counts[i] = g.graph_nodes[graph][i];
    return 0;
}

int tsl_replay(int graph) {
    NEED_OPEN();
    if (graph < 0 || graph >= (int)g.graphs.size()) return tsl_fail(TSL_ERR_ARG, "no such graph");
    CHECK(hipGraphLaunch(g.graphs[graph], g.stream), "hipGraphLaunch");
    return 0;
}

int tsl_event_record(int* event) {
    NEED_OPEN();
    hipEvent_t e;
    CHECK(hipEventCreate(&e), "event");
    CHECK(hipEventRecord(e, g.stream), "record");
    g.events.push_back(e);
    *event = (int)g.events.size() - 1;
    return 0;
}

int tsl_event_elapsed(int start, int end, float* ms) {
    NEED_OPEN();
    if (start < 0 || end < 0 || start >= (int)g.events.size() || end >= (int)g.events.size())
        return tsl_fail(TSL_ERR_ARG, "no such event");
    CHECK(hipEventSynchronize(g.events[end]), "event sync");
    CHECK(hipEventElapsedTime(ms, g.events[start], g.events[end]), "elapsed");
    return 0;
}

}  // extern "C"

// Records event `id` (made by tsl_event_record) again, on the stream: the
// engine's per-step timing reuses one pair of events. Library-internal.
int rt_event_rerecord(int id) {
    NEED_OPEN();
    if (id < 0 || id >= (int)g.events.size()) return tsl_fail(TSL_ERR_ARG, "no such event");
    CHECK(hipEventRecord(g.events[id], g.stream), "record");
    return 0;
}

// The engine's per-step transfers through pinned host buffers (library-
// internal): an upload that is only enqueued (ordered before the step's
// kernels on the stream; the caller keeps the buffer unchanged until a later
// synchronisation), and a download that enqueues and waits once.
int rt_host_alloc(size_t n, void** p) {
    NEED_OPEN();
    CHECK(hipHostMalloc(p, n, hipHostMallocDefault), "pinned host buffer");
    return 0;
}
int rt_host_free(void* p) {
    if (p) CHECK(hipHostFree(p), "pinned host buffer");
    return 0;
}
int rt_upload_async(uint64_t dst, const void* pinned, size_t n) {
    NEED_OPEN();
    if (n == 0) return 0;
    CHECK(hipMemcpyAsync((void*)dst, pinned, n, hipMemcpyHostToDevice, g.stream), "upload");
    return 0;
}
int rt_download_pinned(void* pinned, uint64_t src, size_t n) {
    NEED_OPEN();
    if (n) CHECK(hipMemcpyAsync(pinned, (const void*)src, n, hipMemcpyDeviceToHost, g.stream), "download");
    CHECK(hipStreamSynchronize(g.stream), "download");
    return 0;
}
