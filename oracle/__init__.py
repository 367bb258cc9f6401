"""TEST INFRASTRUCTURE ONLY: Python access to the CPU oracle.

The oracle (oracle/interp.cpp, oracle/llm.cpp) restates tessel's reference
interpreter (src/interp.rs) per kernel, and src/llm/{mod,reference}.rs. Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker: the product (tessel_amd) never does.

Arrays are numpy: f16 tensors as np.float16 (the same bits the kernels
read), f32 as np.float32, i32 as np.int32. Each wrapper returns the output
array(s) the kernel writes.
"""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build():
    """Compiles oracle/liboracle.so (g++, no fast-math, no FMA contraction)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I64 = ctypes.c_int64
F32 = ctypes.c_float
INT = ctypes.c_int


def _declare(L):
    L.tsl_ref_f32_to_f16.argtypes = [F32]
    L.tsl_ref_f32_to_f16.restype = ctypes.c_uint16
    L.tsl_ref_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.tsl_ref_f16_to_f32.restype = F32
    L.tsl_ref_rng_new.argtypes = [ctypes.c_uint64]
    L.tsl_ref_rng_new.restype = ctypes.c_uint64
    L.tsl_ref_rng_bits.argtypes = [P]
    L.tsl_ref_rng_bits.restype = ctypes.c_uint64
    L.tsl_ref_rng_uniform.argtypes = [P]
    L.tsl_ref_rng_uniform.restype = F32
    L.tsl_ref_rng_tensor.argtypes = [P, I64, F32, INT, P]
    L.tsl_ref_matmul.argtypes = [P, P, P] + [I64] * 9 + [INT]
    L.tsl_ref_matmul_f32.argtypes = [P, P, P] + [I64] * 6
    L.tsl_ref_linear_bias.argtypes = [P, P, P, P] + [I64] * 4
    for n in ("tsl_ref_llm_linear", "tsl_ref_linear_residual", "tsl_ref_logits"):
        getattr(L, n).argtypes = [P, P, P] + [I64] * 4
    L.tsl_ref_gate_up.argtypes = [P, P, P, P] + [I64] * 4
    L.tsl_ref_add.argtypes = [P, P, P, I64]
    L.tsl_ref_softmax.argtypes = [P, P, I64, I64, I64, INT]
    L.tsl_ref_rmsnorm_basic.argtypes = [P, P, P, I64, I64, F32, I64, INT]
    L.tsl_ref_embed.argtypes = [P, P, P, I64, I64, I64]
    L.tsl_ref_rmsnorm.argtypes = [P, P, P, I64, I64, F32, I64]
    L.tsl_ref_rmsnorm_rows.argtypes = [P, P, P, P, I64, I64, I64, F32, I64]
    L.tsl_ref_rope_q.argtypes = [P] * 5 + [I64] * 6
    L.tsl_ref_kv_write.argtypes = [P] * 9 + [I64] * 7
    L.tsl_ref_flash_attention.argtypes = [P] * 4 + [I64] * 3 + [F32, I64, I64, INT]
    L.tsl_ref_prefill_attention.argtypes = [P] * 5 + [I64] * 4 + [F32, I64, I64, INT]
    L.tsl_ref_decode_attention.argtypes = [P] * 6 + [I64] * 7 + [F32, INT]
    L.tsl_ref_weights_random.argtypes = [P, ctypes.c_uint64, P, P, P, P]
    L.tsl_ref_rope_tables.argtypes = [P, P, P]
    L.tsl_ref_argmax.argtypes = [P, I64]
    L.tsl_ref_argmax.restype = I64
    L.tsl_ref_forward.argtypes = [P] * 6 + [I64, P]


def _p(a):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


# ---------------------------------------------------------------- half / Rng

def f32_to_f16_bits(x):
    return lib().tsl_ref_f32_to_f16(float(x))


def f16_bits_to_f32(h):
    return lib().tsl_ref_f16_to_f32(int(h))


class Rng:
    """The xorshift Rng of src/bench.rs:13-35 (and tests/common/mod.rs:7-23)."""

    def __init__(self, seed):
        self.state = ctypes.c_uint64(lib().tsl_ref_rng_new(seed))

    def bits(self):
        return lib().tsl_ref_rng_bits(ctypes.byref(self.state))

    def uniform(self):
        return lib().tsl_ref_rng_uniform(ctypes.byref(self.state))

    def below(self, n):
        return self.bits() % n

    def tensor(self, dtype, shape, scale=1.0):
        """Rng::tensor: uniform * scale rounded to dtype ('f32', 'f16', 'i32')."""
        n = int(np.prod(shape)) if len(shape) else 1
        code, npdt = {"f32": (0, np.float32), "f16": (1, np.float16), "i32": (2, np.int32)}[dtype]
        out = np.empty(n, dtype=npdt)
        lib().tsl_ref_rng_tensor(ctypes.byref(self.state), n, scale, code, _p(out))
        return out.reshape(shape)


# ---------------------------------------------------------------- kernels

def matmul(A, B, BM=128, BN=128, BK=32, G=8, threads=1, first_pid=0, npids=-1, C=None):
    M, K = A.shape
    N = B.shape[1]
    if C is None:
        C = np.zeros((M, N), np.float16)
    lib().tsl_ref_matmul(_p(A), _p(B), _p(C), M, N, K, BM, BN, BK, G, first_pid, npids, threads)
    return C


def matmul_f32(A, B, BM=64, BN=64, BK=16):
    M, K = A.shape
    N = B.shape[1]
    C = np.zeros((M, N), np.float32)
    lib().tsl_ref_matmul_f32(_p(A), _p(B), _p(C), M, N, K, BM, BN, BK)
    return C


def linear_bias(X, W, b, BK=32):
    M, K = X.shape
    N = W.shape[0]
    Y = np.zeros((M, N), np.float16)
    lib().tsl_ref_linear_bias(_p(X), _p(W), _p(b), _p(Y), M, N, K, BK)
    return Y


def llm_linear(X, W, BK=64):
    M, K = X.shape
    N = W.shape[0]
    Y = np.zeros((M, N), np.float16)
    lib().tsl_ref_llm_linear(_p(X), _p(W), _p(Y), M, N, K, BK)
    return Y


def linear_residual(X, W, R, BK=64):
    M, K = X.shape
    N = W.shape[0]
    R = np.ascontiguousarray(R, np.float32).copy()
    lib().tsl_ref_linear_residual(_p(X), _p(W), _p(R), M, N, K, BK)
    return R


def logits(X, W, BK=64):
    M, K = X.shape
    N = W.shape[0]
    Y = np.zeros((M, N), np.float32)
    lib().tsl_ref_logits(_p(X), _p(W), _p(Y), M, N, K, BK)
    return Y


def gate_up(X, Wg, Wu, BK=64):
    M, K = X.shape
    F = Wg.shape[0]
    Y = np.zeros((M, F), np.float16)
    lib().tsl_ref_gate_up(_p(X), _p(Wg), _p(Wu), _p(Y), M, F, K, BK)
    return Y


def add(X, Y):
    Z = np.zeros_like(X)
    lib().tsl_ref_add(_p(X), _p(Y), _p(Z), X.size)
    return Z


def softmax(X, BC=1024, threads=1):
    R, C = X.shape
    Y = np.zeros_like(X)
    lib().tsl_ref_softmax(_p(X), _p(Y), R, C, BC, threads)
    return Y


def rmsnorm_basic(X, W, eps, BC=1024, threads=1):
    R, C = X.shape
    Y = np.zeros_like(X)
    lib().tsl_ref_rmsnorm_basic(_p(X), _p(W), _p(Y), R, C, eps, BC, threads)
    return Y


def embed(tok, E):
    T = tok.shape[0]
    V, Dm = E.shape
    X = np.zeros((T, Dm), np.float32)
    lib().tsl_ref_embed(_p(tok), _p(E), _p(X), T, V, Dm)
    return X


def rmsnorm(X, W, eps, BC=2048):
    T, Dm = X.shape
    Y = np.zeros((T, Dm), np.float16)
    lib().tsl_ref_rmsnorm(_p(X), _p(W), _p(Y), T, Dm, eps, BC)
    return Y


def rmsnorm_rows(X, idx, W, eps, BC=2048):
    T, Dm = X.shape
    B = idx.shape[0]
    Y = np.zeros((B, Dm), np.float16)
    lib().tsl_ref_rmsnorm_rows(_p(X), _p(idx), _p(W), _p(Y), T, B, Dm, eps, BC)
    return Y


def rope_q(QKV, pos, C, S, H, D):
    T, W = QKV.shape
    NPOS, D2 = C.shape
    Q = np.zeros((T, H, D), np.float16)
    lib().tsl_ref_rope_q(_p(QKV), _p(pos), _p(C), _p(S), _p(Q), T, W, NPOS, D2, H, D)
    return Q


def kv_write(QKV, pos, slot, C, S, Kc, Vc, K, V):
    """Returns updated copies of (Kc, Vc, K, V)."""
    T, W = QKV.shape
    NPOS, D2 = C.shape
    NS, G, D = Kc.shape
    Kc, Vc, K, V = (np.array(a, copy=True) for a in (Kc, Vc, K, V))
    lib().tsl_ref_kv_write(_p(QKV), _p(pos), _p(slot), _p(C), _p(S), _p(Kc), _p(Vc), _p(K), _p(V),
                           T, W, NPOS, D2, NS, G, D)
    return Kc, Vc, K, V


def flash_attention(Q, K, V, scale, BM=64, BN=64, threads=1):
    H, S, D = Q.shape
    O = np.zeros_like(Q)
    lib().tsl_ref_flash_attention(_p(Q), _p(K), _p(V), _p(O), H, S, D, scale, BM, BN, threads)
    return O


def prefill_attention(Q, K, V, starts, scale, BM=64, BN=64, threads=1):
    S, H, D = Q.shape
    G = K.shape[1]
    O = np.zeros_like(Q)
    lib().tsl_ref_prefill_attention(_p(Q), _p(K), _p(V), _p(starts), _p(O), S, H, G, D, scale, BM, BN, threads)
    return O


def decode_attention(Q, Kc, Vc, table, lens, scale, threads=1):
    """decode_attention (G < H) or paged_attention (G == H)."""
    B, H, D = Q.shape
    NP, P, G, _ = Kc.shape
    MP = table.shape[1]
    O = np.zeros_like(Q)
    lib().tsl_ref_decode_attention(_p(Q), _p(Kc), _p(Vc), _p(table), _p(lens), _p(O),
                                   B, H, D, NP, P, G, MP, scale, threads)
    return O


# ---------------------------------------------------------------- LLM

class Config(ctypes.Structure):
    """src/llm/mod.rs:15-28 (layout of include/tessel.h tsl_config)."""

    _fields_ = [(n, ctypes.c_int32) for n in ("dim", "layers", "heads", "kv_heads", "head_dim", "ffn", "vocab")] + [
        ("eps", ctypes.c_float), ("rope_theta", ctypes.c_float),
        ("max_pos", ctypes.c_int32), ("bos", ctypes.c_int32), ("eos", ctypes.c_int32)]

    @staticmethod
    def tiny():
        """Config::tiny (src/llm/mod.rs:37-52)."""
        return Config(64, 2, 4, 2, 16, 128, 256, 1e-5, 10000.0, 256, 1, 2)

    @staticmethod
    def tinyllama():
        """TinyLlama-1.1B's shape."""
        return Config(2048, 22, 32, 4, 64, 5632, 32000, 1e-5, 10000.0, 2048, 1, 2)

    def qkv(self):
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def layer_elems(self):
        d, hd = self.dim, self.heads * self.head_dim
        return d + self.qkv() * d + d * hd + d + 2 * self.ffn * d + d * self.ffn


def weights_random(cfg, seed):
    """Weights::random: (embed, layers (flat, layer after layer), norm, head) as float16."""
    embed = np.zeros(cfg.vocab * cfg.dim, np.float16)
    layers = np.zeros(cfg.layers * cfg.layer_elems(), np.float16)
    norm = np.zeros(cfg.dim, np.float16)
    head = np.zeros(cfg.vocab * cfg.dim, np.float16)
    lib().tsl_ref_weights_random(ctypes.byref(cfg), seed, _p(embed), _p(layers), _p(norm), _p(head))
    return embed, layers, norm, head


def rope_tables(cfg):
    h = cfg.head_dim // 2
    c = np.zeros((cfg.max_pos, h), np.float32)
    s = np.zeros((cfg.max_pos, h), np.float32)
    lib().tsl_ref_rope_tables(ctypes.byref(cfg), _p(c), _p(s))
    return c, s


def argmax(xs):
    xs = np.ascontiguousarray(xs, np.float32)
    return int(lib().tsl_ref_argmax(_p(xs), xs.size))


def forward(cfg, weights, tokens):
    """reference::forward: logits [n, vocab] after each token."""
    embed, layers, norm, head = weights
    tokens = np.ascontiguousarray(tokens, np.int32)
    out = np.zeros((tokens.size, cfg.vocab), np.float32)
    if lib().tsl_ref_forward(ctypes.byref(cfg), _p(embed), _p(layers), _p(norm), _p(head), _p(tokens), tokens.size,
                             _p(out)) != 0:
        raise ValueError(f"forward: {tokens.size} tokens, more than max_pos = {cfg.max_pos}")
    return out


def paged_case(rng, b, h, d, p, lens, g=None):
    """tests/common/mod.rs:119-173 paged_case (its inputs; G = h unless g is
    given): q, Kc, Vc, table, lens, scale. Pages are handed out in a
    scrambled (Fisher-Yates) order."""
    g = h if g is None else g
    mp = max(max((l + p - 1) // p for l in lens), 1)
    np_ = sum((l + p - 1) // p for l in lens) + 3
    q = rng.tensor("f16", [b, h, d], 1.0)
    kc = rng.tensor("f16", [np_, p, g, d], 1.0)
    vc = rng.tensor("f16", [np_, p, g, d], 1.0)
    order = list(range(np_))
    for i in range(np_ - 1, 0, -1):
        u = np.float32(rng.uniform())
        j = int((u + np.float32(1.0)) * np.float32(0.5) * np.float32(i + 1)) % (i + 1)
        order[i], order[j] = order[j], order[i]
    table = np.zeros((b, mp), np.int32)
    nxt = 0
    for s in range(b):
        for n in range((lens[s] + p - 1) // p):
            table[s, n] = order[nxt]
            nxt += 1
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    return q, kc, vc, table, np.array(lens, np.int32), scale
