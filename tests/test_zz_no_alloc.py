"""tsl_decode_attention_noalloc, the decode_attention entry point that
allocates nothing (its partial states live in a library-owned device array):
through the C ABI it must give exactly what tsl_launch of a decode_attention
handle gives (the same kernels), on consecutive calls that share the array,
the second smaller than the first, and stay within the oracle's parity bar.
Kernels: kernels/llm.tl:150-172."""

import ctypes

import numpy as np
import pytest

import oracle
import tessel_amd as T
from tests.refs import parity

pytestmark = pytest.mark.gpu


def _case(seed, b, h, g, d, p, lo, hi):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, b).astype(np.int32)
    need = (lens + p - 1) // p
    mp = int(need.max())
    npages = int(need.sum())
    perm = rng.permutation(npages).astype(np.int32)
    table = np.zeros((b, mp), np.int32)
    o = 0
    for i in range(b):
        table[i, :need[i]] = perm[o:o + need[i]]
        o += need[i]
    q = rng.standard_normal((b, h, d)).astype(np.float16)
    kc = rng.standard_normal((npages, p, g, d)).astype(np.float16)
    vc = rng.standard_normal((npages, p, g, d)).astype(np.float16)
    return q, kc, vc, table, lens, float(np.float32(1.0) / np.sqrt(np.float32(d)))


def _both(q, kc, vc, table, lens, scale):
    b, h, d = q.shape
    npg, p, g, _ = kc.shape
    mp = table.shape[1]
    bufs = [T.tensor(x) for x in (q, kc, vc, table, lens)]
    o1, o2 = T.alloc(q.nbytes), T.alloc(q.nbytes)
    T.fill_nan(o1)
    T.fill_nan(o2)
    k = T.kernel("llm", "decode_attention", [q.shape, kc.shape, vc.shape, table.shape, lens.shape, q.shape])
    T.launch(k, bufs + [o1, T.F32(scale)])
    T.check(T.lib().tsl_decode_attention_noalloc(*[x.ptr for x in bufs], o2.ptr, ctypes.c_float(scale), b, h, g, d,
                                                 npg, p, mp))
    got1 = T.read_array(o1, np.float16, q.shape)
    got2 = T.read_array(o2, np.float16, q.shape)
    for x in bufs + [o1, o2]:
        T.free(x)
    return got1, got2


@pytest.mark.parametrize("cases", [
    # The benchmark decode shape (balanced stream path), then a smaller call (fewer
    # sequences, shorter tables: the chunked path) on the same scratch.
    [(1, 64, 32, 8, 128, 16, 128, 4096), (2, 12, 32, 8, 128, 16, 100, 1500)],
    # The TinyLlama engine's decode shape (D 64, G 4), then a smaller one.
    [(3, 32, 32, 4, 64, 16, 500, 700), (4, 5, 32, 4, 64, 16, 3, 90)],
])
def test_noalloc_matches_the_allocating_launch(gpu, cases):
    for i, c in enumerate(cases):
        print("noalloc decode case", c, flush=True)
        q, kc, vc, table, lens, scale = _case(*c)
        want, got = _both(q, kc, vc, table, lens, scale)
        assert np.array_equal(want.view(np.uint16), got.view(np.uint16)), f"call {i}: differs from tsl_launch"
        if i == 1:  # the smaller call against the oracle too
            parity("noalloc decode", got, oracle.decode_attention(q, kc, vc, table, lens, scale))


def test_noalloc_rejects_shapes_beyond_its_scratch(gpu):
    # 1024 sequences x 8 kv heads of D 128 need ~138 MB of states (> 64 MiB).
    rc = T.lib().tsl_decode_attention_noalloc(0, 0, 0, 0, 0, 0, ctypes.c_float(0.1), 1024, 32, 8, 128, 65536, 16,
                                              256)
    assert rc == -2 and "scratch" in T.lib().tsl_last_error().decode()
    rc = T.lib().tsl_decode_attention_noalloc(0, 0, 0, 0, 0, 0, ctypes.c_float(0.1), 4, 32, 8, 128, 64, 12, 16)
    assert rc == -2  # page size not a power of two
