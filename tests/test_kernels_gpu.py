"""The HIP kernels, launched through the C ABI, against the CPU oracle on
identical seeded inputs: the reference's own test shapes (tests/interp.rs,
tests/emu.rs, tests/llm.rs:108-187) and the benchmark workloads. Tolerance for
float outputs (written in refs.parity): relative Frobenius error <= 1e-3
and max |diff| <= 2e-2; integer, index and copy results bit-exact."""

import numpy as np
import pytest

import oracle
import tessel_amd as T
from tests.refs import assert_close, attention_ref, matmul_ref, paged_ref, parity

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _open(gpu):
    yield


def _say(*a):
    print("[case]", *a, flush=True)


# ---------------------------------------------------------------- matmul.tl

@pytest.mark.parametrize("m,k,n", [(512, 512, 512), (100, 70, 90), (256, 256, 256), (1, 16, 8), (130, 264, 200)])
def test_matmul_vs_oracle(m, k, n):
    _say("matmul", m, k, n)
    r = oracle.Rng(7 + m)
    a, b = r.tensor("f16", [m, k]), r.tensor("f16", [k, n])
    want = oracle.matmul(a, b, 128, 128, 32, 8, threads=8)
    got = T.run("matmul", "matmul", [a, b, np.zeros((m, n), np.float16)], outputs=[2])[2]
    parity("matmul", got, want)
    assert_close("matmul vs f64", got, matmul_ref(a, b), 2e-3)


def test_matmul_exact_integers():
    _say("matmul integers")
    rng = np.random.default_rng(4)
    m, k, n = 300, 136, 264
    a = rng.integers(-4, 5, (m, k)).astype(np.float16)
    b = rng.integers(-4, 5, (k, n)).astype(np.float16)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float16)
    got = T.run("matmul", "matmul", [a, b, np.zeros((m, n), np.float16)], outputs=[2])[2]
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n", [1024, 2048, 4096])
def test_matmul_large_sampled(n):
    # The benchmark GEMM inputs: A, B ~ N(0,1)/sqrt(K); checked at 512 sampled entries
    # against f64 (as src/bench.rs:86-98 does) and, on a block of rows, against the oracle.
    _say("matmul large", n)
    rng = np.random.default_rng(n)
    a = (rng.standard_normal((n, n)) / np.sqrt(n)).astype(np.float16)
    b = (rng.standard_normal((n, n)) / np.sqrt(n)).astype(np.float16)
    got = T.run("matmul", "matmul", [a, b, np.zeros((n, n), np.float16)], outputs=[2])[2]
    i = rng.integers(0, n, 512)
    j = rng.integers(0, n, 512)
    want = np.einsum("sk,ks->s", a[i].astype(np.float64), b[:, j].astype(np.float64))
    assert np.abs(got[i, j].astype(np.float64) - want).max() <= 2e-3 * max(1.0, np.abs(want).max())
    rows = slice(n // 2, n // 2 + 128)
    want_rows = oracle.matmul(np.ascontiguousarray(a[rows]), b, 128, 128, 32, 8, threads=8)
    parity("matmul rows", got[rows], want_rows)


@pytest.mark.parametrize("m,k,n", [(3900, 1024, 4000), (4000, 1000, 3900), (1000, 1000, 1000), (2000, 1024, 2040),
                                   (2040, 1000, 2000)])
def test_matmul_tiles_ragged_exact(m, k, n):
    # The 256 x 256 tiles with ragged M and N: the ping-pong form (K % 64 == 0)
    # and the two-stage form (a partial last K step); 32 x 128 tiles (about
    # 1024^3) with ragged M, N and K; 128 x 128 tiles (about 2048^3) in the
    # ping-pong form (K % 128 == 0) and the three-stage form. Integer operands make
    # every f32 sum exact, so the f16 outputs must equal the rounded integers.
    _say("matmul large tiles", m, k, n)
    rng = np.random.default_rng(m + k)
    a = rng.integers(-3, 4, (m, k)).astype(np.float16)
    b = rng.integers(-3, 4, (k, n)).astype(np.float16)
    want = (a.astype(np.float32) @ b.astype(np.float32)).astype(np.float16)
    got = T.run("matmul", "matmul", [a, b, np.zeros((m, n), np.float16)], outputs=[2])[2]
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("name", ["linear", "linear_residual", "logits"])
def test_llm_matmuls_large_tiles_ragged(name):
    # X W^T on the 256 x 256 ping-pong tiles (ragged M and N) with each plain
    # epilogue, against f64.
    _say("llm mm large tiles", name)
    m, k, n = 3900, 512, 4000
    r = oracle.Rng(900)
    x = r.tensor("f16", [m, k], 1.0)
    w = r.tensor("f16", [n, k], 1.0 / np.sqrt(k))
    prod = x.astype(np.float64) @ w.astype(np.float64).T
    if name == "linear_residual":
        res = r.tensor("f32", [m, n], 1.0)
        args, want = [x, w, res.copy()], res + prod
    elif name == "logits":
        args, want = [x, w, np.zeros((m, n), np.float32)], prod
    else:
        args, want = [x, w, np.zeros((m, n), np.float16)], prod
    got = T.run("llm", name, args, outputs=[2])[2]
    parity(f"{name} {m}x{k}x{n}", got, want)


def test_matmul_f32_and_linear_bias():
    _say("matmul_f32, linear")
    r = oracle.Rng(12)
    m, k, n = 100, 70, 90
    a, b = r.tensor("f32", [m, k]), r.tensor("f32", [k, n])
    got = T.run("matmul", "matmul_f32", [a, b, np.zeros((m, n), np.float32)], outputs=[2])[2]
    assert_close("matmul_f32", got, oracle.matmul_f32(a, b), 1e-5)
    x, w, bias = r.tensor("f16", [m, k]), r.tensor("f16", [n, k]), r.tensor("f16", [n])
    got = T.run("matmul", "linear", [x, w, bias, np.zeros((m, n), np.float16)], outputs=[3])[3]
    parity("linear bias", got, oracle.linear_bias(x, w, bias))


@pytest.mark.parametrize("m,k,n", [(3900, 512, 4000), (1000, 1000, 1000)])
def test_linear_bias_large_tiles_ragged(m, k, n):
    # matmul.tl's biased linear on the 256 x 256 ping-pong tiles (ragged M
    # and N) and on the smaller tiled forms, against f64.
    _say("linear bias large tiles", m, k, n)
    r = oracle.Rng(901 + m)
    x, w = r.tensor("f16", [m, k], 1.0), r.tensor("f16", [n, k], 1.0 / np.sqrt(k))
    bias = r.tensor("f16", [n], 1.0)
    got = T.run("matmul", "linear", [x, w, bias, np.zeros((m, n), np.float16)], outputs=[3])[3]
    want = x.astype(np.float64) @ w.astype(np.float64).T + bias.astype(np.float64)
    parity(f"linear bias {m}x{k}x{n}", got, want)


# ---------------------------------------------------------------- llm.tl matmuls

MM_CASES = ["linear", "linear_residual", "logits", "gate_up"]


def _mm_args(r, name, m, k, n, wscale=0.1):
    x = r.tensor("f16", [m, k], 1.0)
    w = r.tensor("f16", [n, k], wscale)
    if name == "linear":
        return [x, w, np.zeros((m, n), np.float16)], oracle.llm_linear(x, w)
    if name == "linear_residual":
        res = r.tensor("f32", [m, n], 1.0)
        return [x, w, res], oracle.linear_residual(x, w, res)
    if name == "logits":
        return [x, w, np.zeros((m, n), np.float32)], oracle.logits(x, w)
    w2 = r.tensor("f16", [n, k], wscale)
    return [x, w, w2, np.zeros((m, n), np.float16)], oracle.gate_up(x, w, w2)


@pytest.mark.parametrize("m", [16, 32, 64])
@pytest.mark.parametrize("name", MM_CASES)
def test_every_tuning_candidate(name, m):
    # tests/llm.rs:108-187: each tile configuration the reference's tuner may
    # pick, within 1e-2 of the largest output. Here the launchers choose tiles
    # from the shape, so every candidate's meta (a distinct cache key) runs
    # the same code: the outputs must also be bit-identical across them.
    _say("mm candidates", name, m)
    r = oracle.Rng(5)
    k, n = 256, 96
    args, want = _mm_args(r, name, m, k, n)
    first = None
    for meta, warps in T.mm_candidates(m, name == "gate_up"):
        got = T.run("llm", name, [a.copy() for a in args], meta=meta, warps=warps, outputs=[len(args) - 1])
        got = got[len(args) - 1]
        first = got if first is None else first
        assert np.array_equal(got.view(np.uint8), first.view(np.uint8)), (name, m, meta)
        scale = np.abs(want).max()
        err = np.abs(got.astype(np.float64) - want.astype(np.float64)).max()
        assert err <= 1e-2 * scale, (name, m, meta, warps, err, scale)
        parity(f"{name} m={m} {meta}", got, want)


@pytest.mark.parametrize("m", [1, 16, 32, 48, 64, 128, 512, 1024])
@pytest.mark.parametrize("name", MM_CASES)
def test_llm_matmuls_tinyllama_shapes(name, m):
    _say("llm mm", name, m)
    r = oracle.Rng(100 + m)
    k, n = {"linear": (2048, 2560), "linear_residual": (5632, 2048), "logits": (2048, 4000),
            "gate_up": (2048, 5632)}[name]
    args, want = _mm_args(r, name, m, k, n, wscale=1.0 / np.sqrt(k))
    got = T.run("llm", name, args, outputs=[len(args) - 1])[len(args) - 1]
    parity(f"{name} m={m}", got, want)


@pytest.mark.parametrize("name", MM_CASES)
@pytest.mark.parametrize("m,k,n", [(40, 192, 100), (7, 4160, 33), (64, 64, 1), (40, 2176, 100), (3, 384, 17),
                                   (17, 4352, 50), (32, 2048, 5000), (20, 1024, 4500), (5, 128, 40), (9, 256, 70)])
def test_llm_matmuls_ragged_few_rows(name, m, k, n):
    # Few-row (decode-sized) products with ragged M and N, one K step, a long
    # K that is split across workgroups, and (K % 128 == 0) the LDS-staged
    # blocks with uneven K slices and a partial last block of rows; more
    # blocks than CUs at K = 1024 or 2048 take the persistent form. K = 128,
    # 256 and 384 leave wavefronts without a k step of their own (they still
    # load a share of the block).
    _say("llm mm ragged", name, m, k, n)
    r = oracle.Rng(300 + m + n)
    args, want = _mm_args(r, name, m, k, n, wscale=1.0 / np.sqrt(k))
    got = T.run("llm", name, args, outputs=[len(args) - 1])[len(args) - 1]
    parity(f"{name} {m}x{k}x{n}", got, want)


@pytest.mark.parametrize("name", MM_CASES)
@pytest.mark.parametrize("m,k,n", [(200, 4160, 300), (130, 4200, 260)])
def test_llm_matmuls_ragged_split_tiles(name, m, k, n):
    # Prefill-sized products whose 128 x 128 tiles are split over K (uneven
    # slices, a partial last K step, ragged M and N).
    _say("llm mm split tiles", name, m, k, n)
    r = oracle.Rng(400 + m + n)
    args, want = _mm_args(r, name, m, k, n, wscale=1.0 / np.sqrt(k))
    got = T.run("llm", name, args, outputs=[len(args) - 1])[len(args) - 1]
    parity(f"{name} {m}x{k}x{n}", got, want)


@pytest.mark.parametrize("name", ["linear", "linear_residual", "logits"])
@pytest.mark.parametrize("m,k,n", [(900, 1000, 1500), (1000, 1000, 2050)])
def test_llm_matmuls_prefill_tiles_ragged(name, m, k, n):
    # Prefill-sized X W^T on 128 x 64 tiles: one round of workgroups (8
    # wavefronts, 192 tiles) and more than one (4 wavefronts, 264 tiles), with
    # ragged M and N and a partial last K step.
    _say("llm mm prefill tiles", name, m, k, n)
    r = oracle.Rng(500 + m + n)
    args, want = _mm_args(r, name, m, k, n, wscale=1.0 / np.sqrt(k))
    got = T.run("llm", name, args, outputs=[len(args) - 1])[len(args) - 1]
    parity(f"{name} {m}x{k}x{n}", got, want)


def test_split_k_products_repeat_bit_identically():
    # The K-split partials are summed in slice order: repeated launches agree
    # bit for bit.
    _say("split-k repeat")
    r = oracle.Rng(77)
    args, want = _mm_args(r, "linear", 32, 5632, 2048, wscale=1.0 / np.sqrt(5632))
    outs = [T.run("llm", "linear", [a.copy() for a in args], outputs=[2])[2] for _ in range(3)]
    for o in outs[1:]:
        np.testing.assert_array_equal(o.view(np.uint16), outs[0].view(np.uint16))
    parity("split-k linear", outs[0], want)
    args, want = _mm_args(r, "linear_residual", 512, 5632, 2048, wscale=1.0 / np.sqrt(5632))
    outs = [T.run("llm", "linear_residual", [a.copy() for a in args], outputs=[2])[2] for _ in range(3)]
    for o in outs[1:]:
        np.testing.assert_array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    parity("split-k tiles linear_residual", outs[0], want)


# ---------------------------------------------------------------- attention

# The small cases take the key-split form (at most 256 query blocks x heads);
# the last two, the unsplit form at D = 128 and D = 32.
@pytest.mark.parametrize("h,s,d", [(2, 150, 32), (2, 100, 32), (1, 40, 16), (4, 300, 64), (2, 200, 128),
                                   (32, 1100, 128), (24, 1400, 32)])
def test_flash_attention_vs_oracle(h, s, d):
    _say("flash", h, s, d)
    r = oracle.Rng(4 + s)
    q, k, v = (r.tensor("f16", [h, s, d]) for _ in range(3))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    want = oracle.flash_attention(q, k, v, scale, threads=8)
    got = T.run("attention", "flash_attention", [q, k, v, np.zeros_like(q)], [T.F32(scale)], outputs=[3])[3]
    parity("flash", got, want)
    assert_close("flash vs f64", got, attention_ref(q, k, v, scale), 5e-3)


@pytest.mark.parametrize("s", [512, 1024])
def test_flash_attention_baseline_shapes(s):
    # The benchmark attention shape (H 32, D 64) against the oracle.
    _say("flash baseline", s)
    rng = np.random.default_rng(s)
    q, k, v = (rng.standard_normal((32, s, 64)).astype(np.float16) for _ in range(3))
    want = oracle.flash_attention(q, k, v, 0.125, threads=8)
    got = T.run("attention", "flash_attention", [q, k, v, np.zeros_like(q)], [T.F32(0.125)], outputs=[3])[3]
    parity("flash baseline", got, want)


@pytest.mark.parametrize("name", ["flash_attention", "prefill_attention"])
@pytest.mark.parametrize("s,h", [(300, 4), (2000, 4), (2000, 24)])
def test_attention_scores_that_outgrow_the_running_max(name, s, h):
    # Keys of later blocks scaled up 12x (scores jump by far more than 2^16
    # in the exp2 domain): p against the stale running max overflows f16, and
    # the block is redone through its max. Short and long sequences (both
    # key-split forms, and at 24 heads the form with the scale folded into Q),
    # plain and prefill (GQA, two packed prompts).
    _say("attention growth", name, s, h)
    rng = np.random.default_rng(s + 7)
    if name == "flash_attention":
        q, k, v = (rng.standard_normal((h, s, 64)).astype(np.float16) for _ in range(3))
        k[:, s // 3:s // 3 + 40] *= np.float16(12)
        k[:, 2 * s // 3:] *= np.float16(3)
        want = oracle.flash_attention(q, k, v, 0.125, threads=8)
        got = T.run("attention", name, [q, k, v, np.zeros_like(q)], [T.F32(0.125)], outputs=[3])[3]
    else:
        q = rng.standard_normal((s, 2 * h, 64)).astype(np.float16)
        k, v = (rng.standard_normal((s, h // 2, 64)).astype(np.float16) for _ in range(2))
        k[s // 3:s // 3 + 40] *= np.float16(12)
        starts = np.where(np.arange(s) < s // 2, 0, s // 2).astype(np.int32)
        want = oracle.prefill_attention(q, k, v, starts, 0.125, threads=8)
        got = T.run("llm", name, [q, k, v, starts, np.zeros_like(q)], [T.F32(0.125)], outputs=[4])[4]
    parity("attention growth", got, want)


@pytest.mark.parametrize("s", [2048, 4096])
def test_flash_attention_long_sampled(s):
    # Long sequences: sampled query rows against the f64 closed form
    # (src/bench.rs:135-160 checks 4 rows); 16 rows of varied heads here.
    _say("flash long", s)
    rng = np.random.default_rng(s)
    q, k, v = (rng.standard_normal((32, s, 64)).astype(np.float16) for _ in range(3))
    got = T.run("attention", "flash_attention", [q, k, v, np.zeros_like(q)], [T.F32(0.125)], outputs=[3])[3]
    for _ in range(16):
        hh, i = int(rng.integers(0, 32)), int(rng.integers(0, s))
        sc = k[hh, :i + 1].astype(np.float64) @ q[hh, i].astype(np.float64) * 0.125
        e = np.exp(sc - sc.max())
        want = e @ v[hh, :i + 1].astype(np.float64) / e.sum()
        parity(f"flash row {hh},{i}", got[hh, i], want)


@pytest.mark.parametrize("s", [2048, 4096])
def test_flash_attention_long_whole_heads_vs_oracle(s):
    # The benchmark attention shape at its long sizes: the 32-head launch, with four
    # whole heads (every row) against the interpreter restatement of
    # kernels/attention.tl:4-24 (heads are independent programs, so the
    # oracle runs on just those heads' slices).
    _say("flash long heads", s)
    rng = np.random.default_rng(s + 1)
    q, k, v = (rng.standard_normal((32, s, 64)).astype(np.float16) for _ in range(3))
    got = T.run("attention", "flash_attention", [q, k, v, np.zeros_like(q)], [T.F32(0.125)], outputs=[3])[3]
    heads = [0, 9, 22, 31]
    sl = lambda x: np.ascontiguousarray(x[heads])
    want = oracle.flash_attention(sl(q), sl(k), sl(v), 0.125, threads=16)
    parity(f"flash S={s} heads {heads}", got[heads], want)


def _packed(seed, lens, h, g, d):
    r = oracle.Rng(seed)
    s = sum(lens)
    q = r.tensor("f16", [s, h, d])
    k = r.tensor("f16", [s, g, d])
    v = r.tensor("f16", [s, g, d])
    starts = np.concatenate([np.full(l, sum(lens[:i]), np.int32) for i, l in enumerate(lens)])
    return q, k, v, starts


@pytest.mark.parametrize("lens,h,g,d", [([90], 4, 2, 16), ([70, 20], 4, 2, 16), ([512, 512], 32, 4, 64),
                                         ([300, 5, 130, 64], 8, 2, 64), ([1000], 32, 4, 64),
                                         ([600, 7, 700, 300], 32, 4, 64), ([1500, 40], 32, 8, 128)])
def test_prefill_attention_vs_oracle(lens, h, g, d):
    _say("prefill", lens, h, g, d)
    q, k, v, starts = _packed(11 + len(lens), lens, h, g, d)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    want = oracle.prefill_attention(q, k, v, starts, scale, threads=8)
    got = T.run("llm", "prefill_attention", [q, k, v, starts, np.zeros_like(q)], [T.F32(scale)], outputs=[4])[4]
    parity("prefill", got, want)


def test_paged_attention_reference_case():
    # tests/interp.rs:126-136 and tests/emu.rs:174-175.
    _say("paged")
    r = oracle.Rng(5)
    q, kc, vc, table, lens, scale = oracle.paged_case(r, 3, 2, 32, 16, [37, 1, 64])
    want = oracle.decode_attention(q, kc, vc, table, lens, scale)
    got = T.run("attention", "paged_attention", [q, kc, vc, table, lens, np.zeros_like(q)], [T.F32(scale)],
                outputs=[5])[5]
    parity("paged", got, want)
    assert_close("paged vs f64", got, paged_ref(q, kc, vc, table, lens, scale), 3e-3)


@pytest.mark.parametrize("b,h,d,p,lo,hi", [(6, 16, 64, 16, 1, 2000), (3, 32, 128, 32, 0, 4000), (5, 8, 128, 16, 900, 1500)])
def test_paged_attention_long_tables(b, h, d, p, lo, hi):
    # paged_attention (G = H) with tables longer than 64 pages: the balanced
    # form, 8 heads at a time (16 and 32 heads) or all 8, one query head each.
    _say("paged long", b, h, d, p)
    q, kc, vc, table, lens, scale = decode_case(9 + b, b=b, h=h, g=h, d=d, p=p, lo=lo, hi=hi,
                                                mp=max(65, (hi + p - 1) // p))
    want = oracle.decode_attention(q, kc, vc, table, lens, scale, threads=8)
    got = T.run("attention", "paged_attention", [q, kc, vc, table, lens, np.zeros_like(q)], [T.F32(scale)],
                outputs=[5])[5]
    parity("paged long", got, want)


def decode_case(seed, b=64, h=32, g=8, d=128, p=16, lo=128, hi=4096, mp=None):
    """The benchmark decode workload: lens ~ U[lo, hi], pages assigned by a seeded
    permutation into int32 block tables, KV pool N(0,1) f16."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, b).astype(np.int32)
    need = (lens + p - 1) // p
    mp = int(need.max()) if mp is None else mp
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


def _decode(q, kc, vc, table, lens, scale):
    return T.run("llm", "decode_attention", [q, kc, vc, table, lens, np.zeros_like(q)], [T.F32(scale)],
                 outputs=[5])[5]


@pytest.mark.parametrize("cfg", [dict(b=64, h=32, g=8, d=128, p=16),
                                 dict(b=8, h=32, g=4, d=64, p=16, lo=1, hi=700),
                                 dict(b=5, h=4, g=2, d=16, p=8, lo=0, hi=60),
                                 dict(b=3, h=8, g=8, d=32, p=16, lo=1, hi=300),
                                 dict(b=6, h=16, g=1, d=128, p=64, lo=1, hi=3000),
                                 dict(b=9, h=8, g=4, d=64, p=32, lo=0, hi=2100),
                                 # tables longer than 64 pages take the balanced (persistent) path:
                                 # fewer units than workgroups, many short sequences (lens 0
                                 # among them) under a long table, P 64, 3-stage rings
                                 dict(b=1, h=32, g=8, d=128, p=16, lo=1100, hi=1100),
                                 dict(b=40, h=32, g=8, d=64, p=16, lo=0, hi=40, mp=80),
                                 dict(b=3, h=16, g=4, d=128, p=64, lo=1, hi=9000),
                                 dict(b=17, h=32, g=4, d=128, p=16, lo=2000, hi=5000),
                                 # 16 and 32 kv heads: 8 at a time (head groups as sequences of their own)
                                 dict(b=5, h=32, g=16, d=128, p=16, lo=100, hi=3000),
                                 dict(b=3, h=32, g=32, d=64, p=32, lo=0, hi=4000)])
def test_decode_attention_vs_oracle(cfg):
    _say("decode", cfg)
    q, kc, vc, table, lens, scale = decode_case(1, **cfg)
    want = oracle.decode_attention(q, kc, vc, table, lens, scale, threads=8)
    got = _decode(q, kc, vc, table, lens, scale)
    parity("decode", got, want)


def test_decode_attention_repeat_launches():
    """Multi-chunk sequences write per-chunk partial states into the handle's
    scratch and a second kernel merges them: back-to-back launches on one
    handle (reusing that scratch) agree bit for bit, and with the oracle."""
    _say("decode repeat")
    q, kc, vc, table, lens, scale = decode_case(4, b=12, h=32, g=8, d=128, p=16, lo=300, hi=4096)
    T.open()
    kern = T.kernel("llm", "decode_attention", [list(q.shape), list(kc.shape), list(vc.shape), list(table.shape),
                                                 list(lens.shape), list(q.shape)])
    bufs = [T.tensor(x) for x in (q, kc, vc, table, lens)] + [T.alloc(q.nbytes), T.F32(scale)]
    outs = []
    for _ in range(3):
        T.launch(kern, bufs)
        outs.append(T.read_array(bufs[5], np.float16, q.shape))
    for o in outs[1:]:
        np.testing.assert_array_equal(o.view(np.uint16), outs[0].view(np.uint16))
    parity("decode repeat", outs[0], oracle.decode_attention(q, kc, vc, table, lens, scale, threads=8))
    for x in bufs[:6]:
        T.free(x)


@pytest.mark.parametrize("mp", [None, 100])
def test_decode_attention_indexing_properties(mp):
    # mp None: tables of at most 64 pages (the single-chunk form); 100: the
    # balanced form, whose range boundaries move with every sequence's length.
    _say("decode properties", mp)
    q, kc, vc, table, lens, scale = decode_case(2, b=16, h=32, g=8, d=128, p=16, lo=1, hi=1000, mp=mp)
    base = _decode(q, kc, vc, table, lens, scale)
    # The same tokens at other pool positions: bit-identical (only the token order matters).
    perm = np.random.default_rng(3).permutation(kc.shape[0])
    inv = np.argsort(perm).astype(np.int32)
    got = _decode(q, np.ascontiguousarray(kc[perm]), np.ascontiguousarray(vc[perm]), inv[table], lens, scale)
    np.testing.assert_array_equal(got.view(np.uint16), base.view(np.uint16))
    # Pages outside the pool read as zeros (scores 0, values 0), as the oracle says.
    t2 = table.copy()
    t2[3, 0] = kc.shape[0] + 5
    t2[5, 1] = -7
    want = oracle.decode_attention(q, kc, vc, t2, lens, scale, threads=8)
    parity("decode oob pages", _decode(q, kc, vc, t2, lens, scale), want)
    # lens 0 gives NaN rows; the rest unchanged (bit for bit where the work
    # split does not depend on the lengths, else within the tolerance).
    l0 = lens.copy()
    l0[[2, 9]] = 0
    got = _decode(q, kc, vc, table, l0, scale)
    assert np.isnan(got[[2, 9]].astype(np.float32)).all()
    keep = [i for i in range(16) if i not in (2, 9)]
    if mp is None:
        np.testing.assert_array_equal(got[keep].view(np.uint16), base[keep].view(np.uint16))
    else:
        parity("decode lens 0 rest", got[keep], base[keep])
    # NaN garbage past lens inside a sequence's last page: the .tl loads whole
    # pages, so V's reaches the output (p = 0 times NaN), while K's is masked
    # off before it counts.
    ragged = np.flatnonzero(lens % 16 != 0)
    bv, bk = int(ragged[0]), int(ragged[1])
    kn, vn = kc.copy(), vc.copy()
    vn[table[bv, (lens[bv] - 1) // 16], lens[bv] % 16] = np.nan
    kn[table[bk, (lens[bk] - 1) // 16], lens[bk] % 16] = np.nan
    want = oracle.decode_attention(q, kn, vn, table, lens, scale, threads=8)
    assert np.isnan(want[bv].astype(np.float32)).any() and not np.isnan(want[bk].astype(np.float32)).any()
    parity("decode nan past lens", _decode(q, kn, vn, table, lens, scale), want)
    # Tokens past the table's MP * P read page 0 (the interpreter's out-of-range load).
    w = 8 if mp is None else 70
    tb = np.ascontiguousarray(table[:, :w])
    l3 = np.minimum(lens + (0 if mp is None else 200), w * 16 + 40).astype(np.int32)
    want = oracle.decode_attention(q, kc, vc, tb, l3, scale, threads=8)
    parity("decode past table", _decode(q, kc, vc, tb, l3, scale), want)


# ---------------------------------------------------------------- rows

@pytest.mark.parametrize("rows,cols,bc", [(10, 700, 1024), (4096, 4096, 4096), (7, 5000, 8192), (3, 40, 16),
                                         (9, 3000, 4096), (5, 4096, 4096)])
def test_softmax(rows, cols, bc):
    _say("softmax", rows, cols, bc)
    r = oracle.Rng(2)
    x = r.tensor("f32", [rows, cols], 4.0)
    want = oracle.softmax(x, BC=bc, threads=8)
    got = T.run("basic", "softmax", [x, np.zeros_like(x)], meta=[("BC", bc)], outputs=[1])[1]
    parity("softmax", got, want)
    assert np.abs(got - want).max() <= 1e-6


def test_softmax_special_values():
    # Whole 4096-column rows (the per-chunk form): -inf over every chunk of
    # some lanes and at the row's end, a row of -inf, +inf and NaN entries,
    # against the oracle (NaN positions included).
    _say("softmax special values")
    r = oracle.Rng(5)
    x = r.tensor("f32", [8, 4096], 4.0)
    x[1, :1024] = -np.inf
    x[2, 3000:] = -np.inf
    x[3, :] = -np.inf
    x[4, 17] = np.inf
    x[5, 4000] = np.nan
    x[6, ::2] = -np.inf
    x[7, :] = -1e30
    x[7, 5] = -1e29
    want = oracle.softmax(x, BC=4096, threads=8)
    got = T.run("basic", "softmax", [x, np.zeros_like(x)], meta=[("BC", 4096)], outputs=[1])[1]
    parity("softmax special", got, want)
    ok = ~np.isnan(want)
    assert np.abs(got[ok] - want[ok]).max() <= 1e-6


@pytest.mark.parametrize("rows,cols,bc", [(10, 700, 1024), (4096, 4096, 4096), (5, 9000, 16384), (4, 100, 64),
                                         (13, 2048, 2048), (6, 4096, 4096)])
def test_rmsnorm_basic(rows, cols, bc):
    _say("rmsnorm basic", rows, cols, bc)
    r = oracle.Rng(3)
    x = r.tensor("f16", [rows, cols], 2.0)
    w = r.tensor("f16", [cols], 1.0)
    want = oracle.rmsnorm_basic(x, w, 1e-5, BC=bc, threads=8)
    got = T.run("basic", "rmsnorm", [x, w, np.zeros_like(x)], [T.F32(1e-5)], meta=[("BC", bc)], outputs=[2])[2]
    parity("rmsnorm", got, want)


def test_add_exact():
    r = oracle.Rng(1)
    for n in (3000, 1 << 20, 5):
        x, y = r.tensor("f32", [n]), r.tensor("f32", [n])
        got = T.run("basic", "add", [x, y, np.zeros_like(x)], outputs=[2])[2]
        np.testing.assert_array_equal(got, x + y)


@pytest.mark.parametrize("t,dm", [(16, 2048), (5, 64), (32, 2048), (3, 1000)])
def test_llm_rows(t, dm):
    _say("llm rows", t, dm)
    r = oracle.Rng(8)
    bc = 1 << (dm - 1).bit_length()
    x = r.tensor("f32", [t, dm], 3.0)
    w = r.tensor("f16", [dm], 1.0)
    got = T.run("llm", "rmsnorm", [x, w, np.zeros((t, dm), np.float16)], [T.F32(1e-5)], meta=[("BC", bc)],
                outputs=[2])[2]
    parity("llm rmsnorm", got, oracle.rmsnorm(x, w, 1e-5, BC=bc))
    idx = np.array([t - 1, 0, t // 2, 0], np.int32)
    got = T.run("llm", "rmsnorm_rows", [x, idx, w, np.zeros((4, dm), np.float16)], [T.F32(1e-5)],
                meta=[("BC", bc)], outputs=[3])[3]
    parity("rmsnorm_rows", got, oracle.rmsnorm_rows(x, idx, w, 1e-5, BC=bc))
    v = 300
    e = r.tensor("f16", [v, dm])
    tok = np.array([(i * 37) % v for i in range(t - 1)] + [v + 3], np.int32)
    got = T.run("llm", "embed", [tok, e, np.zeros((t, dm), np.float32)], meta=[("BD", min(bc, 1024))],
                outputs=[2])[2]
    np.testing.assert_array_equal(got, oracle.embed(tok, e))


@pytest.mark.parametrize("m,k,n,mode", [(32, 5632, 2048, "split"), (32, 2048, 2048, "own split"),
                                        (7, 4160, 36, "split"), (40, 11008, 4096, "split"),
                                        (5, 1024, 1000, "own split"), (7, 4160, 33, "pair"), (128, 2048, 2048, "pair"),
                                        (200, 4160, 300, "pair"), (512, 5632, 2048, "pair")])
def test_fused_linear_residual_rmsnorm(m, k, n, mode):
    # The engine's fused launch (fused/linear_residual_rmsnorm): R += X W^T,
    # then Y = rmsnorm(R) Wn, against the oracle and against llm/linear_residual
    # followed by llm/rmsnorm. "pair": bits of exactly that pair (prefill
    # shapes split over K end in the reduce-and-normalise kernel too).
    # "split": K is split as linear_residual splits it, so R and Y have the
    # pair's bits too. "own split": a split linear_residual does not make, so
    # R and Y are within the float tolerance.
    _say("fused linear_residual_rmsnorm", m, k, n)
    r = oracle.Rng(500 + m + n)
    x = r.tensor("f16", [m, k], 1.0)
    w = r.tensor("f16", [n, k], 1.0 / np.sqrt(k))
    res = r.tensor("f32", [m, n], 1.0)
    wn = r.tensor("f16", [n], 1.0)
    bc = 1 << (n - 1).bit_length()
    eps = [T.F32(1e-5)]
    out = T.run("fused", "linear_residual_rmsnorm", [x, w, res.copy(), wn, np.zeros((m, n), np.float16)], eps,
                meta=[("BC", bc)], outputs=[2, 4])
    pr = T.run("llm", "linear_residual", [x, w, res.copy()], outputs=[2])[2]
    py = T.run("llm", "rmsnorm", [pr, wn, np.zeros((m, n), np.float16)], eps, meta=[("BC", bc)], outputs=[2])[2]
    want_r = oracle.linear_residual(x, w, res.copy())
    parity("fused R", out[2], want_r)
    parity("fused Y", out[4], oracle.rmsnorm(want_r.astype(np.float32), wn, 1e-5, BC=bc))
    if mode in ("split", "pair"):
        np.testing.assert_array_equal(out[2].view(np.uint32), pr.view(np.uint32))
        np.testing.assert_array_equal(out[4].view(np.uint16), py.view(np.uint16))


def test_argmax_rows_vs_the_sequential_scan():
    # fused/argmax (the scheduler's next token) against src/llm/mod.rs:132-140
    # restated (oracle.argmax): first index of the largest value under `>`,
    # a NaN at index 0 wins, later NaNs never do, +0 and -0 tie.
    _say("argmax rows")
    rng = np.random.default_rng(9)
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    rows = [np.array([1, 3, 3, 2], np.float32), np.array([nan, 5, 7], np.float32),
            np.array([2, nan, 7, nan, 7], np.float32), np.array([-0.0, 0.0, -0.0], np.float32),
            np.array([0.0, -0.0], np.float32), np.array([-inf, -inf, -inf], np.float32),
            np.array([1, nan, nan, nan], np.float32), np.array([-1, -2, inf, inf], np.float32),
            np.array([5], np.float32)]
    for v in (4, 37, 1000, 32000, 32003):
        rows.append(rng.integers(0, 6, v).astype(np.float32))  # many ties
        x = rng.standard_normal(v).astype(np.float32)
        x[rng.integers(0, v, 3)] = nan
        rows.append(x)
        rows.append(np.full(v, -inf, np.float32))
    for r in rows:
        for b in (1, 3):  # several rows of the same values at once
            x = np.tile(r, (b, 1))
            got = T.run("fused", "argmax", [x, np.zeros(b, np.int32)], outputs=[1])[1]
            want = oracle.argmax(r)
            assert (got == want).all(), (r[:8], got, want)


@pytest.mark.parametrize("cfgname,t", [("tinyllama", 1), ("tinyllama", 32), ("tinyllama", 40), ("tinyllama", 64),
                                       ("tinyllama", 80), ("tiny", 16)])
def test_fused_qkv_rope_kv(cfgname, t):
    # The engine's fused launch (fused/qkv_rope_kv): llm/linear, then
    # llm/rope_q and llm/kv_write of its QKV. Decode-sized TinyLlama batches
    # run the one-kernel form (rotation in the projection's epilogue); t = 80
    # and the tiny config (dim 64) launch the three. Either way Q, K, V and
    # the cache are the bits of the three launches. Slots outside the cache
    # and positions outside the tables are included.
    _say("fused qkv_rope_kv", cfgname, t)
    cfg = getattr(oracle.Config, cfgname)()
    c, s = oracle.rope_tables(cfg)
    H, G, D, dm, W = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.dim, cfg.qkv()
    r = oracle.Rng(21 + t)
    x = r.tensor("f16", [t, dm], 1.0)
    wq = r.tensor("f16", [W, dm], 1.0 / np.sqrt(dm))
    pos = np.array([(i * 97) % cfg.max_pos for i in range(t)], np.int32)
    pos[0] = cfg.max_pos + 5  # outside the tables: rotated values are 0
    NS = 3 * t + 7
    slot = np.array([(i * 7) % NS for i in range(t)], np.int32)
    slot[-1] = NS  # dropped
    if t > 1:
        slot[-2] = -1
    Kc = r.tensor("f16", [NS, G, D])
    Vc = r.tensor("f16", [NS, G, D])
    z = lambda *sh: np.zeros(sh, np.float16)
    args = [x, wq, z(t, W), pos, slot, c, s, z(t, H, D), Kc, Vc, z(t, G, D), z(t, G, D)]
    got = T.run("fused", "qkv_rope_kv", [a.copy() for a in args])
    qkv = T.run("llm", "linear", [x, wq, z(t, W)], outputs=[2])[2]
    want = T.run("fused", "rope_kv", [qkv, pos, slot, c, s, z(t, H, D), Kc.copy(), Vc.copy(), z(t, G, D), z(t, G, D)])
    for gi, wi, name in ((7, 5, "Q"), (8, 6, "Kc"), (9, 7, "Vc"), (10, 8, "K"), (11, 9, "V")):
        np.testing.assert_array_equal(got[gi].view(np.uint16), want[wi].view(np.uint16), err_msg=name)
    parity("fused Q", got[7], oracle.rope_q(oracle.llm_linear(x, wq), pos, c, s, H, D))


def _ss_ref(r):
    """SS[b][m]: the squares of R[m][8 b .. 8 b + 7] added in column order in f32."""
    m, n = r.shape
    nb = (n + 7) // 8
    pad = np.zeros((m, nb * 8), np.float32)
    pad[:, :n] = r
    sq = (pad * pad).reshape(m, nb, 8)
    acc = np.zeros((m, nb), np.float32)
    for j in range(8):
        acc = (acc + sq[:, :, j]).astype(np.float32)
    return np.ascontiguousarray(acc.T)


def _prenorm(r, m, ko, dm):
    """fused/linear_residual_prenorm on seeded inputs, checked: R against the
    oracle, Y = f16(R Wn) and the sums of squares bit-exact against their
    definitions from the returned R. Returns (Y, SS, the oracle's R, Wn)."""
    x = r.tensor("f16", [m, ko], 1.0)
    w = r.tensor("f16", [dm, ko], 1.0 / np.sqrt(ko))
    res = r.tensor("f32", [m, dm], 1.0)
    wn = r.tensor("f16", [dm], 1.0)
    nb = (dm + 7) // 8
    out = T.run("fused", "linear_residual_prenorm",
                [x, w, res.copy(), wn, np.zeros((m, dm), np.float16), np.zeros((nb, m), np.float32),
                 np.zeros(1, np.int32)], outputs=[2, 4, 5, 6])
    assert out[6][0] == 0  # no overflow flagged
    want_r = oracle.linear_residual(x, w, res.copy())
    parity("prenorm R", out[2], want_r)
    y_def = (out[2].astype(np.float32) * wn.astype(np.float32)).astype(np.float16)
    np.testing.assert_array_equal(out[4].view(np.uint16), y_def.view(np.uint16))
    np.testing.assert_array_equal(out[5].view(np.uint32), _ss_ref(out[2]).view(np.uint32))
    return out[4], out[5], want_r, wn


@pytest.mark.parametrize("m,ko,dm", [(32, 2048, 2048), (5, 192, 100)])
def test_fused_prenorm_flags_f16_overflow(m, ko, dm):
    # Y = f16(R Wn) overflows where |R Wn| >= 65520: one row's residual entry
    # set to 3e4 with its norm weight 4 must set OVF[0] (the fused kernel at
    # 32 x 2048, the fallback at 5 x 100); R stays exact against the oracle.
    _say("fused prenorm overflow flag", m, ko, dm)
    r = oracle.Rng(77 + m)
    x = r.tensor("f16", [m, ko], 1.0)
    w = r.tensor("f16", [dm, ko], 1.0 / np.sqrt(ko))
    res = r.tensor("f32", [m, dm], 1.0)
    res[m // 2, dm // 3] = 3e4
    wn = r.tensor("f16", [dm], 1.0)
    wn[dm // 3] = 4.0
    nb = (dm + 7) // 8
    out = T.run("fused", "linear_residual_prenorm",
                [x, w, res.copy(), wn, np.zeros((m, dm), np.float16), np.zeros((nb, m), np.float32),
                 np.zeros(1, np.int32)], outputs=[2, 4, 6])
    parity("prenorm R", out[2], oracle.linear_residual(x, w, res.copy()))
    assert np.isinf(out[4][m // 2, dm // 3])
    assert out[6][0] == 1


@pytest.mark.parametrize("m,ko,dm,f", [(32, 2048, 2048, 5632), (17, 5632, 2048, 5632), (9, 1024, 1024, 4000),
                                       (40, 2048, 2048, 5632), (100, 192, 100, 300)])
def test_fused_prenorm_then_gate_up_rs(m, ko, dm, f):
    # The engine's decode-step pair for the MLP input: the o projection leaves
    # Y = f16(R Wn) and per-8-column sums of squares (linear_residual_prenorm),
    # and gate_up_rs scales each row's products by 1 / rms(R): against the
    # oracle's linear_residual -> rmsnorm -> gate_up. M <= 32 with K = 1024 or
    # 2048 and F / 8 > the CUs take the fused kernels; the others the fallbacks.
    # Two launches of the pair agree bit for bit.
    _say("fused prenorm + gate_up_rs", m, ko, dm, f)
    r = oracle.Rng(810 + m + f)
    y, ss, want_r, wn = _prenorm(r, m, ko, dm)
    wg = r.tensor("f16", [f, dm], 1.0 / np.sqrt(dm))
    wu = r.tensor("f16", [f, dm], 1.0 / np.sqrt(dm))
    eps = [T.F32(1e-5)]
    got = [T.run("fused", "gate_up_rs", [y, ss, wg, wu, np.zeros((m, f), np.float16)], eps, outputs=[4])[4]
           for _ in range(2)]
    np.testing.assert_array_equal(got[0].view(np.uint16), got[1].view(np.uint16))
    bc = 1 << (dm - 1).bit_length()
    h = oracle.rmsnorm(want_r.astype(np.float32), wn, 1e-5, BC=bc)
    parity("gate_up_rs", got[0], oracle.gate_up(h, wg, wu))


@pytest.mark.parametrize("cfgname,t", [("tinyllama", 32), ("tinyllama", 7), ("tinyllama", 40), ("tiny", 16)])
def test_fused_prenorm_then_qkv_rs_rope_kv(cfgname, t):
    # The engine's decode-step pair for the next layer's attention input: the
    # down projection leaves Y = f16(R Wn) and the sums of squares, and
    # qkv_rs_rope_kv scales each row's QKV sums by 1 / rms(R) before the
    # f16 rounding, the rotation and the cache write: against the oracle's
    # rmsnorm -> llm/linear -> rope_q / kv_write chain (within the float
    # tolerance; slots and positions outside the tables included; cache slots
    # nobody writes bit-exact). t = 40 and the tiny config take the
    # fallbacks.
    _say("fused prenorm + qkv_rs_rope_kv", cfgname, t)
    cfg = getattr(oracle.Config, cfgname)()
    c, s = oracle.rope_tables(cfg)
    H, G, D, dm, W = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.dim, cfg.qkv()
    r = oracle.Rng(31 + t)
    y, ss, want_r, wn = _prenorm(r, t, cfg.ffn, dm)
    wq = r.tensor("f16", [W, dm], 1.0 / np.sqrt(dm))
    pos = np.array([(i * 97) % cfg.max_pos for i in range(t)], np.int32)
    pos[0] = cfg.max_pos + 5
    NS = 3 * t + 7
    slot = np.array([(i * 7) % NS for i in range(t)], np.int32)
    slot[-1] = NS
    slot[-2] = -1
    Kc = r.tensor("f16", [NS, G, D])
    Vc = r.tensor("f16", [NS, G, D])
    z = lambda *sh: np.zeros(sh, np.float16)
    got = T.run("fused", "qkv_rs_rope_kv",
                [y, wq, z(t, W), pos, slot, c, s, z(t, H, D), Kc.copy(), Vc.copy(), z(t, G, D), z(t, G, D), ss],
                [T.F32(cfg.eps)])
    # The oracle's chain: rmsnorm of R, llm/linear, then llm/rope_q and
    # llm/kv_write of that QKV (src/llm/engine.rs launch order).
    bc = 1 << (dm - 1).bit_length()
    h = oracle.rmsnorm(want_r.astype(np.float32), wn, cfg.eps, BC=bc)
    qkv = oracle.llm_linear(h, wq)  # (the fused kernel leaves its QKV argument unwritten)
    want_q = oracle.rope_q(qkv, pos, c, s, H, D)
    wKc, wVc, wK, wV = oracle.kv_write(qkv, pos, slot, c, s, Kc.copy(), Vc.copy(), z(t, G, D), z(t, G, D))
    for i, name, want in ((7, "Q", want_q), (8, "Kc", wKc), (9, "Vc", wVc), (10, "K", wK), (11, "V", wV)):
        parity(f"qkv_rs {name}", got[i], want)
    # Slots outside [0, NS) (the last two rows) write nothing: every cache
    # slot no row wrote keeps its bits.
    written = set(int(x) for x in slot if 0 <= x < NS)
    untouched = [i for i in range(NS) if i not in written]
    np.testing.assert_array_equal(got[8][untouched].view(np.uint16), Kc[untouched].view(np.uint16))
    np.testing.assert_array_equal(got[9][untouched].view(np.uint16), Vc[untouched].view(np.uint16))
    # A position past the rotary tables (row 0) rotates by zeros, as the
    # oracle's rope_q does: its Q row is all zero on both sides.
    assert not want_q[0].any() and not got[7][0].any()


@pytest.mark.parametrize("cfgname", ["tiny", "tinyllama"])
def test_rope_and_kv_write(cfgname):
    _say("rope/kv_write", cfgname)
    cfg = getattr(oracle.Config, cfgname)()
    c, s = oracle.rope_tables(cfg)
    H, G, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    Tn, W = 16, cfg.qkv()
    r = oracle.Rng(13)
    qkv = r.tensor("f16", [Tn, W])
    pos = np.array([(i * 97) % cfg.max_pos for i in range(Tn)], np.int32)
    q = T.run("llm", "rope_q", [qkv, pos, c, s, np.zeros((Tn, H, D), np.float16)], outputs=[4])[4]
    want = oracle.rope_q(qkv, pos, c, s, H, D)
    parity("rope_q", q, want)
    assert np.abs(q.astype(np.float32) - want.astype(np.float32)).max() <= 2e-3 * max(1, np.abs(want).max())
    NS = 40
    slot = np.array([(i * 7) % NS for i in range(Tn - 2)] + [NS, -1], np.int32)  # last two dropped
    Kc = r.tensor("f16", [NS, G, D])
    Vc = r.tensor("f16", [NS, G, D])
    K = np.zeros((Tn, G, D), np.float16)
    V = np.zeros((Tn, G, D), np.float16)
    out = T.run("llm", "kv_write", [qkv, pos, slot, c, s, Kc, Vc, K, V])
    wKc, wVc, wK, wV = oracle.kv_write(qkv, pos, slot, c, s, Kc, Vc, K, V)
    np.testing.assert_array_equal(out[6], wVc)  # values: copies, bit-exact
    np.testing.assert_array_equal(out[8], wV)
    parity("kv_write K", out[7], wK)
    parity("kv_write Kc", out[5], wKc)
    untouched = [i for i in range(NS) if i not in set(slot[:Tn - 2].tolist())]
    np.testing.assert_array_equal(out[5][untouched], Kc[untouched])
    # The engine's fused launch (fused/rope_kv) writes exactly what the two do.
    # (It takes 8 columns per thread when D = 2 D2 with D2 % 8 == 0, as both
    # configs here; positions outside the tables rotate by zeros.)
    for pp in (pos, np.where(np.arange(Tn) % 5 == 3, cfg.max_pos + 3, pos).astype(np.int32)):
        q = T.run("llm", "rope_q", [qkv, pp, c, s, np.zeros((Tn, H, D), np.float16)], outputs=[4])[4]
        out = T.run("llm", "kv_write", [qkv, pp, slot, c, s, Kc, Vc, K, V])
        fz = T.run("fused", "rope_kv", [qkv, pp, slot, c, s, np.zeros((Tn, H, D), np.float16), Kc, Vc, K, V])
        for got, ref in ((fz[5], q), (fz[6], out[5]), (fz[7], out[6]), (fz[8], out[7]), (fz[9], out[8])):
            np.testing.assert_array_equal(got.view(np.uint16), ref.view(np.uint16))


# ---------------------------------------------------------------- graph replay

def test_graph_replay_of_kernels_with_scratch():
    # Handles that own scratch (split-K projection partials, chunked decode
    # states) recorded into one graph and replayed several times, with eager
    # work on the stream between replays: every replay matches the eager run.
    _say("graph replay")
    T.open()
    r = oracle.Rng(21)
    x = r.tensor("f16", [32, 5632], 1.0)
    w = r.tensor("f16", [2048, 5632], 1.0 / np.sqrt(5632))
    lin = T.kernel("llm", "linear", [[32, 5632], [2048, 5632], [32, 2048]])
    q, kc, vc, table, lens, scale = decode_case(6, b=16, h=32, g=8, d=128, p=16, lo=1000, hi=4096)
    dec = T.kernel("llm", "decode_attention", [list(q.shape), list(kc.shape), list(vc.shape), list(table.shape),
                                               list(lens.shape), list(q.shape)])
    lb = [T.tensor(x), T.tensor(w), T.alloc(32 * 2048 * 2)]
    db = [T.tensor(a) for a in (q, kc, vc, table, lens)] + [T.alloc(q.nbytes), T.F32(scale)]
    T.launch(lin, lb)
    T.launch(dec, db)
    T.sync()
    want_l = T.read_array(lb[2], np.float16, (32, 2048))
    want_d = T.read_array(db[5], np.float16, q.shape)
    parity("graph linear eager", want_l, oracle.llm_linear(x, w))
    parity("graph decode eager", want_d, oracle.decode_attention(q, kc, vc, table, lens, scale, threads=8))
    T.capture_begin()
    T.launch(lin, lb)
    T.launch(dec, db)
    g = T.capture_end()
    nodes = T.graph_nodes(g)
    assert nodes["kernel"] >= 2 and nodes["memset"] == nodes["memcpy"] == nodes["other"] == 0, nodes
    other = T.kernel("llm", "linear", [[32, 5632], [2048, 5632], [32, 2048]])
    ob = [T.tensor(x[::-1].copy()), lb[1], T.alloc(32 * 2048 * 2)]
    for i in range(3):
        for buf in (lb[2], db[5]):
            T.fill_nan(buf)  # replays must rewrite the outputs
        T.replay(g)
        T.launch(other, ob)  # eager work between replays, on the same handle type
        T.sync()
        np.testing.assert_array_equal(T.read_array(lb[2], np.float16, (32, 2048)).view(np.uint16),
                                      want_l.view(np.uint16))
        np.testing.assert_array_equal(T.read_array(db[5], np.float16, q.shape).view(np.uint16),
                                      want_d.view(np.uint16))
    for b in lb + db[:6] + [ob[0], ob[2]]:
        T.free(b)
