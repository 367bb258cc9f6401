"""The CPU oracle pinned against what it must reproduce: the reference's own
interpreter tests (tests/interp.rs, restated with the f64 closed forms of
tests/common/mod.rs), known answers (src/half.rs:69-78), exact integer
cases, brute force on tiny inputs and invariants a dropped term, a wrong
index or a transposed operand would break."""

import numpy as np
import pytest

import oracle
from tests.refs import assert_close, attention_ref, matmul_ref, packed_causal_ref, paged_ref, rmsnorm_ref, softmax_ref


# ---------------------------------------------------------------- half.rs

def test_half_known_answers():
    # src/half.rs:69-78
    for x in [0.0, 1.0, -2.5, 65504.0, 6.1e-5, 1e-7, 3.140625]:
        h = oracle.f32_to_f16_bits(x)
        assert oracle.f32_to_f16_bits(oracle.f16_bits_to_f32(h)) == h
    assert oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(1.0 + 1.0 / 4096.0)) == 1.0
    assert oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(70000.0)) == float("inf")


def test_half_matches_numpy_rne():
    # numpy's float32 -> float16 is an independent round-to-nearest-even.
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([6.103515625e-05, 5.960464477539063e-08, 2.98e-08, 65519.0, 65520.0, -0.0], np.float32),
    ]).astype(np.float32)
    for x in xs:
        want = int(np.float16(x).view(np.uint16))
        assert oracle.f32_to_f16_bits(float(x)) == want, x
    for h in range(0, 65536, 7):
        f = oracle.f16_bits_to_f32(h)
        want = float(np.uint16(h).view(np.float16))
        assert (f == want) or (np.isnan(f) and np.isnan(want))


# ---------------------------------------------------------------- Rng

def test_rng_matches_xorshift():
    # src/bench.rs:13-35, written out with Python integers.
    s = (7 * 0x9E3779B97F4A7C15 | 1) & (2**64 - 1)
    r = oracle.Rng(7)
    for _ in range(100):
        s ^= (s << 13) & (2**64 - 1)
        s ^= s >> 7
        s ^= (s << 17) & (2**64 - 1)
        assert r.bits() == s
    r = oracle.Rng(3)
    u = np.array([r.uniform() for _ in range(10000)])
    assert u.min() >= -1.0 and u.max() < 1.0 and abs(u.mean()) < 0.03


# ---------------------------------------------------------------- tests/interp.rs

def test_add():
    r = oracle.Rng(1)
    x, y = r.tensor("f32", [3000]), r.tensor("f32", [3000])
    np.testing.assert_array_equal(oracle.add(x, y), x + y)


def test_softmax_and_rmsnorm():
    # tests/interp.rs:34-61
    r = oracle.Rng(2)
    rows, cols = 10, 700
    x = r.tensor("f32", [rows, cols], 4.0)
    y = oracle.softmax(x)
    assert_close("softmax", y, softmax_ref(x), 1e-6)
    np.testing.assert_allclose(y.sum(axis=1), 1.0, atol=1e-5)
    x = r.tensor("f16", [rows, cols], 2.0)
    w = r.tensor("f16", [cols], 1.0)
    y = oracle.rmsnorm_basic(x, w, 1e-5)
    assert_close("rmsnorm", y.astype(np.float32), rmsnorm_ref(x, w, 1e-5), 2e-3)


def test_softmax_partial_block():
    # BC smaller than C: only the first BC columns are written, normalised
    # over those columns (kernels/basic.tl:13-17).
    r = oracle.Rng(9)
    x = r.tensor("f32", [3, 40])
    y = oracle.softmax(x, BC=16)
    assert_close("softmax BC=16", y[:, :16], softmax_ref(x[:, :16]), 1e-6)
    assert (y[:, 16:] == 0).all()


def test_matmuls():
    # tests/interp.rs:63-101
    r = oracle.Rng(3)
    m, k, n = 100, 70, 90
    a, b = r.tensor("f16", [m, k]), r.tensor("f16", [k, n])
    assert_close("matmul", oracle.matmul(a, b, BK=16), matmul_ref(a, b), 2e-3)
    a, b = r.tensor("f32", [m, k]), r.tensor("f32", [k, n])
    assert_close("matmul_f32", oracle.matmul_f32(a, b, BK=16), matmul_ref(a, b), 1e-6)
    x, w, bias = r.tensor("f16", [m, k]), r.tensor("f16", [n, k]), r.tensor("f16", [n])
    want = matmul_ref(x, w, bt=True) + bias.astype(np.float64)[None, :]
    assert_close("linear", oracle.linear_bias(x, w, bias), want, 2e-3)


def test_matmul_exact_integers():
    # Small integers make every partial sum exact: the f16 result is known
    # bit for bit whatever the tile shape or program order.
    rng = np.random.default_rng(4)
    m, k, n = 130, 70, 90
    a = rng.integers(-4, 5, (m, k)).astype(np.float16)
    b = rng.integers(-4, 5, (k, n)).astype(np.float16)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float16)
    for bm, bn, bk, g in [(128, 128, 32, 8), (64, 32, 16, 2), (16, 16, 16, 1)]:
        np.testing.assert_array_equal(oracle.matmul(a, b, bm, bn, bk, g), want)


def test_matmul_program_order_covers_every_tile():
    # The grouped program order of kernels/matmul.tl:8-13 must visit each
    # output tile exactly once: with threads the tiles are disjoint, so a
    # NaN-poisoned C is fully overwritten.
    r = oracle.Rng(5)
    for m, n in [(300, 200), (512, 512), (100, 1000)]:
        a, b = r.tensor("f16", [m, 32]), r.tensor("f16", [32, n])
        c = np.full((m, n), np.nan, np.float16)
        oracle.matmul(a, b, 64, 64, 32, 3, threads=4, C=c)
        assert not np.isnan(c).any()
        assert_close("matmul grouped", c, matmul_ref(a, b), 2e-3)


def test_matmul_tile_rounding_is_per_bk():
    # The f32 accumulator is rounded once per BK-tile: with one K tile
    # (BK >= K) the result is the f16 of the f32 of the f64 dot product.
    r = oracle.Rng(6)
    a, b = r.tensor("f16", [20, 64]), r.tensor("f16", [64, 24])
    want = matmul_ref(a, b).astype(np.float32).astype(np.float16)
    np.testing.assert_array_equal(oracle.matmul(a, b, 16, 16, 64, 1), want)


def test_flash_attention():
    # tests/interp.rs:103-124
    r = oracle.Rng(4)
    h, s, d = 2, 150, 32
    q, k, v = (r.tensor("f16", [h, s, d]) for _ in range(3))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    assert_close("flash attention", oracle.flash_attention(q, k, v, scale), attention_ref(q, k, v, scale), 5e-3)


def test_flash_attention_single_block_is_dense_softmax():
    # With S <= BN there is one key block: the online softmax is the plain one.
    r = oracle.Rng(8)
    q, k, v = (r.tensor("f16", [1, 40, 16]) for _ in range(3))
    assert_close("one block", oracle.flash_attention(q, k, v, 0.25, BM=64, BN=64), attention_ref(q, k, v, 0.25), 2e-3)


def test_paged_attention():
    # tests/interp.rs:126-136 (G == H)
    r = oracle.Rng(5)
    q, kc, vc, table, lens, scale = oracle.paged_case(r, 3, 2, 32, 16, [37, 1, 64])
    got = oracle.decode_attention(q, kc, vc, table, lens, scale)
    assert_close("paged attention", got, paged_ref(q, kc, vc, table, lens, scale), 5e-3)


def test_decode_attention_gqa_and_invariants():
    r = oracle.Rng(10)
    q, kc, vc, table, lens, scale = oracle.paged_case(r, 4, 8, 64, 16, [37, 1, 64, 200], g=2)
    got = oracle.decode_attention(q, kc, vc, table, lens, scale)
    assert_close("decode gqa", got, paged_ref(q, kc, vc, table, lens, scale), 5e-3)
    # Permuting the pool's pages together with the table changes nothing.
    perm = np.random.default_rng(1).permutation(kc.shape[0])
    inv = np.argsort(perm)
    got2 = oracle.decode_attention(q, np.ascontiguousarray(kc[perm]), np.ascontiguousarray(vc[perm]),
                                   inv[table].astype(np.int32), lens, scale)
    np.testing.assert_array_equal(got2.view(np.uint16), got.view(np.uint16))
    # A page outside the pool reads as zeros: scores 0 and values 0.
    t2 = table.copy()
    t2[3, 1] = 10**6
    kz, vz = kc.copy(), vc.copy()
    kz[table[3, 1]] = 0
    vz[table[3, 1]] = 0
    np.testing.assert_array_equal(oracle.decode_attention(q, kc, vc, t2, lens, scale).view(np.uint16),
                                  oracle.decode_attention(q, kz, vz, table, lens, scale).view(np.uint16))
    # lens 0 (a padding row) divides 0 by 0.
    l0 = lens.copy()
    l0[1] = 0
    assert np.isnan(oracle.decode_attention(q, kc, vc, table, l0, scale)[1].astype(np.float32)).all()


def test_prefill_attention_packed():
    # Two prompts packed into one step, the second starting mid-block after
    # a whole 64-key block of the first (tests/llm.rs:189-227's shape).
    r = oracle.Rng(11)
    s, h, g, d = 90, 4, 2, 16
    q = r.tensor("f16", [s, h, d])
    k = r.tensor("f16", [s, g, d])
    v = r.tensor("f16", [s, g, d])
    starts = np.array([0] * 70 + [70] * 20, np.int32)
    got = oracle.prefill_attention(q, k, v, starts, 0.25)
    assert_close("packed prefill", got, packed_causal_ref(q, k, v, starts, 0.25), 5e-3)
    # Rows of one prompt alone give the same as that prompt in its own step.
    alone = oracle.prefill_attention(np.ascontiguousarray(q[70:]), np.ascontiguousarray(k[70:]),
                                     np.ascontiguousarray(v[70:]), np.zeros(20, np.int32), 0.25)
    assert_close("packed vs alone", got[70:], alone.astype(np.float64), 2e-3)


# ---------------------------------------------------------------- llm.tl rows and matmuls

def test_llm_matmuls_against_f64():
    r = oracle.Rng(5)
    m, k, n = 16, 256, 96
    x, w, w2 = r.tensor("f16", [m, k]), r.tensor("f16", [n, k], 0.1), r.tensor("f16", [n, k], 0.1)
    ref = matmul_ref(x, w, bt=True)
    assert_close("linear", oracle.llm_linear(x, w), ref, 2e-3)
    assert_close("logits", oracle.logits(x, w), ref, 1e-5)
    res = r.tensor("f32", [m, n])
    assert_close("linear_residual", oracle.linear_residual(x, w, res), ref + res, 1e-5)
    g, u = ref, matmul_ref(x, w2, bt=True)
    assert_close("gate_up", oracle.gate_up(x, w, w2), g / (1 + np.exp(-g)) * u, 2e-3)


def test_rows_kernels():
    r = oracle.Rng(12)
    t, dm, v = 5, 48, 30
    e = r.tensor("f16", [v, dm])
    tok = np.array([3, 0, 29, 7, 40], np.int32)  # 40 is outside the vocabulary
    x = oracle.embed(tok, e)
    np.testing.assert_array_equal(x[:4], e[tok[:4]].astype(np.float32))
    assert (x[4] == 0).all()
    xr = r.tensor("f32", [t, dm], 3.0)
    w = r.tensor("f16", [dm])
    y = oracle.rmsnorm(xr, w, 1e-5, BC=64)
    assert_close("llm rmsnorm", y, rmsnorm_ref(xr, w, 1e-5), 2e-3)
    idx = np.array([4, 0, 2], np.int32)
    np.testing.assert_array_equal(oracle.rmsnorm_rows(xr, idx, w, 1e-5, BC=64).view(np.uint16),
                                  y[idx].view(np.uint16))


def test_rope_and_kv_write():
    cfg = oracle.Config.tiny()
    c, s = oracle.rope_tables(cfg)
    h = cfg.head_dim // 2
    inv = cfg.rope_theta ** (-(2.0 * np.arange(h)) / cfg.head_dim)
    ang = np.arange(cfg.max_pos)[:, None] * inv[None, :]
    np.testing.assert_allclose(c, np.cos(ang), atol=2e-7)
    np.testing.assert_allclose(s, np.sin(ang), atol=2e-7)
    r = oracle.Rng(13)
    H, G, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    T, W = 6, cfg.qkv()
    qkv = r.tensor("f16", [T, W])
    pos = np.array([0, 1, 2, 50, 255, 3], np.int32)
    q = oracle.rope_q(qkv, pos, c, s, H, D).astype(np.float64)
    x = qkv.astype(np.float64)
    for t in range(T):
        for hh in range(H):
            a, b = x[t, hh * D:hh * D + h], x[t, hh * D + h:(hh + 1) * D]
            want = np.concatenate([a * c[pos[t]] - b * s[pos[t]], b * c[pos[t]] + a * s[pos[t]]])
            np.testing.assert_allclose(q[t, hh], want, atol=2e-3)
    NS = 16
    slot = np.array([3, 9, 15, 16, 0, -1], np.int32)  # 16 and -1 are out of range: dropped
    Kc = np.zeros((NS, G, D), np.float16)
    Vc = np.zeros((NS, G, D), np.float16)
    K = np.zeros((T, G, D), np.float16)
    V = np.zeros((T, G, D), np.float16)
    Kc, Vc, K, V = oracle.kv_write(qkv, pos, slot, c, s, Kc, Vc, K, V)
    for t in range(T):
        for g in range(G):
            k0 = W - 2 * G * D + g * D
            a, b = x[t, k0:k0 + h], x[t, k0 + h:k0 + D]
            want = np.concatenate([a * c[pos[t]] - b * s[pos[t]], b * c[pos[t]] + a * s[pos[t]]])
            np.testing.assert_allclose(K[t, g].astype(np.float64), want, atol=2e-3)
            np.testing.assert_array_equal(V[t, g], qkv[t, k0 + G * D:k0 + G * D + D])
            if 0 <= slot[t] < NS:
                np.testing.assert_array_equal(Kc[slot[t], g], K[t, g])
                np.testing.assert_array_equal(Vc[slot[t], g], V[t, g])
    written = set(int(x) for x in slot if 0 <= x < NS)
    for sl in range(NS):
        if sl not in written:
            assert (Kc[sl] == 0).all() and (Vc[sl] == 0).all()


# ---------------------------------------------------------------- llm/mod.rs, reference.rs

def test_argmax_first_on_ties():
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    rng = np.random.default_rng(3)
    for _ in range(50):
        x = rng.integers(0, 5, 40).astype(np.float32)
        assert oracle.argmax(x) == int(np.argmax(x))


def test_weights_random_shape_and_scale():
    cfg = oracle.Config.tiny()
    embed, layers, norm, head = oracle.weights_random(cfg, 7)
    assert (norm == 1).all()
    le = cfg.layer_elems()
    l0 = layers[:le]
    assert (l0[:cfg.dim] == 1).all()
    wqkv = l0[cfg.dim:cfg.dim + cfg.qkv() * cfg.dim].astype(np.float32)
    s = 1 / np.sqrt(np.float32(cfg.dim))
    assert np.abs(wqkv).max() <= s and np.abs(wqkv).max() > 0.9 * s
    assert np.abs(embed.astype(np.float32)).max() <= 8 * s * 1.001
    # The first wqkv entry is the Rng's first uniform * scale.
    r = oracle.Rng(7)
    assert wqkv[0] == np.float16(np.float32(r.uniform()) * s).astype(np.float32)


def test_weights_random_draw_order():
    """Every tensor of Weights::random in the draw order of src/llm/mod.rs:80-108: per layer
    wqkv, wo, wg, wu, wd (norms are ones, no draws), then embed (f16 of the draw, times 8,
    rounded again), then lm_head; each matrix draws rows x cols uniforms scaled by
    1/sqrt(cols) in f32. A swapped pair of draws (wg/wu, embed/lm_head) fails here."""
    for cfg, seed in ((oracle.Config.tiny(), 7), (oracle.Config.tiny(), 123)):
        embed, layers, norm, head = oracle.weights_random(cfg, seed)
        r = oracle.Rng(seed)

        def m(rows, cols):
            sc = np.float32(1) / np.sqrt(np.float32(cols))
            return r.tensor("f16", [rows * cols], float(sc))

        d, ff, hd, nh = cfg.dim, cfg.ffn, cfg.head_dim, cfg.heads
        want_layers = []
        for _ in range(cfg.layers):
            ones = np.ones(d, np.float16)
            wqkv, wo = m(cfg.qkv(), d), m(d, nh * hd)
            wg, wu, wd = m(ff, d), m(ff, d), m(d, ff)
            want_layers += [ones, wqkv, wo, ones, wg, wu, wd]
        want_embed = (m(cfg.vocab, d).astype(np.float32) * np.float32(8)).astype(np.float16)
        want_head = m(cfg.vocab, d)
        assert np.array_equal(layers.view(np.uint16), np.concatenate(want_layers).view(np.uint16))
        assert np.array_equal(embed.view(np.uint16), want_embed.view(np.uint16))
        assert np.array_equal(head.view(np.uint16), want_head.view(np.uint16))
        assert (norm == 1).all()


def _np_forward(cfg, w, tokens):
    """An independent f64 numpy model of src/llm/reference.rs."""
    embed, layers, norm, head = (a.astype(np.float64) for a in w)
    d, hd, nh, ng, ff = cfg.dim, cfg.head_dim, cfg.heads, cfg.kv_heads, cfg.ffn
    c, s = (t.astype(np.float64) for t in oracle.rope_tables(cfg))
    E = embed.reshape(cfg.vocab, d)
    le = cfg.layer_elems()
    qr = cfg.qkv()

    def rms(x, wt):
        return x / np.sqrt((x * x).mean() + cfg.eps) * wt

    def rope(x, p):
        x = x.reshape(-1, hd).copy()
        a, b = x[:, :hd // 2].copy(), x[:, hd // 2:].copy()
        x[:, :hd // 2] = a * c[p] - b * s[p]
        x[:, hd // 2:] = b * c[p] + a * s[p]
        return x

    L = []
    for li in range(cfg.layers):
        o = li * le
        parts = []
        for n in (d, qr * d, d * nh * hd, d, ff * d, ff * d, d * ff):
            parts.append(layers[o:o + n])
            o += n
        L.append(parts)
    ks = [[] for _ in range(cfg.layers)]
    vs = [[] for _ in range(cfg.layers)]
    out = []
    for p, t in enumerate(tokens):
        x = E[t].copy()
        for li, (n1, wqkv, wo, n2, wg, wu, wd) in enumerate(L):
            h = rms(x, n1)
            qkv = wqkv.reshape(qr, d) @ h
            q = rope(qkv[:nh * hd], p)
            k = rope(qkv[nh * hd:(nh + ng) * hd], p)
            ks[li].append(k)
            vs[li].append(qkv[(nh + ng) * hd:].reshape(ng, hd))
            K, V = np.stack(ks[li]), np.stack(vs[li])
            o_ = np.zeros((nh, hd))
            for hh in range(nh):
                g = hh // (nh // ng)
                sc = K[:, g] @ q[hh] / np.sqrt(hd)
                e = np.exp(sc - sc.max())
                o_[hh] = e @ V[:, g] / e.sum()
            x = x + wo.reshape(d, nh * hd) @ o_.reshape(-1)
            h = rms(x, n2)
            g_, u_ = wg.reshape(ff, d) @ h, wu.reshape(ff, d) @ h
            x = x + wd.reshape(d, ff) @ (g_ / (1 + np.exp(-g_)) * u_)
        out.append(head.reshape(cfg.vocab, d) @ rms(x, norm))
    return np.array(out)


def test_reference_forward_against_f64():
    cfg = oracle.Config.tiny()
    w = oracle.weights_random(cfg, 7)
    toks = [1, 17, 200, 33, 5, 99, 64, 3, 250, 12]
    got = oracle.forward(cfg, w, toks)
    want = _np_forward(cfg, w, toks)
    rel = np.abs(got - want).max() / np.abs(want).max()
    assert rel < 1e-4, rel


def test_reference_forward_is_causal_and_token_blocked_exactly():
    """forward runs layer by layer over every token in 16-token blocks; the
    logits after token i must not depend on later tokens or on the block a
    token falls in: a prefix's logits equal, bit for bit, the same rows of
    the longer run (37 tokens: three blocks, the last ragged). A history
    longer than max_pos is an error, as the reference's table index is."""
    cfg = oracle.Config.tiny()
    w = oracle.weights_random(cfg, 5)
    toks = [(i * 37 + 3) % cfg.vocab for i in range(37)]
    full = oracle.forward(cfg, w, toks)
    for k in (1, 15, 16, 17, 33):
        np.testing.assert_array_equal(oracle.forward(cfg, w, toks[:k]).view(np.uint32), full[:k].view(np.uint32))
    with pytest.raises(ValueError):
        oracle.forward(cfg, w, [1] * (cfg.max_pos + 1))
