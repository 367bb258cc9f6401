"""Plain f64 references of the kernels, restating tests/common/mod.rs:45-173
(softmax_ref, rmsnorm_ref, matmul_ref, attention_ref, paged_case's expected
output) and its assert_close (:37-43). They share no code with the oracle
or the HIP kernels; tests use them to pin both."""

import numpy as np


def assert_close(what, got, want, tol):
    """max |got - want| <= tol * max(1, max |want|), and no NaN (tests/common/mod.rs:37-43)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert not np.isnan(got).any(), f"{what}: NaN in output"
    d = float(np.max(np.abs(got - want))) if got.size else 0.0
    s = float(np.max(np.abs(want))) if want.size else 0.0
    assert d <= tol * max(s, 1.0), f"{what}: max |diff| {d} (largest {s}, tolerance {tol})"


def parity(what, got, want, rel_fro=1e-3, max_abs=2e-2):
    """The north-star fp16 parity bar: relative Frobenius error <= 1e-3 and
    max |diff| <= 2e-2 (NaN only where the oracle has NaN)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    gn, wn = np.isnan(got), np.isnan(want)
    assert (gn == wn).all(), f"{what}: NaN positions differ ({gn.sum()} vs {wn.sum()})"
    g, w = got[~gn], want[~wn]
    if g.size == 0:
        return 0.0, 0.0
    diff = g - w
    denom = np.linalg.norm(w)
    rel = float(np.linalg.norm(diff) / denom) if denom > 0 else float(np.linalg.norm(diff))
    mx = float(np.max(np.abs(diff)))
    assert rel <= rel_fro and mx <= max_abs, f"{what}: rel Frobenius {rel:.3e} (<= {rel_fro}), max |diff| {mx:.3e} (<= {max_abs})"
    return rel, mx


def softmax_ref(x):
    x = np.asarray(x, np.float32)
    m = x.max(axis=1, keepdims=True)
    e = np.exp((x - m).astype(np.float64))
    return e / e.sum(axis=1, keepdims=True)


def rmsnorm_ref(x, w, eps):
    x = np.asarray(x, np.float64)
    ms = (x * x).sum(axis=1, keepdims=True) / x.shape[1]
    return x / np.sqrt(ms + float(np.float32(eps))) * np.asarray(w, np.float64)[None, :]


def matmul_ref(a, b, bt=False):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return a @ (b.T if bt else b)


def attention_ref(q, k, v, scale):
    """Causal attention per head; q, k, v [h, s, d]."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    h, s, d = q.shape
    sc = np.einsum("hid,hjd->hij", q, k) * float(scale)
    mask = np.tril(np.ones((s, s), bool))
    sc = np.where(mask[None], sc, -np.inf)
    m = sc.max(axis=2, keepdims=True)
    e = np.exp(sc - m)
    return np.einsum("hij,hjd->hid", e, v) / e.sum(axis=2, keepdims=True)


def paged_ref(q, kc, vc, table, lens, scale):
    """paged_case's expected output (tests/common/mod.rs:139-162), with the
    GQA head map h // (H // G) of kernels/llm.tl:154."""
    q, kc, vc = (np.asarray(t, np.float64) for t in (q, kc, vc))
    b, h, d = q.shape
    p, g = kc.shape[1], kc.shape[2]
    out = np.zeros((b, h, d))
    for s in range(b):
        n = int(lens[s])
        if n == 0:
            out[s] = np.nan
            continue
        t = np.arange(n)
        pages = table[s, t // p]
        for hh in range(h):
            gg = hh // (h // g)
            k = kc[pages, t % p, gg]
            v = vc[pages, t % p, gg]
            sc = k @ q[s, hh] * float(scale)
            e = np.exp(sc - sc.max())
            out[s, hh] = e @ v / e.sum()
    return out


def packed_causal_ref(q, k, v, starts, scale):
    """Attention of packed prompts: row r sees keys starts[r] .. r; q [S,H,D],
    k, v [S,G,D], query head h reads kv head h // (H // G)."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    s, h, d = q.shape
    g = k.shape[1]
    out = np.zeros_like(q)
    for r in range(s):
        lo = int(starts[r])
        for hh in range(h):
            gg = hh // (h // g)
            sc = k[lo:r + 1, gg] @ q[r, hh] * float(scale)
            e = np.exp(sc - sc.max())
            out[r, hh] = e @ v[lo:r + 1, gg] / e.sum()
    return out


def f16(x):
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float16)
