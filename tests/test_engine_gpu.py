"""The engine (every step a sequence of the HIP llm.tl kernels) against the
f32 reference model, on a small random Llama: tests/llm.rs:25-83 and
:189-227 restated, plus graph replay against eager launches."""

import numpy as np
import pytest

import oracle
import tessel_amd as T

pytestmark = pytest.mark.gpu


def limits(page=8, pages=32, max_tokens=16, max_seq_pages=8):
    return T.Limits(page, pages, max_tokens, max_seq_pages)


def rel(got, want):
    return np.abs(got - want).max() / np.abs(want).max()


def test_prefill_and_batched_decode_match_the_reference(gpu):
    cfg = T.Config.tiny()
    w = T.weights_random(cfg, 7)
    e = T.Engine(cfg, limits(), w)
    prompt = [1, 17, 200, 33, 5, 99, 64, 3, 250, 12]
    n = len(prompt)
    got = e.step(prompt, list(range(n)), list(range(n)), T.Engine.PREFILL, want=[n - 1])
    ocfg = oracle.Config.tiny()
    want = oracle.forward(ocfg, w, prompt)
    err = rel(got[0], want[n - 1])
    print(f"prefill: logits within {err:.2e} of the reference", flush=True)
    assert err < 2e-2
    reqs = [([1, 5, 9], 6), (prompt, 4), ([1, 100, 101, 102, 103, 104, 105], 9)]
    outs, st = e.generate(reqs, 3)
    assert st.largest_batch == 3
    exact = 0
    for (p, m), toks in zip(reqs, outs):
        assert len(toks) == m
        seq = list(p)
        for t in toks:
            l = oracle.forward(ocfg, w, seq)[-1]
            best = oracle.argmax(l)
            scale = np.abs(l).max()
            assert t == best or l[best] - l[t] < 2e-2 * scale, (t, best)
            exact += t == best
            seq.append(t)
    print(f"generation: {exact} of {st.generated} tokens the reference's own choice", flush=True)
    e.close()


def test_wide_model_shape_against_the_reference(gpu):
    # A Llama-7B-wide shape (dim 4096, head_dim 128, GQA 32/8, ffn 11008),
    # two layers and a small vocabulary: projections with K > 2048 (split
    # QKV without the fused rotation, split gate_up, down at K = 11008), the
    # 4096-column reduce-and-normalise, and decode attention at D = 128.
    vals = (4096, 2, 32, 8, 128, 11008, 4000, 1e-5, 10000.0, 512, 1, 2)
    cfg, ocfg = T.Config(*vals), oracle.Config(*vals)
    w = T.weights_random(cfg, 21)
    e = T.Engine(cfg, limits(page=16, pages=16, max_tokens=32, max_seq_pages=4), w)
    prompt = [1, 17, 200, 33, 5, 99, 64, 3, 250, 12, 3000, 7]
    n = len(prompt)
    got = e.step(prompt, list(range(n)), list(range(n)), T.Engine.PREFILL, want=[n - 1])
    want = oracle.forward(ocfg, w, prompt)
    err = rel(got[0], want[n - 1])
    print(f"wide prefill: logits within {err:.2e} of the reference", flush=True)
    assert err < 2e-2
    reqs = [(prompt, 3), ([1, 2, 3, 4, 5], 3)]
    outs, st = e.generate(reqs, 2)
    e.close()
    assert st.largest_batch == 2
    for (p, m), toks in zip(reqs, outs):
        assert len(toks) == m
        seq = list(p)
        for t in toks:
            l = oracle.forward(ocfg, w, seq)[-1]
            best = oracle.argmax(l)
            assert t == best or l[best] - l[t] < 2e-2 * np.abs(l).max(), (t, best)
            seq.append(t)


def test_packed_prefill_matches_one_prompt_per_step(gpu):
    cfg = T.Config.tiny()
    w = T.weights_random(cfg, 11)
    lim = limits(page=8, pages=64, max_tokens=128, max_seq_pages=16)
    long = [1 + (i * 37 % 250) for i in range(70)]
    short = [1, 9, 42, 7, 200, 13, 5, 77, 31, 64, 2, 150, 99, 3, 18, 240, 6, 11, 120, 45]
    reqs = [(long, 4), (short, 4)]
    e = T.Engine(cfg, lim, w)
    packed, st = e.generate(reqs, 2, packed=True)
    assert st.prefill_steps == 1
    e.close()
    e = T.Engine(cfg, lim, w)
    single, st = e.generate(reqs, 2, packed=False)
    assert st.prefill_steps == 2
    e.close()
    assert packed == single


def test_graph_replay_matches_eager(gpu):
    cfg = T.Config.tiny()
    w = T.weights_random(cfg, 5)
    reqs = [([1, 2, 3, 4, 5], 12), ([9, 8, 7], 10), ([100 + i for i in range(12)], 8)]
    outs = []
    for graphs in (False, True):
        e = T.Engine(cfg, limits(pages=64), w, graphs=graphs)
        e.step_times(True)
        outs.append(e.generate(reqs, 3)[0])
        # Every decode step was timed, as a replay or as eager launches (the
        # first step of each batch size is launched eagerly, then captured).
        tm = e.step_times(False)
        n = tm["graph"][0] + tm["eager"][0]
        print(f"graphs={graphs}: step spans {tm}", flush=True)
        assert n > 0 and all(ms > 0 for k, ms in tm.values() if k)
        assert (tm["graph"][0] > 0) == graphs
        if graphs:
            # The recorded decode steps are kernel launches only (no memset
            # or copy nodes): each layer's QKV, attention (+ merge), o and
            # down projections with their norms, gate_up; then embed, norm,
            # final norm, logits and argmax.
            gs = e.graphs()
            assert gs
            for rows, g in gs.items():
                nodes = T.graph_nodes(g)
                print(f"decode graph for {rows} rows: {nodes}", flush=True)
                assert nodes["memset"] == nodes["memcpy"] == nodes["other"] == 0
                assert nodes["kernel"] >= 5 * cfg.layers + 5
        e.close()
    assert outs[0] == outs[1]


def test_engine_from_a_bf16_checkpoint(gpu, tmp_path):
    # A checkpoint as another writer stores it (BF16, Hugging Face names),
    # read by the loader, runs through the engine like the reference model
    # with the same (converted) weights.
    import json
    import torch
    from safetensors.torch import save_file
    cfg = T.Config.tiny()
    w = T.weights_random(cfg, 9)
    T.save_checkpoint(str(tmp_path / "f16"), cfg, w)
    from safetensors.torch import load_file
    t = load_file(str(tmp_path / "f16" / "model.safetensors"))
    save_file({k: v.to(torch.float32).to(torch.bfloat16) for k, v in t.items()}, str(tmp_path / "model.safetensors"))
    with open(tmp_path / "f16" / "config.json") as f:
        conf = json.load(f)
    with open(tmp_path / "config.json", "w") as f:
        json.dump(conf, f)
    c2, w2 = T.load_checkpoint(str(tmp_path))
    assert w2[3] is not None
    e = T.Engine(c2, limits(), w2)
    prompt = [1, 7, 99, 42, 3, 128, 200]
    n = len(prompt)
    got = e.step(prompt, list(range(n)), list(range(n)), T.Engine.PREFILL, want=[n - 1])
    want = oracle.forward(oracle.Config.tiny(), w2, prompt)
    err = rel(got[0], want[n - 1])
    print(f"bf16 checkpoint prefill: logits within {err:.2e} of the reference", flush=True)
    assert err < 2e-2
    e.close()


def test_close_then_launch():
    # Closing an engine frees exactly its own allocations (its step inputs
    # are views into one arena): a kernel launched afterwards reports no
    # error left behind by the close.
    cfg = T.Config.tiny()
    w = T.weights_random(cfg, 4)
    e = T.Engine(cfg, T.Limits(16, 64, 64, 8), w)
    e.generate([([1, 2, 3], 3)], 1)
    e.close()
    a = np.ones((64, 64), np.float16)
    c = T.run("matmul", "matmul", [a, a, np.zeros((64, 64), np.float16)], outputs=[2])[2]
    assert (c == 64).all()


def _tinyllama_engine(seqs=32, prompt=512, new=128, graphs=True):
    # The headline engine workload: TinyLlama-1.1B shape, Weights::random(7)
    # (the library's generator, equal to the oracle's bit for bit:
    # tests/test_abi.py), page 16, 1024-token steps.
    cfg = T.Config.tinyllama()
    w = T.weights_random(cfg, 7)
    mp = (prompt + new + 15) // 16
    e = T.Engine(cfg, T.Limits(16, seqs * mp + 64, 1024, mp), w, graphs=graphs)
    return cfg, w, e


def test_tinyllama_shape_against_the_reference(gpu):
    """Config 5's model (22 layers, 32/4 heads, D 64, FFN 5632, vocab 32000)
    against reference::forward (src/llm/reference.rs) at real context
    lengths: prefill logits of a 124-token prompt at three rows, then four
    prompts of 109-188 tokens packed into one prefill step (multi-page
    tables, 7-12 pages each) and 10 greedy steps at batch 4 whose positions
    each cross a 16-token page boundary; every token is the reference's
    argmax or within 2e-2 of its scale (tests/llm.rs:26-82)."""
    lens = (124, 157, 188, 109)
    new = 10
    cfg, w, e = _tinyllama_engine(seqs=4, prompt=max(lens), new=new)
    ocfg = oracle.Config.tinyllama()
    rng = np.random.default_rng(3)
    prompts = [rng.integers(3, cfg.vocab, n).tolist() for n in lens]
    for n in lens:  # positions n .. n + new - 2 feed decode steps; each run crosses a page boundary
        assert (n - 1) // 16 != (n + new - 2) // 16
    p1 = prompts[0]
    n = len(p1)
    rows = (0, 63, n - 1)
    got = e.step(p1, list(range(n)), list(range(n)), T.Engine.PREFILL, want=list(rows))
    reqs = [(p, new) for p in prompts]
    outs, st = e.generate(reqs, 4)
    e.close()
    print(f"tinyllama: {st.prefill_steps} prefill step(s), {st.decode_steps} decode steps", flush=True)
    assert st.prefill_steps == 1 and st.largest_batch == 4 and [len(o) for o in outs] == [new] * 4
    exact = total = 0
    for k, ((p, m), toks) in enumerate(zip(reqs, outs)):
        seq = list(p) + toks[:-1]
        ref = oracle.forward(ocfg, w, seq)  # logits after every position of the history
        if k == 0:
            for row, r in zip(got, rows):
                err = rel(row, ref[r])
                print(f"tinyllama prefill row {r}: logits within {err:.2e} of the reference", flush=True)
                assert err < 2e-2
        for i, t in enumerate(toks):
            l = ref[len(p) - 1 + i]
            best = oracle.argmax(l)
            scale = np.abs(l).max()
            assert t == best or l[best] - l[t] < 2e-2 * scale, (k, i, t, best)
            exact += t == best
            total += 1
    print(f"tinyllama generation: {exact} of {total} tokens the reference's own choice", flush=True)


def test_tinyllama_full_config_properties(gpu):
    """Config 5 at full size (32 prompts of 512 random ids, 128 greedy
    steps): two of the streams token by token against the reference model,
    packed prefill (two prompts per 1024-token step) and one prompt per step
    generate the same token streams, graph replay equals eager launches,
    every request gets 128 tokens (or stops at eos), and the statistics count
    what ran."""
    cfg, w, e = _tinyllama_engine()
    rng = np.random.default_rng(5)
    reqs = [(rng.integers(3, cfg.vocab, 512).tolist(), 128) for _ in range(32)]
    packed, st = e.generate(reqs, 32)
    # Two of the 32 streams (the first and the last request) against
    # reference::forward over their whole 639-token histories: every token of
    # the 32-row decode is the reference's argmax or within 2e-2 of its scale.
    ocfg = oracle.Config.tinyllama()
    for k in (0, 31):
        p, toks = reqs[k][0], packed[k]
        ref = oracle.forward(ocfg, w, list(p) + toks[:-1])
        exact = 0
        for i, t in enumerate(toks):
            l = ref[len(p) - 1 + i]
            best = oracle.argmax(l)
            assert t == best or l[best] - l[t] < 2e-2 * np.abs(l).max(), (k, i, t, best)
            exact += t == best
        print(f"config 5 request {k}: {exact} of {len(toks)} tokens the reference's own choice", flush=True)
    del w
    print(f"config 5: {st.generated} tokens, {st.prefill_steps} prefill + {st.decode_steps} decode steps", flush=True)
    assert st.prefill_steps == 16 and st.prompt_tokens == 32 * 512 and st.largest_batch == 32
    assert st.generated == sum(len(o) for o in packed)
    assert st.decode_tokens == st.generated - 32
    for o in packed:
        assert len(o) == 128 or (len(o) < 128 and o[-1] == cfg.eos and cfg.eos not in o[:-1])
    e.set(False, True)
    eager, _ = e.generate(reqs, 32)
    assert eager == packed
    e.set(True, True)
    single, st1 = e.generate(reqs, 32, packed=False)
    assert st1.prefill_steps == 32
    e.close()
    same = sum(a == b for a, b in zip(single, packed))
    print(f"config 5: one prompt per step == packed for {same} of 32 requests", flush=True)
    assert single == packed


def test_engine_rejects_bad_requests_and_starts(gpu):
    # max_new 0 and a request larger than the page pool are refused before
    # any step runs; packed starts must be 0 at row 0 and, at every later
    # row, the previous row's start (same sequence) or the row itself (a new
    # one): a start outside the rows would address K/V before or past the
    # step.
    cfg = T.Config.tiny()
    e = T.Engine(cfg, limits(), T.weights_random(cfg, 3))
    with pytest.raises(RuntimeError, match="max_new must be at least 1"):
        e.generate([([1, 2, 3], 2), ([4, 5], 0)], 2)
    with pytest.raises(RuntimeError, match="does not fit"):
        T.Engine.generate(e, [([1] * 16, 300)], 1)
    # [0, 0, 1, 1]: row 2 claims a sequence starting at row 1, which belongs
    # to the sequence that starts at row 0.
    for bad in ([0, 0, -1, 3], [0, 0, 3, 3], [0, 1, 0, 3], [0, 0, 1, 1], [1, 1, 2, 3]):
        with pytest.raises(RuntimeError, match="starts"):
            e.step([1, 2, 3, 4], [0, 1, 0, 1], [0, 1, 2, 3], T.Engine.PACKED, starts=bad, want=[3])
    got = e.step([1, 2, 3, 4], [0, 1, 0, 1], [0, 1, 2, 3], T.Engine.PACKED, starts=[0, 0, 2, 2], want=[1, 3])
    assert np.isfinite(got).all()
    e.close()


def test_deferred_norm_overflow_recomputes_the_step(gpu):
    """Decode steps defer each rmsnorm into the next projection through
    Y = f16(R Wn). With embeddings (the residual's start) up to 2000 and
    norm weights of 40, R Wn overflows f16 (|R Wn| >= 65520) while
    rmsnorm(R) Wn stays below ~70: the
    engine must notice and recompute the step with the norms applied first,
    so its tokens stay the reference's (src/llm/reference.rs normalises
    first). Without the overflow no step is recomputed."""
    cfg = T.Config.tiny()
    emb, lay, nrm, head = T.weights_random(cfg, 13)
    ocfg = oracle.Config.tiny()
    prompt = [1, 17, 200, 33, 5]
    for big in (False, True):
        e_w = emb.copy()
        l_w = lay.copy()
        if big:
            e_w = (e_w.astype(np.float32) * (2000 / np.abs(e_w.astype(np.float32)).max())).astype(np.float16)
            per = l_w.size // cfg.layers
            d, qr = cfg.dim, cfg.qkv() * cfg.dim
            hd = cfg.heads * cfg.head_dim
            for li in range(cfg.layers):  # every norm weight (attn_norm and mlp_norm) 40
                b = li * per
                l_w[b:b + d] = 40
                n2 = b + d + qr + d * hd
                l_w[n2:n2 + d] = 40
        w = (e_w, l_w, nrm, head)
        e = T.Engine(cfg, limits(), w)
        outs, st = e.generate([(prompt, 6), ([4, 9, 100], 5)], 2)
        fb = e.fallbacks()
        e.close()
        print(f"big={big}: {fb} of {st.decode_steps} decode steps recomputed", flush=True)
        if not big:
            assert fb == 0
            continue
        assert fb == st.decode_steps > 0
        for p, toks in zip((prompt, [4, 9, 100]), outs):
            seq = list(p)
            for t in toks:
                l = oracle.forward(ocfg, w, seq)[-1]
                assert np.isfinite(l).all()
                best = oracle.argmax(l)
                assert t == best or l[best] - l[t] < 2e-2 * np.abs(l).max(), (t, best)
                seq.append(t)
