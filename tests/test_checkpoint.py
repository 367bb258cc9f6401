"""Hugging Face checkpoints (src/llm/safetensors.rs): config.json, single
and sharded safetensors, F16/BF16/F32 tensors, the reference's save layout
and error wording (tests/llm.rs:86-102 checkpoints_round_trip). Host code:
these run without a GPU. Checkpoints in other dtypes are written with the
`safetensors` package (an independent writer) and the expected f16 values
come from numpy's round-to-nearest-even conversion."""

import json
import os

import numpy as np
import pytest

import tessel_amd as T


def _names(cfg):
    """(name, shape) of every tensor, in the tsl_weights_random layout order."""
    dm, hd = cfg.dim, cfg.head_dim
    out = []
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        out += [(p + "input_layernorm.weight", (dm,)),
                (p + "self_attn.q_proj.weight", (cfg.heads * hd, dm)),
                (p + "self_attn.k_proj.weight", (cfg.kv_heads * hd, dm)),
                (p + "self_attn.v_proj.weight", (cfg.kv_heads * hd, dm)),
                (p + "self_attn.o_proj.weight", (dm, cfg.heads * hd)),
                (p + "post_attention_layernorm.weight", (dm,)),
                (p + "mlp.gate_proj.weight", (cfg.ffn, dm)),
                (p + "mlp.up_proj.weight", (cfg.ffn, dm)),
                (p + "mlp.down_proj.weight", (dm, cfg.ffn))]
    return out


def _config_json(cfg, tied=True, **extra):
    d = {"model_type": "llama", "hidden_size": cfg.dim, "num_hidden_layers": cfg.layers,
         "num_attention_heads": cfg.heads, "num_key_value_heads": cfg.kv_heads, "head_dim": cfg.head_dim,
         "intermediate_size": cfg.ffn, "vocab_size": cfg.vocab, "rms_norm_eps": 1e-5, "rope_theta": 10000.0,
         "max_position_embeddings": cfg.max_pos, "bos_token_id": cfg.bos, "eos_token_id": cfg.eos,
         "rope_scaling": None, "tie_word_embeddings": tied}
    d.update(extra)
    return d


def _hf_tensors(cfg, seed, head=True):
    """Random f32 tensors of a Llama checkpoint, HF names."""
    rng = np.random.default_rng(seed)
    t = {"model.embed_tokens.weight": rng.standard_normal((cfg.vocab, cfg.dim), np.float32),
         "model.norm.weight": rng.standard_normal(cfg.dim, np.float32)}
    if head:
        t["lm_head.weight"] = rng.standard_normal((cfg.vocab, cfg.dim), np.float32)
    for n, s in _names(cfg):
        t[n] = rng.standard_normal(s, np.float32) * 0.05
    return t


def _expected_layers(cfg, f16):
    """The flat layer array the loader should produce from per-name f16 arrays."""
    parts = []
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        parts += [f16[p + "input_layernorm.weight"], f16[p + "self_attn.q_proj.weight"],
                  f16[p + "self_attn.k_proj.weight"], f16[p + "self_attn.v_proj.weight"],
                  f16[p + "self_attn.o_proj.weight"], f16[p + "post_attention_layernorm.weight"],
                  f16[p + "mlp.gate_proj.weight"], f16[p + "mlp.up_proj.weight"], f16[p + "mlp.down_proj.weight"]]
    return np.concatenate([a.reshape(-1) for a in parts])


def _bits(a):
    return np.ascontiguousarray(a, np.float16).view(np.uint16)


def test_round_trip_through_the_reference_layout(tmp_path):
    # tests/llm.rs:86-102: save(w) then load gives back the same weights and config.
    cfg = T.Config.tiny()
    w = T.weights_random(cfg, 3)
    d = str(tmp_path / "ckpt")
    T.save_checkpoint(d, cfg, w)
    c2, (e, l, n, h) = T.load_checkpoint(d)
    for f in ("dim", "layers", "heads", "kv_heads", "head_dim", "ffn", "vocab", "max_pos", "bos", "eos"):
        assert getattr(c2, f) == getattr(cfg, f), f
    assert c2.eps == cfg.eps and c2.rope_theta == cfg.rope_theta
    for got, want in ((e, w[0]), (l, w[1]), (n, w[2]), (h, w[3])):
        np.testing.assert_array_equal(_bits(got), _bits(want))
    # The file is a safetensors file another reader accepts, HF names and shapes.
    from safetensors.numpy import load_file
    t = load_file(os.path.join(d, "model.safetensors"))
    assert t["model.layers.1.self_attn.k_proj.weight"].shape == (cfg.kv_heads * cfg.head_dim, cfg.dim)
    assert t["model.layers.0.mlp.down_proj.weight"].dtype == np.float16
    # Tied: no lm_head.weight written, and none read back.
    T.save_checkpoint(d, cfg, (w[0], w[1], w[2], None))
    _, (_, _, _, h2) = T.load_checkpoint(d)
    assert h2 is None
    assert json.load(open(os.path.join(d, "config.json")))["tie_word_embeddings"] is True


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_other_writers_dtypes_and_shards(tmp_path, dtype):
    import torch
    from safetensors.torch import save_file
    cfg = T.Config.tiny()
    tens = _hf_tensors(cfg, 11)
    tdt = getattr(torch, dtype)
    tt = {k: torch.from_numpy(v).to(tdt) for k, v in tens.items()}
    # Two shards and an index, as large checkpoints come.
    names = sorted(tt)
    shard = {n: ("model-00001-of-00002.safetensors" if i % 2 == 0 else "model-00002-of-00002.safetensors")
             for i, n in enumerate(names)}
    for f in set(shard.values()):
        save_file({n: tt[n].contiguous() for n in names if shard[n] == f}, str(tmp_path / f),
                  metadata={"format": "pt"})
    json.dump({"metadata": {"total_size": 0}, "weight_map": shard}, open(tmp_path / "model.safetensors.index.json", "w"))
    json.dump(_config_json(cfg, tied=False), open(tmp_path / "config.json", "w"))
    c2, (e, l, n, h) = T.load_checkpoint(str(tmp_path))
    # The f16 the loader must produce: the stored values (as f32), rounded to nearest even.
    f16 = {k: v.to(torch.float32).numpy().astype(np.float16) for k, v in tt.items()}
    np.testing.assert_array_equal(_bits(e), _bits(f16["model.embed_tokens.weight"].reshape(-1)))
    np.testing.assert_array_equal(_bits(h), _bits(f16["lm_head.weight"].reshape(-1)))
    np.testing.assert_array_equal(_bits(n), _bits(f16["model.norm.weight"]))
    np.testing.assert_array_equal(_bits(l), _bits(_expected_layers(cfg, f16)))


def test_f32_rounding_edges(tmp_path):
    # Round to nearest even at ties, overflow to inf, subnormals, NaN to the quiet NaN.
    from safetensors.numpy import save_file
    cfg = T.Config.tiny()
    tens = _hf_tensors(cfg, 5, head=False)
    special = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65520.0, 70000.0, -1e-7, 6e-8, 2.0 ** -25,
                        3 * 2.0 ** -26, np.inf, -np.inf, np.nan, -0.0], np.float32)
    emb = tens["model.embed_tokens.weight"].reshape(-1)
    emb[:special.size] = special
    save_file(tens, str(tmp_path / "model.safetensors"))
    json.dump(_config_json(cfg), open(tmp_path / "config.json", "w"))
    _, (e, _, _, h) = T.load_checkpoint(str(tmp_path))
    assert h is None
    got = _bits(e)[:special.size]
    with np.errstate(over="ignore"):
        want = _bits(special.astype(np.float16))
    want[10] = 0x7E00  # NaN: the quiet NaN, positive sign (src/half.rs)
    np.testing.assert_array_equal(got, want)


def test_config_defaults_and_rules(tmp_path):
    d = {"hidden_size": 64, "num_hidden_layers": 2, "num_attention_heads": 4, "intermediate_size": 128,
         "vocab_size": 256, "eos_token_id": [7, 9], "max_position_embeddings": 100000}
    json.dump(d, open(tmp_path / "config.json", "w"))
    c = T.checkpoint_config(str(tmp_path))
    assert (c.kv_heads, c.head_dim, c.bos, c.eos, c.max_pos) == (4, 16, 1, 7, 8192)
    assert abs(c.eps - 1e-6) < 1e-12 and c.rope_theta == 10000.0
    d["head_dim"] = None  # a non-number counts as absent
    d["eos_token_id"] = None
    json.dump(d, open(tmp_path / "config.json", "w"))
    c = T.checkpoint_config(str(tmp_path))
    assert (c.head_dim, c.eos) == (16, -1)
    d["rope_scaling"] = {"type": "linear", "factor": 2.0}
    json.dump(d, open(tmp_path / "config.json", "w"))
    with pytest.raises(T.TesselError, match="rope_scaling is not supported"):
        T.checkpoint_config(str(tmp_path))
    del d["rope_scaling"], d["vocab_size"]
    json.dump(d, open(tmp_path / "config.json", "w"))
    with pytest.raises(T.TesselError, match="config.json: no vocab_size"):
        T.checkpoint_config(str(tmp_path))


def _write(tmp_path, cfg, tens, **cfg_extra):
    from safetensors.numpy import save_file
    save_file(tens, str(tmp_path / "model.safetensors"))
    json.dump(_config_json(cfg, **cfg_extra), open(tmp_path / "config.json", "w"))


def test_checkpoint_errors(tmp_path):
    cfg = T.Config.tiny()
    base = {k: v.astype(np.float16) for k, v in _hf_tensors(cfg, 2).items()}
    t = dict(base)
    t["model.layers.0.self_attn.q_proj.bias"] = np.zeros(cfg.heads * cfg.head_dim, np.float16)
    _write(tmp_path, cfg, t)
    with pytest.raises(T.TesselError, match=r"q_proj.bias: models with biases are not supported"):
        T.load_checkpoint(str(tmp_path))
    t = dict(base)
    t["model.layers.1.mlp.up_proj.weight"] = np.zeros((cfg.ffn, cfg.dim + 1), np.float16)
    _write(tmp_path, cfg, t)
    with pytest.raises(T.TesselError, match=r"up_proj.weight: shape \[128, 65\], expected \[128, 64\]"):
        T.load_checkpoint(str(tmp_path))
    t = dict(base)
    del t["model.norm.weight"]
    _write(tmp_path, cfg, t)
    with pytest.raises(T.TesselError, match="checkpoint has no model.norm.weight"):
        T.load_checkpoint(str(tmp_path))
    t = dict(base)
    t["model.norm.weight"] = np.zeros(cfg.dim, np.int16)
    _write(tmp_path, cfg, t)
    with pytest.raises(T.TesselError, match="model.norm.weight: dtype I16 not supported"):
        T.load_checkpoint(str(tmp_path))


def test_json_parser():
    # tests/llm.rs:99-100: escapes and non-ASCII text survive.
    out = json.loads(T.json_roundtrip(r'{"a": [1, -2.5e3, true, null], "b": "x\"é😀y"}'))
    assert out == {"a": [1.0, -2500.0, True, None], "b": 'x"é😀y'}
    out = json.loads(T.json_roundtrip(r'{"u": "é😀\n\t\/", "e": {}, "n": [], "x": 1e-7}'))
    assert out == {"u": "é😀\n\t/", "e": {}, "n": [], "x": 1e-7}
    for bad, where in (('{"a": }', "byte 6"), ('[1, 2', "expected ',' or ']' at byte 5"), ('{"a": 1} x', "trailing data at byte 9"),
                       ('"\\q"', "bad escape"), ("01x", "trailing")):
        with pytest.raises(T.TesselError, match=where):
            T.json_roundtrip(bad)
