"""The command line (src/main.rs): usage, llm-tiny and the llm argument
errors run on the host; bench and llm on the GPU print the reference's
JSON lines (src/bench.rs:398-405, src/main.rs:297-313)."""

import json
import os
import subprocess
import sys

import numpy as np
import pytest

import tessel_amd as T
from tessel_amd import cli

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _cli(*args, timeout=600):
    return subprocess.run([sys.executable, "-m", "tessel_amd", *args], cwd=ROOT, capture_output=True, text=True,
                          timeout=timeout)


def test_usage_and_formatting():
    r = _cli()
    assert r.returncode == 0 and "llm-tiny" in r.stdout
    # Rust's {:?} of the meta list and {:e} / {:.3e} of floats.
    assert cli.config_name([("BM", 128), ("BN", 64)], 4) == '[("BM", 128), ("BN", 64)] warps 4'
    assert [cli.rust_e(x) for x in (0.1, 1.0, -2.5e-7, 123456.0, 0.0)] == ["1e-1", "1e0", "-2.5e-7", "1.23456e5",
                                                                            "0e0"]
    assert cli.rust_e(0.000123456, 3) == "1.235e-4" and cli.rust_e(0.0, 3) == "0.000e0"


def test_rng_matches_the_reference_generator():
    # bench::Rng (src/bench.rs:13-35) through the library equals the oracle's.
    import oracle
    a, b = T.Rng(7), oracle.Rng(7)
    assert [a.bits() for _ in range(5)] == [b.bits() for _ in range(5)]
    np.testing.assert_array_equal(a.tensor("f16", [33, 7], 2.0).view(np.uint16),
                                  b.tensor("f16", [33, 7], 2.0).view(np.uint16))
    np.testing.assert_array_equal(a.tensor("f32", [100], 4.0), b.tensor("f32", [100], 4.0))
    assert a.below(1000) == b.below(1000)


def test_llm_tiny_writes_a_checkpoint(tmp_path):
    d = tmp_path / "tiny"
    r = _cli("llm-tiny", str(d))
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == f"wrote a tiny random Llama to {d}"
    cfg, (e, l, n, h) = T.load_checkpoint(str(d))
    w = T.weights_random(T.Config.tiny(), 1)
    np.testing.assert_array_equal(l.view(np.uint16), w[1].view(np.uint16))


def test_llm_argument_errors(tmp_path):
    assert "--prompts is required" in _cli("llm", str(tmp_path)).stderr
    r = _cli("llm", str(tmp_path), "--prompts", "p.json", "--device", "emu")
    assert r.returncode == 1 and "unknown device emu" in r.stderr
    p = tmp_path / "p.json"
    p.write_text('{"a": 1}')
    assert f"{p}: not a JSON list" in _cli("llm", str(tmp_path), "--prompts", str(p)).stderr
    p.write_text("[[1, 2], 3]")
    assert "each prompt is a list of token ids" in _cli("llm", str(tmp_path), "--prompts", str(p)).stderr
    p.write_text("[[1, 2]]")
    r = _cli("llm", str(tmp_path / "none"), "--prompts", str(p))
    assert r.returncode == 1 and r.stderr.startswith("tessel: ")


@pytest.mark.gpu
def test_bench_quick_lines(tmp_path):
    out = tmp_path / "b.jsonl"
    tuned = tmp_path / "tuned.tsv"
    r = _cli("bench", "--quick", "--iters", "20", "--json", str(out), "--tuned", str(tuned))
    assert r.returncode == 0, r.stderr
    rows = [json.loads(x) for x in r.stdout.splitlines()]
    assert [x["kind"] for x in rows] == ["gemm", "attention", "softmax", "rmsnorm"]
    for x in rows:
        assert set(x) >= {"kind", "label", "engine", "device", "median_ms", "min_ms", "tflops", "gbps", "rel_err",
                          "sm_mhz", "config", "tried"}
        assert x["rel_err"] < 2e-2 and x["median_ms"] > 0, x
    # Tiles follow from the shape: one candidate per case runs distinct code,
    # and only it is timed.
    assert rows[0]["label"] == "1024x1024x1024"
    assert all(len(x["tried"]) == 1 and x["tiles"] == "by shape" for x in rows)
    assert [json.loads(x) for x in out.read_text().splitlines()] == rows
    # The tuned file keeps the choice: a second run times only it.
    r = _cli("bench", "--quick", "--iters", "5", "--tuned", str(tuned))
    rows2 = [json.loads(x) for x in r.stdout.splitlines()]
    assert all(len(x["tried"]) == 1 and x["config"] == y["config"] for x, y in zip(rows2, rows))


@pytest.mark.gpu
def test_llm_on_a_tiny_checkpoint(tmp_path):
    d = tmp_path / "tiny"
    assert _cli("llm-tiny", str(d)).returncode == 0
    prompts = [[1, 5, 9, 3], [2, 7], [4, 4, 4, 4, 4, 4]]
    p = tmp_path / "p.json"
    p.write_text(json.dumps(prompts))
    r = _cli("llm", str(d), "--prompts", str(p), "--max-new", "6", "--batch", "2", "--warmup", "--json",
             str(tmp_path / "o.json"), "--logits", str(tmp_path / "l.json"), "--profile")
    assert r.returncode == 0, r.stderr
    line = json.loads(r.stdout)
    assert line["engine"] == "tessel" and line["requests"] == 3 and line["batch"] == 2
    assert line["prompt_tokens"] == 12 and len(line["first_token_s"]) == 3
    assert json.loads((tmp_path / "o.json").read_text()) == line
    # --profile: every launch of a third run timed, by phase and kernel.
    prof = line["profile"]
    assert {x["phase"] for x in prof} == {"prefill", "decode"}
    assert any(x["kernel"].startswith("decode_attention -> [") for x in prof)
    assert all(x["launches"] > 0 and x["ms"] > 0 for x in prof)
    assert "decode, kernel time by kernel" in r.stderr
    # The same generation through the library.
    T.open()
    cfg, w = T.load_checkpoint(str(d))
    lim = T.Limits(16, 1024, 1024, max(cfg.max_pos // 16, 1))
    e = T.Engine(cfg, lim, w)
    outs, _ = e.generate([(q, 6) for q in prompts], 2)
    e.close()
    assert line["outputs"] == outs
    logits = json.loads((tmp_path / "l.json").read_text())
    assert len(logits) == cfg.vocab


def test_distinct_configs_keeps_one_per_code():
    # Candidates differing only in tiles or warps run the same code (one is
    # kept); a different column chunk (BC, read by the row kernels) is
    # different code.
    from tessel_amd.cli import distinct_configs
    c = [([("BM", 64), ("BN", 64)], 4), ([("BM", 128), ("BN", 64)], 8)]
    assert distinct_configs(c) == c[:1]
    r = [([("BR", 1), ("BC", 1024)], 4), ([("BR", 2), ("BC", 1024)], 4), ([("BR", 1), ("BC", 2048)], 8)]
    assert distinct_configs(r) == [r[0], r[2]]
