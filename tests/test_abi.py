"""The C ABI without a GPU: the library loads and exports every entry point
include/tessel.h declares; tsl_kernel specialises kernels the way
src/ir.rs:970-1043 and src/gpu.rs:148-172 do (cache key, shape and meta
checks) before any device is touched; the product's Weights::random
equals the oracle's bit for bit; the product never reaches the oracle."""

import os
import re

import numpy as np
import pytest

import oracle
import tessel_amd as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "tessel.h")).read()
    return sorted(set(re.findall(r"\b(tsl_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = T.lib()
    syms = header_symbols()
    assert len(syms) >= 27
    for s in syms:
        assert hasattr(L, s), f"{s} declared in include/tessel.h but not exported"
    assert sorted(T.EXPORTS) == syms


def test_kernel_key_matches_the_reference_format():
    k = T.kernel("matmul", "matmul", [[512, 512], [512, 512], [512, 512]], [("BM", 64), ("BN", 64)], 4)
    assert k.key == 'matmul/matmul [[512, 512], [512, 512], [512, 512]] [("BM", 64), ("BN", 64)] 4'
    k2 = T.kernel("matmul", "matmul", [[512, 512], [512, 512], [512, 512]], [("BM", 64), ("BN", 64)], 4)
    assert k2.handle == k.handle
    k3 = T.kernel("llm", "rope_q", [[16, 96], [16], [256, 8], [256, 8], [16, 4, 16]], [], 1)
    assert k3.key == "llm/rope_q [[16, 96], [16], [256, 8], [256, 8], [16, 4, 16]] [] 1"


@pytest.mark.parametrize("args,msg", [
    (("matmul", "matmul", [[4, 8], [9, 4], [4, 4]], []), "dimension K is 8 and 9"),
    (("matmul", "matmul", [[4, 8], [8, 4]], []), "no shape given for array C"),
    (("matmul", "matmul", [[4, 8], [8, 4], [4]], []), "C has 2 dimensions"),
    (("matmul", "matmul", [[4, 8], [8, 4], [4, 4]], [("BQ", 16)]), "no meta constant BQ"),
    (("matmul", "matmul", [[4, 8], [8, 4], [4, 4]], [("BM", 48)]), "powers of two"),
    (("matmul", "nope", [], []), "no kernel nope"),
    (("nofile", "matmul", [], []), "no kernel file nofile"),
    (("llm", "rope_q", [[16, 96], [16], [256, 6], [256, 6], [16, 4, 12]], []), "powers of two"),
])
def test_kernel_specialisation_errors(args, msg):
    with pytest.raises(T.TesselError, match=msg):
        T.kernel(*args)


def test_launch_arity_is_checked():
    k = T.kernel("basic", "add", [[8], [8], [8]])
    with pytest.raises(T.TesselError, match="2 arguments for 3 parameters"):
        T.launch(k, [T.Buf(0, 32), T.Buf(0, 32)])


def test_weights_random_matches_the_oracle():
    for cfg in (T.Config.tiny(), T.Config(96, 1, 6, 2, 16, 160, 300, 1e-5, 10000.0, 64, 1, 2)):
        got = T.weights_random(cfg, 7)
        ocfg = oracle.Config(*[getattr(cfg, f) for f, _ in cfg._fields_])
        want = oracle.weights_random(ocfg, 7)
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g.view(np.uint16), w.view(np.uint16))


def test_mm_candidates_match_the_reference_lists():
    # src/llm/engine.rs:106-147: defaults first; gate_up never takes (32,16,256).
    assert T.mm_candidates(16, False)[0] == ([("BM", 16), ("BN", 64), ("BK", 64)], 4)
    assert len(T.mm_candidates(32, False)) == 8 and len(T.mm_candidates(32, True)) == 7
    assert T.mm_candidates(64, True)[0] == ([("BM", 64), ("BN", 64), ("BK", 32)], 4)
    assert [T.padded(n) for n in (1, 16, 17, 100, 512)] == [16, 16, 32, 128, 512]


def test_product_never_reaches_the_oracle():
    for dirpath, _, files in os.walk(os.path.join(ROOT, "tessel_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "liboracle" not in text and "tsl_ref_" not in text, f
    text = open(os.path.join(ROOT, "include", "tessel.h")).read()
    assert "tsl_ref_" not in text
