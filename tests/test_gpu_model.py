"""Decoder parity: the device runner vs the CPU oracle on the same GGUF file.

Greedy tokens must be identical (temperature_sample(., 0) semantics, last max
wins); the final logits within max-abs 2e-2 / rel-L2 1e-3.  Small models run
the oracle live; the full TinyLlama-shape model is checked against the
oracle's committed golden tokens (tests/golden/).
"""
import json
import os

import numpy as np
import pytest

from tensorlogic_amd import Model
from tensorlogic_amd.gguf import GGML_Q4_0, GGML_Q8_0
from tensorlogic_amd import synth as S

from test_gpu_ops import assert_close

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

TINY_LLAMA = dict(n_layers=2, hidden=256, inter=512, n_heads=4, n_kv=2, vocab=1000)
TINY_PHI2 = dict(n_layers=2, hidden=320, inter=1280, n_heads=4, vocab=1000, rot=32)


def _compare(dev, oracle, path, arch, prompt, n_decode, max_ctx=256):
    om = oracle.Model(path, arch=arch, max_ctx=max_ctx)
    ref_toks, margins, ref_logits = om.generate(prompt, n_decode)
    om.close()
    m = Model(dev, path, arch=arch, max_ctx=max_ctx)
    for use_graph in (False, True):
        toks = m.generate(prompt, n_decode, use_graph=use_graph)
        mism = np.nonzero(toks != ref_toks)[0]
        assert mism.size == 0, (f"graph={use_graph}: first mismatch at step {mism[0]}: "
                                f"{toks[mism[0]]} vs {ref_toks[mism[0]]} (oracle margin {margins[mism[0]]:.3g})")
        assert_close(m.logits(), ref_logits, what="final logits")
    # host-driven prefill / decode API gives the same stream
    m.reset()
    t = m.prefill(prompt)
    seq = [t]
    for _ in range(min(n_decode, 8)):
        t = m.decode(t)
        seq.append(t)
    assert seq == list(ref_toks[:len(seq)])
    m.close()


@pytest.mark.parametrize("qtype", [GGML_Q4_0, GGML_Q8_0])
def test_tiny_llama_greedy(dev, oracle, tmp_path, qtype):
    path = str(tmp_path / "tiny_llama.gguf")
    S.write_llama_gguf(path, seed=21, qtype=qtype, **TINY_LLAMA)
    prompt = S.token_ids(21, "prompt", 46, TINY_LLAMA["vocab"])
    _compare(dev, oracle, path, 0, prompt, 32)


def test_tiny_phi2_greedy(dev, oracle, tmp_path):
    path = str(tmp_path / "tiny_phi2.gguf")
    S.write_phi2_gguf(path, seed=22, **TINY_PHI2)
    prompt = S.token_ids(22, "prompt", 40, TINY_PHI2["vocab"])
    _compare(dev, oracle, path, 1, prompt, 24)


def test_long_prompt_chunked_prefill(dev, oracle, tmp_path):
    # more prompt tokens than one prefill chunk holds (512 rows)
    path = str(tmp_path / "tiny_llama_long.gguf")
    S.write_llama_gguf(path, seed=23, **TINY_LLAMA)
    prompt = S.token_ids(23, "prompt", 600, TINY_LLAMA["vocab"])
    _compare(dev, oracle, path, 0, prompt, 8, max_ctx=700)


def _golden(name):
    p = os.path.join(GOLDEN, name)
    if not os.path.exists(p):
        pytest.skip(f"{name} not generated")
    with open(p) as f:
        return json.load(f)


def test_tinyllama_full_golden_tokens(dev, tmp_path):
    """TinyLlama-1.1B shape, Q4_0, 46-token prompt, 128 greedy steps (config 4)."""
    g = _golden("tinyllama_q4_0_tokens.json")
    path = str(tmp_path / "tinyllama.gguf")
    S.write_llama_gguf(path, seed=g["seed"], **S.TINYLLAMA_ARGS)
    prompt = np.array(g["prompt"], np.int32)
    m = Model(dev, path, arch=0, max_ctx=256)
    toks = m.generate(prompt, g["n_decode"], use_graph=True)
    ref = np.array(g["tokens"], np.int32)
    mism = np.nonzero(toks != ref)[0]
    assert mism.size == 0, f"first mismatch at step {mism[0]}: {toks[mism[0]]} vs {ref[mism[0]]}"
    assert_close(m.logits(), np.array(g["last_logits"], np.float16), what="final logits")
    m.close()
