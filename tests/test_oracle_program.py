"""Pins oracle/program.py -- debug/chat_demo_with_kvcache.tl composed one TL
builtin at a time -- against the oracle's decoder runner (tlo_model), an
independent restatement of the same model: in both semantics (the program as
written: decode rows rotated at position 0, rms_norm eps 1e-6; and absolute
positions with the file's eps) every logit of the prefill and of each decode
step agrees bit for bit.  The runner is itself pinned against a float64
numpy decoder (test_oracle_decoder.py).  CPU only.
"""
import numpy as np
import pytest

from oracle.program import ChatDemoKVCache, ChatDemoOptimized
from tensorlogic_amd import synth as S

# head_dim 64, so the program's literal `* 0.125` is 1 / sqrt(head_dim)
SMALL = dict(n_layers=2, hidden=256, inter=512, n_heads=4, n_kv=2, vocab=500)


@pytest.fixture(scope="module")
def model_path(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("prog") / "small.gguf")
    S.write_llama_gguf(p, seed=31, norm_mean=1.0, **SMALL)
    return p


def _runner_stream(oracle, path, literal, prompt, n):
    m = oracle.Model(path, arch=0, max_ctx=64)
    m.set_program_semantics(literal)
    _, lg = m.forward(np.asarray(prompt, np.int32), 0)
    out = [lg]
    for step in range(n):
        tok = oracle.argmax_last(lg)
        _, lg = m.forward(np.asarray([tok], np.int32), len(prompt) + step)
        out.append(lg)
    m.close()
    return out


@pytest.mark.parametrize("literal", [True, False])
def test_program_composition_equals_runner(oracle, model_path, literal):
    prompt = S.token_ids(31, "prompt", 12, SMALL["vocab"])
    n = 6
    ref = _runner_stream(oracle, model_path, literal, prompt, n)
    prog = ChatDemoKVCache(model_path, "program" if literal else "absolute", 1e-6 if literal else 1e-5)
    lg = prog.prefill(prompt)[0]
    for step in range(n + 1):
        assert np.array_equal(lg.view(np.uint16), ref[step].view(np.uint16)), f"step {step}"
        if step < n:
            lg = prog.decode(oracle.argmax_last(lg))[0]


def test_program_semantics_differ_from_absolute(oracle, model_path):
    """The two semantics agree on the prompt and part at the first decode
    step (rotation at 0 vs at the token's position), so the tests above
    distinguish them."""
    prompt = S.token_ids(31, "prompt", 12, SMALL["vocab"])
    a = ChatDemoKVCache(model_path, "program", 1e-6)
    b = ChatDemoKVCache(model_path, "absolute", 1e-6)
    la, lb = a.prefill(prompt)[0], b.prefill(prompt)[0]
    assert np.array_equal(la.view(np.uint16), lb.view(np.uint16))
    t = oracle.argmax_last(la)
    assert not np.array_equal(a.decode(t)[0].view(np.uint16), b.decode(t)[0].view(np.uint16))


def test_program_semantics_are_llama_only(oracle, tmp_path):
    p = str(tmp_path / "phi.gguf")
    S.write_phi2_gguf(p, seed=32, n_layers=1, hidden=128, inter=256, n_heads=2, vocab=64, rot=32)
    m = oracle.Model(p, arch=1, max_ctx=16)
    with pytest.raises(ValueError):
        m.set_program_semantics(True)
    m.close()


def test_optimized_loop_equals_cached_absolute(oracle, model_path):
    """examples/chat_demo_optimized.tl recomputes every row each step (no
    cache), with rope over the full sequence (row s at position s) and the
    builtin rms_norm eps 1e-6: per output row the oracle's arithmetic does
    not depend on how many rows a call holds, so each step's logits equal
    the cached program's at absolute positions with eps 1e-6 bit for bit --
    and those differ from the program-as-written decode (rows at position
    0), so the check tells the two apart."""
    prompt = S.token_ids(31, "prompt", 12, SMALL["vocab"])
    n = 5
    gen, logits, _ = ChatDemoOptimized(model_path, 1e-6).generate(prompt, max_steps=n, temperature=0.0, eos=-1)
    assert len(gen) == len(prompt) + n and len(logits) == n
    cached = ChatDemoKVCache(model_path, "absolute", 1e-6)
    lit = ChatDemoKVCache(model_path, "program", 1e-6)
    lg, ll = cached.prefill(prompt)[0], lit.prefill(prompt)[0]
    differs = False
    for step in range(n):
        assert np.array_equal(logits[step].view(np.uint16), lg.view(np.uint16)), f"step {step}"
        assert int(gen[len(prompt) + step]) == oracle.argmax_last(lg)
        differs |= not np.array_equal(lg.view(np.uint16), ll.view(np.uint16))
        if step < n - 1:
            tok = int(gen[len(prompt) + step])
            lg, ll = cached.decode(tok)[0], lit.decode(tok)[0]
    assert differs


def test_optimized_loop_stops_at_eos_and_samples(oracle, model_path):
    """The loop ends before appending EOS; at T = 0.8 each step's id is the
    inverse-CDF pick of softmax(logits / T) for that step's draw."""
    prompt = S.token_ids(31, "prompt", 12, SMALL["vocab"])
    prog = ChatDemoOptimized(model_path, 1e-6)
    gen, logits, draws = prog.generate(prompt, max_steps=4, temperature=0.8, seed=3, eos=-1)
    for step, (lg, u) in enumerate(zip(logits, draws)):
        assert int(gen[len(prompt) + step]) == oracle.sample_temperature(lg, 0.8, u)
    first = int(gen[len(prompt)])
    gen2, logits2, _ = prog.generate(prompt, max_steps=4, temperature=0.8, seed=3, eos=first)
    assert len(gen2) == len(prompt) and len(logits2) == 1
