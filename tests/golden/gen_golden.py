"""Writes the golden fixtures of tests/golden/ by running the CPU oracle.

    python tests/golden/gen_golden.py [--only NAME]

tinyllama_q4_0_tokens.json -- config 4: the TinyLlama-1.1B-shape Q4_0 model
    of tensorlogic_amd.synth.write_llama_gguf(seed=4), 46-token prompt
    token_ids(4, "prompt", 46, 32000), 128 greedy decode steps: the 129
    oracle tokens, the top1-top2 logit margin of each step, the 8 largest
    logits of each step (ids and f16 values, from a step-by-step forward
    that must reproduce the greedy stream) and the final logits (f16
    values).  The GPU test regenerates the same file from the seed and
    compares.
phi2_q8_0_tokens.json -- config 5: the Phi-2-shape Q8_0 model of
    write_phi2_gguf(seed=5), 512-token prompt token_ids(5, "prompt", 512,
    51200), 256 greedy decode steps, recorded the same way.
synth_checksums.json -- sha256 of fixed generator draws, pinning the seeded
    generator across machines.

Final logits are stored as base64 of their f16 bytes (little-endian).
"""
from __future__ import annotations

import argparse
import base64
import hashlib
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from tensorlogic_amd import synth as S  # noqa: E402


def synth_checksums():
    draws = {
        "q4_0_blocks(1,'W',64,256)": S.q4_0_blocks(1, "W", 64, 256).tobytes(),
        "q8_0_blocks(1,'W',64,256)": S.q8_0_blocks(1, "W", 64, 256).tobytes(),
        "normal_f16(1,'x',(4,2048))": S.normal_f16(1, "x", (4, 2048)).tobytes(),
        "token_ids(4,'prompt',46,32000)": S.token_ids(4, "prompt", 46, 32000).tobytes(),
    }
    return {k: hashlib.sha256(v).hexdigest() for k, v in draws.items()}


def record_tokens(path, arch, prompt, n_decode, max_ctx, top=8):
    """Oracle greedy stream + per-step top logits (step-wise forward, which
    must reproduce the generate() stream)."""
    t0 = time.time()
    m = O.Model(path, arch=arch, max_ctx=max_ctx)
    toks, margins, logits = m.generate(prompt, n_decode)
    m.reset()
    top_ids, top_vals = [], []
    _, lg = m.forward(prompt, 0)
    for step in range(n_decode + 1):
        order = np.argsort(-lg.astype(np.float32), kind="stable")[:top]
        top_ids.append([int(i) for i in order])
        top_vals.append([float(lg[i]) for i in order])
        if O.argmax_last(lg) != toks[step]:
            raise RuntimeError(f"step-wise forward diverged from generate at step {step}")
        if step < n_decode:
            _, lg = m.forward(np.array([toks[step]], np.int32), len(prompt) + step)
    m.close()
    print(f"oracle: {time.time() - t0:.1f} s", file=sys.stderr)
    return {
        "prompt": prompt.tolist(),
        "n_decode": n_decode,
        "tokens": toks.tolist(),
        "margins": [float(x) for x in margins],
        f"top{top}_ids": top_ids,
        f"top{top}_logits": top_vals,
        "last_logits_f16_b64": base64.b64encode(logits.astype("<f2").tobytes()).decode(),
    }


def tinyllama_tokens(n_decode=128, seed=4):
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "tinyllama.gguf")
        S.write_llama_gguf(path, seed=seed, **S.TINYLLAMA_ARGS)
        prompt = S.token_ids(seed, "prompt", 46, S.TINYLLAMA_ARGS["vocab"])
        rec = record_tokens(path, 0, prompt, n_decode, 256)
    return {"config": "TinyLlama-1.1B shape, Q4_0 linear weights, seed 4", "seed": seed, **rec}


def phi2_tokens(n_decode=256, seed=5):
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "phi2.gguf")
        S.write_phi2_gguf(path, seed=seed, **S.PHI2_ARGS)
        prompt = S.token_ids(seed, "prompt", 512, S.PHI2_ARGS["vocab"])
        rec = record_tokens(path, 1, prompt, n_decode, 800)
    return {"config": "Phi-2 shape, Q8_0 linear weights, seed 5", "seed": seed, **rec}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", default="")
    a = ap.parse_args()
    jobs = {"synth_checksums.json": synth_checksums,
            "tinyllama_q4_0_tokens.json": tinyllama_tokens,
            "phi2_q8_0_tokens.json": phi2_tokens}
    for name, fn in jobs.items():
        if a.only and a.only != name:
            continue
        data = fn()   # computed before the file is opened: no partial fixture
        tmp = os.path.join(HERE, name + ".tmp")
        with open(tmp, "w") as f:
            json.dump(data, f)
        os.replace(tmp, os.path.join(HERE, name))
        print(f"wrote {name}", file=sys.stderr)


if __name__ == "__main__":
    main()
