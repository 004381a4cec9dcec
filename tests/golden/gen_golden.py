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
tinyllama_q4_0_margins_tokens.json -- the config-4 architecture with real
    logit margins (RMSNorm weights 1 + N(0, 0.02), zero-mean Q4_0 codes;
    see tinyllama_margins_tokens), recorded the same way plus each step's
    top-2 margin in f16 ulps, and the same model run by the oracle with
    every fp32 sum taken in descending order (ACC_F32_REV): its per-step
    top-8 deviation teacher-forced and its free-running greedy stream -- how
    far a second, equally valid fp32 summation order moves this model.
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
        "q4_0_blocks(1,'W',64,256,zero_mean)": S.q4_0_blocks(1, "W", 64, 256, zero_mean=True).tobytes(),
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
        rec.update(reorder_final_logits(path, 0, prompt, rec, 256))
    return {"config": "TinyLlama-1.1B shape, Q4_0 linear weights, seed 4", "seed": seed, **rec}


def reordered_oracle(path, prompt, rec, n_decode, top=8):
    """The oracle with every fp32 sum in descending order (ACC_F32_REV) on
    the same model: per-step deviation of its top-k logits from rec's, in
    f16 ulps of the top logit, on rec's own token stream (teacher-forced),
    and its free-running greedy stream."""
    ids = np.array(rec[f"top{top}_ids"], np.int64)
    vals = np.array(rec[f"top{top}_logits"], np.float64)
    toks = np.array(rec["tokens"], np.int32)
    m = O.Model(path, arch=0, max_ctx=256, acc=O.ACC_F32_REV)
    dev = []
    _, lg = m.forward(prompt, 0)
    for step in range(n_decode + 1):
        ulp = 2.0 ** (np.floor(np.log2(max(abs(vals[step][0]), 2.0 ** -14))) - 10)
        dev.append(float(np.abs(lg.astype(np.float64)[ids[step]] - vals[step]).max() / ulp))
        if step < n_decode:
            _, lg = m.forward(np.array([toks[step]], np.int32), len(prompt) + step)
    m.reset()
    rtoks, _, _ = m.generate(prompt, n_decode)
    m.close()
    bad = np.nonzero(rtoks != toks)[0]
    return {"reorder_dev_ulps": dev, "reorder_tokens": rtoks.tolist(),
            "reorder_first_divergence": int(bad[0]) if bad.size else n_decode + 1}


def reorder_final_logits(path, arch, prompt, rec, max_ctx):
    """The reordered oracle (ACC_F32_REV) teacher-forced on rec's token
    stream: the relative L2 distance of its final logits from rec's -- how
    far a second, equally valid fp32 summation order moves the end-to-end
    logits of this model."""
    toks = np.array(rec["tokens"], np.int32)
    n_decode = rec["n_decode"]
    m = O.Model(path, arch=arch, max_ctx=max_ctx, acc=O.ACC_F32_REV)
    _, lg = m.forward(prompt, 0)
    for step in range(n_decode):
        _, lg = m.forward(np.array([toks[step]], np.int32), len(prompt) + step)
    m.close()
    ref = np.frombuffer(base64.b64decode(rec["last_logits_f16_b64"]), "<f2").astype(np.float64)
    got = lg.astype(np.float64)
    return {"reorder_last_logits_rel_l2": float(np.linalg.norm(got - ref) / np.linalg.norm(ref))}


def tinyllama_margins_tokens(n_decode=128, seed=8):
    """Config-4 shape (22 layers, 2048 / 5632, 32 / 4 heads, vocab 32000),
    Q4_0, with RMSNorm weights 1 + N(0, 0.02) and Q4_0 codes symmetric about
    8 (synth.write_llama_gguf(zero_mean=True)): logits of a few units, so
    the greedy stream is diverse and its top-2 margins are real.  The seed
    is the one of seeds 5..16 whose smallest margin over the 129 steps,
    in f16 ulps of the top logit, comes latest and is largest."""
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "tinyllama_margins.gguf")
        S.write_llama_gguf(path, seed=seed, norm_mean=1.0, zero_mean=True, **S.TINYLLAMA_ARGS)
        prompt = S.token_ids(seed, "prompt", 46, S.TINYLLAMA_ARGS["vocab"])
        rec = record_tokens(path, 0, prompt, n_decode, 256)
        rec.update(reordered_oracle(path, prompt, rec, n_decode))
        rec.update(reorder_final_logits(path, 0, prompt, rec, 256))
    top = np.array(rec["top8_logits"], np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(top[:, 0]), 2.0 ** -14))) - 10)
    rec["margin_ulps"] = [float(v) for v in (top[:, 0] - top[:, 1]) / ulp]
    rec["min_margin_ulps"] = float(min(rec["margin_ulps"]))
    return {"config": "TinyLlama-1.1B shape, Q4_0 (codes 1..15), RMSNorm weights 1 + N(0, 0.02), seed "
                      f"{seed}", "seed": seed, **rec}


def phi2_tokens(n_decode=256, seed=5):
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "phi2.gguf")
        S.write_phi2_gguf(path, seed=seed, **S.PHI2_ARGS)
        prompt = S.token_ids(seed, "prompt", 512, S.PHI2_ARGS["vocab"])
        rec = record_tokens(path, 1, prompt, n_decode, 800)
        rec.update(reorder_final_logits(path, 1, prompt, rec, 800))
    return {"config": "Phi-2 shape, Q8_0 linear weights, seed 5", "seed": seed, **rec}


def augment_reorder(name):
    """Adds reorder_last_logits_rel_l2 to an existing token file without
    recomputing the rest (the model is regenerated from its seed)."""
    fp = os.path.join(HERE, name)
    rec = json.load(open(fp))
    seed = rec["seed"]
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "m.gguf")
        if name.startswith("phi2"):
            S.write_phi2_gguf(path, seed=seed, **S.PHI2_ARGS)
            arch, max_ctx = 1, 800
        elif "margins" in name:
            S.write_llama_gguf(path, seed=seed, norm_mean=1.0, zero_mean=True, **S.TINYLLAMA_ARGS)
            arch, max_ctx = 0, 256
        else:
            S.write_llama_gguf(path, seed=seed, **S.TINYLLAMA_ARGS)
            arch, max_ctx = 0, 256
        rec.update(reorder_final_logits(path, arch, np.array(rec["prompt"], np.int32), rec, max_ctx))
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", default="")
    ap.add_argument("--augment-reorder", action="store_true",
                    help="only add reorder_last_logits_rel_l2 to the existing token files")
    a = ap.parse_args()
    jobs = {"synth_checksums.json": synth_checksums,
            "tinyllama_q4_0_tokens.json": tinyllama_tokens,
            "tinyllama_q4_0_margins_tokens.json": tinyllama_margins_tokens,
            "phi2_q8_0_tokens.json": phi2_tokens}
    for name, fn in jobs.items():
        if a.only and a.only != name:
            continue
        if a.augment_reorder and not name.endswith("_tokens.json"):
            continue
        # computed before the file is opened: no partial fixture
        data = augment_reorder(name) if a.augment_reorder else fn()
        tmp = os.path.join(HERE, name + ".tmp")
        with open(tmp, "w") as f:
            json.dump(data, f)
        os.replace(tmp, os.path.join(HERE, name))
        print(f"wrote {name}", file=sys.stderr)


if __name__ == "__main__":
    main()
