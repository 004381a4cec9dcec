"""The seeded generator is a fixed function of (seed, name, purpose): draws
hash to the committed checksums, so the GPU box, this container and the
oracle all see the same bytes.  CPU only."""
import hashlib
import json
import os

import numpy as np

from tensorlogic_amd import synth as S

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "synth_checksums.json")


def test_generator_checksums():
    ref = json.load(open(GOLDEN))
    draws = {
        "q4_0_blocks(1,'W',64,256)": S.q4_0_blocks(1, "W", 64, 256).tobytes(),
        "q8_0_blocks(1,'W',64,256)": S.q8_0_blocks(1, "W", 64, 256).tobytes(),
        "q4_0_blocks(1,'W',64,256,zero_mean)": S.q4_0_blocks(1, "W", 64, 256, zero_mean=True).tobytes(),
        "normal_f16(1,'x',(4,2048))": S.normal_f16(1, "x", (4, 2048)).tobytes(),
        "token_ids(4,'prompt',46,32000)": S.token_ids(4, "prompt", 46, 32000).tobytes(),
    }
    assert {k: hashlib.sha256(v).hexdigest() for k, v in draws.items()} == ref


def test_distributions_match_the_configs():
    # config 1: Q4_0 scales in [1e-3, 2e-2], nibbles uniform 0..15
    b = S.q4_0_blocks(2, "W", 256, 2048).reshape(-1, 18)
    d = b[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    assert d.min() >= 1e-3 - 1e-6 and d.max() <= 2e-2 + 1e-5
    nib = np.concatenate([b[:, 2:] & 15, b[:, 2:] >> 4]).ravel()
    assert np.abs(np.bincount(nib, minlength=16) / nib.size - 1 / 16).max() < 2e-3
    # zero-mean Q4_0 codes: uniform 1..15, so (q - 8) is symmetric about 0
    z = S.q4_0_blocks(2, "W", 256, 2048, zero_mean=True).reshape(-1, 18)
    nz = np.concatenate([z[:, 2:] & 15, z[:, 2:] >> 4]).ravel()
    cnt = np.bincount(nz, minlength=16)
    assert cnt[0] == 0 and np.abs(cnt[1:] / nz.size - 1 / 15).max() < 2e-3
    assert np.array_equal(z[:, :2], b[:, :2])   # same scales as the full-range draw
    # config 2: Q8_0 scales in [1e-3, 1e-2], codes uniform in [-127, 127]
    b = S.q8_0_blocks(2, "W", 256, 2048).reshape(-1, 34)
    q = b[:, 2:].copy().view(np.int8).astype(np.int32).ravel()
    assert q.min() == -127 and q.max() == 127
    x = S.normal_f16(2, "x", (64, 2048)).astype(np.float64)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02
    ids = S.token_ids(2, "ids", 100000, 32000)
    assert ids.min() >= 0 and ids.max() < 32000
