"""Pins the CPU oracle (oracle/liboracle.so) before it is trusted as the
parity checker.  CPU only.

Each oracle function is checked against (a) the known answers the
reference's own tests hold for it, and (b) what the mathematics fixes,
computed independently in numpy / float64 (closed forms, brute force over
every code, invariants), chosen so that a plausible mistake -- a swapped
nibble half, a wrong sign or pair index, a transposed operand, a dropped
eps or scale -- fails at least one check.  Functions with nothing but the
reference's Metal transcendentals to compare to are pinned by closed form
within a stated f16 tolerance (see the module docstrings of each group).
"""
import numpy as np
import pytest

from tensorlogic_amd import synth as S

# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------


def h(x):
    return np.asarray(x, np.float16)


def _ulp16(x):
    """f16 spacing at |x| (2^-24 below the normal range)."""
    a = np.abs(np.asarray(x, np.float64))
    return 2.0 ** (np.floor(np.log2(np.maximum(a, 2.0 ** -14))) - 10)


def ulps(a, b):
    """Distance in f16 units in the last place (sign-magnitude aware)."""
    ai = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    bi = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


def q4_block(d, nibbles):
    """One GGUF Q4_0 block from 32 nibble codes (element j < 16 in the low
    half of byte j, element j + 16 in its high half)."""
    nib = np.asarray(nibbles, np.uint8)
    b = np.empty(18, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:] = (nib[:16] & 0xF) | ((nib[16:] & 0xF) << 4)
    return b


def q8_block(d, codes):
    b = np.empty(34, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:] = np.asarray(codes, np.int8).view(np.uint8)
    return b


# ---------------------------------------------------------------------------
# binary16 conversion (`half` 2.7.1 from_f32 / to_f32: IEEE RNE)
# ---------------------------------------------------------------------------
def test_f16_conversion_matches_ieee(oracle):
    # every f16 bit pattern converts up exactly like numpy's IEEE conversion
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.h2f(bits)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    # f32 -> f16: ties, subnormals, overflow, random values
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 200000),
        (np.arange(2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),   # subnormal ties
        np.float32([65504.0, 65519.99, 65520.0, 1e9, -1e9, 0.0, -0.0, 2.0 ** -25, 2.0 ** -26,
                    1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]),
    ]).astype(np.float32)
    got = oracle.f2h(xs)
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------------------
# dequantisation (gguf.rs:22-112): bit-exact
# ---------------------------------------------------------------------------
def test_dequant_reference_known_answers(oracle):
    # gguf.rs:622-640: Q8_0, scale 1, codes 0..31 -> 0, 1, 2
    y = oracle.dequant(q8_block(1.0, np.arange(32)), 8).astype(np.float32)
    assert y[0] == 0.0 and y[1] == 1.0 and y[2] == 2.0
    # gguf.rs:663-690: two Q8_0 blocks, scales 1 and 2 -> y[10] = 10, y[32] = 0, y[42] = 20
    two = np.concatenate([q8_block(1.0, np.arange(32)), q8_block(2.0, np.arange(32))])
    y = oracle.dequant(two, 8).astype(np.float32)
    assert (y[0], y[10], y[32], y[42]) == (0.0, 10.0, 0.0, 20.0)
    # gguf.rs:692-714: Q4_0, scale 0.5, every byte 0xFF -> (15 - 8) * 0.5 = 3.5
    blk = np.full(18, 0xFF, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    assert np.all(oracle.dequant(blk, 2).astype(np.float32) == 3.5)
    # gguf.rs:642-661: byte 0x01 in a scale-1 block: element 0 = 1 - 8, element 16 = 0 - 8
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2] = 0x01
    y = oracle.dequant(blk, 2).astype(np.float32)
    assert y[0] == -7.0 and y[16] == -8.0 and y[1] == -8.0


def test_dequant_q4_0_element_order_and_all_codes(oracle):
    # element j carries code j % 16 with distinct halves: a swapped nibble half
    # or a transposed element order fails here
    codes = np.array([j % 16 for j in range(16)] + [15 - (j % 16) for j in range(16)], np.uint8)
    y = oracle.dequant(q4_block(1.0, codes), 2).astype(np.float32)
    assert np.array_equal(y, codes.astype(np.float32) - 8.0)
    # brute force: every code x 4096 scales (normal, subnormal, extremes)
    rng = np.random.default_rng(1)
    scales = np.concatenate([rng.uniform(1e-3, 2e-2, 2000), rng.uniform(-4, 4, 2000),
                             [6.1e-5, 5.96e-8, 65504.0, -65504.0, 0.0, -0.0] + [2.0 ** -k for k in range(90)]])
    scales = h(scales).astype(np.float32)
    blocks, ref = [], []
    for d in scales:
        c = rng.integers(0, 16, 32).astype(np.uint8)
        blocks.append(q4_block(d, c))
        ref.append(((c.astype(np.float32) - 8.0) * np.float32(d)).astype(np.float16))
    got = oracle.dequant(np.concatenate(blocks), 2)
    assert np.array_equal(got.view(np.uint16), np.concatenate(ref).view(np.uint16))


def test_dequant_q8_0_all_codes(oracle):
    rng = np.random.default_rng(2)
    codes = np.arange(-128, 128).astype(np.int8).reshape(8, 32)
    blocks, ref = [], []
    for d in h(np.concatenate([rng.uniform(1e-3, 1e-2, 300), rng.uniform(-300, 300, 100),
                               [5.96e-8, 65504.0]])).astype(np.float32):
        for c in codes:
            blocks.append(q8_block(d, c))
            ref.append((c.astype(np.float32) * np.float32(d)).astype(np.float16))
    got = oracle.dequant(np.concatenate(blocks), 8)
    assert np.array_equal(got.view(np.uint16), np.concatenate(ref).view(np.uint16))


def q6k_block(d, sc, codes):
    """One GGUF Q6_K super-block from 256 six-bit codes, written from the
    block's element-index form: element e = 128 n + 32 j + l keeps its low
    4 bits in nibble j // 2 of ql[64 n + 32 (j % 2) + l], its high 2 bits in
    bits 2 j .. 2 j + 1 of qh[32 n + l], and its scale in sc[e // 16]."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for e, q in enumerate(codes):
        n, j, l = e // 128, (e % 128) // 32, e % 32
        ql[64 * n + 32 * (j % 2) + l] |= (int(q) & 15) << (4 * (j // 2))
        qh[32 * n + l] |= (int(q) >> 4) << (2 * j)
    return np.concatenate([ql, qh, np.asarray(sc, np.int8).view(np.uint8),
                           np.frombuffer(np.float16(d).tobytes(), np.uint8)])


def test_dequant_q6_k_layout(oracle):
    # distinct codes and distinct scales per 16-element group: a swapped
    # nibble, bit pair, ql half or scale index fails here (no reference test
    # covers Q6_K; gguf.rs:128-212 is the only statement of it)
    codes = (np.arange(256) * 7 + 3) % 64
    y = oracle.dequant(q6k_block(1.0, np.ones(16), codes), 14).astype(np.float32)
    assert np.array_equal(y, codes.astype(np.float32) - 32.0)
    sc = np.arange(1, 17) * np.where(np.arange(16) % 2, -1, 1)
    y = oracle.dequant(q6k_block(0.5, sc, codes), 14).astype(np.float64)
    assert np.array_equal(y, 0.5 * np.repeat(sc, 16) * (codes - 32.0))


def test_dequant_q6_k_arithmetic(oracle):
    # d * sc * (q - 32) needs at most 11 + 7 + 5 bits, so the reference's f32
    # products are exact and the value is the correctly rounded f16 of the
    # exact product -- checked in float64 over every code, both scale signs,
    # and f16 scales from subnormal to the largest finite
    rng = np.random.default_rng(3)
    ds = h(np.concatenate([rng.uniform(2e-5, 1e-4, 40), rng.uniform(-2, 2, 20),
                           [5.96e-8, 6.1e-5, 65504.0, -65504.0, 0.0]])).astype(np.float64)
    blocks, ref = [], []
    for d in ds:
        sc = rng.integers(-128, 128, 16)
        codes = np.concatenate([np.arange(64)] * 4)
        rng.shuffle(codes)
        blocks.append(q6k_block(d, sc, codes))
        with np.errstate(over="ignore"):
            ref.append((d * np.repeat(sc, 16) * (codes - 32.0)).astype(np.float16))
    got = oracle.dequant(np.concatenate(blocks), 14)
    assert np.array_equal(got.view(np.uint16), np.concatenate(ref).view(np.uint16))


def test_dequant_q6_k_synthetic_rows(oracle):
    # the seeded generator's blocks decode within the scale bounds it drew
    from tensorlogic_amd import synth as S
    blk = S.q6_k_blocks(9, "pin_q6k", 4, 512)
    y = oracle.dequant(blk, 14).astype(np.float32)
    assert y.size == 4 * 512 and np.isfinite(y).all() and np.abs(y).max() <= 1e-4 * 100 * 32 * 1.001


# ---------------------------------------------------------------------------
# linear = matmul_transposed_b (matmul.rs:241-311, unified.metal:4291-4348)
# ---------------------------------------------------------------------------
def test_matmul_reference_known_answers(oracle):
    # tests/test_gpu_operations.rs:81-94: [[1,2],[3,4]] @ [[5,6],[7,8]] = [[19,22],[43,50]];
    # linear takes W[N,K] = b^T
    a = h([[1, 2], [3, 4]])
    bt = h([[5, 7], [6, 8]])
    assert oracle.linear(a, bt).astype(np.float32).tolist() == [[19, 22], [43, 50]]
    # src/ops/tests.rs:248-300: identity
    x = S.normal_f16(30, "x", (5, 50))
    assert np.array_equal(oracle.linear(x, np.eye(50, dtype=np.float16)), x)


def test_linear_fp32_accumulation_closed_form(oracle):
    # rectangular [50, 122] as src/ops/tests.rs:302-377; fp32 sum in k order,
    # one RNE to f16: within 1 ulp of the float64 product, and a transposed
    # W (W^T instead of W) or a dropped bias fails
    x = S.normal_f16(31, "x", (3, 50))
    w = S.normal_f16(31, "w", (122, 50), 0.0, 0.2)
    b = S.normal_f16(31, "b", (122,))
    y = oracle.linear(x, w, b)
    prod = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float16)
    ref = (prod.astype(np.float64) + b.astype(np.float64)).astype(np.float16)
    assert ulps(y, ref).max() <= 1
    # quantised W: same as the f16 product with the dequantised matrix
    blocks = S.q4_0_blocks(31, "wq", 64, 256)
    xq = S.normal_f16(31, "xq", (4, 256))
    wd = oracle.dequant(blocks, 2).reshape(64, 256)
    assert np.array_equal(oracle.linear_q(xq, blocks, 2, 64), oracle.linear(xq, wd))
    ref = (xq.astype(np.float64) @ wd.astype(np.float64).T).astype(np.float16)
    assert ulps(oracle.linear_q(xq, blocks, 2, 64), ref).max() <= 1


def test_linear_f16_accumulation_is_matmul_cpu(oracle):
    # matmul_cpu (matmul.rs:201-228): `sum += a * b` on half::f16, i.e. the
    # product and every partial sum rounded to f16 -- numpy float16 scalar
    # arithmetic rounds exactly that way
    x = S.normal_f16(32, "x", (2, 40))
    w = S.normal_f16(32, "w", (7, 40))
    got = oracle.linear(x, w, acc=oracle.ACC_F16)
    ref = np.empty((2, 7), np.float16)
    for m in range(2):
        for n in range(7):
            s = np.float16(0)
            for k in range(40):
                s = np.float16(s + np.float16(x[m, k] * w[n, k]))
            ref[m, n] = s
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_linear_reversed_fp32_order(oracle):
    # ACC_F32_REV sums k in descending order: on integer-valued inputs every
    # partial sum is exact, so both orders agree bit for bit; on random
    # inputs both stay within 1 ulp of the float64 product and differ
    # somewhere (an order-insensitive implementation would not), and a
    # reversed attention matches the forward one within the same bound
    x = (S.token_ids(33, "xi", 3 * 64, 7).reshape(3, 64) - 3).astype(np.float16)
    w = (S.token_ids(33, "wi", 5 * 64, 5).reshape(5, 64) - 2).astype(np.float16)
    assert np.array_equal(oracle.linear(x, w, acc=oracle.ACC_F32_REV).view(np.uint16),
                          oracle.linear(x, w).view(np.uint16))
    x = S.normal_f16(33, "x", (16, 2048))
    w = S.normal_f16(33, "w", (64, 2048), 0.0, 0.2)
    fwd, rev = oracle.linear(x, w), oracle.linear(x, w, acc=oracle.ACC_F32_REV)
    ref = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float16)
    assert ulps(fwd, ref).max() <= 1 and ulps(rev, ref).max() <= 1
    assert not np.array_equal(fwd.view(np.uint16), rev.view(np.uint16))
    q = S.normal_f16(33, "q", (4, 8, 64))
    k = S.normal_f16(33, "k", (40, 2, 64))
    v = S.normal_f16(33, "v", (40, 2, 64))
    a = oracle.attention(q, k, v, 36, 0.125, True)
    b = oracle.attention(q, k, v, 36, 0.125, True, acc=oracle.ACC_F32_REV)
    assert ulps(a, b).max() <= 2


def test_linear_f32_fused_sums(oracle):
    """linear() on f32 operands: one fused multiply-add per term in k order
    over the kernel's zero-padded 32-wide tiles, then the bias add.
    (1) Small integers: every product and partial sum is exact, so the result
    is numpy's integer matmul whatever the order or fusion -- a transposed
    operand, a dropped term or a wrong bias index fails.  (2) Values on a
    2^-12 grid in [-4, 4]: products need up to 29 bits, so a separately
    rounded product and a fused one differ, while a float64 running sum of
    f32 partials plus the exact product is exact, and rounding it to f32
    once per step is the fused multiply-add -- the oracle equals that
    emulation bit for bit and differs somewhere from the unfused order."""
    rng = np.random.default_rng(41)
    xi = rng.integers(-7, 8, size=(5, 37)).astype(np.float32)
    wi = rng.integers(-7, 8, size=(9, 37)).astype(np.float32)
    bi = rng.integers(-50, 51, size=9).astype(np.float32)
    want = (xi.astype(np.int64) @ wi.astype(np.int64).T + bi.astype(np.int64)).astype(np.float32)
    assert np.array_equal(oracle.linear_f32(xi, wi, bi), want)
    assert np.array_equal(oracle.linear_f32(xi, wi), (xi.astype(np.int64) @ wi.astype(np.int64).T).astype(np.float32))
    x = (rng.integers(-2 ** 14, 2 ** 14, size=(4, 45)) * 2.0 ** -12).astype(np.float32)
    w = (rng.integers(-2 ** 14, 2 ** 14, size=(6, 45)) * 2.0 ** -12).astype(np.float32)
    got = oracle.linear_f32(x, w)
    fused = np.zeros((4, 6), np.float32)
    unfused = np.zeros((4, 6), np.float32)
    for m in range(4):
        for n in range(6):
            sf = su = np.float32(0.0)
            for k in range(64):   # 45 terms padded to two 32-wide tiles
                a = float(x[m, k]) if k < 45 else 0.0
                b = float(w[n, k]) if k < 45 else 0.0
                sf = np.float32(float(sf) + a * b)
                su = np.float32(su + np.float32(a * b))
            fused[m, n], unfused[m, n] = sf, su
    assert np.array_equal(got.view(np.uint32), fused.view(np.uint32))
    assert not np.array_equal(fused.view(np.uint32), unfused.view(np.uint32))


# ---------------------------------------------------------------------------
# RMSNorm (normalization.rs:199-250, unified.metal:1785-1831)
# ---------------------------------------------------------------------------
def test_rms_norm_known_answer_and_closed_form(oracle):
    # tests/test_gpu_operations.rs:184-205: [1,2,3,4] / sqrt(mean = 7.5)
    y = oracle.rms_norm(h([[1, 2, 3, 4]]), h([1, 1, 1, 1]), 1e-6).astype(np.float64)
    assert np.allclose(y, np.array([1, 2, 3, 4]) / np.sqrt(7.5 + 1e-6), atol=1e-3)
    # tests/test_attention_math.rs:444-510: rows of [34, 2048] come out with RMS ~ 1
    x = S.normal_f16(33, "x", (34, 2048), 0.0, 3.0)
    w = S.normal_f16(33, "w", (2048,), 1.0, 0.02)
    y = oracle.rms_norm(x, np.ones(2048, np.float16), 1e-5).astype(np.float64)
    assert np.allclose(np.sqrt((y ** 2).mean(-1)), 1.0, atol=2e-3)
    # closed form in float64 (eps inside the root, weight applied after)
    xf = x.astype(np.float64)
    ref = (xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-5) * w.astype(np.float64)).astype(np.float16)
    assert ulps(oracle.rms_norm(x, w, 1e-5), ref).max() <= 1
    # eps matters: a row of tiny values
    t = h(np.full((1, 8), 1e-3))
    assert np.allclose(oracle.rms_norm(t, h(np.ones(8)), 1e-2).astype(np.float64),
                       1e-3 / np.sqrt(1e-6 + 1e-2), rtol=2e-3)


def test_layer_norm_closed_form(oracle):
    x = S.normal_f16(34, "x", (5, 2560), 0.5, 2.0)
    w = S.normal_f16(34, "w", (2560,), 1.0, 0.1)
    b = S.normal_f16(34, "b", (2560,), 0.0, 0.1)
    xf = x.astype(np.float64)
    mu = xf.mean(-1, keepdims=True)
    ref = ((xf - mu) / np.sqrt(((xf - mu) ** 2).mean(-1, keepdims=True) + 1e-5) * w.astype(np.float64)
           + b.astype(np.float64)).astype(np.float16)
    assert ulps(oracle.layer_norm(x, w, b, 1e-5), ref).max() <= 1


# ---------------------------------------------------------------------------
# RoPE (rope_f16 unified.metal:2355-2418, interleaved pairs)
# ---------------------------------------------------------------------------
def _rope64(x, offset, theta, layout, rot):
    """float64 rotation; pair (2i, 2i+1) or (i, i + rot/2)."""
    S_, H, D = x.shape
    rot = rot or D
    out = x.astype(np.float64).copy()
    i = np.arange(rot // 2)
    freq = 1.0 / theta ** (2 * i / rot)
    for s in range(S_):
        ang = (offset + s) * freq
        c, sn = np.cos(ang), np.sin(ang)
        i0, i1 = (2 * i, 2 * i + 1) if layout == 0 else (i, i + rot // 2)
        x0, x1 = x[s][:, i0].astype(np.float64), x[s][:, i1].astype(np.float64)
        out[s][:, i0] = x0 * c - x1 * sn
        out[s][:, i1] = x0 * sn + x1 * c
    return out


def test_rope_reference_cpu_check(oracle):
    # tests/test_shader_mathematical_correctness.rs:66-101,158-185: seq 3,
    # heads 2, dim 8, x = sin(0.1 i), tolerance 1e-2
    x = h(np.sin(0.1 * np.arange(48)).reshape(3, 2, 8))
    y = oracle.rope(x, 0).astype(np.float64)
    ref = _rope64(x, 0, 10000.0, 0, 0)
    assert np.abs(y - ref).max() <= 1e-2
    assert ulps(y.astype(np.float16), ref.astype(np.float16)).max() <= 1


def test_rope_properties(oracle):
    # position 0 is the identity (src/ops/rope.rs:505-540)
    x = S.normal_f16(35, "x", (1, 32, 64))
    assert np.array_equal(oracle.rope(x, 0), x)
    # magnitude of each (3, 4) pair stays 5 (test_shader_mathematical_correctness.rs:189-225)
    x = h(np.tile([3.0, 4.0], 64).reshape(2, 1, 64))
    y = oracle.rope(x, 0).astype(np.float64).reshape(-1, 2)
    assert np.allclose(np.hypot(y[:, 0], y[:, 1]), 5.0, atol=1e-1)
    # TinyLlama head layout at position 34 (tests/test_attention_math.rs:382-441),
    # both layouts and a partial rotary (Phi-2: 32 of 80 dims)
    # (the reference evaluates freq and angle in f32, so the angle carries
    # ~2^-24 |angle| of rounding, and f32 products of a near-cancelling pair
    # are exact only to 2^-24 of the pair's size: the bound is 1 f16 ulp of
    # the result plus |x| (2^-20 + 2^-22 |angle|); a wrong sign, pair,
    # layout or position is off by O(|x|))
    for shape, off, layout, rot in (((1, 32, 64), 34, 0, 0), ((4, 4, 64), 1000, 1, 0), ((3, 2, 80), 511, 1, 32)):
        x = S.normal_f16(36, f"x{shape}", shape)
        y = oracle.rope(x, off, 10000.0, layout, rot).astype(np.float64)
        ref = _rope64(x, off, 10000.0, layout, rot)
        max_ang = off + shape[0]
        bound = _ulp16(ref) + (2.0 ** -20 + 2.0 ** -22 * max_ang) * np.abs(x).max(-1, keepdims=True)
        assert np.all(np.abs(y - ref) <= bound), (shape, layout)
        if rot:
            assert np.array_equal(y[..., rot:], x[..., rot:])
    # the interleaved and half-rotation layouts differ (a swapped layout fails)
    x = S.normal_f16(37, "x", (2, 2, 8))
    assert not np.array_equal(oracle.rope(x, 5, 10000.0, 0), oracle.rope(x, 5, 10000.0, 1))


def test_rope_table_closed_form(oracle):
    cs = oracle.rope_table(64, 64, 10000.0).astype(np.float64)
    i = np.arange(32)
    ang = np.arange(64)[:, None] * (1.0 / 10000.0 ** (2 * i / 64))[None, :]
    assert np.allclose(cs[..., 0], np.cos(ang), atol=2e-6)
    assert np.allclose(cs[..., 1], np.sin(ang), atol=2e-6)


# ---------------------------------------------------------------------------
# softmax / activations
# ---------------------------------------------------------------------------
def test_softmax_known_answer_and_invariants(oracle):
    # src/ops/activations.rs:100-102: [1, 2, 3] -> [0.0900, 0.2446, 0.6650]
    y = oracle.softmax(h([[1, 2, 3]])).astype(np.float64)
    assert np.allclose(y, [[0.0900, 0.2446, 0.6650]], atol=1e-3)
    x = S.normal_f16(38, "x", (16, 300), 0.0, 4.0)
    y = oracle.softmax(x).astype(np.float64)
    assert np.allclose(y.sum(-1), 1.0, atol=1e-2)
    xf = x.astype(np.float64)
    e = np.exp(xf - xf.max(-1, keepdims=True))
    ref = (e / e.sum(-1, keepdims=True)).astype(np.float16)
    assert ulps(y.astype(np.float16), ref).max() <= 2    # exp stored f16, then divided
    # masked (-10000) entries get 0; an all-non-finite row becomes uniform
    m = h([[0.5, -10000.0, 1.0, -10000.0]])
    y = oracle.softmax(m).astype(np.float64)
    assert y[0, 1] == 0 and y[0, 3] == 0
    y = oracle.softmax(h([[np.inf, -np.inf, np.nan]])).astype(np.float64)
    assert np.allclose(y, 1 / 3, atol=1e-3)


def test_activations_closed_form(oracle):
    x = S.normal_f16(39, "x", (5632,), 0.0, 4.0)
    u = S.normal_f16(39, "u", (5632,))
    xf = x.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-xf))
    assert ulps(oracle.sigmoid(x), sig.astype(np.float16)).max() <= 1
    # sigma(0) = 0.5 (src/ops/tests.rs:640-659)
    assert float(oracle.sigmoid(h([0.0]))[0]) == 0.5
    # TL silu(x) = x * sigmoid(x) with the sigmoid stored f16 first
    s16 = sig.astype(np.float16).astype(np.float64)
    assert np.array_equal(oracle.silu(x), (xf * s16).astype(np.float16))
    sw = (xf * s16).astype(np.float16).astype(np.float64) * u.astype(np.float64)
    assert np.array_equal(oracle.swiglu(x, u), sw.astype(np.float16))
    # gelu (tanh form): 1 + tanh(.) cancels for x << 0, where the f32 formula
    # is exact only to ~2^-24 absolute; a dropped cubic term is off by 1e-3
    g = 0.5 * xf * (1 + np.tanh(np.sqrt(2 / np.pi) * (xf + 0.044715 * xf ** 3)))
    err = np.abs(oracle.gelu(x).astype(np.float64) - g)
    assert np.all(err <= np.maximum(_ulp16(g), 2e-7 * np.abs(xf)))
    # f16 elementwise: f16(a op b), exactly numpy float16 arithmetic
    assert np.array_equal(oracle.add(x, u), x + u)
    assert np.array_equal(oracle.mul(x, u), x * u)
    assert np.array_equal(oracle.mul_scalar(x, 0.125), x * np.float16(0.125))


# ---------------------------------------------------------------------------
# attention (chat_demo_optimized.tl:52-97 op sequence)
# ---------------------------------------------------------------------------
def test_attention_closed_form_and_gqa(oracle):
    Sq, J, H, Hkv, D, q0 = 5, 12, 8, 2, 16, 7
    q = S.normal_f16(40, "q", (Sq, H, D))
    k = S.normal_f16(40, "k", (J, Hkv, D))
    v = S.normal_f16(40, "v", (J, Hkv, D))
    got = oracle.attention(q, k, v, q0, 0.25, True).astype(np.float64)
    # float64 closed form: query head h uses KV head h // (H/Hkv) (np.repeat
    # expands [J, Hkv, D] -> [J, H, D] exactly as broadcast_to does)
    ke = np.repeat(k.astype(np.float64), H // Hkv, axis=1)
    ve = np.repeat(v.astype(np.float64), H // Hkv, axis=1)
    sc = np.einsum("ihd,jhd->ihj", q.astype(np.float64), ke) * 0.25
    pos = q0 + np.arange(Sq)
    sc = np.where(np.arange(J)[None, None, :] > pos[:, None, None], -10000.0, sc)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("ihj,jhd->ihd", p, ve)
    assert np.abs(got - ref).max() < 2e-2
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 5e-3
    # the other GQA mapping (h % Hkv) is measurably different
    kw = np.tile(k.astype(np.float64), (1, H // Hkv, 1))
    wrong = np.einsum("ihd,jhd->ihj", q.astype(np.float64), kw)
    assert not np.allclose(wrong, np.einsum("ihd,jhd->ihj", q.astype(np.float64), ke))
    # einsum known values (tests/test_einsum_f16_comprehensive.rs:45-135 pattern):
    # one key -> output equals that key's V row regardless of the scores
    got1 = oracle.attention(q[:1], k[:1], v[:1], 0, 0.25, True)
    assert np.array_equal(got1, np.repeat(v[:1], H // Hkv, axis=1))


def test_embedding_and_argmax(oracle):
    table = S.normal_f16(41, "t", (100, 16))
    ids = np.array([3, 99, 0, 3], np.int32)
    assert np.array_equal(oracle.embedding(table, ids), table[ids])
    with pytest.raises(IndexError):
        oracle.embedding(table, [100])
    # temperature_sample(., 0) takes Iterator::max_by: the LAST maximum wins
    lg = np.zeros(50, np.float16)
    lg[[4, 9, 31]] = 2.0
    assert oracle.argmax_last(lg) == 31
    lg = S.normal_f16(41, "lg", (32000,))
    assert oracle.argmax_last(lg) == int(np.argmax(lg.astype(np.float32)))


# ---------------------------------------------------------------------------
# temperature_sample with T > 1e-4 (builtin_sampling.rs:178-215)
# ---------------------------------------------------------------------------
def test_sampler_known_answer_boundaries(oracle):
    # softmax([1, 2, 3]) = [0.0900, 0.2447, 0.6652] (activations.rs:100-102
    # quotes 0.0900, 0.2446, 0.6650): the inverse CDF switches at 0.0900 and
    # 0.3348
    lg = np.array([1, 2, 3], np.float16)
    assert [oracle.sample_temperature(lg, 1.0, r) for r in (0.0, 0.0899, 0.0901, 0.3345, 0.3349, 0.99)] == \
        [0, 0, 1, 1, 2, 2]
    # T scales the logits before the softmax: T = 2 -> softmax([0.5, 1, 1.5])
    assert oracle.sample_temperature(lg, 2.0, 0.18) == 0 and oracle.sample_temperature(lg, 2.0, 0.19) == 1


def test_sampler_distribution(oracle):
    # the inverse CDF over a grid of draws reproduces softmax(x / T) computed
    # in float64 (a dropped scale, a wrong max shift or an off-by-one index
    # shows as a frequency error far above the grid's 1/4096)
    rng = np.random.default_rng(7)
    lg = h(rng.normal(0, 2, 50))
    for T in (0.5, 0.8, 1.7):
        x = lg.astype(np.float64) / np.float64(np.float32(T))
        p = np.exp(x - x.max())
        p /= p.sum()
        grid = (np.arange(4096) + 0.5) / 4096
        toks = np.array([oracle.sample_temperature(lg, T, float(r)) for r in grid])
        freq = np.bincount(toks, minlength=50) / 4096
        assert np.abs(freq - p).max() < 2.0 / 4096 + 1e-6


def test_sampler_uniform_is_splitmix64(oracle):
    # splitmix64 seeded with 0 first returns 0xE220A8397B1DCDAF (Steele, Lea,
    # Flood 2014); the draw is its top 24 bits
    assert oracle.sample_uniform(0, 0) == 0xE220A8 / 2 ** 24
    r = np.array([oracle.sample_uniform(11, c) for c in range(20000)])
    assert r.min() >= 0.0 and r.max() < 1.0 and abs(r.mean() - 0.5) < 0.01
