"""Pins the oracle's restatements of the TensorF32 arms of rms_norm,
softmax, rope, sigmoid and the attention einsums (unified.metal:1129-1135,
1961-2036, 2202-2340, 2420-2482, 2702-2768) before the device parity tests
trust them.  CPU only.

Each is checked against the reference's own known answers where its tests
hold them (activations.rs:669-700 and :844-870, rope.rs:599-640, the
[1, 2, 3, 4] RMSNorm of tests/test_gpu_operations.rs:184-205) and against an
independent computation chosen so that a plausible mistake fails: float64
closed forms; the f16 oracle (already pinned) for the rotation's angles;
integer operands, whose sums are exact in any order, for the einsums; and
step-by-step emulations of the summation order (fused multiply-adds, the
256-partial tree) on grids where a different order or an unfused product
gives different bits -- each emulation is also shown to differ from the
alternative it rules out.
"""
import ctypes.util

import numpy as np
import pytest


def f32(x):
    return np.asarray(x, np.float32)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def ulps(got, ref):
    """|got - ref| in units of the f32 spacing at |ref|."""
    ref = f32(ref)
    return np.abs(got.astype(np.float64) - ref.astype(np.float64)) / np.spacing(np.abs(ref)).astype(np.float64)


def fused_sum(vals_a, vals_b, s=0.0):
    """Running f32 sum with one fused multiply-add per term: the float64 sum
    of the f32 partial and the exact product (exact on the grids used here),
    rounded to f32 once per step."""
    s = np.float32(s)
    for a, b in zip(vals_a, vals_b):
        s = np.float32(float(s) + float(a) * float(b))
    return s


def unfused_sum(vals_a, vals_b):
    s = np.float32(0.0)
    for a, b in zip(vals_a, vals_b):
        s = np.float32(s + np.float32(float(a) * float(b)))
    return s


def grid(rng, shape, frac_bits=12, lim=2.0):
    """Values on a 2^-frac_bits grid in (-lim, lim): products are exact in
    float64 and need more than 24 bits, so fused and unfused sums differ."""
    n = int(lim * 2 ** frac_bits)
    return (rng.integers(-n + 1, n, size=shape) * 2.0 ** -frac_bits).astype(np.float32)


# ---------------------------------------------------------------------------
# rms_norm (rms_norm_simple_f32 / rms_norm_f32)
# ---------------------------------------------------------------------------
def test_rms_norm_f32_known_answer(oracle):
    # tests/test_gpu_operations.rs:184-205: [1, 2, 3, 4] / sqrt(7.5 + eps)
    y = oracle.rms_norm_f32(f32([[1, 2, 3, 4]]), f32([1, 1, 1, 1]), 1e-6)
    want = np.array([1, 2, 3, 4], np.float64) / np.sqrt(7.5 + 1e-6)
    assert np.all(ulps(y[0], want) <= 2)
    # the weight multiplies after the normalisation, element by element
    y2 = oracle.rms_norm_f32(f32([[1, 2, 3, 4]]), f32([2, 0, -1, 0.5]), 1e-6)
    assert np.all(ulps(y2[0], want * np.array([2, 0, -1, 0.5])) <= 2)


def _rms_ref(xr, w, eps, order):
    n = xr.size
    if order == "reference":
        if n <= 256:
            sq = fused_sum(xr, xr)
        else:
            part = [fused_sum(xr[t::256], xr[t::256]) for t in range(256)]
            st = 128
            while st:
                for t in range(st):
                    part[t] = np.float32(part[t] + part[t + st])
                st >>= 1
            sq = part[0]
    elif order == "sequential":
        sq = fused_sum(xr, xr)
    else:   # unfused products, reference order
        if n <= 256:
            sq = unfused_sum(xr, xr)
        else:
            part = [unfused_sum(xr[t::256], xr[t::256]) for t in range(256)]
            st = 128
            while st:
                for t in range(st):
                    part[t] = np.float32(part[t] + part[t + st])
                st >>= 1
            sq = part[0]
    mean_sq = np.float32(sq / np.float32(n))
    rms = np.float32(np.sqrt(np.float32(mean_sq + np.float32(eps)), dtype=np.float32))
    inv = np.float32(np.float32(1.0) / rms)
    return ((xr * inv).astype(np.float32) * w).astype(np.float32)


@pytest.mark.parametrize("n", [200, 4096])
def test_rms_norm_f32_summation_order(oracle, n):
    """Rows of n <= 256: one fused running sum in element order; longer rows:
    256 strided fused partial sums, then the halving tree.  The oracle equals
    that emulation bit for bit; for the long row the emulation differs from
    a sequential sum, and for both from unfused products (unit weights and
    16 rows, so that a sum differing in its last bits shows in the output
    bits of some row after the square root and the reciprocal)."""
    rng = np.random.default_rng(7 + n)
    R = 16
    x = grid(rng, (R, n))
    w = np.ones(n, np.float32)
    got = oracle.rms_norm_f32(x, w, 1e-5)
    wv = grid(rng, (n,), 8, 2.0)   # and with a weight, the emulation still holds
    gotw = oracle.rms_norm_f32(x[:2], wv, 1e-5)
    for r in range(2):
        assert np.array_equal(bits(gotw[r]), bits(_rms_ref(x[r], wv, 1e-5, "reference")))
    for r in range(R):
        want = _rms_ref(x[r], w, 1e-5, "reference")
        assert np.array_equal(bits(got[r]), bits(want))
    assert any(not np.array_equal(bits(_rms_ref(x[r], w, 1e-5, "reference")),
                                  bits(_rms_ref(x[r], w, 1e-5, "unfused"))) for r in range(R))
    if n > 256:
        assert any(not np.array_equal(bits(_rms_ref(x[r], w, 1e-5, "reference")),
                                      bits(_rms_ref(x[r], w, 1e-5, "sequential"))) for r in range(R))


def test_rms_norm_f32_closed_form(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 2048)).astype(np.float32) * 3
    w = rng.standard_normal(2048).astype(np.float32)
    y = oracle.rms_norm_f32(x, w, 1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(y - want) / (np.abs(want) + 1e-30)) < 2e-6


# ---------------------------------------------------------------------------
# softmax (softmax_simple_f32 / softmax_f32)
# ---------------------------------------------------------------------------
def test_softmax_f32_known_answer(oracle):
    # activations.rs:669-700: [1, 2, 3, 4] sums to 1 and keeps the order
    y = oracle.softmax_f32(f32([1, 2, 3, 4]))
    assert abs(float(y.sum()) - 1.0) < 1e-6
    assert np.all(np.diff(y) > 0)
    e = np.exp(np.array([1, 2, 3, 4], np.float64) - 4)
    assert np.all(ulps(y, e / e.sum()) <= 4)


def test_softmax_f32_masked_and_degenerate_rows(oracle):
    x = f32([[0.5, -np.inf, 1.5, np.nan],            # non-finite entries take no weight
             [-np.inf, -np.inf, -np.inf, -np.inf],    # nothing finite: max 0, every e 0 -> uniform
             [np.nan, np.nan, np.nan, np.nan]])
    y = oracle.softmax_f32(x)
    e = np.exp(np.array([0.5, 1.5]) - 1.5)
    assert y[0, 1] == 0 and y[0, 3] == 0
    assert np.all(ulps(y[0, [0, 2]], e / e.sum()) <= 4)
    assert np.array_equal(y[1], f32([0.25] * 4)) and np.array_equal(y[2], f32([0.25] * 4))


def test_softmax_f32_element_order_sum(oracle):
    """The reference sums e in element order on one thread.  With e from the
    same libm expf the oracle calls, e / (running sum in element order) is
    the oracle's output bit for bit; the reversed-order sum gives other
    bits at this length."""
    import ctypes
    expf = ctypes.CDLL(ctypes.util.find_library("m")).expf
    expf.restype, expf.argtypes = ctypes.c_float, [ctypes.c_float]
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(3000) * 4).astype(np.float32)
    y = oracle.softmax_f32(x[None])[0]
    mx = x.max()
    e = np.array([expf(float(np.float32(v - mx))) for v in x], np.float32)
    s = np.float32(0)
    for v in e:
        s = np.float32(s + v)
    r = np.float32(0)
    for v in e[::-1]:
        r = np.float32(r + v)
    assert s != r
    assert np.array_equal(bits(y), bits(e / s))
    assert not np.array_equal(bits(y), bits(e / r))


# ---------------------------------------------------------------------------
# rope (rope_f32)
# ---------------------------------------------------------------------------
def test_rope_f32_magnitude(oracle):
    # rope.rs:599-640: pairs (3, 4) keep length 5 at position 0 of a 64-dim head
    x = np.tile(f32([3, 4]), 32).reshape(1, 1, 64)
    y = oracle.rope_f32(x, 0)
    assert np.array_equal(y, x)   # position 0: cos 1, sin 0, exactly
    y = oracle.rope_f32(x, 17)
    mag = np.sqrt(y[0, 0, 0::2].astype(np.float64) ** 2 + y[0, 0, 1::2].astype(np.float64) ** 2)
    assert np.max(np.abs(mag - 5.0)) < 5.0 * 4e-7


@pytest.mark.parametrize("layout,rot", [(0, 0), (1, 0), (0, 32), (1, 32)])
def test_rope_f32_matches_the_f16_oracle_and_float64(oracle, layout, rot):
    """Same angles and rotation as the f16 rope: on f16-representable inputs
    the f32 result rounded to f16 is the f16 oracle's output bit for bit; and
    each pair is the float64 rotation within a few f32 ulps."""
    rng = np.random.default_rng(5 + layout + rot)
    S, H, D, off = 7, 3, 64, 300
    x16 = (rng.standard_normal((S, H, D)) * 2).astype(np.float16)
    y = oracle.rope_f32(x16.astype(np.float32), off, 10000.0, layout, rot)
    y16 = oracle.rope(x16, off, 10000.0, layout, rot)
    assert np.array_equal(y.astype(np.float16).view(np.uint16), y16.view(np.uint16))
    r = D if rot == 0 else rot
    half = r // 2
    i = np.arange(half)
    freq = 1.0 / np.power(10000.0, (2.0 * i) / r)
    x = x16.astype(np.float64)
    for s in range(S):
        ang = (off + s) * freq
        c, sn = np.cos(ang), np.sin(ang)
        i0, i1 = (2 * i, 2 * i + 1) if layout == 0 else (i, i + half)
        r0 = x[s][:, i0] * c - x[s][:, i1] * sn
        r1 = x[s][:, i0] * sn + x[s][:, i1] * c
        # (f32 angles near position 300 carry ~3e-5 rad of rounding)
        assert np.max(np.abs(y[s][:, i0] - r0)) < 1e-3
        assert np.max(np.abs(y[s][:, i1] - r1)) < 1e-3
        assert np.array_equal(y[s][:, r:], x16[s][:, r:].astype(np.float32))   # pass-through dims


# ---------------------------------------------------------------------------
# sigmoid (sigmoid_f32)
# ---------------------------------------------------------------------------
def test_sigmoid_f32_known_answers(oracle):
    # activations.rs:844-870: SiLU(0) = 0 through x * sigmoid(x); sigmoid(0) = 1/2
    x = f32([-2, -1, 0, 1, 2])
    s = oracle.sigmoid_f32(x)
    assert s[2] == np.float32(0.5)
    assert (x * s)[2] == 0
    want = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.all(ulps(s, want) <= 2)
    # symmetry sigma(-x) = 1 - sigma(x) within rounding
    assert np.max(np.abs(s[::-1] - (1 - s))) < 1e-7


def test_sigmoid_f32_range(oracle):
    x = f32([-200, -90, -20, 0, 20, 90, 200, np.inf, -np.inf])
    s = oracle.sigmoid_f32(x)
    assert s[0] == 0 and s[-1] == 0 and s[-2] == 1 and s[6] == 1
    assert np.all((s >= 0) & (s <= 1))


# ---------------------------------------------------------------------------
# einsum (einsum_ihd_jhd_ihj_f32 / einsum_ihj_jhd_ihd_f32)
# ---------------------------------------------------------------------------
def test_einsum_f32_integer_operands(oracle):
    """Small integers: every sum is exact in f32, so the results are numpy's
    integer einsums whatever the order -- a transposed operand, a wrong head
    mapping (GQA: head h reads KV head h // 2) or a dropped term fails."""
    rng = np.random.default_rng(2)
    q = rng.integers(-5, 6, (4, 6, 16))
    k = rng.integers(-5, 6, (9, 3, 16))
    p = rng.integers(-5, 6, (4, 6, 9))
    kk = np.repeat(k, 2, axis=1)
    assert np.array_equal(oracle.einsum_scores_f32(q, k), np.einsum("ihd,jhd->ihj", q, kk).astype(np.float32))
    assert np.array_equal(oracle.einsum_context_f32(p, k), np.einsum("ihj,jhd->ihd", p, kk).astype(np.float32))


def test_einsum_f32_fused_index_order(oracle):
    """On a 2^-12 grid the products need more than 24 bits: the oracle is the
    fused running sum in index order (over d for scores, over j for the
    context) bit for bit, which differs somewhere from unfused products."""
    rng = np.random.default_rng(9)
    q, k = grid(rng, (2, 2, 40)), grid(rng, (5, 2, 40))
    sc = oracle.einsum_scores_f32(q, k)
    p, v = grid(rng, (2, 2, 37)), grid(rng, (37, 2, 8))
    ctx = oracle.einsum_context_f32(p, v)
    fs, us = np.zeros_like(sc), np.zeros_like(sc)
    for i in range(2):
        for h in range(2):
            for j in range(5):
                fs[i, h, j] = fused_sum(q[i, h], k[j, h])
                us[i, h, j] = unfused_sum(q[i, h], k[j, h])
    assert np.array_equal(bits(sc), bits(fs)) and not np.array_equal(bits(fs), bits(us))
    fc, uc = np.zeros_like(ctx), np.zeros_like(ctx)
    for i in range(2):
        for h in range(2):
            for d in range(8):
                fc[i, h, d] = fused_sum(p[i, h], v[:, h, d])
                uc[i, h, d] = unfused_sum(p[i, h], v[:, h, d])
    assert np.array_equal(bits(ctx), bits(fc)) and not np.array_equal(bits(fc), bits(uc))


# ---------------------------------------------------------------------------
# layer_norm (layer_norm_f32 / layer_norm_simple_f32)
# ---------------------------------------------------------------------------
def test_layer_norm_f32_known_answers(oracle):
    # normalization.rs:541-600 (basic: [[1, 2, 3], [4, 5, 6]] over the last
    # dim: mean 0, variance 1) and :674-705 (3-D [2, 3, 4] of i / 10)
    y = oracle.layer_norm_f32(f32([[1, 2, 3], [4, 5, 6]]), None, None, 1e-5)
    want = np.array([-1, 0, 1], np.float64) / np.sqrt(2.0 / 3.0 + 1e-5)
    for r in range(2):
        assert np.all(ulps(y[r], want) <= 2) and y[r, 1] == 0
    x3 = (np.arange(24, dtype=np.float64) / 10).astype(np.float32).reshape(2, 3, 4)
    y3 = oracle.layer_norm_f32(x3, None, None, 1e-5)
    assert y3.shape == (2, 3, 4)
    assert np.all(np.abs(y3.astype(np.float64).mean(-1)) < 4e-6)   # (the reference test: 1e-2)
    # :605-670 (affine): [[1, 2], [3, 4]] with w = [2, 3], b = [0.5, 1]
    ya = oracle.layer_norm_f32(f32([[1, 2], [3, 4]]), f32([2, 3]), f32([0.5, 1]), 1e-5)
    t = 1.0 / np.sqrt(0.25 + 1e-5) * 0.5
    assert np.all(ulps(ya, [[-2 * t + 0.5, 3 * t + 1]] * 2) <= 2)


def test_layer_norm_f32_closed_form(oracle):
    """float64 closed form (biased variance, weight then bias): a dropped
    term, the unbiased variance (a 1/n change) or a swapped weight / bias
    fails the 2e-6 relative bound at these sizes."""
    rng = np.random.default_rng(4)
    for n in (64, 2560):
        x = (rng.standard_normal((3, n)) * 2 + 0.5).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        x64 = x.astype(np.float64)
        mu = x64.mean(-1, keepdims=True)
        nz = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(-1, keepdims=True) + 1e-5)
        for ww, bb in ((w, b), (w, None), (None, b), (None, None)):
            want = nz * (ww if ww is not None else 1.0) + (bb if bb is not None else 0.0)
            got = oracle.layer_norm_f32(x, ww, bb, 1e-5)
            assert np.max(np.abs(got - want)) < 2e-6 * max(1.0, np.max(np.abs(want)))
        unbiased = nz * np.sqrt((n - 1) / n)
        assert np.max(np.abs(oracle.layer_norm_f32(x, None, None, 1e-5) - unbiased)) > 1e-5


def _ln_ref(xr, w, b, eps, order="reference"):
    """Step-by-step layer_norm of one f32 row: element-order sum; squared
    deviations in element order, fused (one rounding per term) or not, or as
    256 strided partial sums and a halving tree; y = fma(t, w, b)."""
    n = xr.size
    s = np.float32(0.0)
    for v in xr:
        s = np.float32(s + v)
    mean = np.float32(s / np.float32(n))
    d = (xr - mean).astype(np.float32)
    if order == "reference":
        q = fused_sum(d, d)
    elif order == "unfused":
        q = unfused_sum(d, d)
    else:
        part = [fused_sum(d[t::256], d[t::256]) for t in range(256)]
        st = 128
        while st:
            for t in range(st):
                part[t] = np.float32(part[t] + part[t + st])
            st >>= 1
        q = part[0]
    var = np.float32(q / np.float32(n))
    inv = np.float32(np.float32(1.0) / np.float32(np.sqrt(np.float32(var + np.float32(eps)), dtype=np.float32)))
    t = (d * inv).astype(np.float32)
    return np.array([np.float32(float(a) * float(c) + float(e)) for a, c, e in zip(t, w, b)], np.float32)


@pytest.mark.parametrize("n", [200, 1024])
def test_layer_norm_f32_summation_order(oracle, n):
    """Both sums in element order, the squares fused, the weight and bias one
    fused multiply-add: the oracle equals that emulation bit for bit (grid
    values, so each float64 step of the emulation is exact or rounds once),
    and the emulation differs from unfused squares and from a 256-partial
    tree on some of the 16 rows -- so the test tells those orders apart."""
    rng = np.random.default_rng(17 + n)
    R = 16
    x = grid(rng, (R, n)) + np.float32(0.25)
    w = np.ones(n, np.float32)
    b = np.zeros(n, np.float32)
    got = oracle.layer_norm_f32(x, w, b, 1e-5)
    refs = [_ln_ref(x[r], w, b, 1e-5) for r in range(R)]
    for r in range(R):
        assert np.array_equal(bits(got[r]), bits(refs[r]))
    assert any(not np.array_equal(bits(refs[r]), bits(_ln_ref(x[r], w, b, 1e-5, "unfused"))) for r in range(R))
    assert any(not np.array_equal(bits(refs[r]), bits(_ln_ref(x[r], w, b, 1e-5, "tree"))) for r in range(R))
    # with a weight and a bias on the grid: one fused multiply-add per element
    wv, bv = grid(rng, (n,), 8), grid(rng, (n,), 8)
    gotw = oracle.layer_norm_f32(x[:2], wv, bv, 1e-5)
    for r in range(2):
        assert np.array_equal(bits(gotw[r]), bits(_ln_ref(x[r], wv, bv, 1e-5)))


# ---------------------------------------------------------------------------
# gelu (gelu_f32), silu / swiglu, add / mul / mul_scalar, apply_attention_mask
# ---------------------------------------------------------------------------
def test_gelu_f32_known_answers_and_closed_form(oracle):
    # activations.rs:900-940: GELU(0) = 0, GELU(-2) ~ -0.0454, GELU(-1) ~
    # -0.1587, GELU(1) ~ 0.8413, GELU(2) ~ 1.9545
    y = oracle.gelu_f32(f32([-2, -1, 0, 1, 2]))
    assert y[2] == 0
    assert np.all(np.abs(y - f32([-0.0454, -0.1587, 0, 0.8413, 1.9545])) < 2e-4)
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(4000) * 4).astype(np.float32)
    g = oracle.gelu_f32(x)
    v = x.astype(np.float64)
    want = 0.5 * v * (1 + np.tanh(0.7978845608 * (v + 0.044715 * v ** 3)))
    # (for x << 0, 1 + tanh cancels: the f32 steps then carry ~|x| * 2^-24 absolute error)
    assert np.all(np.abs(g - want) <= 4e-6 * np.abs(want) + 3e-7 * np.abs(v))
    # the tanh form's odd part: gelu(x) - gelu(-x) = x
    assert np.max(np.abs((g - oracle.gelu_f32(-x)) - x) / np.maximum(np.abs(x), 1.0)) < 2e-6


def test_silu_swiglu_f32(oracle):
    # activations.rs:844-870: silu(x) = x * sigmoid(x), silu(0) = 0
    x = f32([-2, -1, 0, 1, 2])
    s = oracle.silu_f32(x)
    assert s[2] == 0
    want = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.all(ulps(s, want) <= 3)
    # composed of the oracle's own f32 steps: sigmoid, then one product each
    rng = np.random.default_rng(10)
    g = (rng.standard_normal(1000) * 3).astype(np.float32)
    u = rng.standard_normal(1000).astype(np.float32)
    sg = oracle.sigmoid_f32(g)
    assert np.array_equal(bits(oracle.silu_f32(g)), bits(g * sg))
    assert np.array_equal(bits(oracle.swiglu_f32(g, u)), bits((g * sg).astype(np.float32) * u))


def test_add_mul_mask_f32(oracle):
    # one IEEE operation each: integers and halves add and multiply exactly
    a, b = f32([1.5, -2, 3, 0.25]), f32([0.5, 4, -3, 8])
    assert np.array_equal(oracle.add_f32(a, b), f32([2, 2, 0, 8.25]))
    assert np.array_equal(oracle.mul_f32(a, b), f32([0.75, -8, -9, 2]))
    # the f32 scalar is not rounded to f16: 0.1 stays 0.1f
    assert oracle.mul_scalar_f32(f32([1.0]), 0.1)[0] == np.float32(0.1)
    assert np.float32(np.float16(0.1)) != np.float32(0.1)
    # masking.rs:325-355: scores [1, 2, 3, 4], mask [1, 0, 1, 1]
    m = oracle.apply_attention_mask_f32(f32([[1, 2], [3, 4]]), f32([[1, 0], [1, 1]]))
    assert np.array_equal(m, f32([[1, -10000], [3, 4]]))
    # a [I, J] mask over [I, H, J] scores masks every head alike
    sc = np.arange(12, dtype=np.float32).reshape(2, 3, 2)
    mm = oracle.apply_attention_mask_f32(sc, f32([[1, 0], [0, 1]]))
    assert np.all(mm[0, :, 1] == -10000) and np.all(mm[1, :, 0] == -10000)
    assert np.array_equal(mm[0, :, 0], sc[0, :, 0]) and np.array_equal(mm[1, :, 1], sc[1, :, 1])
