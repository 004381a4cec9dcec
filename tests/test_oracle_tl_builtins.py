"""Pins the oracle's restatements of the TL builtins around the attention
path -- causal_mask, slice_last, broadcast_to, rope(x, cos, sin) and the
precompute_rope_* tables -- before the device parity tests trust them.
CPU only.

Each is checked against the known answers of the reference's own tests
where they exist (tests/test_attention_mask.rs, tests/test_slice_last.rs,
tests/test_broadcasting.rs) and against an independent computation:
numpy's tril / indexing / broadcast_to, and closed forms for the rotation
(quarter turns, identity at position 0, preserved pair length) chosen so
that a wrong sign, a wrong table column or a transposed operand fails.
"""
import numpy as np
import pytest

from tensorlogic_amd import synth as S


def h(x):
    return np.asarray(x, np.float16)


# ---------------------------------------------------------------------------
# causal_mask
# ---------------------------------------------------------------------------
def test_causal_mask_known_answer(oracle):
    # tests/test_attention_mask.rs:37-62
    m = oracle.causal_mask(3)
    assert m.shape == (3, 3) and m.dtype == np.float16
    assert np.array_equal(m, h([[1, 0, 0], [1, 1, 0], [1, 1, 1]]))
    # tests/test_attention_mask.rs:101-114: one token attends to itself
    assert np.array_equal(oracle.causal_mask(1), h([[1]]))


@pytest.mark.parametrize("n", [2, 5, 46, 129])
def test_causal_mask_is_lower_triangle(oracle, n):
    m = oracle.causal_mask(n)
    assert np.array_equal(m, np.tril(np.ones((n, n), np.float16)))
    # tests/test_attention_mask.rs:116-140: n(n+1)/2 ones
    assert int((m == 1).sum()) == n * (n + 1) // 2 and int((m == 0).sum()) == n * (n - 1) // 2


# ---------------------------------------------------------------------------
# slice_last
# ---------------------------------------------------------------------------
def test_slice_last_known_answers(oracle):
    # tests/test_slice_last.rs:100-131: [2, 3, 4] of 1..24 -> 13..24 as [3, 4]
    x = np.arange(1, 25, dtype=np.float32).reshape(2, 3, 4)
    y = oracle.slice_last(x, 0)
    assert y.shape == (3, 4) and np.array_equal(y, np.arange(13, 25, dtype=np.float32).reshape(3, 4))
    # the same in f16 (tests/test_slice_last.rs:135-158)
    assert np.array_equal(oracle.slice_last(h(x), 0), h(x[-1]))
    # 1-D: the last element (slice.rs:42-50)
    assert np.array_equal(oracle.slice_last(h([4, 5, 6]), 0), h([6]))


@pytest.mark.parametrize("shape", [(5, 7), (46, 2048), (3, 2, 4, 5), (1, 32, 64)])
def test_slice_last_matches_indexing(oracle, shape):
    x = S.normal_f16(61, f"sl{shape}", shape)
    assert np.array_equal(oracle.slice_last(x, 0), x[-1])
    xi = np.arange(np.prod(shape), dtype=np.int32).reshape(shape)
    assert np.array_equal(oracle.slice_last(xi, 0), xi[-1])


def test_slice_last_rejects_what_the_reference_rejects(oracle):
    x = h(np.zeros((2, 3)))
    with pytest.raises(ValueError):
        oracle.slice_last(x, 1)   # slice.rs:36-40: only axis 0
    with pytest.raises(ValueError):
        oracle.slice_last(x, 2)   # slice.rs:29-33: axis out of bounds


# ---------------------------------------------------------------------------
# broadcast_to
# ---------------------------------------------------------------------------
def test_broadcast_known_answers(oracle):
    # tests/test_broadcasting.rs:14-27: [1] -> [5], all 42
    assert np.array_equal(oracle.broadcast_to(h([42.0]), (5,)), h([42.0] * 5))
    # tests/test_broadcasting.rs:29-54: [3] -> [4, 3], every row 1 2 3
    assert np.array_equal(oracle.broadcast_to(h([1, 2, 3]), (4, 3)), h([[1, 2, 3]] * 4))
    # column vector [3, 1] -> [3, 4] (tests/test_broadcasting.rs:78-109)
    assert np.array_equal(oracle.broadcast_to(h([[1], [2], [3]]), (3, 4)), h([[1] * 4, [2] * 4, [3] * 4]))


@pytest.mark.parametrize("src,dst", [((3,), (4, 3)), ((4, 1), (4, 6)), ((1, 5), (3, 5)), ((2, 1, 4), (3, 2, 5, 4)),
                                     ((7, 4, 1, 64), (7, 4, 8, 64)), ((1,), (2, 3, 4)), ((6, 5), (6, 5)),
                                     ((1, 1, 1), (2, 3, 4))])
def test_broadcast_matches_numpy(oracle, src, dst):
    x = S.normal_f16(62, f"bc{src}", src)
    assert np.array_equal(oracle.broadcast_to(x, dst), np.broadcast_to(x, dst))
    xi = np.arange(np.prod(src), dtype=np.int32).reshape(src)
    assert np.array_equal(oracle.broadcast_to(xi, dst), np.broadcast_to(xi, dst))


@pytest.mark.parametrize("src,dst", [((3,), (4, 2)), ((2, 3), (3,)), ((2, 3), (4, 3, 3)), ((5, 1), (4, 5, 2, 3))])
def test_broadcast_rejects_incompatible_shapes(oracle, src, dst):
    # shape.rs:37-49 -> TensorError::ShapeMismatch
    with pytest.raises(ValueError):
        oracle.broadcast_to(h(np.zeros(src)), dst)


# ---------------------------------------------------------------------------
# precompute_rope_* and rope(x, cos, sin)
# ---------------------------------------------------------------------------
def test_precompute_rope_closed_form(oracle):
    D, L, base = 64, 40, 10000.0
    c, s = oracle.precompute_rope(D, L, base, False), oracle.precompute_rope(D, L, base, True)
    assert c.shape == (L, D) and s.shape == (L, D)
    # each value stored twice: columns 2i and 2i+1 (builtin_tensor.rs:676-681)
    assert np.array_equal(c[:, 0::2], c[:, 1::2]) and np.array_equal(s[:, 0::2], s[:, 1::2])
    # position 0: cos 1, sin 0
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    # pair 0 has theta 1: cos(pos), sin(pos) exactly rounded to f16
    pos = np.arange(L, dtype=np.float64)
    assert np.array_equal(c[:, 0], h(np.cos(pos))) and np.array_equal(s[:, 0], h(np.sin(pos)))
    # every entry within one f16 ulp of the float64 angle (the f32 angle
    # carries ~2^-24 relative rounding)
    th = 1.0 / base ** (np.arange(0, D, 2) / D)
    ang = pos[:, None] * th[None, :]
    for got, ref in ((c[:, 0::2], np.cos(ang)), (s[:, 0::2], np.sin(ang))):
        err = np.abs(got.astype(np.float64) - ref)
        assert np.all(err <= 2.0 ** -11 * np.maximum(np.abs(ref), 2.0 ** -14) + 1e-6 * (1 + pos[:, None]))


def test_rope_cos_sin_quarter_turn_pins_sign_and_column(oracle):
    """x = (1, 0) in every pair; the tables turn only column 1 by a quarter
    (cos 0, sin 1), every other column is the identity.  rope_candle_f16
    reads pair i's cos/sin at column i (unified.metal:5161-5166), so exactly
    pair 1 (elements 2, 3) becomes (0, 1): a sign error gives (0, -1), a
    kernel reading column 2i would leave pair 1 alone and turn nothing."""
    S_, H, D = 2, 3, 8
    x = np.zeros((S_, H, D), np.float16)
    x[..., 0::2] = 1
    c = np.ones((S_, D), np.float16)
    s = np.zeros((S_, D), np.float16)
    c[:, 1], s[:, 1] = 0, 1
    y = oracle.rope_cos_sin(x, c, s)
    ref = x.copy()
    ref[..., 2], ref[..., 3] = 0, 1
    assert np.array_equal(y, ref)


def test_rope_cos_sin_properties(oracle):
    D, S_, H = 64, 12, 4
    c, s = oracle.precompute_rope(D, 16, 10000.0, False), oracle.precompute_rope(D, 16, 10000.0, True)
    x = S.normal_f16(63, "rcs", (S_, H, D))
    y = oracle.rope_cos_sin(x, c, s)
    # position 0 (row 0 of the tables) is the identity
    assert np.array_equal(y[0], x[0])
    # each pair keeps its length (the f16 tables carry ~2^-11 relative
    # rounding in cos and sin, the f16 stores another 2^-11 per element)
    xf, yf = x.astype(np.float64), y.astype(np.float64)
    n0 = np.hypot(xf[..., 0::2], xf[..., 1::2])
    n1 = np.hypot(yf[..., 0::2], yf[..., 1::2])
    assert np.all(np.abs(n1 - n0) <= 4 * 2.0 ** -11 * n0 + 2.0 ** -14)
    # with the duplicated tables, pair i turns by the angle of pair i // 2
    # (the table column-i read), in float64 within f16 rounding
    th = 1.0 / 10000.0 ** (np.arange(0, D, 2) / D)
    ang = np.arange(S_)[:, None] * th[np.arange(D // 2) // 2][None, :]
    cc, ss = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    r0 = xf[..., 0::2] * cc - xf[..., 1::2] * ss
    r1 = xf[..., 0::2] * ss + xf[..., 1::2] * cc
    tol = 4 * 2.0 ** -11 * (np.abs(xf[..., 0::2]) + np.abs(xf[..., 1::2])) + 2.0 ** -14
    assert np.all(np.abs(yf[..., 0::2] - r0) <= tol) and np.all(np.abs(yf[..., 1::2] - r1) <= tol)


def test_rope_cos_sin_rejects_bad_shapes(oracle):
    x = h(np.zeros((4, 2, 8)))
    with pytest.raises(ValueError):
        oracle.rope_cos_sin(x, h(np.ones((3, 8))), h(np.zeros((3, 8))))   # fewer table rows than positions
    with pytest.raises(ValueError):
        oracle.rope_cos_sin(x, h(np.ones((4, 6))), h(np.zeros((4, 6))))   # table width != head_dim
    with pytest.raises(ValueError):
        oracle.rope_cos_sin(h(np.zeros((4, 2, 7))), h(np.ones((4, 7))), h(np.zeros((4, 7))))   # odd head_dim


# ---------------------------------------------------------------------------
# einsum("ihd,jhd->ihj"), einsum("ihj,jhd->ihd"), apply_attention_mask: the
# attention steps one builtin at a time, as debug/chat_demo_with_kvcache.tl
# calls them
# ---------------------------------------------------------------------------
def test_einsum_known_answers(oracle):
    # tests/test_einsum_f16_comprehensive.rs:45-89: q [2,1,2], k [3,1,2]
    q = h([[[1, 2]], [[3, 4]]])
    k = h([[[1, 0]], [[0, 1]], [[1, 1]]])
    assert np.array_equal(oracle.einsum_scores(q, k), h([[[1, 2, 3]], [[3, 4, 7]]]))
    # :92-135: attn [2,1,3], v [3,1,2] -> [[0.7, 0.5]], [[0.7, 0.8]] (within 1e-2)
    p = h([[[0.5, 0.3, 0.2]], [[0.2, 0.3, 0.5]]])
    for acc in (oracle.ACC_F32, oracle.ACC_F16):
        out = oracle.einsum_context(p, k, acc).astype(np.float32)
        assert out.shape == (2, 1, 2)
        assert np.allclose(out, [[[0.7, 0.5]], [[0.7, 0.8]]], atol=1e-2)


@pytest.mark.parametrize("I,J,H,Hkv,D", [(5, 9, 8, 2, 16), (1, 40, 4, 4, 64), (7, 7, 6, 3, 80)])
def test_einsum_vs_float64(oracle, I, J, H, Hkv, D):
    """Against float64 with the expansion written out as the programs do it
    (K reshaped to [J, Hkv, 1, D] and broadcast to [J, Hkv, H/Hkv, D]): a
    transposed operand or the wrong KV head for a query head fails."""
    q = S.normal_f16(80, "eq", (I, H, D))
    k = S.normal_f16(80, "ek", (J, Hkv, D))
    v = S.normal_f16(80, "ev", (J, Hkv, D))
    kx = np.broadcast_to(k[:, :, None, :], (J, Hkv, H // Hkv, D)).reshape(J, H, D).astype(np.float64)
    vx = np.broadcast_to(v[:, :, None, :], (J, Hkv, H // Hkv, D)).reshape(J, H, D).astype(np.float64)
    sc = oracle.einsum_scores(q, k)
    ref = np.einsum("ihd,jhd->ihj", q.astype(np.float64), kx)
    # one f32 sum of D products, one f16 rounding: within one f16 ulp
    assert np.all(np.abs(sc.astype(np.float64) - ref) <= np.maximum(2.0 ** -24, np.abs(ref) * 2.0 ** -10))
    p = oracle.softmax(sc)
    ctx = oracle.einsum_context(p, v)
    ref = np.einsum("ihj,jhd->ihd", p.astype(np.float64), vx)
    assert np.all(np.abs(ctx.astype(np.float64) - ref) <= np.maximum(2.0 ** -24, np.abs(ref) * 2.0 ** -10))


def test_apply_attention_mask_known_answers(oracle):
    # tests/test_attention_mask.rs:267-292, :296-319, :323-343, :347-373
    assert np.array_equal(oracle.apply_attention_mask(h([[1, 2], [3, 4]]), h([[1, 0], [1, 1]])),
                          h([[1, -10000], [3, 4]]))
    assert np.array_equal(oracle.apply_attention_mask(h([[1, 2, 3]]), h([[1, 1, 1]])), h([[1, 2, 3]]))
    assert np.all(oracle.apply_attention_mask(h([[1, 2], [3, 4]]), np.zeros((2, 2), np.float16)) == -10000)
    got = oracle.apply_attention_mask(np.ones((4, 4), np.float16), oracle.causal_mask(4))
    assert np.array_equal(got, np.where(np.tril(np.ones((4, 4))) == 1, 1.0, -10000.0).astype(np.float16))
    with pytest.raises(ValueError):            # the reference requires equal shapes (masking.rs:36-43)
        oracle.apply_attention_mask(h([[1, 2]]), h([[1], [1]]))


@pytest.mark.parametrize("acc", [0, 1])
@pytest.mark.parametrize("S_,H,Hkv,D,q0", [(12, 8, 2, 64, 0), (1, 8, 2, 64, 11), (30, 4, 4, 16, 0)])
def test_einsum_program_composition_is_the_fused_oracle(oracle, acc, S_, H, Hkv, D, q0):
    """The program's steps -- einsum, * 0.125, apply_attention_mask with a
    causal_mask broadcast over heads (all ones for the single decode row),
    softmax, einsum -- composed from the one-builtin functions equal
    tlo_attention (pinned against float64 in test_oracle_pinning.py) bit
    for bit."""
    J = q0 + S_
    q = S.normal_f16(81, "cq", (S_, H, D))
    k = S.normal_f16(81, "ck", (J, Hkv, D))
    v = S.normal_f16(81, "cv", (J, Hkv, D))
    sc = oracle.mul_scalar(oracle.einsum_scores(q, k), 0.125)
    if S_ == J:
        mask = np.broadcast_to(oracle.causal_mask(S_).reshape(S_, 1, S_), (S_, H, S_))
    else:   # decode: causal_mask(1) broadcast to [1, H, J] (chat_demo_with_kvcache.tl:265-268)
        mask = np.broadcast_to(oracle.causal_mask(1).reshape(1, 1, 1), (1, H, J))
    p = oracle.softmax(oracle.apply_attention_mask(sc, np.ascontiguousarray(mask)))
    out = oracle.einsum_context(p, v, acc)
    fused = oracle.attention(q, k, v, q0, 0.125, True, acc)
    assert np.array_equal(out.view(np.uint16), fused.view(np.uint16))


# ---------------------------------------------------------------------------
# argmax (Tensor::argmax, reduce.rs:585-668)
# ---------------------------------------------------------------------------
def test_argmax_reference_known_answers(oracle):
    # tests/test_reduce_ops.rs:385-398, 418-441, 463-482, 519-525
    assert oracle.tensor_argmax(h([3, 7, 2, 9, 1])).tolist() == [3.0]
    assert oracle.tensor_argmax(h([[1, 5, 3], [9, 2, 7]]), 1).tolist() == [1.0, 0.0]
    assert oracle.tensor_argmax(h([[1, 5], [9, 2]]), 1, True).shape == (2, 1)
    with pytest.raises(ValueError):
        oracle.tensor_argmax(h(np.ones((2, 3))), 10)


def test_argmax_first_maximum_and_specials(oracle):
    inf, nan = np.inf, np.nan
    # ties: the first index; -0 and +0 are equal; NaN never beats anything
    assert oracle.tensor_argmax(h([1, 4, 4, 2])).tolist() == [1.0]
    assert oracle.tensor_argmax(h([-0.0, 0.0, -1])).tolist() == [0.0]
    assert oracle.tensor_argmax(h([1, nan, 3, nan])).tolist() == [2.0]
    # the whole-tensor scan starts from element 0's value: a NaN there is never beaten
    assert oracle.tensor_argmax(h([nan, 5, 7])).tolist() == [0.0]
    # along a dim the scan starts from -inf: NaN and -inf never win, index 0 if nothing does
    assert oracle.tensor_argmax(h([[nan, 5, 7], [-inf, -inf, nan], [-inf, -3, -inf]]), 1).tolist() == [2.0, 0.0, 1.0]
    assert oracle.tensor_argmax(np.array([-inf, -inf], np.float32)).tolist() == [0.0]
    # the index is stored as T::from_f64: f16 rounds to nearest even above 2048
    x = np.zeros(4000, np.float16)
    for i, want in ((2049, 2048.0), (3001, 3000.0), (3003, 3004.0), (2047, 2047.0)):
        x[:] = 0
        x[i] = 1
        assert oracle.tensor_argmax(x).tolist() == [want]
        assert oracle.tensor_argmax(x.astype(np.float32)).tolist() == [float(i)]
    # reducing the only dim without keepdim: the reference's from_vec([i], []) fails
    with pytest.raises(ValueError):
        oracle.tensor_argmax(h([1, 2]), 0)
    assert oracle.tensor_argmax(h([1, 2]), 0, True).tolist() == [1.0]


@pytest.mark.parametrize("shape,dim", [((17,), None), ((6, 9), None), ((6, 9), 0), ((6, 9), 1), ((1, 40), 1),
                                       ((4, 3, 5), 0), ((4, 3, 5), 1), ((4, 3, 5), 2), ((2, 3, 4, 5), 2),
                                       ((3, 1, 4), 2), ((5, 2, 3), None)])
@pytest.mark.parametrize("dt", [np.float16, np.float32])
def test_argmax_matches_numpy(oracle, shape, dim, dt):
    """numpy's argmax also returns the first maximum (no NaNs here; -inf
    entries and all--inf lines included).  The reference lays the results
    out with the first kept dim varying fastest, i.e. numpy's result array
    with its axes reversed, flattened, in the kept dims' shape."""
    rng = np.random.default_rng(len(shape) * 10 + (dim or 0))
    x = rng.integers(-4, 5, size=shape).astype(dt)   # many ties
    x[x == -4] = -np.inf
    if dim is not None and x.ndim > 1:
        first = [slice(None)] * x.ndim
        first[0 if dim else -1] = 0
        x[tuple(first)] = -np.inf   # some lines with nothing above -inf
    got = oracle.tensor_argmax(x, dim)
    if dim is None:
        want = np.array([np.argmax(x.ravel())], np.float64)
    else:
        r = np.argmax(x, axis=dim)
        want = r.transpose(tuple(reversed(range(r.ndim)))).ravel().reshape(r.shape)
    assert got.shape == want.shape
    assert np.array_equal(got.astype(np.float64), want.astype(dt).astype(np.float64))
