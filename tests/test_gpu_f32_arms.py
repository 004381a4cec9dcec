"""Device parity of the TensorF32 arms of rms_norm, layer_norm, softmax,
rope, sigmoid, silu, gelu, add / mul / mul_scalar, apply_attention_mask,
embedding and the attention einsums (unified.metal:678-694, 934-992,
1051-1062, 1129-1135, 1833-2036, 2202-2340, 2420-2482, 2702-2768, 4491-4503)
through libtlhip.so's C ABI, against the CPU oracle on the same inputs.

Bars: rms_norm, layer_norm, rope, the einsums, add / mul / mul_scalar, the
mask and the embedding gather take the reference's summation order and
rounding steps on both sides (sqrt and division correctly rounded), so they
are bit-exact.  softmax, sigmoid, silu and gelu call exp or tanh, which the
device's math library and the host's libm round differently in the last
bit (softmax's sum is taken in the reference's element order on both
sides): those are bounded at 8 f32 ulps per element (f32 relative error
~5e-7, far inside the 1e-3 relative-L2 bar of the f16 path); gelu for x <<
0, where 1 + tanh cancels, at 8 ulps of 0.5 |x| instead.  Operand dtypes
must agree: a mix is the reference's TypeError (DtypeError here).
"""
import numpy as np
import pytest

from tensorlogic_amd import F16, F32, TLHipError
from tensorlogic_amd.tensor import einsum, embedding

pytestmark = pytest.mark.gpu
ULPS = 8


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_ulps(got, ref, what, bound=ULPS):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape, what
    same_nonfinite = (~np.isfinite(ref)) & (got.view(np.uint32) == ref.view(np.uint32))
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    sp = np.spacing(np.maximum(np.abs(ref), np.float32(2.0 ** -126))).astype(np.float64)
    u = np.where(same_nonfinite, 0.0, err / sp)
    assert np.all(u <= bound), f"{what}: {u.max():.1f} f32 ulps (bound {bound})"


def rnd(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


@pytest.mark.parametrize("rows,n", [(3, 64), (5, 256), (4, 257), (2, 2048), (1, 5000), (7, 1)])
def test_rms_norm_f32(dev, oracle, rows, n):
    x = rnd(rows * 7 + n, (rows, n), 3.0)
    w = rnd(n, (n,))
    got = dev.tensor(x, F32).rms_norm([n], dev.tensor(w, F32), 1e-6).numpy()
    assert got.dtype == np.float32
    assert np.array_equal(bits(got), bits(oracle.rms_norm_f32(x, w, 1e-6)))


@pytest.mark.parametrize("rows,n", [(3, 4), (5, 256), (4, 257), (2, 1000), (1, 32000)])
def test_softmax_f32(dev, oracle, rows, n):
    x = rnd(rows + n, (rows, n), 4.0)
    got = dev.tensor(x, F32).softmax().numpy()
    assert got.dtype == np.float32
    assert_ulps(got, oracle.softmax_f32(x), f"softmax f32 [{rows}, {n}]")


def test_softmax_f32_masked_and_degenerate_rows(dev, oracle):
    x = np.array([[0.5, -np.inf, 1.5, np.nan, -3.0],
                  [-np.inf] * 5,
                  [np.nan] * 5,
                  [1e30, 1e30, -1e30, 0.0, 1e30]], np.float32)
    got = dev.tensor(x, F32).softmax().numpy()
    ref = oracle.softmax_f32(x)
    assert np.array_equal(bits(got[1:3]), bits(ref[1:3]))   # uniform 1/n, exactly
    assert got[0, 1] == 0 and got[0, 3] == 0
    assert_ulps(got, ref, "softmax f32 masked rows")


@pytest.mark.parametrize("S,H,D,offset,layout,rot", [
    (1, 1, 64, 0, 0, 0), (7, 4, 64, 300, 0, 0), (5, 3, 80, 17, 1, 32), (46, 32, 64, 0, 0, 0),
    (3, 2, 128, 1000, 1, 0), (4, 5, 64, 9, 0, 16)])
def test_rope_f32(dev, oracle, S, H, D, offset, layout, rot):
    x = rnd(S * H + D + offset, (S, H, D), 2.0)
    got = dev.tensor(x, F32).rope(offset, 10000.0, layout, rot).numpy()
    assert got.dtype == np.float32
    assert np.array_equal(bits(got), bits(oracle.rope_f32(x, offset, 10000.0, layout, rot)))


def test_rope_f32_magnitude(dev):
    # rope.rs:599-640: pairs (3, 4) keep length 5
    x = np.tile(np.array([3, 4], np.float32), 32).reshape(1, 1, 64)
    y = dev.tensor(x, F32).rope(0).numpy()
    assert np.array_equal(y, x)
    y = dev.tensor(x, F32).rope(123).numpy().astype(np.float64)
    assert np.max(np.abs(np.hypot(y[0, 0, 0::2], y[0, 0, 1::2]) - 5.0)) < 5.0 * 4e-7


@pytest.mark.parametrize("n", [5, 1000, 65537])
def test_sigmoid_f32(dev, oracle, n):
    x = rnd(n, (n,), 6.0)
    if n == 5:
        x = np.array([-2, -1, 0, 1, 2], np.float32)   # activations.rs:844-870
    got = dev.tensor(x, F32).sigmoid().numpy()
    assert got.dtype == np.float32
    assert_ulps(got, oracle.sigmoid_f32(x), f"sigmoid f32 n={n}", 4)
    if n == 5:
        assert got[2] == np.float32(0.5)


@pytest.mark.parametrize("I,J,H,Hkv,D", [(1, 47, 32, 4, 64), (5, 9, 4, 4, 16), (46, 46, 8, 2, 80), (3, 130, 6, 3, 128)])
def test_einsum_f32(dev, oracle, I, J, H, Hkv, D):
    q = rnd(I + J, (I, H, D))
    k = rnd(I + J + 1, (J, Hkv, D))
    p = np.abs(rnd(I + J + 2, (I, H, J))) / J
    v = rnd(I + J + 3, (J, Hkv, D))
    sc = einsum("ihd,jhd->ihj", dev.tensor(q, F32), dev.tensor(k, F32)).numpy()
    ctx = einsum("ihj,jhd->ihd", dev.tensor(p, F32), dev.tensor(v, F32)).numpy()
    assert sc.dtype == np.float32 and ctx.dtype == np.float32
    assert np.array_equal(bits(sc), bits(oracle.einsum_scores_f32(q, k)))
    assert np.array_equal(bits(ctx), bits(oracle.einsum_context_f32(p, v)))


def test_f32_arms_refuse_mixed_dtypes(dev):
    x32 = dev.tensor(np.ones((2, 8), np.float32), F32)
    w16 = dev.tensor(np.ones(8, np.float16), F16)
    with pytest.raises(TLHipError) as e:
        x32.rms_norm([8], w16)
    assert e.value.kind == "DtypeError"
    q32 = dev.tensor(np.ones((2, 2, 8), np.float32), F32)
    k16 = dev.tensor(np.ones((3, 2, 8), np.float16), F16)
    with pytest.raises(TLHipError) as e:
        einsum("ihd,jhd->ihj", q32, k16)
    assert e.value.kind == "DtypeError"


@pytest.mark.parametrize("rows,n,affine", [(3, 64, "wb"), (5, 256, "w"), (4, 257, "b"), (2, 2560, "wb"),
                                           (1, 5000, ""), (7, 1, "wb")])
def test_layer_norm_f32(dev, oracle, rows, n, affine):
    x = rnd(rows * 3 + n, (rows, n), 2.0) + np.float32(0.3)
    w = rnd(n + 1, (n,)) if "w" in affine else None
    b = rnd(n + 2, (n,)) if "b" in affine else None
    got = dev.tensor(x, F32).layer_norm(dev.tensor(w, F32) if w is not None else None,
                                        dev.tensor(b, F32) if b is not None else None, 1e-5).numpy()
    assert got.dtype == np.float32
    assert np.array_equal(bits(got), bits(oracle.layer_norm_f32(x, w, b, 1e-5)))


@pytest.mark.parametrize("n", [5, 1000, 65537])
def test_gelu_silu_f32(dev, oracle, n):
    x = rnd(n + 5, (n,), 4.0)
    if n == 5:
        x = np.array([-2, -1, 0, 1, 2], np.float32)   # activations.rs:900-940
    g = dev.tensor(x, F32).gelu().numpy()
    assert g.dtype == np.float32
    ref = oracle.gelu_f32(x)
    # 1 + tanh cancels for x << 0: 8 ulps of 0.5 |x| there
    sp = np.spacing(np.maximum(np.maximum(np.abs(ref), 0.5 * np.abs(x)), np.float32(2.0 ** -126)))
    assert np.all(np.abs(g.astype(np.float64) - ref) <= ULPS * sp.astype(np.float64)), "gelu f32"
    if n == 5:
        assert g[2] == 0
    s = dev.tensor(x, F32).silu().numpy()
    assert_ulps(s, oracle.silu_f32(x), f"silu f32 n={n}")
    u = rnd(n + 6, (n,))
    sm = dev.tensor(x, F32).silu_mul(dev.tensor(u, F32)).numpy()
    assert_ulps(sm, oracle.swiglu_f32(x, u), f"silu_mul f32 n={n}")


@pytest.mark.parametrize("shape", [(7,), (3, 257), (46, 2048)])
def test_add_mul_scalar_f32(dev, oracle, shape):
    a = rnd(sum(shape), shape, 3.0)
    b = rnd(sum(shape) + 1, shape)
    ta, tb = dev.tensor(a, F32), dev.tensor(b, F32)
    for got, ref in ((ta.add(tb), oracle.add_f32(a, b)), (ta.mul(tb), oracle.mul_f32(a, b)),
                     (ta.mul_scalar(0.1), oracle.mul_scalar_f32(a, 0.1))):
        got = got.numpy()
        assert got.dtype == np.float32
        assert np.array_equal(bits(got), bits(ref))
    row = rnd(7, (shape[-1],))   # a bias-style row repeated over the last dim
    assert np.array_equal(bits(ta.add(dev.tensor(row, F32)).numpy()), bits(oracle.add_f32(a, row)))


def test_apply_attention_mask_f32(dev, oracle):
    # masking.rs:325-355
    sc = dev.tensor(np.array([[1, 2], [3, 4]], np.float32), F32)
    m = dev.tensor(np.array([[1, 0], [1, 1]], np.float32), F32)
    got = sc.apply_attention_mask(m).numpy()
    assert got.dtype == np.float32 and np.array_equal(got, np.array([[1, -10000], [3, 4]], np.float32))
    # a causal [I, J] mask over [I, H, J] scores, and a same-shape mask with -0 / NaN entries
    I, H, J = 46, 32, 46
    s3 = rnd(1, (I, H, J), 3.0)
    cm = np.tril(np.ones((I, J), np.float32))
    assert np.array_equal(bits(dev.tensor(s3, F32).apply_attention_mask(dev.tensor(cm, F32)).numpy()),
                          bits(oracle.apply_attention_mask_f32(s3, cm)))
    mm = np.where(rnd(2, (I, H, J)) > 0, np.float32(1), np.float32(-0.0)).astype(np.float32)
    mm[0, 0, :3] = np.nan
    assert np.array_equal(bits(dev.tensor(s3, F32).apply_attention_mask(dev.tensor(mm, F32)).numpy()),
                          bits(oracle.apply_attention_mask_f32(s3, mm)))


@pytest.mark.parametrize("V,Hd", [(100, 64), (50, 30)])
def test_embedding_f32(dev, V, Hd):
    table = rnd(V + Hd, (V, Hd))
    ids = np.array([3, 0, V - 1, 3, 17], np.int32)
    got = embedding(dev.tensor(table, F32), ids).numpy()
    assert got.dtype == np.float32 and np.array_equal(bits(got), bits(table[ids]))
    with pytest.raises(TLHipError) as e:
        embedding(dev.tensor(table, F32), np.array([V], np.int32))
    assert e.value.kind == "IndexOutOfBounds"


def test_more_f32_arms_refuse_mixed_dtypes(dev):
    x32 = dev.tensor(np.ones((2, 8), np.float32), F32)
    x16 = dev.tensor(np.ones((2, 8), np.float16), F16)
    w16 = dev.tensor(np.ones(8, np.float16), F16)
    for call in (lambda: x32.layer_norm(w16, None), lambda: x32.add(x16), lambda: x32.mul(x16),
                 lambda: x32.silu_mul(x16), lambda: x32.apply_attention_mask(x16)):
        with pytest.raises(TLHipError) as e:
            call()
        assert e.value.kind == "DtypeError"
