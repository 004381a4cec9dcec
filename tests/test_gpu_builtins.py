"""Device parity of the TL builtins around the attention path: causal_mask,
slice_last, broadcast_to, precompute_rope_* and rope(x, cos, sin), through
libtlhip.so's C ABI against the CPU oracle on the same inputs.  All of
them are data movement or one rounded f32 rotation per pair, so the bar
is bit-exact; error cases return the reference's TensorError kinds.
"""
import numpy as np
import pytest

from tensorlogic_amd import F16, F32, I32, TLHipError
from tensorlogic_amd import synth as S
from tensorlogic_amd.tensor import causal_mask, precompute_rope_cos, precompute_rope_sin

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16 if a.dtype == np.float16 else np.uint32)


@pytest.mark.parametrize("n", [1, 3, 7, 46, 301, 2048])
def test_causal_mask(dev, oracle, n):
    got = causal_mask(dev, n).numpy()
    assert np.array_equal(bits(got), bits(oracle.causal_mask(n)))


def test_causal_mask_needs_square_output(dev):
    out = dev.empty((3, 4))
    with pytest.raises(TLHipError) as e:
        from tensorlogic_amd._lib import call
        call("tlhip_causal_mask", dev.h, out.h)
    assert e.value.kind == "InvalidDimension"


@pytest.mark.parametrize("shape", [(5,), (2, 3, 4), (46, 2048), (3, 2, 4, 5), (1, 32, 64), (7, 1)])
@pytest.mark.parametrize("dtype", [F16, F32, I32])
def test_slice_last(dev, oracle, shape, dtype):
    np_t = {F16: np.float16, F32: np.float32, I32: np.int32}[dtype]
    if dtype == I32:
        x = np.arange(np.prod(shape), dtype=np.int32).reshape(shape) * 7 - 3
    else:
        x = S.normal_f16(64, f"sl{shape}", shape).astype(np_t)
    got = dev.tensor(x, dtype).slice_last(0).numpy()
    ref = oracle.slice_last(x, 0)
    assert got.shape == ref.shape and np.array_equal(bits(got), bits(ref))


def test_slice_last_errors(dev):
    x = dev.tensor(np.zeros((2, 3), np.float16))
    for axis in (1, 2):   # slice.rs:29-40: out of bounds / only axis 0
        with pytest.raises(TLHipError) as e:
            x.slice_last(axis)
        assert e.value.kind == "InvalidOperation"


@pytest.mark.parametrize("src,dst", [((1,), (5,)), ((3,), (4, 3)), ((3, 1), (3, 4)), ((2, 1, 4), (3, 2, 5, 4)),
                                     ((40, 4, 1, 64), (40, 4, 8, 64)), ((1, 1, 1), (2, 3, 4)), ((6, 5), (6, 5)),
                                     ((46, 1, 46), (46, 32, 46))])
@pytest.mark.parametrize("dtype", [F16, F32])
def test_broadcast_to(dev, oracle, src, dst, dtype):
    np_t = np.float16 if dtype == F16 else np.float32
    x = S.normal_f16(65, f"bc{src}", src).astype(np_t)
    got = dev.tensor(x, dtype).broadcast_to(dst).numpy()
    ref = oracle.broadcast_to(x, dst)
    assert got.shape == tuple(dst) and np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("src,dst", [((3,), (4, 2)), ((2, 3), (3,)), ((5, 1), (4, 5, 2, 3))])
def test_broadcast_to_shape_mismatch(dev, src, dst):
    x = dev.tensor(np.zeros(src, np.float16))
    with pytest.raises(TLHipError) as e:
        x.broadcast_to(dst)
    assert e.value.kind == "ShapeMismatch"


@pytest.mark.parametrize("D,L", [(64, 2048), (80, 600), (8, 3)])
def test_precompute_rope_tables(dev, oracle, D, L):
    for fn, want_sin in ((precompute_rope_cos, False), (precompute_rope_sin, True)):
        got = fn(dev, D, L, 10000.0).numpy()
        assert np.array_equal(bits(got), bits(oracle.precompute_rope(D, L, 10000.0, want_sin)))


@pytest.mark.parametrize("S_,H,D,L", [(46, 32, 64, 64), (1, 4, 64, 2048), (512, 32, 80, 600), (3, 2, 8, 3)])
def test_rope_cos_sin(dev, oracle, S_, H, D, L):
    """The TL program's precompute_rope_* tables fed to rope(x, cos, sin)."""
    x = S.normal_f16(66, f"rcs{S_}", (S_, H, D))
    c, s = precompute_rope_cos(dev, D, L), precompute_rope_sin(dev, D, L)
    got = dev.tensor(x).rope_candle(c, s).numpy()
    ref = oracle.rope_cos_sin(x, c.numpy(), s.numpy())
    assert np.array_equal(bits(got), bits(ref))


def test_rope_cos_sin_arbitrary_tables(dev, oracle):
    # tables that are not rotations (any f16 values), so every product matters
    x = S.normal_f16(67, "rcsx", (20, 4, 16))
    c = S.normal_f16(68, "rcsc", (24, 16))
    s = S.normal_f16(69, "rcss", (24, 16))
    got = dev.tensor(x).rope_candle(dev.tensor(c), dev.tensor(s)).numpy()
    assert np.array_equal(bits(got), bits(oracle.rope_cos_sin(x, c, s)))


def test_rope_cos_sin_errors(dev):
    x = dev.tensor(np.zeros((4, 2, 8), np.float16))
    for cs_shape in ((3, 8), (4, 6)):   # rope.rs:43-55
        c = dev.tensor(np.ones(cs_shape, np.float16))
        with pytest.raises(TLHipError) as e:
            x.rope_candle(c, c)
        assert e.value.kind == "InvalidOperation"
    with pytest.raises(TLHipError) as e:   # rope.rs:22-26: 3-D input only
        dev.tensor(np.zeros((4, 8), np.float16)).rope_candle(dev.tensor(np.ones((4, 8), np.float16)),
                                                            dev.tensor(np.ones((4, 8), np.float16)))
    assert e.value.kind == "InvalidOperation"


# ---------------------------------------------------------------------------
# argmax() builtin (Tensor::argmax, reduce.rs:585-668): indices are small
# integers stored in the input dtype, so the bar is bit-exact.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,dim,keepdim", [((5,), None, False), ((5,), None, True), ((2, 3), 1, False),
                                               ((2, 3), 1, True), ((2, 3), 0, False), ((6, 9), None, True),
                                               ((4, 3, 5), 0, False), ((4, 3, 5), 1, True), ((4, 3, 5), 2, False),
                                               ((2, 3, 4, 5), 2, False), ((64, 32000), 1, False),
                                               ((3, 5000), None, False), ((2, 70000), 1, False),
                                               ((300, 7), 0, True), ((1, 1), 0, False)])
@pytest.mark.parametrize("dtype", [F16, F32])
def test_tensor_argmax(dev, oracle, shape, dim, keepdim, dtype):
    np_t = np.float16 if dtype == F16 else np.float32
    rng = np.random.default_rng(int(np.prod(shape)) % 1000 + (dim or 0))
    x = rng.integers(-40, 41, size=shape).astype(np_t)   # ties everywhere
    flat = x.reshape(-1)
    flat[rng.integers(0, flat.size, size=max(1, flat.size // 50))] = np.nan
    flat[rng.integers(0, flat.size, size=max(1, flat.size // 50))] = -np.inf
    flat[rng.integers(0, flat.size, size=max(1, flat.size // 50))] = np.float16(-0.0)
    if dim is None and flat.size > 2:
        flat[0] = 1.0   # (a NaN at element 0 has a test of its own)
    t = dev.tensor(x, dtype)
    got = t.argmax(dim, keepdim)
    want = oracle.tensor_argmax(x, dim, keepdim)
    if dim is None and not keepdim:
        assert got == int(want[0])
    else:
        g = got.numpy()
        assert g.shape == want.shape and g.dtype == want.dtype
        assert np.array_equal(bits(g), bits(want))


def test_tensor_argmax_specials(dev, oracle):
    inf, nan = np.inf, np.nan
    for arr, dim in (([nan, 5, 7], None), ([[nan, 5, 7], [-inf, -inf, nan], [-inf, -3, -inf]], 1),
                     ([-0.0, 0.0, -1], None), ([[1, 4, 4, 2]], 1)):
        for dt, np_t in ((F16, np.float16), (F32, np.float32)):
            x = np.array(arr, np_t)
            got = dev.tensor(x, dt).argmax(dim, True)
            want = oracle.tensor_argmax(x, dim, True)
            assert np.array_equal(bits(got.numpy()), bits(want)), (arr, dim, dt)
    # f16 indices above 2048 round to nearest even, as T::from_f64 does
    x = np.zeros((1, 4000), np.float16)
    x[0, 3003] = 1
    assert dev.tensor(x).argmax() == 3004
    assert dev.tensor(x.astype(np.float32), F32).argmax() == 3003


def test_tensor_argmax_errors(dev):
    from tensorlogic_amd._lib import call
    t = dev.tensor(np.ones((2, 3), np.float16))
    with pytest.raises(TLHipError) as e:
        t.argmax(10)
    assert e.value.kind == "InvalidDimension"
    with pytest.raises(TLHipError) as e:
        dev.tensor(np.ones(4, np.float16)).argmax(0)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(TLHipError) as e:   # a result of the wrong shape
        call("tlhip_tensor_argmax", dev.h, t.h, 1, 0, dev.empty((3,)).h)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(TLHipError) as e:
        dev.tensor(np.ones((2, 3), np.int32), I32).argmax()
    assert e.value.kind == "DtypeError"
