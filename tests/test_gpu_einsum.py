"""Device parity of einsum(equation, tensors...) through libtlhip.so's C ABI
(tlhip_einsum / tlhip_einsum_shape): every equation other than the two
attention einsums runs general_einsum_cpu's f16 arithmetic
(einsum.rs:207-333) on the device, bit-exact against the oracle's
restatement on the same inputs; the attention equations route to their
kernels; errors follow the reference's checks.
"""
import numpy as np
import pytest

from tensorlogic_amd import F16, F32, TLHipError
from tensorlogic_amd.tensor import einsum

pytestmark = pytest.mark.gpu


def h(x):
    return np.asarray(x, np.float16)


def run(dev, eq, ops, dtype=F16):
    return einsum(eq, *[dev.tensor(o, dtype) for o in ops]).numpy()


def test_reference_known_answers(dev):
    # einsum.rs:428-620
    a = h([[1, 2], [3, 4]])
    assert np.array_equal(run(dev, "ij,jk->ik", [a, h([[5, 6], [7, 8]])]), h([[19, 22], [43, 50]]))
    t = run(dev, "ij->ji", [h([[1, 2, 3], [4, 5, 6]])])
    assert t.shape == (3, 2) and np.array_equal(t, h([[1, 4], [2, 5], [3, 6]]))
    assert np.array_equal(run(dev, "ii->", [a]), h([5]))
    assert np.array_equal(run(dev, "ij,ij->ij", [a, h([[2, 3], [4, 5]])]), h([[2, 6], [12, 20]]))
    assert np.array_equal(run(dev, "i,j->ij", [h([1, 2]), h([3, 4])]), h([[3, 4], [6, 8]]))
    x = h(np.arange(1, 9).reshape(2, 2, 2))
    assert np.array_equal(run(dev, "bij,bjk->bik", [x, h(np.stack([np.eye(2)] * 2))]), x)


@pytest.mark.parametrize("eq,shapes", [
    ("ij,jk->ik", [(33, 65), (65, 31)]),
    ("ij,jk->ik", [(4, 2048), (2048, 3)]),
    ("ii->i", [(40, 40)]),
    ("ii->", [(300, 300)]),
    ("ijk->kj", [(3, 40, 50)]),
    ("bij,bjk->bik", [(4, 16, 64), (4, 64, 24)]),
    ("i,i->", [(5000,), (5000,)]),
    ("ij,j->i", [(300, 700), (700,)]),
    ("ij,jk,kl->il", [(6, 20), (20, 30), (30, 5)]),
    ("ijk->i", [(7, 40, 50)]),
    ("abc,cd,a->bd", [(3, 8, 9), (9, 4), (3,)]),
    ("ab,cb", [(30, 40), (20, 40)]),
    ("ijkl->lkji", [(2, 3, 4, 5)]),
    ("i,j,k->ijk", [(5,), (6,), (7,)]),
])
def test_general_equations_bit_exact(dev, oracle, eq, shapes):
    rng = np.random.default_rng(len(eq) * 131 + sum(map(sum, shapes)))
    ops = [h(rng.standard_normal(s) * 1.5) for s in shapes]
    got = run(dev, eq, ops)
    want = oracle.einsum_general(eq, *ops)
    assert got.dtype == np.float16 and got.shape == want.shape
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), f"{eq} {shapes}"


def test_integer_operands_match_numpy(dev):
    rng = np.random.default_rng(3)
    for eq, shapes in [("ij,jk->ik", [(9, 11), (11, 6)]), ("bij,bjk->bik", [(3, 5, 7), (3, 7, 4)]),
                       ("ij,jk,kl->il", [(3, 4), (4, 5), (5, 2)]), ("iij->j", [(5, 5, 3)])]:
        ops = [rng.integers(-3, 4, s) for s in shapes]
        got = run(dev, eq, [h(o) for o in ops])
        assert np.array_equal(got.astype(np.int64), np.einsum(eq, *ops)), eq


def test_attention_equations_route_to_their_kernels(dev, oracle):
    rng = np.random.default_rng(4)
    q = h(rng.standard_normal((5, 8, 64)))
    k = h(rng.standard_normal((9, 8, 64)))
    got = run(dev, "ihd,jhd->ihj", [q, k])
    assert np.array_equal(got.view(np.uint16), oracle.einsum_scores(q, k).view(np.uint16))
    p = h(np.abs(rng.standard_normal((5, 8, 9))) / 9)
    ctx = run(dev, "ihj,jhd->ihd", [p, k])
    assert ctx.shape == (5, 8, 64)
    q32, k32 = q.astype(np.float32), k.astype(np.float32)
    s32 = run(dev, "ihd,jhd->ihj", [q32, k32], F32)
    assert s32.dtype == np.float32
    assert np.array_equal(s32.view(np.uint32), oracle.einsum_scores_f32(q32, k32).view(np.uint32))


def test_errors(dev):
    a = dev.tensor(h(np.ones((2, 3))))
    b = dev.tensor(h(np.ones((4, 5))))
    for eq, ops, kind in [("ij,jk->ik", [a, b], "ShapeMismatch"),      # j: 3 vs 4
                          ("ij,jk->ik", [a], "InvalidOperation"),       # operand count
                          ("ij->j->i", [a], "InvalidOperation"),        # too many arrows
                          ("ijk->i", [a], "InvalidOperation"),          # spec longer than the rank
                          ("ij->iz", [a], "InvalidOperation"),          # unknown output index
                          ("ij->ii", [a], "InvalidOperation")]:         # repeated output index
        with pytest.raises(TLHipError) as e:
            einsum(eq, *ops)
        assert e.value.kind == kind, eq
    # a summation space beyond the general kernel's bound is refused up front
    big = dev.tensor(h(np.ones((2048, 2048))))
    with pytest.raises(TLHipError) as e:
        einsum("ij,kl->", big, big)
    assert e.value.kind == "InvalidOperation"
    f = dev.tensor(np.ones((3, 5), np.float32), F32)
    with pytest.raises(TLHipError) as e:
        einsum("ij,jk->ik", a, f)
    assert e.value.kind == "DtypeError"
    with pytest.raises(TLHipError) as e:
        einsum("ij->ji", f)
    assert e.value.kind == "InvalidOperation"
