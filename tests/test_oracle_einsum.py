"""Pins the oracle's restatement of the general einsum (parse_einsum_equation,
infer_output_spec and general_einsum_cpu, einsum.rs:84-333) before the
device parity tests trust it.  CPU only.

Checked against the reference's own known answers (einsum.rs:428-620:
matmul, transpose, trace, element-wise and outer products, batch matmul);
against numpy's integer einsum on small integers, where every product and
partial sum is an integer below 2048 and so exact in f16 in any order (a
transposed operand, a wrong diagonal stride or a dropped term fails); and
for the rounding, against the oracle's f16-accumulation matmul
(matmul_cpu, already pinned bit for bit against a numpy f16 loop), which
"ij,jk->ik" must equal bit for bit.
"""
import numpy as np
import pytest

from oracle import oracle as O


def h(x):
    return np.asarray(x, np.float16)


def test_parse():
    assert O.einsum_parse("ij,jk->ik") == (["ij", "jk"], "ik")
    assert O.einsum_parse(" ij , jk ") == (["ij", "jk"], "ik")   # implicit: indices occurring once, sorted
    assert O.einsum_parse("ba,ca") == (["ba", "ca"], "bc")
    assert O.einsum_parse("ii") == (["ii"], "")
    with pytest.raises(ValueError):
        O.einsum_parse("ij->j->i")


def test_reference_known_answers():
    a = h([[1, 2], [3, 4]])
    b = h([[5, 6], [7, 8]])
    assert np.array_equal(O.einsum_general("ij,jk->ik", a, b), h([[19, 22], [43, 50]]))
    t = O.einsum_general("ij->ji", h([[1, 2, 3], [4, 5, 6]]))
    assert t.shape == (3, 2) and np.array_equal(t.reshape(-1)[:4], h([1, 4, 2, 5]))
    assert np.array_equal(O.einsum_general("ii->", a), h([5]))
    assert np.array_equal(O.einsum_general("ij,ij->ij", a, h([[2, 3], [4, 5]])), h([[2, 6], [12, 20]]))
    assert np.array_equal(O.einsum_general("i,j->ij", h([1, 2]), h([3, 4])), h([[3, 4], [6, 8]]))
    x = h(np.arange(1, 9).reshape(2, 2, 2))
    eye = h(np.stack([np.eye(2)] * 2))
    bm = O.einsum_general("bij,bjk->bik", x, eye)
    assert bm.shape == (2, 2, 2) and np.array_equal(bm, x)


@pytest.mark.parametrize("eq,shapes", [
    ("ij,jk->ik", [(5, 7), (7, 3)]),
    ("ii->i", [(6, 6)]),
    ("ijk->kj", [(3, 4, 5)]),
    ("bij,bjk->bik", [(2, 3, 4), (2, 4, 5)]),
    ("i,i->", [(9,), (9,)]),
    ("ij,j->i", [(4, 6), (6,)]),
    ("ij,jk,kl->il", [(3, 4), (4, 5), (5, 2)]),
    ("ijk,ikl->jl", [(3, 2, 4), (3, 4, 5)]),
    ("ihd,jhd->ihj", [(3, 2, 4), (5, 2, 4)]),
    ("ab,cb", [(3, 4), (2, 4)]),
])
def test_integer_operands_match_numpy(eq, shapes):
    rng = np.random.default_rng(len(eq) + sum(map(len, shapes)))
    ops = [rng.integers(-3, 4, s) for s in shapes]
    got = O.einsum_general(eq, *[h(o) for o in ops])
    want = np.einsum(eq, *ops)
    assert np.abs(want).max() < 2048
    assert np.array_equal(got.astype(np.int64).reshape(-1), np.asarray(want).reshape(-1))


def test_f16_accumulation_matches_matmul_cpu():
    rng = np.random.default_rng(5)
    a = h(rng.standard_normal((6, 300)))
    b = h(rng.standard_normal((300, 7)))
    got = O.einsum_general("ij,jk->ik", a, b)
    want = O.linear(a, np.ascontiguousarray(b.T), acc=O.ACC_F16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # and f16 accumulation differs from an f32 sum rounded once at this length
    assert not np.array_equal(got.view(np.uint16), O.linear(a, np.ascontiguousarray(b.T)).view(np.uint16))


def test_nested_levels_sum_separately():
    """Two summed indices: each inner level's f16 sum is rounded before it
    joins the outer one.  On data where that matters, the result differs
    from one flat f16 running sum over all terms, and equals the two-level
    sum computed here by hand."""
    rng = np.random.default_rng(8)
    x = h(rng.standard_normal((2, 40, 50)) * 8)
    got = O.einsum_general("ijk->i", x)
    flats = []
    for i in range(2):
        outer = np.float16(0)
        flat = np.float16(0)
        for j in range(40):
            inner = np.float16(0)
            for k in range(50):
                inner = np.float16(inner + x[i, j, k])
                flat = np.float16(flat + x[i, j, k])
            outer = np.float16(outer + inner)
        assert got[i] == outer
        flats.append(flat)
    assert any(got[i] != flats[i] for i in range(2))
