"""tlhip_linear_noalloc: linear() with its split-K workspace in a fixed device
array instead of pool memory.  Through the C ABI, its output must equal
tlhip_linear's bit for bit (same split, same kernels) and the oracle's within
the linear bars, on consecutive calls where a later call is smaller than an
earlier one (the array keeps the previous call's partials), and it must
refuse what it cannot do without allocating."""

import numpy as np
import pytest

from tensorlogic_amd import Q4_0, Q6_K, Q8_0, TLHipError
from tensorlogic_amd import _lib as L
from tensorlogic_amd import synth as S

from test_gpu_ops import assert_close

pytestmark = pytest.mark.gpu


def _linear_pair(dev, oracle, qt, M, N, K, seed):
    """(noalloc output, tlhip_linear output, oracle) for one shape."""
    gen = {Q4_0: S.q4_0_blocks, Q8_0: S.q8_0_blocks}[qt]
    blocks = gen(seed, f"na_W{N}x{K}", N, K)
    x = S.normal_f16(seed, f"na_x{M}x{K}", (M, K))
    w = dev.quantized(blocks, (N, K), qt)
    tx = dev.tensor(x)
    y_na = dev.empty((M, N))
    y_ref = dev.empty((M, N))
    L.call("tlhip_linear_noalloc", dev.h, tx.h, w.h, None, y_na.h)
    L.call("tlhip_linear", dev.h, tx.h, w.h, None, y_ref.h)
    ref = oracle.linear_q(x, blocks, 2 if qt == Q4_0 else 8, N)
    return y_na.numpy(), y_ref.numpy(), ref


# (qt, M, N, K): split-K GEMMs of both kernels (M <= 64: the skinny GEMM,
# unsplit at 176 weight-row tiles, 4 and 8 slices at 64 and 8 tiles; M > 64:
# 2 slices), then a smaller call reusing the array, then a GEMV
@pytest.mark.parametrize("calls", [
    [(Q8_0, 46, 5632, 2048), (Q8_0, 20, 2048, 2048)],
    [(Q4_0, 512, 2048, 2048), (Q4_0, 130, 256, 2048)],
    [(Q4_0, 64, 2048, 5632), (Q8_0, 5, 256, 2048), (Q4_0, 1, 2048, 2048)],
    # the largest partial set the split policy picks: 80 tiles x 4 slices of
    # 128 x 128 fp32 = 20 MiB, the whole array (Phi-2 fc2 at a 512-row
    # prefill), then a smaller split
    [(Q4_0, 512, 2560, 10240), (Q8_0, 256, 512, 2048)],
])
def test_linear_noalloc_matches_linear(dev, oracle, calls):
    for i, (qt, M, N, K) in enumerate(calls):
        got, ref_dev, ref = _linear_pair(dev, oracle, qt, M, N, K, 40 + i)
        assert np.array_equal(got.view(np.uint16), ref_dev.view(np.uint16)), f"call {i}: {M}x{N}x{K}"
        assert_close(got, ref, what=f"linear_noalloc call {i} {M}x{N}x{K}")


def test_linear_noalloc_with_bias_repeated(dev, oracle):
    """Bias epilogue through the skinny GEMM's split (8 slices), twice in a
    row on the same tensors: the second call reads only what it wrote
    itself.  The
    activations are N(0, 0.25) so that outputs stay below 8, where the bias
    add's second f16 rounding is within the 2e-2 bar."""
    M, N, K = 33, 512, 4096
    blocks = S.q8_0_blocks(48, "na_Wb", N, K)
    x = S.normal_f16(48, "na_xb", (M, K), 0.0, 0.25)
    b = S.normal_f16(48, "na_b", (N,))
    w, tx, tb = dev.quantized(blocks, (N, K), Q8_0), dev.tensor(x), dev.tensor(b)
    ref = oracle.linear(x, oracle.dequant(blocks, 8).reshape(N, K), b)
    outs = []
    for _ in range(2):
        y = dev.empty((M, N))
        L.call("tlhip_linear_noalloc", dev.h, tx.h, w.h, tb.h, y.h)
        outs.append(y.numpy())
    y_ref = dev.empty((M, N))
    L.call("tlhip_linear", dev.h, tx.h, w.h, tb.h, y_ref.h)
    for o in outs:
        assert np.array_equal(o.view(np.uint16), y_ref.numpy().view(np.uint16))
    assert_close(outs[0], ref, what="linear_noalloc with bias")


def test_linear_noalloc_refusals(dev):
    """What needs an allocation is refused with a clear error, and shape
    errors are the same as tlhip_linear's."""
    blocks = S.q6_k_blocks(49, "na_W6", 64, 256)
    w6 = dev.quantized(blocks, (64, 256), Q6_K)
    x = dev.tensor(S.normal_f16(49, "na_x6", (8, 256)))
    y = dev.empty((8, 64))
    with pytest.raises(TLHipError) as e:
        L.call("tlhip_linear_noalloc", dev.h, x.h, w6.h, None, y.h)
    assert e.value.kind == "InvalidOperation" and "Q6_K" in str(e.value)
    x1 = dev.tensor(S.normal_f16(49, "na_x6b", (1, 256)))
    y1 = dev.empty((1, 64))
    L.call("tlhip_linear_noalloc", dev.h, x1.h, w6.h, None, y1.h)   # M <= 4: the GEMV needs no workspace
    y1r = dev.empty((1, 64))
    L.call("tlhip_linear", dev.h, x1.h, w6.h, None, y1r.h)
    assert np.array_equal(y1.numpy().view(np.uint16), y1r.numpy().view(np.uint16))
    xb = dev.tensor(np.zeros((2, 128), np.float16))
    with pytest.raises(TLHipError) as e:
        L.call("tlhip_linear_noalloc", dev.h, xb.h, w6.h, None, y.h)
    assert e.value.kind == "InvalidOperation"
    assert L.lib().tlhip_linear_noalloc(None, x.h, w6.h, None, y.h) == 9
