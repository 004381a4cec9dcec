"""Operator parity: libtlhip.so on the device vs the CPU oracle, same seeded inputs.

Bars (north star): dequantised weights and pure data movement bit-exact;
matmul / layer outputs within max-abs 2e-2 and relative L2 1e-3 of the
fp32-accumulated oracle (the oracle stores f16 exactly where the reference
does).  Elementwise ops that evaluate exp/tanh are held to 1 f16 ulp.
"""
import json
import os

import numpy as np
import pytest

from tensorlogic_amd import F16, Q4_0, Q6_K, Q8_0, ROPE_INTERLEAVED, ROPE_NEOX, TLHipError
from tensorlogic_amd import synth as S
from tensorlogic_amd.tensor import KVCache, attention, einsum, embedding, temperature_sample

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL_L2 = 1e-3


def f16_ulp(x):
    """Spacing of f16 values at |x| (2^-24 in the subnormal range)."""
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def _log_figures(rec):
    """Append one parity record (JSON line) to $TL_PARITY_LOG when it is set."""
    path = os.environ.get("TL_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")


def assert_close(got, ref, max_abs=MAX_ABS, rel_l2=REL_L2, what=""):
    """The north star's bars: plain relative L2 ||got - ref|| / ||ref|| <= 1e-3
    and max-abs <= 2e-2.

    One named relaxation of the max-abs bar: where the reference value is
    beyond |32|, one f16 ulp (2^-5 and up) is itself coarser than 2e-2, and
    two fp32 sums taken in different orders round to neighbouring f16 values
    now and then, so there the element bound is one f16 ulp of the reference
    value.  The rel-L2 is asserted plain; the rel-L2 of each element's
    difference beyond one f16 ulp is reported beside it as a diagnostic."""
    g = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    assert g.shape == r.shape, what
    assert np.all(np.isfinite(g)) or not np.all(np.isfinite(r)), f"{what}: non-finite output"
    d = np.abs(g - r)
    ma = float(d.max()) if d.size else 0.0
    nr = max(np.linalg.norm(r), 1e-30)
    rl = float(np.linalg.norm(d) / nr) if d.size else 0.0
    rl_ulp = float(np.linalg.norm(np.maximum(d - f16_ulp(r), 0.0)) / nr) if d.size else 0.0
    bound = np.maximum(max_abs, f16_ulp(r))
    bad = np.nonzero(d > bound)[0]
    _log_figures({"what": what, "n": int(d.size), "max_abs": ma, "rel_l2": rl, "rel_l2_beyond_ulp": rl_ulp,
                  "max_ref": float(np.abs(r).max()) if d.size else 0.0})
    assert bad.size == 0 and rl <= rel_l2, (f"{what}: max_abs {ma:.3e} rel_l2 {rl:.3e} (beyond 1 ulp "
                                           f"{rl_ulp:.3e}); {bad.size} elements beyond max(2e-2, 1 ulp)")
    return ma, rl


# Named exemption of the rel-L2 bar: end-to-end decoder logits.
LOGITS_REORDER_RATIO = 1.5


def assert_logits_close(got, ref, reorder_rel_l2, what="final logits"):
    """End-to-end decoder logits, after every layer and decode step of a
    model.  The north star's bars are for matmul and layer outputs (held
    plain by assert_close everywhere else); at the end of a decoder the f16
    roundings of every earlier op have compounded, and two equally valid
    fp32 summation orders already differ by about the 1e-3 bar there: the
    oracle with every sum in descending order (ACC_F32_REV) is 0.80-1.0e-3
    from the oracle on the 2-layer program models.  So the rel-L2 bound here
    is max(1e-3, 1.5 x the reordered oracle's own distance on the same model
    and token stream), reorder_rel_l2; the max-abs bar is assert_close's."""
    bound = max(REL_L2, LOGITS_REORDER_RATIO * reorder_rel_l2)
    _log_figures({"what": f"{what} (reordered oracle)", "reorder_rel_l2": float(reorder_rel_l2), "bound": bound})
    return assert_close(got, ref, rel_l2=bound, what=f"{what} (reordered oracle at {reorder_rel_l2:.3e})")


def reorder_rel_l2(oracle, path, arch, prompt, ref_toks, ref_logits, max_ctx, literal=None):
    """The reordered oracle (ACC_F32_REV) teacher-forced on ref_toks: the
    relative L2 distance of its final logits from ref_logits."""
    m = oracle.Model(path, arch=arch, max_ctx=max_ctx, acc=oracle.ACC_F32_REV)
    if literal is not None:
        m.set_program_semantics(literal)
    prompt = np.asarray(prompt, np.int32)
    _, lg = m.forward(prompt, 0)
    for step in range(len(ref_toks) - 1):
        _, lg = m.forward(np.array([ref_toks[step]], np.int32), len(prompt) + step)
    m.close()
    r = np.asarray(ref_logits, np.float64).ravel()
    return float(np.linalg.norm(np.asarray(lg, np.float64).ravel() - r) / np.linalg.norm(r))


def ulp_diff(a, b):
    ai = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    bi = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


# ---------------------------------------------------------------------------
# dequantisation (bit-exact)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qt,gen,shape", [(Q4_0, S.q4_0_blocks, (2048, 2048)),
                                          (Q8_0, S.q8_0_blocks, (256, 5632)),
                                          (Q4_0, S.q4_0_blocks, (3, 32))])
def test_dequant_bit_exact(dev, oracle, qt, gen, shape):
    blocks = gen(1, "W", *shape)
    w = dev.quantized(blocks, shape, qt)
    assert np.array_equal(w.numpy(), blocks), "packed round trip"
    got = w.dequantize().numpy().view(np.uint16)
    ref = oracle.dequant(blocks, 2 if qt == Q4_0 else 8).view(np.uint16).reshape(shape)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("shape", [(1, 256), (7, 768), (64, 2048), (1000, 2560)])
def test_dequant_q6_k_bit_exact(dev, oracle, shape):
    """Q6_K super-blocks (gguf.rs:128-212) re-laid out on the device: the
    packed round trip returns the GGUF bytes and the device dequantisation is
    the oracle's, bit for bit."""
    blocks = S.q6_k_blocks(3, f"W6k{shape}", *shape)
    w = dev.quantized(blocks, shape, Q6_K)
    assert np.array_equal(w.numpy(), blocks), "packed round trip"
    got = w.dequantize().numpy().view(np.uint16)
    ref = oracle.dequant(blocks, 14).view(np.uint16).reshape(shape)
    assert np.array_equal(got, ref)


def test_q6_k_extreme_scales(dev, oracle):
    # largest |sc|, both signs, every code, large and subnormal d
    rng = np.random.default_rng(5)
    blocks = S.q6_k_blocks(4, "W6kx", 4, 512, dlo=1e-7, dhi=8.0, smax=128)
    blocks = blocks.reshape(-1, 210)
    blocks[:, :192] = rng.integers(0, 256, (blocks.shape[0], 192), dtype=np.uint8)
    blocks[0, 192:208] = np.array([-128, 127] * 8, np.int8).view(np.uint8)
    blocks = blocks.reshape(-1)
    got = dev.quantized(blocks, (4, 512), Q6_K).dequantize().numpy().view(np.uint16)
    assert np.array_equal(got, oracle.dequant(blocks, 14).view(np.uint16).reshape(4, 512))


def test_dequant_reference_known_answers(dev):
    # gguf.rs:622-718: Q8_0 scale 1 -> 0,1,2; two blocks scale 1/2 -> y[42] = 20;
    # Q4_0 scale 0.5, all nibbles 0xF -> 3.5 everywhere.
    q8 = np.zeros(68, np.uint8)
    q8[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    q8[2:34] = np.arange(32)
    q8[34:36] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    q8[36:68] = np.arange(32)
    y = dev.quantized(q8, (1, 64), Q8_0).dequantize().numpy().astype(np.float32).ravel()
    assert y[0] == 0 and y[1] == 1 and y[2] == 2 and y[10] == 10 and y[32] == 0 and y[42] == 20
    q4 = np.full(18, 0xFF, np.uint8)
    q4[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    y = dev.quantized(q4, (1, 32), Q4_0).dequantize().numpy().astype(np.float32)
    assert np.all(y == 3.5)


# ---------------------------------------------------------------------------
# linear: GEMV (M <= 4) and MFMA GEMM (M > 4)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qt", [Q4_0, Q8_0])
@pytest.mark.parametrize("M,N,K", [(1, 2048, 2048), (1, 5632, 2048), (1, 2048, 5632), (2, 256, 2048),
                                   (3, 512, 1024), (4, 1000, 2048), (1, 37, 64), (1, 2560, 10240),
                                   (1, 2560, 2560), (1, 1030, 2560), (1, 10240, 2560), (1, 32771, 2048)])
def test_linear_quant_gemv(dev, oracle, qt, M, N, K):
    gen = S.q4_0_blocks if qt == Q4_0 else S.q8_0_blocks
    blocks = gen(2, f"W{N}x{K}", N, K)
    x = S.normal_f16(2, f"x{M}x{K}", (M, K))
    w = dev.quantized(blocks, (N, K), qt)
    y = dev.tensor(x).linear(w).numpy()
    ref = oracle.linear_q(x, blocks, 2 if qt == Q4_0 else 8, N)
    assert_close(y, ref, what=f"gemv {qt} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(1, 32000, 2048), (3, 1000, 2560), (4, 512, 5632), (2, 77, 256),
                                   (20, 300, 768)])
def test_linear_q6_k(dev, oracle, M, N, K):
    """Q6_K weights: the fused dequant-GEMV for M <= 4, the dequantised f16
    copy through the MFMA GEMM above; fp32 accumulation of the reference's
    f16 weights either way."""
    blocks = S.q6_k_blocks(6, f"W6k{N}x{K}", N, K)
    x = S.normal_f16(6, f"x6k{M}x{K}", (M, K))
    w = dev.quantized(blocks, (N, K), Q6_K)
    y = dev.tensor(x).linear(w).numpy()
    ref = oracle.linear_q(x, blocks, 14, N)
    assert_close(y, ref, what=f"q6_k linear {M}x{N}x{K}")


def test_linear_q6_k_copy_follows_upload(dev, oracle):
    """The f16 copy a Q6_K weight keeps for the GEMM (M > 4) is made once,
    gives the same bits on the next call, and is replaced when the weight's
    contents are uploaded again."""
    M, N, K = 12, 200, 512
    b1 = S.q6_k_blocks(8, "W6c1", N, K)
    b2 = S.q6_k_blocks(8, "W6c2", N, K)
    x = S.normal_f16(8, "x6c", (M, K))
    w = dev.quantized(b1, (N, K), Q6_K)
    tx = dev.tensor(x)
    y1 = tx.linear(w).numpy()
    assert np.array_equal(tx.linear(w).numpy().view(np.uint16), y1.view(np.uint16))
    assert_close(y1, oracle.linear_q(x, b1, 14, N), what="q6_k first contents")
    from tensorlogic_amd._lib import call
    import ctypes as C
    bb = np.ascontiguousarray(b2)
    call("tlhip_tensor_upload", dev.h, w.h, bb.ctypes.data_as(C.c_void_p), bb.nbytes)
    assert_close(tx.linear(w).numpy(), oracle.linear_q(x, b2, 14, N), what="q6_k after re-upload")


@pytest.mark.parametrize("qt", [Q4_0, Q8_0, F16])
@pytest.mark.parametrize("M,N,K", [(46, 5632, 2048), (5, 64, 64), (64, 256, 512), (130, 96, 2048),
                                   (512, 512, 2048), (33, 100, 96), (17, 2048, 5632), (64, 130, 160),
                                   (8, 40, 32), (512, 2048, 5632), (200, 384, 1024), (65, 256, 128),
                                   # config 2's remaining cells: M = 46 on W_down, M = 512 on W_up/gate
                                   (46, 2048, 5632), (512, 5632, 2048),
                                   # skinny path (M <= 64, K % 64 == 0): ragged N, one to four
                                   # 16-row M tiles, K parts of unequal length; up to 128 tiles of
                                   # 32 rows also split K over workgroups (2 to 5 slices here)
                                   (7, 77, 256), (20, 300, 768), (63, 1000, 384), (5, 2048, 2048),
                                   (48, 2560, 2048), (33, 11264, 2048), (9, 500, 320), (12, 640, 1472),
                                   (64, 4096, 2048)])
def test_linear_gemm(dev, oracle, qt, M, N, K):
    x = S.normal_f16(3, f"x{M}x{K}", (M, K))
    if qt == F16:
        wh = S.normal_f16(3, f"W{N}x{K}", (N, K), 0.0, 0.05)
        w = dev.tensor(wh)
        ref = oracle.linear(x, wh)
    else:
        gen = S.q4_0_blocks if qt == Q4_0 else S.q8_0_blocks
        blocks = gen(3, f"W{N}x{K}", N, K)
        w = dev.quantized(blocks, (N, K), qt)
        ref = oracle.linear_q(x, blocks, 2 if qt == Q4_0 else 8, N)
    y = dev.tensor(x).linear(w).numpy()
    assert_close(y, ref, what=f"gemm {qt} {M}x{N}x{K}")


@pytest.mark.parametrize("qt,M,N,K", [(Q8_0, 46, 5632, 2048), (Q4_0, 512, 2048, 5632), (F16, 33, 256, 4096),
                                      (Q4_0, 46, 2048, 5632), (F16, 12, 640, 1472)])
def test_gemm_split_k_deterministic(dev, oracle, qt, M, N, K):
    """Split-K GEMMs sum their fp32 slices in slice order: repeated calls
    give identical bits (no order depends on scheduling).  The skinny
    GEMM's split (the last workgroup of a tile to arrive adds the slices)
    also resets its arrival counters: every repeat is correct."""
    x = S.normal_f16(7, f"xs{M}x{K}", (M, K))
    if qt == F16:
        wh = S.normal_f16(7, f"Ws{N}x{K}", (N, K), 0.0, 0.05)
        w = dev.tensor(wh)
        ref = oracle.linear(x, wh)
    else:
        gen = S.q4_0_blocks if qt == Q4_0 else S.q8_0_blocks
        blocks = gen(7, f"Ws{N}x{K}", N, K)
        w = dev.quantized(blocks, (N, K), qt)
        ref = oracle.linear_q(x, blocks, 2 if qt == Q4_0 else 8, N)
    tx = dev.tensor(x)
    outs = [tx.linear(w).numpy() for _ in range(5)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint16), outs[0].view(np.uint16))
    assert_close(outs[0], ref, what=f"split-K gemm {qt} {M}x{N}x{K}")


def test_linear_bias_and_f16_odd_shapes(dev, oracle):
    # src/ops/tests.rs:248-377 uses a rectangular [50, 122] case
    x = S.normal_f16(4, "x", (3, 50))
    w = S.normal_f16(4, "w", (122, 50), 0.0, 0.2)
    b = S.normal_f16(4, "b", (122,))
    for M in (1, 3):
        got = dev.tensor(x[:M]).linear(dev.tensor(w), dev.tensor(b)).numpy()
        assert_close(got, oracle.linear(x[:M], w, b), what=f"f16 linear M={M}")


@pytest.mark.parametrize("qt", [Q4_0, Q8_0, F16])
@pytest.mark.parametrize("N,K", [(37, 96), (1025, 2048), (300, 5632), (2, 32), (1030, 5632), (2560, 2560), (1030, 2560),
                                 (32771, 2048)])
def test_linear_one_row_bias(dev, oracle, qt, N, K):
    """One activation row with a bias: the compact M = 1 GEMV (rows per wave
    1 or 2, blocks past the row read as zero weights: K = 96 and 5632 leave
    lanes without a block, K = 32 all but one); from 1024 rows the
    epilogue-specialised instantiations, two rows per wave at K = 2048 (Q4_0
    from 32768 rows: four, the last wave with three rows) and one at
    K = 5632 (three 64-block passes), with idle waves in the last workgroup
    at N = 1030."""
    x = S.normal_f16(9, f"x1b{K}", (1, K))
    b = S.normal_f16(9, f"b1b{N}", (N,))
    if qt == F16:
        wh = S.normal_f16(9, f"W1b{N}x{K}", (N, K), 0.0, 0.05)
        w = dev.tensor(wh)
        ref = oracle.linear(x, wh, b)
    else:
        gen = S.q4_0_blocks if qt == Q4_0 else S.q8_0_blocks
        blocks = gen(9, f"W1b{N}x{K}", N, K)
        w = dev.quantized(blocks, (N, K), qt)
        ref = oracle.linear_q(x, blocks, 2 if qt == Q4_0 else 8, N, b)
    got = dev.tensor(x).linear(w, dev.tensor(b)).numpy()
    assert_close(got, ref, what=f"one-row linear + bias {qt} {N}x{K}")


@pytest.mark.parametrize("M,N,K,with_bias", [(1, 64, 64, False), (3, 100, 37, True), (46, 256, 2048, True),
                                             (130, 96, 200, False), (64, 65, 33, True), (1, 2048, 5632, False)])
def test_linear_f32(dev, oracle, M, N, K, with_bias):
    """linear() on TensorF32 operands: the reference f32 kernel's fused sums
    in k order and the separate bias add, bit for bit."""
    from tensorlogic_amd import F32
    rng = np.random.default_rng(M * 7 + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if with_bias else None
    got = dev.tensor(x, F32).linear(dev.tensor(w, F32), dev.tensor(b, F32) if with_bias else None).numpy()
    want = oracle.linear_f32(x, w, b)
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_linear_f32_dtype_mix_is_an_error(dev):
    from tensorlogic_amd import F32
    x32 = dev.tensor(np.ones((2, 32), np.float32), F32)
    with pytest.raises(TLHipError) as e:
        x32.linear(dev.tensor(np.ones((4, 32), np.float16)))
    assert e.value.kind == "DtypeError"
    with pytest.raises(TLHipError) as e:
        x32.linear(dev.tensor(np.ones((4, 31), np.float32), F32))
    assert e.value.kind == "InvalidOperation"


def test_kvcache_f32(dev):
    """KVCache::new_f32: set / append / get_k / get_v on f32 rows, bit for
    bit; an f16 row is refused, and so is attention over the f32 cache."""
    from tensorlogic_amd import F32
    c = KVCache(dev, 2, 16, 2, 8, dtype=F32)
    rng = np.random.default_rng(3)
    k0, v0 = rng.standard_normal((5, 2, 8)).astype(np.float32), rng.standard_normal((5, 2, 8)).astype(np.float32)
    k1, v1 = rng.standard_normal((2, 2, 8)).astype(np.float32), rng.standard_normal((2, 2, 8)).astype(np.float32)
    c.set(1, dev.tensor(k0, F32), dev.tensor(v0, F32))
    c.append(1, dev.tensor(k1, F32), dev.tensor(v1, F32))
    gk, gv = c.get_k(1).numpy(), c.get_v(1).numpy()
    assert gk.dtype == np.float32 and gk.shape == (7, 2, 8)
    assert np.array_equal(gk, np.concatenate([k0, k1])) and np.array_equal(gv, np.concatenate([v0, v1]))
    with pytest.raises(TLHipError) as e:
        c.append(1, dev.tensor(k1), dev.tensor(v1))
    assert e.value.kind == "DtypeError"
    with pytest.raises(TLHipError) as e:
        c.attention(dev.tensor(rng.standard_normal((1, 4, 8)).astype(np.float32), F32), 1, 0.35)
    assert e.value.kind == "DtypeError"


def test_matmul_known_answer(dev):
    # tests/test_gpu_operations.rs:81-94: [[1,2],[3,4]] @ [[5,6],[7,8]]
    a = dev.tensor(np.array([[1, 2], [3, 4]], np.float16))
    b = dev.tensor(np.array([[5, 6], [7, 8]], np.float16))
    assert a.matmul(b).numpy().astype(np.float32).tolist() == [[19, 22], [43, 50]]


@pytest.mark.parametrize("M,K,N", [(33, 65, 130), (1, 64, 33), (5, 32, 1), (46, 2048, 5632), (512, 2048, 2048),
                                   (7, 100, 31)])
def test_matmul_oracle(dev, oracle, M, K, N):
    """matmul(a, b) = a[M,K] @ b[K,N] (matmul.rs:22-60, builtin_math.rs:36-60)
    at shapes that cross the transpose's 32 x 32 tiles with ragged edges, and
    at the config-2 / prefill shapes.  Two checks: the oracle's fp32-
    accumulated product of a and b^T (the rel-L2 / max-abs bars), and
    integer-valued operands in {-1, 0, 1}, whose products and sums are exact
    in fp32 and in f16 (|sum| <= K <= 2048), so the result must equal numpy's
    integer product bit for bit -- a transposed or shifted element of b fails
    it whatever the summation order."""
    a = S.normal_f16(31, f"mma{M}x{K}", (M, K))
    b = S.normal_f16(31, f"mmb{K}x{N}", (K, N))
    y = dev.tensor(a).matmul(dev.tensor(b)).numpy()
    assert y.shape == (M, N)
    ref = oracle.linear(a, np.ascontiguousarray(b.T))
    assert_close(y, ref, what=f"matmul {M}x{K} @ {K}x{N}")
    rng = np.random.default_rng(M * 7 + K * 3 + N)
    ai = rng.integers(-1, 2, (M, K)).astype(np.int64)
    bi = rng.integers(-1, 2, (K, N)).astype(np.int64)
    yi = dev.tensor(ai.astype(np.float16)).matmul(dev.tensor(bi.astype(np.float16))).numpy()
    assert np.array_equal(yi.astype(np.int64), ai @ bi)


@pytest.mark.parametrize("M,K,N", [(33, 65, 130), (46, 2048, 300), (1, 7, 5)])
def test_matmul_f32(dev, oracle, M, K, N):
    """matmul on TensorF32 operands (builtin_math.rs:55-58): every output is
    the k-ordered fused sum of matmul_tiled_32x32_f32 / matmul_tiled_f32 /
    matmul_f32 (unified.metal:337-500; zero padding adds nothing), i.e. the
    oracle's f32 linear of a and b^T, bit for bit."""
    from tensorlogic_amd import F32
    rng = np.random.default_rng(M + 3 * K + 5 * N)
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    got = dev.tensor(a, F32).matmul(dev.tensor(b, F32)).numpy()
    want = oracle.linear_f32(a, np.ascontiguousarray(b.T))
    assert got.dtype == np.float32 and got.shape == (M, N)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(TLHipError) as e:
        dev.tensor(a, F32).matmul(dev.tensor(b.astype(np.float16)))
    assert e.value.kind == "DtypeError"


def test_matmul_shape_errors(dev):
    """matmul.rs:27-42: rank != 2 and an inner-dimension mismatch are both
    InvalidOperation."""
    a = dev.tensor(np.zeros((2, 3), np.float16))
    with pytest.raises(TLHipError) as e:
        a.matmul(dev.tensor(np.zeros((4, 5), np.float16)))
    assert e.value.kind == "InvalidOperation"
    with pytest.raises(TLHipError) as e:
        a.matmul(dev.tensor(np.zeros((3,), np.float16)))
    assert e.value.kind == "InvalidOperation"


def test_linear_shape_errors(dev):
    x = dev.tensor(np.zeros((2, 64), np.float16))
    w = dev.tensor(np.zeros((8, 32), np.float16))
    with pytest.raises(TLHipError) as e:
        x.linear(w)
    assert e.value.kind == "InvalidOperation"


# ---------------------------------------------------------------------------
# normalisation, RoPE, softmax, elementwise
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,n", [(1, 2048), (46, 2048), (34, 2048), (3, 4), (5, 2560), (3, 24), (2, 6144),
                                    (1, 8192), (2, 8200), (2048, 2048)])
def test_rms_norm(dev, oracle, rows, n):
    x = S.normal_f16(5, "x", (rows, n))
    w = S.normal_f16(5, "w", (n,), 1.0, 0.02)
    got = dev.tensor(x).rms_norm([n], dev.tensor(w), 1e-5).numpy()
    ref = oracle.rms_norm(x, w, 1e-5)
    assert ulp_diff(got, ref).max() <= 1
    assert_close(got, ref)


def test_rms_norm_known_answer(dev):
    # tests/test_gpu_operations.rs:184-205: [1,2,3,4] / sqrt(7.5)
    x = dev.tensor(np.array([[1, 2, 3, 4]], np.float16))
    got = x.rms_norm([4], dev.tensor(np.ones(4, np.float16)), 1e-6).numpy().astype(np.float32).ravel()
    assert np.allclose(got, np.array([1, 2, 3, 4]) / np.sqrt(7.5), atol=1e-3)


@pytest.mark.parametrize("rows,n", [(7, 2560), (46, 2048), (2, 24), (3, 100), (2, 8192), (1, 9000)])
def test_layer_norm(dev, oracle, rows, n):
    x = S.normal_f16(6, "x", (rows, n), 0.3, 2.0)
    w = S.normal_f16(6, "w", (n,), 1.0, 0.1)
    b = S.normal_f16(6, "b", (n,), 0.0, 0.1)
    got = dev.tensor(x).layer_norm(dev.tensor(w), dev.tensor(b), 1e-5).numpy()
    ref = oracle.layer_norm(x, w, b, 1e-5)
    assert ulp_diff(got, ref).max() <= 1
    assert_close(got, ref)


@pytest.mark.parametrize("S_,H,D,off,layout,rot", [
    (3, 2, 8, 0, ROPE_INTERLEAVED, 0),       # test_shader_mathematical_correctness.rs:66-101
    (46, 32, 64, 0, ROPE_INTERLEAVED, 0), (1, 32, 64, 34, ROPE_INTERLEAVED, 0),
    (2048, 4, 64, 0, ROPE_NEOX, 0), (5, 32, 80, 511, ROPE_NEOX, 32),
    # config 3 at S = 2048: Q [2048, 32, 64] in both layouts, K [2048, 4, 64]
    (2048, 32, 64, 0, ROPE_INTERLEAVED, 0), (2048, 32, 64, 0, ROPE_NEOX, 0), (2048, 4, 64, 0, ROPE_INTERLEAVED, 0)])
def test_rope(dev, oracle, S_, H, D, off, layout, rot):
    if (S_, H, D) == (3, 2, 8):
        x = np.sin(0.1 * np.arange(S_ * H * D)).astype(np.float16).reshape(S_, H, D)
    else:
        x = S.normal_f16(7, "x", (S_, H, D))
    got = dev.tensor(x).rope(off, 10000.0, layout, rot).numpy()
    ref = oracle.rope(x, off, 10000.0, layout, rot)
    # cos/sin come from the same table formula; the rotation is rounded the same way
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("rows,n", [(1, 3), (32, 46), (4, 2048), (2, 32000)])
def test_softmax(dev, oracle, rows, n):
    x = S.normal_f16(8, "x", (rows, n), 0.0, 3.0)
    got = dev.tensor(x).softmax().numpy()
    ref = oracle.softmax(x)
    assert ulp_diff(got, ref).max() <= 1
    assert np.allclose(got.astype(np.float32).sum(-1), 1.0, atol=2e-2)


def test_softmax_known_answer_and_masked(dev):
    got = dev.tensor(np.array([[1, 2, 3]], np.float16)).softmax().numpy().astype(np.float32)
    assert np.allclose(got, [[0.0900, 0.2446, 0.6650]], atol=1e-3)
    x = np.array([[np.inf, -np.inf, np.nan]], np.float16)   # degenerate row -> uniform
    got = dev.tensor(x).softmax().numpy().astype(np.float32)
    assert np.allclose(got, 1 / 3, atol=1e-3)


def test_elementwise(dev, oracle):
    x = S.normal_f16(9, "x", (4, 5632), 0.0, 4.0)
    u = S.normal_f16(9, "u", (4, 5632))
    tx, tu = dev.tensor(x), dev.tensor(u)
    for got, ref in ((tx.sigmoid(), oracle.sigmoid(x)), (tx.silu(), oracle.silu(x)),
                     (tx.gelu(), oracle.gelu(x)), (tx.silu_mul(tu), oracle.swiglu(x, u))):
        assert ulp_diff(got.numpy(), ref).max() <= 1
    for got, ref in ((tx + tu, oracle.add(x, u)), (tx * tu, oracle.mul(x, u)),
                     (tx * 0.125, oracle.mul_scalar(x, 0.125))):
        assert np.array_equal(got.numpy().view(np.uint16), ref.view(np.uint16))
    # sigma(0) = 0.5 (src/ops/tests.rs:640-659)
    assert float(dev.tensor(np.zeros(4, np.float16)).sigmoid().numpy()[0]) == 0.5


def test_mask_and_einsums(dev, oracle):
    Sq, H, Hkv, D = 9, 4, 2, 16
    q = S.normal_f16(10, "q", (Sq, H, D))
    k = S.normal_f16(10, "k", (Sq, Hkv, D))
    v = S.normal_f16(10, "v", (Sq, Hkv, D))
    sc = einsum("ihd,jhd->ihj", dev.tensor(q), dev.tensor(k)) * 0.25
    mask = np.tril(np.ones((Sq, Sq), np.float16))
    p = sc.apply_attention_mask(dev.tensor(mask)).softmax()
    out = einsum("ihj,jhd->ihd", p, dev.tensor(v)).numpy()
    ref = oracle.attention(q, k, v, 0, 0.25, True)
    assert_close(out, ref, what="einsum attention")
    fused = attention(dev.tensor(q), dev.tensor(k), dev.tensor(v), 0, 0.25, True).numpy()
    assert_close(fused, ref, what="fused attention")


@pytest.mark.parametrize("I,J,H,Hkv,D", [(1, 190, 32, 32, 64), (1, 47, 32, 4, 64), (46, 46, 32, 4, 64),
                                         (1, 300, 32, 32, 80), (3, 257, 8, 2, 128), (2, 1, 4, 4, 64),
                                         (5, 700, 4, 1, 80)])
def test_einsums_head_dims(dev, oracle, I, J, H, Hkv, D):
    """The program's two einsums (einsum.rs:653-886, unified.metal:2524-2684)
    at the head dims the 8-lanes-per-row kernels take (64 / 80 / 128), with
    and without GQA, key counts that leave partial key groups and passes
    (J = 1, 47, 257, 700), against the oracle's restatement of each."""
    q = S.normal_f16(17, f"eq{I}{H}{D}", (I, H, D))
    k = S.normal_f16(17, f"ek{J}{Hkv}{D}", (J, Hkv, D))
    v = S.normal_f16(17, f"ev{J}{Hkv}{D}", (J, Hkv, D))
    sc = einsum("ihd,jhd->ihj", dev.tensor(q), dev.tensor(k)).numpy()
    assert sc.shape == (I, H, J)
    assert_close(sc, oracle.einsum_scores(q, k), what=f"einsum scores {I}x{J} H{H}/{Hkv} D{D}")
    rng = np.random.default_rng(I * 31 + J)
    p = rng.random((I, H, J)).astype(np.float32)
    p = (p / p.sum(-1, keepdims=True)).astype(np.float16)
    out = einsum("ihj,jhd->ihd", dev.tensor(p), dev.tensor(v)).numpy()
    assert out.shape == (I, H, D)
    assert_close(out, oracle.einsum_context(p, v), what=f"einsum context {I}x{J} H{H}/{Hkv} D{D}")


# S < 128 runs the one-workgroup-per-row kernels; S >= 128 the matrix-core
# prefill kernels (two q-tiles per head pair of waves under causal masking,
# key halves split between the waves, transposed V): the staged one (K / V
# tiles copied to LDS once per workgroup) when the GQA group is a multiple
# of the workgroup's 4 heads (2 at head_dim 128), the direct one otherwise.
@pytest.mark.parametrize("Sq,J,H,Hkv,D,q0,causal", [
    (1, 174, 32, 4, 64, 173, True), (46, 46, 32, 4, 64, 0, True), (1, 768, 32, 32, 80, 767, True),
    (31, 31, 4, 4, 64, 0, True), (64, 100, 8, 8, 80, 36, True), (97, 97, 8, 2, 128, 0, True),
    (45, 77, 8, 4, 64, 0, False),
    (128, 128, 4, 4, 64, 0, True), (300, 300, 8, 4, 64, 0, True), (2048, 2048, 4, 1, 64, 0, True),
    (512, 512, 4, 4, 80, 0, True), (160, 200, 8, 8, 80, 40, True), (129, 129, 5, 1, 128, 0, True),
    (200, 200, 6, 3, 64, 0, True), (128, 300, 4, 4, 80, 0, False), (250, 90, 4, 2, 128, 0, False),
    # single-row kernels for other head dims around their 256 / 512-key passes
    (1, 100, 8, 8, 80, 99, True), (1, 300, 4, 4, 80, 299, True), (1, 513, 4, 2, 128, 512, True),
    (3, 600, 4, 2, 80, 597, True), (2, 1100, 4, 4, 80, 0, False),
    # config 3 at its head layout: 32 query / 4 KV heads (GQA group 8), D = 64
    (2048, 2048, 32, 4, 64, 0, True), (1, 2048, 32, 4, 64, 2047, True), (256, 1024, 32, 4, 64, 768, True),
    # one row over 1025..2048 keys: 256-key chunks and the combine kernel
    (1, 1025, 4, 4, 80, 1024, True), (1, 1500, 8, 2, 128, 1499, True), (1, 1999, 32, 4, 64, 0, False),
    # staged kernel at head dims 80 and 128, ragged key counts, odd tile counts
    (300, 300, 8, 2, 80, 0, True), (200, 150, 8, 2, 80, 0, False), (129, 129, 4, 2, 128, 0, True),
    (256, 333, 8, 2, 128, 77, True), (160, 1000, 8, 1, 64, 840, True)])
def test_attention(dev, oracle, Sq, J, H, Hkv, D, q0, causal):
    q = S.normal_f16(11, "q", (Sq, H, D))
    k = S.normal_f16(11, "k", (J, Hkv, D))
    v = S.normal_f16(11, "v", (J, Hkv, D))
    got = attention(dev.tensor(q), dev.tensor(k), dev.tensor(v), q0, 1 / np.sqrt(D), causal).numpy()
    ref = oracle.attention(q, k, v, q0, 1 / np.sqrt(D), causal)
    assert_close(got, ref, what=f"attention S={Sq} J={J} D={D} causal={causal}")


@pytest.mark.parametrize("Sq,J,H,Hkv,D,causal", [
    # one row past the one-workgroup kernels' 8,192-key score row: key-chunked split
    (1, 8193, 8, 2, 64, True), (1, 10000, 32, 4, 64, True), (1, 9000, 4, 4, 80, False), (1, 12345, 8, 2, 128, True),
    # several rows: the matrix-core path, which has no key cap of its own
    (2, 8200, 8, 2, 64, True), (46, 10000, 32, 4, 64, True), (130, 9000, 8, 8, 80, True), (5, 8500, 4, 2, 128, False)])
def test_attention_past_8192_keys(dev, oracle, Sq, J, H, Hkv, D, causal):
    """Context beyond 8,192 keys (the reference materialises its scores and
    has no cap): queries at the last Sq positions of J keys."""
    q = S.normal_f16(31, f"lq{J}", (Sq, H, D))
    k = S.normal_f16(31, f"lk{J}", (J, Hkv, D))
    v = S.normal_f16(31, f"lv{J}", (J, Hkv, D))
    q0 = J - Sq
    got = attention(dev.tensor(q), dev.tensor(k), dev.tensor(v), q0, 1 / np.sqrt(D), causal).numpy()
    ref = oracle.attention(q, k, v, q0, 1 / np.sqrt(D), causal)
    assert_close(got, ref, what=f"attention S={Sq} J={J} D={D} causal={causal}")


def test_kvcache_past_8192_keys(dev, oracle):
    """A KV cache of 9,000 rows: decode rows appended past 8,192 keys attend
    the whole cache through the key-chunked path."""
    H, Hkv, D = 8, 2, 64
    c = KVCache(dev, 1, 9000, Hkv, D)
    k0, v0 = S.normal_f16(33, "xk0", (8990, Hkv, D)), S.normal_f16(33, "xv0", (8990, Hkv, D))
    c.set(0, dev.tensor(k0), dev.tensor(v0))
    ks, vs = [k0], [v0]
    scale = 1 / np.sqrt(D)
    for t in range(2):
        k1, v1 = S.normal_f16(34 + t, "xk", (1, Hkv, D)), S.normal_f16(34 + t, "xv", (1, Hkv, D))
        q1 = S.normal_f16(34 + t, "xq", (1, H, D))
        c.append(0, dev.tensor(k1), dev.tensor(v1))
        ks.append(k1)
        vs.append(v1)
        kk, vv = np.concatenate(ks), np.concatenate(vs)
        got = c.attention(dev.tensor(q1), 0, scale).numpy()
        assert_close(got, oracle.attention(q1, kk, vv, kk.shape[0] - 1, scale, True), what=f"long cache decode {t}")


def test_attention_key_count_limit(dev):
    """More keys than any entry point reads, and a head dim the long-row paths
    do not cover, are shape errors (no silent truncation)."""
    q = dev.tensor(np.zeros((1, 2, 64), np.float16))
    kv = dev.empty((65537, 1, 64))
    with pytest.raises(TLHipError) as e:
        attention(q, kv, kv, 65536)
    assert e.value.kind == "InvalidDimension"
    q96 = dev.tensor(np.zeros((1, 2, 96), np.float16))
    kv96 = dev.empty((9000, 1, 96))
    with pytest.raises(TLHipError) as e:
        attention(q96, kv96, kv96, 8999)
    assert e.value.kind == "InvalidDimension"


@pytest.mark.parametrize("Sq,H", [(8, 4), (64, 4), (160, 4), (160, 8), (300, 8)])
def test_attention_degenerate_rows(dev, oracle, Sq, H):
    """Rows whose every score overflows f16 take the reference softmax's
    uniform 1/J weights (non-causal, so no -10000 masked scores exist);
    S >= 128 with 8 heads on 2 KV heads runs the staged matrix-core kernel."""
    Hkv, D, J = 2, 64, 40
    q = S.normal_f16(12, "q", (Sq, H, D))
    q[::3] = np.float16(120.0)
    k = np.abs(S.normal_f16(12, "k", (J, Hkv, D))) + np.float16(100.0)
    v = S.normal_f16(12, "v", (J, Hkv, D))
    got = attention(dev.tensor(q), dev.tensor(k), dev.tensor(v), 0, 0.125, False).numpy()
    ref = oracle.attention(q, k, v, 0, 0.125, False)
    assert np.isfinite(got).all()
    assert_close(got, ref, what=f"degenerate attention S={Sq}")


def test_embedding_and_argmax(dev, oracle):
    table = S.normal_f16(12, "t", (320, 64), 0.0, 0.02)
    ids = S.token_ids(12, "ids", 46, 320)
    got = embedding(dev.tensor(table), ids).numpy()
    assert np.array_equal(got, oracle.embedding(table, ids))
    with pytest.raises(TLHipError) as e:
        embedding(dev.tensor(table), [320])
    assert e.value.kind == "IndexOutOfBounds"
    # quantized table rows are dequantised bit-exactly
    blocks = S.q4_0_blocks(12, "tq", 320, 64)
    got = embedding(dev.quantized(blocks, (320, 64), Q4_0), ids).numpy()
    assert np.array_equal(got, oracle.dequant(blocks, 2).reshape(320, 64)[ids])
    blocks = S.q6_k_blocks(12, "tq6", 320, 512)
    got = embedding(dev.quantized(blocks, (320, 512), Q6_K), ids).numpy()
    assert np.array_equal(got, oracle.dequant(blocks, 14).reshape(320, 512)[ids])
    # last-max tie-break (builtin_sampling.rs:170-176)
    logits = np.zeros(32000, np.float16)
    logits[[5, 17, 31000]] = 3.0
    assert temperature_sample(dev.tensor(logits), 0.0) == 31000 == oracle.argmax_last(logits)
    lg = S.normal_f16(12, "lg", (3, 32000))
    assert temperature_sample(dev.tensor(lg), 0.0) == oracle.argmax_last(lg[-1])


def _sample_ok(logits, T, r, tok, delta=2e-5):
    """tok is the inverse-CDF pick of r under softmax(x / T) up to f32
    rounding of the running sum: r lies in [cdf[tok-1], cdf[tok]) widened
    by delta (cdf in float64)."""
    x = logits.astype(np.float64) / np.float64(np.float32(T))
    p = np.exp(x - x.max())
    cdf = np.cumsum(p / p.sum())
    lo = cdf[tok - 1] if tok > 0 else 0.0
    return lo - delta <= r < cdf[tok] + delta or (tok == len(cdf) - 1 and r >= cdf[-1] - delta)


@pytest.mark.parametrize("V,T", [(3, 1.0), (1000, 0.8), (32000, 0.8), (51200, 1.5), (32000, 0.05)])
def test_temperature_sample(dev, oracle, V, T):
    """temperature_sample with T > 1e-4 (builtin_sampling.rs:178-215) for the
    draws splitmix64(seed, counter): the oracle's index for the same draw,
    or a neighbour only where the draw sits on a CDF step within f32
    rounding of the running sum."""
    lg = S.normal_f16(13, f"lg{V}", (2, V), 0.0, 3.0)
    t = dev.tensor(lg)
    exact = 0
    n = 60
    for c in range(n):
        r = oracle.sample_uniform(5, c)
        got = temperature_sample(t, T, seed=5, counter=c)
        ref = oracle.sample_temperature(lg[-1], T, r)
        exact += got == ref
        assert got == ref or _sample_ok(lg[-1], T, r, got), f"V={V} T={T} counter={c}: {got} vs {ref}"
    # the f32 running sums (index order in the oracle, slice order on the
    # device) differ by rounding: only draws on a step of the CDF may differ
    assert exact >= 0.8 * n
    assert temperature_sample(t, 1e-5, seed=5) == oracle.argmax_last(lg[-1])


def test_temperature_sample_distribution(dev):
    lg = np.array([0.0, 1.0, 2.0, -1.0, 0.5] * 10, np.float16)
    t = dev.tensor(lg)
    n = 3000
    toks = np.array([temperature_sample(t, 0.7, seed=9, counter=c) for c in range(n)])
    x = lg.astype(np.float64) / np.float64(np.float32(0.7))
    p = np.exp(x - x.max())
    p /= p.sum()
    freq = np.bincount(toks, minlength=lg.size) / n
    # binomial spread: 5 sigma of the largest cell
    assert np.abs(freq - p).max() < 5 * np.sqrt(p.max() * (1 - p.max()) / n)


@pytest.mark.parametrize("H,Hkv,D", [(32, 4, 64), (4, 4, 80)])
def test_kvcache_attention(dev, oracle, H, Hkv, D):
    """The TL cache flow: set a 46-row prompt, attend it (prefill), append one
    row at a time and attend each (decode); every output equals the oracle's
    attention of the same queries at positions len - S .. len - 1."""
    c = KVCache(dev, 1, 64, Hkv, D)
    k0, v0 = S.normal_f16(14, "ck0", (46, Hkv, D)), S.normal_f16(14, "cv0", (46, Hkv, D))
    q0 = S.normal_f16(14, "cq0", (46, H, D))
    c.set(0, dev.tensor(k0), dev.tensor(v0))
    scale = 1 / np.sqrt(D)
    got = c.attention(dev.tensor(q0), 0, scale).numpy()
    assert_close(got, oracle.attention(q0, k0, v0, 0, scale, True), what="cache prefill")
    ks, vs = [k0], [v0]
    for t in range(3):
        k1, v1 = S.normal_f16(15 + t, "ck", (1, Hkv, D)), S.normal_f16(15 + t, "cv", (1, Hkv, D))
        q1 = S.normal_f16(15 + t, "cq", (1, H, D))
        c.append(0, dev.tensor(k1), dev.tensor(v1))
        ks.append(k1)
        vs.append(v1)
        got = c.attention(dev.tensor(q1), 0, scale).numpy()
        kk, vv = np.concatenate(ks), np.concatenate(vs)
        assert_close(got, oracle.attention(q1, kk, vv, kk.shape[0] - 1, scale, True), what=f"cache decode {t}")
    with pytest.raises(TLHipError) as e:   # more query rows than the cache holds
        c.attention(dev.tensor(S.normal_f16(16, "cqx", (60, H, D))), 0, scale)
    assert e.value.kind == "InvalidDimension"


@pytest.mark.parametrize("H,Hkv,D", [(32, 32, 80), (8, 2, 128), (32, 4, 64)])
def test_kvcache_attention_long(dev, oracle, H, Hkv, D):
    """A cache filled in two prompt chunks of 300 rows (the second chunk's
    causal prefill attends from q_pos0 = 300 through the matrix-core kernel),
    then decode rows past 600 keys: for head dims 80 and 128 the one-row
    kernel takes several 256 / 512-key passes with the key count known on the
    host.  Every output equals the oracle's attention at the same positions."""
    c = KVCache(dev, 1, 640, Hkv, D)
    scale = 1 / np.sqrt(D)
    ks, vs = [], []
    for chunk in range(2):
        k0 = S.normal_f16(60 + chunk, "lk", (300, Hkv, D))
        v0 = S.normal_f16(60 + chunk, "lv", (300, Hkv, D))
        q0 = S.normal_f16(60 + chunk, "lq", (300, H, D))
        c.append(0, dev.tensor(k0), dev.tensor(v0))
        ks.append(k0)
        vs.append(v0)
        kk, vv = np.concatenate(ks), np.concatenate(vs)
        got = c.attention(dev.tensor(q0), 0, scale).numpy()
        assert_close(got, oracle.attention(q0, kk, vv, 300 * chunk, scale, True), what=f"chunk {chunk}")
    for t in range(3):
        k1, v1 = S.normal_f16(70 + t, "lk1", (1, Hkv, D)), S.normal_f16(70 + t, "lv1", (1, Hkv, D))
        q1 = S.normal_f16(70 + t, "lq1", (1, H, D))
        c.append(0, dev.tensor(k1), dev.tensor(v1))
        ks.append(k1)
        vs.append(v1)
        kk, vv = np.concatenate(ks), np.concatenate(vs)
        got = c.attention(dev.tensor(q1), 0, scale).numpy()
        assert_close(got, oracle.attention(q1, kk, vv, kk.shape[0] - 1, scale, True), what=f"decode {t}")


def test_kvcache(dev):
    c = KVCache(dev, 2, 16, 4, 8)
    k1, v1 = S.normal_f16(13, "k1", (5, 4, 8)), S.normal_f16(13, "v1", (5, 4, 8))
    k2, v2 = S.normal_f16(13, "k2", (1, 4, 8)), S.normal_f16(13, "v2", (1, 4, 8))
    c.set(1, dev.tensor(k1), dev.tensor(v1))
    c.append(1, dev.tensor(k2), dev.tensor(v2))
    assert c.len(1) == 6 and c.len(0) == 0
    assert np.array_equal(c.get_k(1).numpy(), np.concatenate([k1, k2]))
    assert np.array_equal(c.get_v(1).numpy(), np.concatenate([v1, v2]))
    with pytest.raises(TLHipError):
        c.append(1, dev.tensor(np.zeros((11, 4, 8), np.float16)), dev.tensor(np.zeros((11, 4, 8), np.float16)))
    # V with K's element count but another layout is refused, and nothing is written
    with pytest.raises(TLHipError) as e:
        c.append(1, dev.tensor(k2), dev.tensor(v2.reshape(1, 8, 4)))
    assert e.value.kind == "ShapeMismatch" and c.len(1) == 6


def test_kvcache_limits(dev):
    # a cache longer than attention can read (65,536 keys) is refused at creation
    with pytest.raises(TLHipError) as e:
        KVCache(dev, 1, 65537, 1, 64)
    assert e.value.kind == "InvalidDimension"
    KVCache(dev, 1, 65536, 1, 64)
