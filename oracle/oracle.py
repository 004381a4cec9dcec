"""ctypes wrapper over oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the parity checker or as the timed CPU baseline.  The product
(tensorlogic_amd/, libtlhip.so) never imports it.

Arrays are numpy: f16 tensors are np.float16, ids np.int32, packed GGUF blocks
np.uint8.  Each wrapper names the tl_oracle.h function it calls; the reference
file:line each one restates is given there.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
ACC_F32, ACC_F16, ACC_F32_REV = 0, 1, 2   # ACC_F32_REV: fp32 sums in descending order
ROPE_INTERLEAVED, ROPE_NEOX = 0, 1

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_u16p = C.POINTER(C.c_uint16)
_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)


def _declare(L):
    sz, i, f, vp = C.c_size_t, C.c_int, C.c_float, C.c_void_p
    sig = {
        "tlo_gguf_open": (vp, [C.c_char_p]),
        "tlo_gguf_close": (None, [vp]),
        "tlo_gguf_n_tensors": (i, [vp]),
        "tlo_gguf_tensor_name": (C.c_char_p, [vp, i]),
        "tlo_gguf_tensor": (vp, [vp, C.c_char_p, C.POINTER(i), C.POINTER(i), C.POINTER(C.c_int64),
                                 C.POINTER(sz)]),
        "tlo_gguf_kv_u32": (i, [vp, C.c_char_p, C.POINTER(C.c_uint32)]),
        "tlo_gguf_kv_f32": (i, [vp, C.c_char_p, C.POINTER(C.c_float)]),
        "tlo_einsum_scores": (None, [vp, vp, i, i, i, i, i, vp]),
        "tlo_einsum_context": (None, [vp, vp, i, i, i, i, i, i, vp]),
        "tlo_apply_attention_mask": (None, [vp, vp, sz, vp]),
        "tlo_set_threads": (i, [i]),
        "tlo_h2f": (f, [C.c_uint16]),
        "tlo_f2h": (C.c_uint16, [f]),
        "tlo_h2f_array": (None, [vp, vp, sz]),
        "tlo_f2h_array": (None, [vp, vp, sz]),
        "tlo_dequant_q4_0": (None, [vp, sz, vp]),
        "tlo_dequant_q8_0": (None, [vp, sz, vp]),
        "tlo_dequant_q6_k": (None, [vp, sz, vp]),
        "tlo_linear_f16": (None, [vp, vp, vp, i, i, i, i, vp]),
        "tlo_linear_q": (None, [vp, vp, i, vp, i, i, i, i, vp]),
        "tlo_rms_norm": (None, [vp, vp, i, i, f, vp]),
        "tlo_layer_norm": (None, [vp, vp, vp, i, i, f, vp]),
        "tlo_rope": (None, [vp, i, i, i, i, f, i, i, vp]),
        "tlo_rope_table": (None, [i, i, f, vp]),
        "tlo_softmax": (None, [vp, i, i, vp]),
        "tlo_sigmoid": (None, [vp, sz, vp]),
        "tlo_silu": (None, [vp, sz, vp]),
        "tlo_add": (None, [vp, vp, sz, vp]),
        "tlo_mul": (None, [vp, vp, sz, vp]),
        "tlo_mul_scalar": (None, [vp, f, sz, vp]),
        "tlo_swiglu": (None, [vp, vp, sz, vp]),
        "tlo_gelu": (None, [vp, sz, vp]),
        "tlo_attention": (None, [vp, vp, vp, i, i, i, i, i, i, f, i, i, vp]),
        "tlo_embedding": (i, [vp, i, i, vp, i, vp]),
        "tlo_causal_mask": (None, [i, vp]),
        "tlo_slice_last": (i, [vp, vp, i, i, i, vp]),
        "tlo_linear_f32": (None, [vp, vp, vp, i, i, i, vp]),
        "tlo_rms_norm_f32": (None, [vp, vp, i, i, f, vp]),
        "tlo_softmax_f32": (None, [vp, i, i, vp]),
        "tlo_rope_f32": (None, [vp, i, i, i, i, f, i, i, vp]),
        "tlo_sigmoid_f32": (None, [vp, sz, vp]),
        "tlo_einsum_scores_f32": (None, [vp, vp, i, i, i, i, i, vp]),
        "tlo_einsum_context_f32": (None, [vp, vp, i, i, i, i, i, vp]),
        "tlo_layer_norm_f32": (None, [vp, vp, vp, i, i, f, vp]),
        "tlo_gelu_f32": (None, [vp, sz, vp]),
        "tlo_silu_f32": (None, [vp, sz, vp]),
        "tlo_swiglu_f32": (None, [vp, vp, sz, vp]),
        "tlo_tensor_argmax": (C.c_int64, [vp, vp, i, i, vp]),
        "tlo_broadcast_to": (i, [vp, vp, i, vp, i, i, vp]),
        "tlo_rope_cos_sin": (i, [vp, i, i, i, vp, vp, i, vp]),
        "tlo_precompute_rope": (None, [i, i, f, i, vp]),
        "tlo_argmax_last": (i, [vp, i]),
        "tlo_sample_temperature": (i, [vp, i, C.c_float, C.c_float]),
        "tlo_sample_uniform": (C.c_float, [C.c_uint64, C.c_uint64]),
        "tlo_model_load": (vp, [C.c_char_p, i, i, i, i]),
        "tlo_model_free": (None, [vp]),
        "tlo_model_generate": (i, [vp, vp, i, i, vp, vp, vp]),
        "tlo_model_forward": (i, [vp, vp, i, i, vp, vp]),
        "tlo_model_reset": (None, [vp]),
        "tlo_model_set_program_semantics": (i, [vp, i]),
        "tlo_model_vocab": (i, [vp]),
        "tlo_model_hidden": (i, [vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _h(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16)


def h2f(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().tlo_h2f_array(_p(bits), _p(out), bits.size)
    return out


def f2h(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().tlo_f2h_array(_p(x), _p(out), x.size)
    return out


def set_threads(n: int) -> int:
    """OpenMP threads for the oracle's loops (n <= 0: unchanged); returns the
    count in force."""
    return lib().tlo_set_threads(n)


def dequant(blocks: np.ndarray, gtype: int) -> np.ndarray:
    """GGUF blocks (gtype 2 = Q4_0, 8 = Q8_0, 14 = Q6_K) -> f16 values."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    bb, per = {2: (18, 32), 8: (34, 32), 14: (210, 256)}[gtype]
    nb = blocks.size // bb
    out = np.empty(nb * per, np.float16)
    fn = {2: lib().tlo_dequant_q4_0, 8: lib().tlo_dequant_q8_0, 14: lib().tlo_dequant_q6_k}[gtype]
    fn(_p(blocks), nb, _p(out))
    return out


def linear(x, w, bias=None, acc=ACC_F32) -> np.ndarray:
    x, w = _h(x), _h(w)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float16)
    lib().tlo_linear_f16(_p(x), _p(w), _p(_h(bias)) if bias is not None else None, M, N, K, acc, _p(y))
    return y


def linear_f32(x, w, bias=None) -> np.ndarray:
    """linear() on f32 operands: the reference f32 kernel's fused sums."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    M, K = x.shape
    N = w.shape[0]
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    y = np.empty((M, N), np.float32)
    lib().tlo_linear_f32(_p(x), _p(w), _p(b) if b is not None else None, M, N, K, _p(y))
    return y


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rms_norm_f32(x, w, eps=1e-6) -> np.ndarray:
    """rms_norm on f32 operands (tlo_rms_norm_f32: the reference f32
    kernels' summation order)."""
    x, w = _f(x), _f(w)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().tlo_rms_norm_f32(_p(x), _p(w), x.size // n, n, eps, _p(y))
    return y


def softmax_f32(x) -> np.ndarray:
    x = _f(x)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().tlo_softmax_f32(_p(x), x.size // n, n, _p(y))
    return y


def rope_f32(x, offset=0, theta=10000.0, layout=0, rot_dims=0) -> np.ndarray:
    x = _f(x)
    S, H, D = x.shape[-3], x.shape[-2], x.shape[-1]
    lead = x.size // (S * H * D)
    y = np.empty_like(x)
    xf, yf = x.reshape(lead, S, H, D), y.reshape(lead, S, H, D)
    for i in range(lead):
        lib().tlo_rope_f32(_p(np.ascontiguousarray(xf[i])), S, H, D, offset, theta, layout, rot_dims, _p(yf[i]))
    return y


def sigmoid_f32(x) -> np.ndarray:
    x = _f(x)
    y = np.empty_like(x)
    lib().tlo_sigmoid_f32(_p(x), x.size, _p(y))
    return y


def layer_norm_f32(x, w=None, b=None, eps=1e-5) -> np.ndarray:
    """layer_norm on f32 operands (tlo_layer_norm_f32: per-row sums in
    element order)."""
    x = _f(x)
    n = x.shape[-1]
    wf = _f(w) if w is not None else None
    bf = _f(b) if b is not None else None
    y = np.empty_like(x)
    lib().tlo_layer_norm_f32(_p(x), _p(wf) if wf is not None else None, _p(bf) if bf is not None else None,
                             x.size // n, n, eps, _p(y))
    return y


def _unary_f32(fn, x) -> np.ndarray:
    x = _f(x)
    y = np.empty_like(x)
    getattr(lib(), fn)(_p(x), x.size, _p(y))
    return y


def gelu_f32(x) -> np.ndarray:
    return _unary_f32("tlo_gelu_f32", x)


def silu_f32(x) -> np.ndarray:
    return _unary_f32("tlo_silu_f32", x)


def swiglu_f32(g, u) -> np.ndarray:
    g, u = _f(g), _f(u)
    y = np.empty_like(g)
    lib().tlo_swiglu_f32(_p(g), _p(u), g.size, _p(y))
    return y


def add_f32(a, b) -> np.ndarray:
    """add_f32 / mul_f32 / mul_scalar_f32 (unified.metal:934-992): one IEEE
    f32 operation per element (numpy's float32 arithmetic rounds the same);
    b may be a row repeated over a's last dim."""
    return (_f(a) + _f(b)).astype(np.float32)


def mul_f32(a, b) -> np.ndarray:
    return (_f(a) * _f(b)).astype(np.float32)


def mul_scalar_f32(a, s) -> np.ndarray:
    return (_f(a) * np.float32(s)).astype(np.float32)


def apply_attention_mask_f32(scores, mask) -> np.ndarray:
    """apply_attention_mask_f32 (unified.metal:4491-4503): mask == 0 gives
    -10000; a [I, J] mask applies to every head of [I, H, J] scores."""
    sc, m = _f(scores), _f(mask)
    if m.ndim == 2 and sc.ndim == 3:
        m = m[:, None, :]
    return np.where(m == 0.0, np.float32(-10000.0), sc).astype(np.float32)


def einsum_scores_f32(q, k) -> np.ndarray:
    q, k = _f(q), _f(k)
    I, H, D = q.shape
    J, Hkv, _ = k.shape
    out = np.empty((I, H, J), np.float32)
    lib().tlo_einsum_scores_f32(_p(q), _p(k), I, J, H, Hkv, D, _p(out))
    return out


def einsum_context_f32(p, v) -> np.ndarray:
    p, v = _f(p), _f(v)
    I, H, J = p.shape
    _, Hkv, D = v.shape
    out = np.empty((I, H, D), np.float32)
    lib().tlo_einsum_context_f32(_p(p), _p(v), I, J, H, Hkv, D, _p(out))
    return out


def linear_q(x, blocks, gtype, N, bias=None, acc=ACC_F32) -> np.ndarray:
    x = _h(x)
    M, K = x.shape
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty((M, N), np.float16)
    lib().tlo_linear_q(_p(x), _p(blocks), gtype, _p(_h(bias)) if bias is not None else None,
                       M, N, K, acc, _p(y))
    return y


def rms_norm(x, w, eps=1e-6) -> np.ndarray:
    x, w = _h(x), _h(w)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().tlo_rms_norm(_p(x), _p(w), x.size // n, n, eps, _p(y))
    return y


def layer_norm(x, w, b, eps=1e-5) -> np.ndarray:
    x = _h(x)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().tlo_layer_norm(_p(x), _p(_h(w)) if w is not None else None,
                         _p(_h(b)) if b is not None else None, x.size // n, n, eps, _p(y))
    return y


def rope(x, offset=0, theta=10000.0, layout=ROPE_INTERLEAVED, rot_dims=0) -> np.ndarray:
    x = _h(x)
    S, H, D = x.shape[-3], x.shape[-2], x.shape[-1]
    lead = x.size // (S * H * D)
    y = np.empty_like(x)
    xf, yf = x.reshape(lead, S, H, D), y.reshape(lead, S, H, D)
    for i in range(lead):
        lib().tlo_rope(_p(np.ascontiguousarray(xf[i])), S, H, D, offset, theta, layout, rot_dims,
                       _p(yf[i]))
    return y


def rope_table(max_pos, rot_dims, theta=10000.0) -> np.ndarray:
    cs = np.empty((max_pos, rot_dims // 2, 2), np.float32)
    lib().tlo_rope_table(max_pos, rot_dims, theta, _p(cs))
    return cs


def softmax(x) -> np.ndarray:
    x = _h(x)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().tlo_softmax(_p(x), x.size // n, n, _p(y))
    return y


def _unary(name, x):
    x = _h(x)
    y = np.empty_like(x)
    getattr(lib(), name)(_p(x), x.size, _p(y))
    return y


def sigmoid(x):
    return _unary("tlo_sigmoid", x)


def silu(x):
    return _unary("tlo_silu", x)


def gelu(x):
    return _unary("tlo_gelu", x)


def _binary(name, a, b):
    a, b = _h(a), _h(b)
    y = np.empty_like(a)
    getattr(lib(), name)(_p(a), _p(b), a.size, _p(y))
    return y


def add(a, b):
    return _binary("tlo_add", a, b)


def mul(a, b):
    return _binary("tlo_mul", a, b)


def swiglu(g, u):
    return _binary("tlo_swiglu", g, u)


def mul_scalar(a, s):
    a = _h(a)
    y = np.empty_like(a)
    lib().tlo_mul_scalar(_p(a), s, a.size, _p(y))
    return y


def attention(q, k, v, q_pos0=0, scale=None, causal=True, acc=ACC_F32) -> np.ndarray:
    q, k, v = _h(q), _h(k), _h(v)
    S, H, D = q.shape
    J, Hkv, _ = k.shape
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    out = np.empty_like(q)
    lib().tlo_attention(_p(q), _p(k), _p(v), S, J, H, Hkv, D, q_pos0, float(scale),
                        int(causal), acc, _p(out))
    return out


def einsum_scores(q, k) -> np.ndarray:
    """einsum("ihd,jhd->ihj", q [I,H,D], k [J,Hkv,D]) with the GQA mapping
    (tlo_einsum_scores)."""
    q, k = _h(q), _h(k)
    I, H, D = q.shape
    J, Hkv, _ = k.shape
    out = np.empty((I, H, J), np.float16)
    lib().tlo_einsum_scores(_p(q), _p(k), I, J, H, Hkv, D, _p(out))
    return out


def einsum_parse(equation: str):
    """parse_einsum_equation / infer_output_spec (einsum.rs:84-128): at most
    one "->", inputs split at ',' and trimmed; without "->" the output is
    every index occurring exactly once, sorted.  Returns (input specs,
    output spec)."""
    parts = equation.split("->")
    if len(parts) > 2:
        raise ValueError("Invalid einsum equation: too many arrows")
    ins = [x.strip() for x in parts[0].split(",")]
    if len(parts) == 2:
        return ins, parts[1].strip()
    counts = {}
    for c in parts[0]:
        if c.isalpha():
            counts[c] = counts.get(c, 0) + 1
    return ins, "".join(sorted(c for c, n in counts.items() if n == 1))


def einsum_general(equation: str, *ops) -> np.ndarray:
    """general_einsum_cpu / sum_over_indices (einsum.rs:207-333) on f16
    operands, vectorised over the output elements: the product starts at f16
    one and multiplies the operands' elements in operand order, each product
    rounded to f16 (the `half` crate computes in f32 and rounds, as numpy's
    float16 arithmetic does); the summed indices nest outermost first, each
    level an f16 running sum from +0 of the inner level's results.  The
    reference nests two or more summed indices in HashSet order (random per
    process); this restatement nests them in order of first appearance, the
    order the library fixes.  A scalar result has shape (1,)."""
    ins, out = einsum_parse(equation)
    ops = [_h(o) for o in ops]
    if len(ins) != len(ops):
        raise ValueError(f"Expected {len(ins)} operands, got {len(ops)}")
    dims, order = {}, []
    for spec, o in zip(ins, ops):
        if len(spec) != o.ndim:
            raise ValueError(f"spec {spec} for a {o.ndim}-d operand")
        for c, d in zip(spec, o.shape):
            if c not in dims:
                dims[c] = d
                order.append(c)
            elif dims[c] != d:
                raise ValueError(f"index {c}: {dims[c]} vs {d}")
    out_dims = [dims[c] for c in out]
    sums = [c for c in order if c not in out]
    coords = {c: g.reshape(-1) for c, g in zip(out, np.indices(out_dims))} if out else {}
    n_out = int(np.prod(out_dims)) if out else 1
    flat = [o.reshape(-1) for o in ops]

    def product(vals):
        prod = np.full(n_out, np.float16(1.0), np.float16)
        for spec, o, f in zip(ins, ops, flat):
            lin = np.zeros(n_out, np.int64)
            for c, d in zip(spec, o.shape):
                lin = lin * d + vals[c]
            prod = (prod * f[lin]).astype(np.float16)
        return prod

    def level(li, vals):
        if li == len(sums):
            return product(vals)
        c = sums[li]
        acc = np.zeros(n_out, np.float16)
        for i in range(dims[c]):
            vals[c] = np.full(n_out, i, np.int64)
            acc = (acc + level(li + 1, vals)).astype(np.float16)
        return acc

    res = level(0, dict(coords))
    return res.reshape(out_dims if out else (1,))


def einsum_context(p, v, acc=ACC_F32) -> np.ndarray:
    """einsum("ihj,jhd->ihd", p [I,H,J], v [J,Hkv,D]) (tlo_einsum_context)."""
    p, v = _h(p), _h(v)
    I, H, J = p.shape
    _, Hkv, D = v.shape
    out = np.empty((I, H, D), np.float16)
    lib().tlo_einsum_context(_p(p), _p(v), I, J, H, Hkv, D, acc, _p(out))
    return out


def apply_attention_mask(scores, mask) -> np.ndarray:
    """apply_attention_mask (tlo_apply_attention_mask): same shapes, as the
    reference requires (masking.rs:36-43)."""
    scores, mask = _h(scores), _h(mask)
    if scores.shape != mask.shape:
        raise ValueError(f"apply_attention_mask: {scores.shape} vs {mask.shape}")
    out = np.empty_like(scores)
    lib().tlo_apply_attention_mask(_p(scores), _p(mask), scores.size, _p(out))
    return out


def embedding(table, ids) -> np.ndarray:
    table = _h(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    V, Hd = table.shape
    out = np.empty((ids.size, Hd), np.float16)
    if lib().tlo_embedding(_p(table), V, Hd, _p(ids), ids.size, _p(out)) != 0:
        raise IndexError("token id out of range")
    return out


def causal_mask(n: int) -> np.ndarray:
    out = np.empty((n, n), np.float16)
    lib().tlo_causal_mask(n, _p(out))
    return out


def _shape_arr(shape) -> np.ndarray:
    return np.ascontiguousarray(shape, dtype=np.int64)


def slice_last(x, axis: int = 0) -> np.ndarray:
    """Raises ValueError where the reference returns InvalidOperation."""
    x = np.ascontiguousarray(x)
    out = np.empty(x.shape[1:] if x.ndim > 1 else (1,), x.dtype)
    shp = _shape_arr(x.shape)
    if lib().tlo_slice_last(_p(x), _p(shp), x.ndim, axis, x.itemsize, _p(out)) != 0:
        raise ValueError(f"slice_last: axis {axis} of a {x.ndim}-D tensor")
    return out


def tensor_argmax(x, dim=None, keepdim=False) -> np.ndarray:
    """Tensor::argmax(dim, keepdim) on an f16 (uint16 bits or float16) or f32
    array: the result tensor the reference builds, in x's dtype (indices
    converted with T::from_f64, so f16 indices above 2048 are rounded).
    Raises ValueError where the reference returns an error."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.uint16:
        x = x.view(np.float16)
    xd = np.ascontiguousarray(x, dtype=np.float64)
    shp = _shape_arr(x.shape)
    n_out = 1 if dim is None else int(np.prod([s for i, s in enumerate(x.shape) if i != dim], dtype=np.int64))
    idx = np.zeros(max(n_out, 1), np.int64)
    got = lib().tlo_tensor_argmax(_p(xd), _p(shp), x.ndim, -1 if dim is None else dim, _p(idx))
    if got < 0:
        raise ValueError(f"argmax: dim {dim} of a {x.ndim}-D tensor (or an empty tensor)")
    if dim is None:
        out_shape = (1,) * x.ndim if keepdim else (1,)
    else:
        out_shape = tuple((1 if i == dim else s) for i, s in enumerate(x.shape) if keepdim or i != dim)
        if not out_shape:
            # Tensor::from_vec(1 value, shape []) fails: a shape without dims
            # has numel 0 (tensor_creation.rs:111-118, shape.rs:28-34)
            raise ValueError("argmax: every dim reduced without keepdim (ShapeMismatch)")
    return idx[:got].astype(np.float64).astype(x.dtype).reshape(out_shape)


def broadcast_to(x, shape) -> np.ndarray:
    """Raises ValueError where the reference returns ShapeMismatch."""
    x = np.ascontiguousarray(x)
    out = np.empty(tuple(shape), x.dtype)
    xs, ts = _shape_arr(x.shape), _shape_arr(shape)
    if lib().tlo_broadcast_to(_p(x), _p(xs), x.ndim, _p(ts), len(shape), x.itemsize, _p(out)) != 0:
        raise ValueError(f"broadcast_to: {x.shape} -> {tuple(shape)}")
    return out


def rope_cos_sin(x, cos_t, sin_t) -> np.ndarray:
    x, cos_t, sin_t = _h(x), _h(cos_t), _h(sin_t)
    S, H, D = x.shape
    y = np.empty_like(x)
    if cos_t.shape != sin_t.shape or cos_t.ndim != 2 or cos_t.shape[1] != D or \
            lib().tlo_rope_cos_sin(_p(x), S, H, D, _p(cos_t), _p(sin_t), cos_t.shape[0], _p(y)) != 0:
        raise ValueError("rope(x, cos, sin): shapes")
    return y


def precompute_rope(head_dim: int, max_seq_len: int, base: float, want_sin: bool) -> np.ndarray:
    out = np.empty((max_seq_len, head_dim), np.float16)
    lib().tlo_precompute_rope(head_dim, max_seq_len, base, int(want_sin), _p(out))
    return out


def argmax_last(logits) -> int:
    logits = _h(logits).reshape(-1)
    return int(lib().tlo_argmax_last(_p(logits), logits.size))


def sample_uniform(seed: int, counter: int) -> float:
    return float(lib().tlo_sample_uniform(seed, counter))


def sample_temperature(logits, temperature: float, r: float) -> int:
    logits = _h(logits).reshape(-1)
    return int(lib().tlo_sample_temperature(_p(logits), logits.size, temperature, r))


class GGUF:
    """The oracle's GGUF reader (tlo_gguf_open, tl_oracle.h): None-checked
    open, tensor table, metadata and each tensor's raw bytes."""

    def __init__(self, path: str):
        self.h = lib().tlo_gguf_open(path.encode())
        if not self.h:
            raise ValueError(f"oracle GGUF reader rejected {path}")

    def close(self):
        if self.h:
            lib().tlo_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def names(self):
        return [lib().tlo_gguf_tensor_name(self.h, i).decode() for i in range(lib().tlo_gguf_n_tensors(self.h))]

    def kv_u32(self, key: str):
        v = C.c_uint32()
        return v.value if lib().tlo_gguf_kv_u32(self.h, key.encode(), C.byref(v)) == 0 else None

    def kv_f32(self, key: str):
        v = C.c_float()
        return v.value if lib().tlo_gguf_kv_f32(self.h, key.encode(), C.byref(v)) == 0 else None

    def tensor(self, name: str):
        """(gguf type, row-major dims, raw bytes) of one tensor."""
        t, nd, nb = C.c_int(), C.c_int(), C.c_size_t()
        dims = (C.c_int64 * 4)()
        p = lib().tlo_gguf_tensor(self.h, name.encode(), C.byref(t), C.byref(nd), dims, C.byref(nb))
        if not p:
            raise KeyError(name)
        return t.value, tuple(dims[i] for i in range(nd.value)), C.string_at(p, nb.value)


class Model:
    """The oracle's decoder (tlo_model_*): arch 0 = llama, 1 = phi2."""

    def __init__(self, path: str, arch: int = 0, max_ctx: int = 1024, acc: int = ACC_F32,
                 n_threads: int = 0):
        self.h = lib().tlo_model_load(path.encode(), arch, max_ctx, acc, n_threads)
        if not self.h:
            raise RuntimeError(f"oracle failed to load {path}")
        self.vocab = lib().tlo_model_vocab(self.h)
        self.hidden = lib().tlo_model_hidden(self.h)

    def close(self):
        if self.h:
            lib().tlo_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def generate(self, prompt, n_decode: int):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        toks = np.empty(n_decode + 1, np.int32)
        margins = np.empty(n_decode + 1, np.float32)
        logits = np.empty(self.vocab, np.float16)
        rc = lib().tlo_model_generate(self.h, _p(prompt), prompt.size, n_decode, _p(toks),
                                      _p(margins), _p(logits))
        if rc:
            raise RuntimeError("oracle generate failed")
        return toks, margins, logits

    def forward(self, ids, pos0: int):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        hid = np.empty((ids.size, self.hidden), np.float16)
        logits = np.empty(self.vocab, np.float16)
        if lib().tlo_model_forward(self.h, _p(ids), ids.size, pos0, _p(hid), _p(logits)):
            raise RuntimeError("oracle forward failed")
        return hid, logits

    def reset(self):
        lib().tlo_model_reset(self.h)

    def set_program_semantics(self, literal: bool):
        """debug/chat_demo_with_kvcache.tl as written (decode rows rotated at
        position 0, rms_norm eps 1e-6) or the default (absolute positions,
        the file's eps); see tlo_model_set_program_semantics."""
        if lib().tlo_model_set_program_semantics(self.h, int(literal)) != 0:
            raise ValueError("program semantics are defined for llama models only")
