"""Host-side mirror of the reference's tensor operator surface over the C ABI.

Names and argument meaning follow the reference's `Tensor<f16>` methods and TL
builtins (`src/ops/*.rs`, `src/interpreter/builtin_*.rs`): `matmul_transposed_b`
/ `linear`, `rms_norm(normalized_shape, weight, eps)`, `rope(position_offset)`,
`softmax()`, `sigmoid()`, `embedding(table, ids)`, `KVCache.set/append/get_k/
get_v`, `temperature_sample(logits, 0)`.  Errors surface as TLHipError with
the reference's TensorError kind (ShapeMismatch, InvalidOperation, ...).

Every operation runs on the device through libtlhip.so; nothing here computes
on the host.
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import F16, F32, I32, Q4_0, Q6_K, Q8_0, ROPE_INTERLEAVED, ROPE_NEOX, TLHipError, call, lib

_vp = C.c_void_p
_BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q6_K: 210}


def _shape_arr(shape):
    return (C.c_int64 * len(shape))(*[int(s) for s in shape])


_NP_DTYPE = {F16: np.float16, F32: np.float32, I32: np.int32}


class Device:
    """One device context: a HIP device plus one stream (MetalDevice::new)."""

    def __init__(self, index: int = 0):
        h = _vp()
        call("tlhip_init", index, C.byref(h))
        self.h = h

    def sync(self):
        call("tlhip_sync", self.h)

    def name(self) -> str:
        buf = C.create_string_buffer(256)
        call("tlhip_device_name", self.h, buf, 256)
        return buf.value.decode()

    def set_sync_every_op(self, on: bool):
        call("tlhip_set_sync_every_op", self.h, int(on))

    def close(self):
        if self.h:
            lib().tlhip_shutdown(self.h)
            self.h = None

    # -- tensor creation ----------------------------------------------------
    def empty(self, shape, dtype: int = F16) -> "Tensor":
        h = _vp()
        call("tlhip_tensor_alloc", self.h, dtype, len(shape), _shape_arr(shape), C.byref(h))
        return Tensor(self, h)

    def tensor(self, arr, dtype: int = F16) -> "Tensor":
        """Tensor::from_vec_gpu: upload an array as F16 (float arrays are
        rounded RNE), F32 or I32."""
        a = np.ascontiguousarray(arr, dtype=_NP_DTYPE[dtype])
        t = self.empty(a.shape if a.ndim else (1,), dtype)
        call("tlhip_tensor_upload", self.h, t.h, a.ctypes.data_as(_vp), a.nbytes)
        return t

    def quantized(self, blocks: np.ndarray, shape, qtype: int) -> "Tensor":
        """A packed Q4_0 / Q8_0 / Q6_K weight [N, K] from GGUF block bytes."""
        b = np.ascontiguousarray(blocks, dtype=np.uint8)
        t = self.empty(shape, qtype)
        call("tlhip_tensor_upload", self.h, t.h, b.ctypes.data_as(_vp), b.nbytes)
        return t


class Tensor:
    def __init__(self, dev: Device, h):
        self.dev = dev
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            try:
                lib().tlhip_tensor_free(self.h)
            except Exception:
                pass
            self.h = None

    # -- metadata -------------------------------------------------------------
    def _info(self):
        dt, nd = C.c_int(), C.c_int()
        shp = (C.c_int64 * 8)()
        call("tlhip_tensor_info", self.h, C.byref(dt), C.byref(nd), shp)
        return dt.value, tuple(shp[i] for i in range(nd.value))

    @property
    def shape(self):
        return self._info()[1]

    @property
    def dtype(self):
        return self._info()[0]

    def numel(self):
        return int(np.prod(self.shape))

    def nbytes(self):
        return int(lib().tlhip_tensor_nbytes(self.h))

    # -- transfer ---------------------------------------------------------------
    def numpy(self) -> np.ndarray:
        """sync_and_read: f16 array, or GGUF block bytes for Q types."""
        dt, shape = self._info()
        if dt in _BLOCK_BYTES:
            out = np.empty(self.nbytes(), np.uint8)
        else:
            out = np.empty(shape, _NP_DTYPE[dt])
        call("tlhip_tensor_download", self.dev.h, self.h, out.ctypes.data_as(_vp), out.nbytes)
        return out

    def reshape(self, shape) -> "Tensor":
        h = _vp()
        call("tlhip_tensor_reshape", self.h, len(shape), _shape_arr(shape), C.byref(h))
        return Tensor(self.dev, h)

    # -- ops --------------------------------------------------------------------
    def _new(self, shape):
        return self.dev.empty(shape)

    def _like(self, shape):
        """An output in this tensor's float type (the ops with a TensorF32 arm)."""
        return self.dev.empty(shape, F32 if self.dtype == F32 else F16)

    def dequantize(self) -> "Tensor":
        out = self._new(self.shape)
        call("tlhip_dequantize", self.dev.h, self.h, out.h)
        return out

    def matmul_transposed_b(self, w: "Tensor") -> "Tensor":
        """self[M,K] @ w[N,K]^T (matmul.rs:241-311)."""
        return self.linear(w)

    def linear(self, w: "Tensor", bias: "Tensor | None" = None) -> "Tensor":
        """linear(x, W[, b]) (builtin_math.rs:76-175): f16 (W f16 or quantized)
        or, all operands F32, the TensorF32 arm; the output has x's dtype."""
        M = self.shape[0] if len(self.shape) == 2 else -1
        N = w.shape[0]
        out = self.dev.empty((max(M, 0), N) if M >= 0 else (1, N), F32 if self.dtype == F32 else F16)
        call("tlhip_linear", self.dev.h, self.h, w.h, bias.h if bias is not None else None, out.h)
        return out

    def matmul(self, b: "Tensor") -> "Tensor":
        """matmul(a, b) (builtin_math.rs:36-60, matmul.rs:22-60): a[M,K] @ b[K,N],
        both f16 or both f32; the output has a's dtype."""
        two_d = len(self.shape) == 2 and len(b.shape) == 2
        # (other ranks: the library refuses them with InvalidOperation)
        out = self.dev.empty((self.shape[0], b.shape[1]) if two_d else (1, 1), F32 if self.dtype == F32 else F16)
        call("tlhip_matmul", self.dev.h, self.h, b.h, out.h)
        return out

    def rms_norm(self, normalized_shape: Sequence[int], weight: "Tensor", eps: float = 1e-6) -> "Tensor":
        """Tensor::rms_norm (normalization.rs:42-89): normalized_shape must be
        the trailing dims and match the weight's shape."""
        dims = list(self.shape)
        ns = list(normalized_shape)
        if len(ns) > len(dims) or dims[len(dims) - len(ns):] != ns:
            raise TLHipError(3, f"normalized_shape {ns} does not match tensor shape {dims}")
        if list(weight.shape) != ns:
            raise TLHipError(1, f"expected {ns}, got {list(weight.shape)}")
        if len(ns) != 1:
            x = self.reshape((self.numel() // int(np.prod(ns)), int(np.prod(ns))))
            w = weight.reshape((int(np.prod(ns)),))
            return x.rms_norm([int(np.prod(ns))], w, eps).reshape(self.shape)
        out = self._like(self.shape)
        call("tlhip_rms_norm", self.dev.h, self.h, weight.h, float(eps), out.h)
        return out

    def layer_norm(self, weight=None, bias=None, eps: float = 1e-5) -> "Tensor":
        out = self._like(self.shape)
        call("tlhip_layer_norm", self.dev.h, self.h, weight.h if weight is not None else None,
             bias.h if bias is not None else None, float(eps), out.h)
        return out

    def rope(self, position_offset: int = 0, theta: float = 10000.0, layout: int = ROPE_INTERLEAVED,
             rot_dims: int = 0) -> "Tensor":
        """Tensor::rope (rope.rs:71-118); layout/theta/rot_dims extend it."""
        out = self._like(self.shape)
        call("tlhip_rope", self.dev.h, self.h, int(position_offset), float(theta), int(layout),
             int(rot_dims), out.h)
        return out

    def softmax(self) -> "Tensor":
        out = self._like(self.shape)
        call("tlhip_softmax_lastdim", self.dev.h, self.h, out.h)
        return out

    def _unary(self, fn):
        out = self._like(self.shape)
        call(fn, self.dev.h, self.h, out.h)
        return out

    def sigmoid(self):
        out = self._like(self.shape)
        call("tlhip_sigmoid", self.dev.h, self.h, out.h)
        return out

    def silu(self):
        return self._unary("tlhip_silu")

    def gelu(self):
        return self._unary("tlhip_gelu")

    def silu_mul(self, up: "Tensor") -> "Tensor":
        out = self._like(self.shape)
        call("tlhip_silu_mul", self.dev.h, self.h, up.h, out.h)
        return out

    def add(self, other: "Tensor") -> "Tensor":
        out = self._like(self.shape)
        call("tlhip_add", self.dev.h, self.h, other.h, out.h)
        return out

    def mul(self, other: "Tensor") -> "Tensor":
        out = self._like(self.shape)
        call("tlhip_mul", self.dev.h, self.h, other.h, out.h)
        return out

    def mul_scalar(self, s: float) -> "Tensor":
        out = self._like(self.shape)
        call("tlhip_mul_scalar", self.dev.h, self.h, float(s), out.h)
        return out

    __add__ = add

    def __mul__(self, other):
        return self.mul_scalar(other) if isinstance(other, (int, float)) else self.mul(other)

    def slice_last(self, axis: int = 0) -> "Tensor":
        """Tensor::slice_last (slice.rs:25-60): last index of axis 0; a 1-D
        tensor gives shape [1] (the reference's scalar)."""
        shape = self.shape
        out = self.dev.empty(shape[1:] if len(shape) > 1 else (1,), self.dtype)
        call("tlhip_slice_last", self.dev.h, self.h, int(axis), out.h)
        return out

    def broadcast_to(self, shape) -> "Tensor":
        """Tensor::broadcast_to (broadcast.rs:11-120)."""
        out = self.dev.empty(tuple(shape), self.dtype)
        call("tlhip_broadcast_to", self.dev.h, self.h, out.h)
        return out

    def rope_candle(self, cos: "Tensor", sin: "Tensor") -> "Tensor":
        """rope(x, cos, sin) = Tensor::rope_candle (rope.rs:18-65)."""
        out = self._new(self.shape)
        call("tlhip_rope_cos_sin", self.dev.h, self.h, cos.h, sin.h, out.h)
        return out

    def apply_attention_mask(self, mask: "Tensor") -> "Tensor":
        out = self._like(self.shape)
        call("tlhip_apply_attention_mask", self.dev.h, self.h, mask.h, out.h)
        return out

    def argmax_last(self) -> int:
        r = C.c_int32()
        call("tlhip_argmax", self.dev.h, self.h, C.byref(r))
        return r.value

    def argmax(self, dim: int | None = None, keepdim: bool = False) -> "int | Tensor":
        """The argmax() builtin (builtin_tensor.rs:1438-1490) over
        Tensor::argmax (reduce.rs:585-668): with neither dim nor keepdim the
        index as an integer, read back from the reference's result tensor
        (so an f16 index above 2048 comes back rounded, as there); otherwise
        the result tensor in this tensor's dtype."""
        shape = self.shape
        if dim is None:
            out_shape = (1,) * len(shape) if keepdim else (1,)
        else:
            out_shape = tuple(1 if i == dim else s for i, s in enumerate(shape) if keepdim or i != dim) or (1,)
        out = self.dev.empty(out_shape, self.dtype)
        call("tlhip_tensor_argmax", self.dev.h, self.h, -1 if dim is None else int(dim), int(bool(keepdim)), out.h)
        if dim is None and not keepdim:
            return int(out.numpy().astype(np.float64)[0])
        return out


def einsum(eq: str, *ops: Tensor) -> Tensor:
    """einsum(equation, tensors...) (eval.rs:3264-3318, einsum.rs:39-82):
    the attention equations through their kernels, any other equation as
    the reference's general f16 einsum; a scalar result has shape (1,)."""
    if not ops:
        raise TLHipError(3, "einsum requires at least one tensor")
    arr = (C.c_void_p * len(ops))(*[t.h for t in ops])
    nd = C.c_int()
    shp = (C.c_int64 * 8)()
    call("tlhip_einsum_shape", eq.encode(), arr, len(ops), C.byref(nd), shp)
    out = ops[0]._like(tuple(shp[i] for i in range(nd.value)))
    call("tlhip_einsum", ops[0].dev.h, eq.encode(), arr, len(ops), out.h)
    return out


def attention(q: Tensor, k: Tensor, v: Tensor, q_pos0: int = 0, scale: float | None = None,
              causal: bool = True, out: Tensor | None = None) -> Tensor:
    if scale is None:
        scale = 1.0 / np.sqrt(q.shape[2])
    if out is None:
        out = q.dev.empty(q.shape)
    call("tlhip_attention", q.dev.h, q.h, k.h, v.h, int(q_pos0), float(scale), int(causal), out.h)
    return out


def causal_mask(dev: Device, n: int) -> Tensor:
    """causal_mask(n) (builtin_nn.rs:423-460): [n, n], 1 where j <= i."""
    out = dev.empty((n, n))
    call("tlhip_causal_mask", dev.h, out.h)
    return out


def precompute_rope_cos(dev: Device, head_dim: int, max_seq_len: int, base: float = 10000.0) -> Tensor:
    """precompute_rope_cos (builtin_tensor.rs:610-700): [max_seq_len, head_dim] f16."""
    out = dev.empty((max_seq_len, head_dim))
    call("tlhip_precompute_rope", dev.h, int(head_dim), int(max_seq_len), float(base), 0, out.h)
    return out


def precompute_rope_sin(dev: Device, head_dim: int, max_seq_len: int, base: float = 10000.0) -> Tensor:
    """precompute_rope_sin (builtin_tensor.rs:610-700): [max_seq_len, head_dim] f16."""
    out = dev.empty((max_seq_len, head_dim))
    call("tlhip_precompute_rope", dev.h, int(head_dim), int(max_seq_len), float(base), 1, out.h)
    return out


def embedding(table: Tensor, ids) -> Tensor:
    ids = np.ascontiguousarray(np.atleast_1d(ids), dtype=np.int32)
    out = table.dev.empty((ids.size, table.shape[1]), F32 if table.dtype == F32 else F16)
    call("tlhip_embedding", table.dev.h, table.h, ids.ctypes.data_as(C.POINTER(C.c_int32)), ids.size, out.h)
    return out


def temperature_sample(logits: Tensor, temperature: float, seed: int = 0, counter: int = 0) -> int:
    """temperature_sample(logits, T) (builtin_sampling.rs:66-231): greedy for
    T <= 1e-4, else the inverse-CDF draw of softmax(x / T) for the uniform
    value splitmix64(seed, counter) (the reference's thread_rng is unseeded)."""
    if temperature <= 1e-4:
        return logits.argmax_last()
    out = C.c_int32()
    call("tlhip_temperature_sample", logits.dev.h, logits.h, float(temperature), int(seed), int(counter),
         C.byref(out))
    return out.value


class KVCache:
    """KVCache::new_f16 (or, dtype F32, KVCache::new_f32) with a
    preallocated device buffer per layer."""

    def __init__(self, dev: Device, n_layers: int, max_ctx: int, n_kv_heads: int, head_dim: int,
                 dtype: int = F16):
        self.dev = dev
        h = _vp()
        fn = "tlhip_kvcache_create_f32" if dtype == F32 else "tlhip_kvcache_create"
        call(fn, dev.h, n_layers, max_ctx, n_kv_heads, head_dim, C.byref(h))
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib().tlhip_kvcache_free(self.h)
            self.h = None

    def set(self, layer: int, k: Tensor, v: Tensor):
        call("tlhip_kvcache_set", self.dev.h, self.h, layer, k.h, v.h)

    def append(self, layer: int, k: Tensor, v: Tensor):
        call("tlhip_kvcache_append", self.dev.h, self.h, layer, k.h, v.h)

    def _get(self, layer, which):
        h = _vp()
        call("tlhip_kvcache_get", self.h, layer, which, C.byref(h))
        return Tensor(self.dev, h)

    def get_k(self, layer: int) -> Tensor:
        return self._get(layer, 0)

    def get_v(self, layer: int) -> Tensor:
        return self._get(layer, 1)

    def len(self, layer: int) -> int:
        return lib().tlhip_kvcache_len(self.h, layer)

    def attention(self, q: Tensor, layer: int, scale: float) -> Tensor:
        """Causal attention of q [S, H, D] -- the queries of the layer's last S
        positions -- against the cached K/V (get_k/get_v + the einsum /
        mask / softmax sequence); S = 1 is the decode step."""
        out = self.dev.empty(q.shape)
        fn = "tlhip_attention_decode" if q.shape[0] == 1 else "tlhip_attention_prefill"
        call(fn, self.dev.h, q.h, self.h, int(layer), float(scale), out.h)
        return out


class GGUF:
    def __init__(self, path: str):
        h = _vp()
        call("tlhip_gguf_open", path.encode(), C.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tlhip_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def names(self):
        n = lib().tlhip_gguf_n_tensors(self.h)
        return [lib().tlhip_gguf_tensor_name(self.h, i).decode() for i in range(n)]

    def load_tensor(self, dev: Device, name: str) -> Tensor:
        h = _vp()
        call("tlhip_gguf_load_tensor", dev.h, self.h, name.encode(), C.byref(h))
        return Tensor(dev, h)

    def kv_u32(self, key: str) -> int:
        v = C.c_uint32()
        call("tlhip_gguf_kv_u32", self.h, key.encode(), C.byref(v))
        return v.value


class Model:
    """The decoder runner (tlhip_model_*): arch 0 = llama, 1 = phi2."""

    def __init__(self, dev: Device, path: str, arch: int = 0, max_ctx: int = 1024):
        self.dev = dev
        h = _vp()
        call("tlhip_model_load", dev.h, path.encode(), arch, max_ctx, C.byref(h))
        self.h = h
        d = (C.c_int32 * 8)()
        call("tlhip_model_dims", h, d)
        (self.n_layers, self.hidden, self.inter, self.n_heads, self.n_kv, self.head_dim, self.vocab,
         self.rot) = list(d)

    def close(self):
        if getattr(self, "h", None):
            lib().tlhip_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def reset(self):
        call("tlhip_model_reset", self.h)

    def prefill(self, ids) -> int:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        r = C.c_int32()
        call("tlhip_model_prefill", self.h, ids.ctypes.data_as(C.POINTER(C.c_int32)), ids.size, C.byref(r))
        return r.value

    def decode(self, token: int) -> int:
        r = C.c_int32()
        call("tlhip_model_decode", self.h, int(token), C.byref(r))
        return r.value

    def set_sampling(self, temperature: float, seed: int = 0):
        """Token choice of prefill/decode: greedy for T <= 1e-4 (default),
        else temperature_sample with the draw splitmix64(seed, step)."""
        call("tlhip_model_set_sampling", self.h, float(temperature), int(seed))

    def set_program_semantics(self, literal: bool):
        """debug/chat_demo_with_kvcache.tl as written (decode rows rotated as
        position 0, rms_norm eps 1e-6) or the default (absolute positions,
        the file's eps); llama only."""
        call("tlhip_model_set_program_semantics", self.h, int(literal))

    def generate(self, prompt, n_decode: int, use_graph: bool = True) -> np.ndarray:
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_decode + 1, np.int32)
        call("tlhip_model_generate", self.h, prompt.ctypes.data_as(C.POINTER(C.c_int32)), prompt.size, n_decode,
             int(use_graph), out.ctypes.data_as(C.POINTER(C.c_int32)))
        return out

    def logits(self) -> np.ndarray:
        out = np.empty(self.vocab, np.uint16)
        call("tlhip_model_logits", self.h, out.ctypes.data_as(C.POINTER(C.c_uint16)), out.size)
        return out.view(np.float16)

    def bench_decode(self, prompt, n_decode: int, use_graph: bool = True):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_decode + 1, np.int32)
        pm, dm = C.c_float(), C.c_float()
        call("tlhip_bench_decode", self.h, prompt.ctypes.data_as(C.POINTER(C.c_int32)), prompt.size, n_decode,
             int(use_graph), out.ctypes.data_as(C.POINTER(C.c_int32)), C.byref(pm), C.byref(dm))
        return out, pm.value, dm.value


def bench_linear(dev: Device, x: Tensor, ws: Sequence[Tensor], y: Tensor, iters: int,
                 per_launch: bool = False) -> float:
    """Mean us per linear launch (hipEvents): back-to-back throughput, or
    with per_launch every launch bracketed by its own event pair."""
    arr = (_vp * len(ws))(*[w.h for w in ws])
    us = C.c_float()
    call("tlhip_bench_linear", dev.h, x.h, arr, len(ws), y.h, iters, int(per_launch), C.byref(us))
    return us.value


class Timer:
    """hipEvent pair on the device's stream around asynchronous calls:
    ``with Timer(dev) as t: ...`` then ``t.ms``."""

    def __init__(self, dev: Device):
        self.dev, self.ms = dev, None

    def __enter__(self):
        call("tlhip_timer_start", self.dev.h)
        return self

    def __exit__(self, exc_type, exc, tb):
        if exc_type is None:
            ms = C.c_float()
            call("tlhip_timer_stop", self.dev.h, C.byref(ms))
            self.ms = ms.value
        return False


def bench_copy(dev: Device, nbytes: int, n_buf: int, iters: int) -> float:
    """Mean us per back-to-back plain copy of nbytes (cycling n_buf sources)."""
    us = C.c_float()
    call("tlhip_bench_copy", dev.h, nbytes, n_buf, iters, C.byref(us))
    return us.value
