"""ctypes binding of libtlhip.so (the C ABI in include/tl_hip.h).

The library is loaded from this package directory (built in-tree by
`python -m tensorlogic_amd.build`).  There is no fallback: if the library is
missing or a call fails, a TLHipError is raised.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtlhip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "tl_hip.h")

F16, F32, I32, Q4_0, Q8_0, Q6_K = 0, 1, 2, 3, 4, 5
ROPE_INTERLEAVED, ROPE_NEOX = 0, 1
STATUS = {0: "OK", 1: "ShapeMismatch", 2: "InvalidDimension", 3: "InvalidOperation",
          4: "AllocationError", 5: "IndexOutOfBounds", 6: "LoadError", 7: "DeviceError",
          8: "DtypeError", 9: "InvalidArgument"}


class TLHipError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(msg)
        self.status = status
        self.kind = STATUS.get(status, "Error")


_vp, _i, _f, _sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t
_i64p = C.POINTER(C.c_int64)
_i32p = C.POINTER(C.c_int32)

# name -> (restype, argtypes); status-returning functions use c_int.
SIGNATURES = {
    "tlhip_last_error": (C.c_char_p, []),
    "tlhip_init": (_i, [_i, C.POINTER(_vp)]),
    "tlhip_shutdown": (_i, [_vp]),
    "tlhip_sync": (_i, [_vp]),
    "tlhip_device_name": (_i, [_vp, C.c_char_p, _sz]),
    "tlhip_set_sync_every_op": (_i, [_vp, _i]),
    "tlhip_tensor_alloc": (_i, [_vp, _i, _i, _i64p, C.POINTER(_vp)]),
    "tlhip_tensor_upload": (_i, [_vp, _vp, _vp, _sz]),
    "tlhip_tensor_download": (_i, [_vp, _vp, _vp, _sz]),
    "tlhip_tensor_retain": (_i, [_vp]),
    "tlhip_tensor_free": (_i, [_vp]),
    "tlhip_tensor_info": (_i, [_vp, C.POINTER(_i), C.POINTER(_i), _i64p]),
    "tlhip_tensor_nbytes": (_sz, [_vp]),
    "tlhip_tensor_reshape": (_i, [_vp, _i, _i64p, C.POINTER(_vp)]),
    "tlhip_gguf_open": (_i, [C.c_char_p, C.POINTER(_vp)]),
    "tlhip_gguf_close": (_i, [_vp]),
    "tlhip_gguf_n_tensors": (_i, [_vp]),
    "tlhip_gguf_tensor_name": (C.c_char_p, [_vp, _i]),
    "tlhip_gguf_load_tensor": (_i, [_vp, _vp, C.c_char_p, C.POINTER(_vp)]),
    "tlhip_gguf_kv_u32": (_i, [_vp, C.c_char_p, C.POINTER(C.c_uint32)]),
    "tlhip_gguf_kv_f32": (_i, [_vp, C.c_char_p, C.POINTER(_f)]),
    "tlhip_dequantize": (_i, [_vp, _vp, _vp]),
    "tlhip_linear": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "tlhip_linear_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "tlhip_matmul": (_i, [_vp, _vp, _vp, _vp]),
    "tlhip_rms_norm": (_i, [_vp, _vp, _vp, _f, _vp]),
    "tlhip_layer_norm": (_i, [_vp, _vp, _vp, _vp, _f, _vp]),
    "tlhip_rope": (_i, [_vp, _vp, _i, _f, _i, _i, _vp]),
    "tlhip_softmax_lastdim": (_i, [_vp, _vp, _vp]),
    "tlhip_sigmoid": (_i, [_vp, _vp, _vp]),
    "tlhip_silu": (_i, [_vp, _vp, _vp]),
    "tlhip_silu_mul": (_i, [_vp, _vp, _vp, _vp]),
    "tlhip_gelu": (_i, [_vp, _vp, _vp]),
    "tlhip_add": (_i, [_vp, _vp, _vp, _vp]),
    "tlhip_mul": (_i, [_vp, _vp, _vp, _vp]),
    "tlhip_mul_scalar": (_i, [_vp, _vp, _f, _vp]),
    "tlhip_embedding": (_i, [_vp, _vp, _i32p, _i, _vp]),
    "tlhip_apply_attention_mask": (_i, [_vp, _vp, _vp, _vp]),
    "tlhip_causal_mask": (_i, [_vp, _vp]),
    "tlhip_attention_prefill": (_i, [_vp, _vp, _vp, _i, _f, _vp]),
    "tlhip_attention_decode": (_i, [_vp, _vp, _vp, _i, _f, _vp]),
    "tlhip_slice_last": (_i, [_vp, _vp, _i, _vp]),
    "tlhip_broadcast_to": (_i, [_vp, _vp, _vp]),
    "tlhip_rope_cos_sin": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "tlhip_precompute_rope": (_i, [_vp, _i, _i, _f, _i, _vp]),
    "tlhip_einsum_scores": (_i, [_vp, _vp, _vp, _vp]),
    "tlhip_einsum_context": (_i, [_vp, _vp, _vp, _vp]),
    "tlhip_einsum_shape": (_i, [C.c_char_p, C.POINTER(_vp), _i, C.POINTER(_i), C.POINTER(C.c_int64)]),
    "tlhip_einsum": (_i, [_vp, C.c_char_p, C.POINTER(_vp), _i, _vp]),
    "tlhip_attention": (_i, [_vp, _vp, _vp, _vp, _i, _f, _i, _vp]),
    "tlhip_argmax": (_i, [_vp, _vp, _i32p]),
    "tlhip_tensor_argmax": (_i, [_vp, _vp, _i, _i, _vp]),
    "tlhip_temperature_sample": (_i, [_vp, _vp, _f, C.c_uint64, C.c_uint64, _i32p]),
    "tlhip_kvcache_create": (_i, [_vp, _i, _i, _i, _i, C.POINTER(_vp)]),
    "tlhip_kvcache_create_f32": (_i, [_vp, _i, _i, _i, _i, C.POINTER(_vp)]),
    "tlhip_kvcache_free": (_i, [_vp]),
    "tlhip_kvcache_set": (_i, [_vp, _vp, _i, _vp, _vp]),
    "tlhip_kvcache_append": (_i, [_vp, _vp, _i, _vp, _vp]),
    "tlhip_kvcache_get": (_i, [_vp, _i, _i, C.POINTER(_vp)]),
    "tlhip_kvcache_len": (_i, [_vp, _i]),
    "tlhip_model_load": (_i, [_vp, C.c_char_p, _i, _i, C.POINTER(_vp)]),
    "tlhip_model_free": (_i, [_vp]),
    "tlhip_model_reset": (_i, [_vp]),
    "tlhip_model_prefill": (_i, [_vp, _i32p, _i, _i32p]),
    "tlhip_model_decode": (_i, [_vp, C.c_int32, _i32p]),
    "tlhip_model_generate": (_i, [_vp, _i32p, _i, _i, _i, _i32p]),
    "tlhip_model_logits": (_i, [_vp, C.POINTER(C.c_uint16), _sz]),
    "tlhip_model_dims": (_i, [_vp, _i32p]),
    "tlhip_model_set_sampling": (_i, [_vp, _f, C.c_uint64]),
    "tlhip_model_set_program_semantics": (_i, [_vp, _i]),
    "tlhip_bench_linear": (_i, [_vp, _vp, C.POINTER(_vp), _i, _vp, _i, _i, C.POINTER(_f)]),
    "tlhip_bench_copy": (_i, [_vp, _sz, _i, _i, C.POINTER(_f)]),
    "tlhip_bench_decode": (_i, [_vp, _i32p, _i, _i, _i, _i32p, C.POINTER(_f), C.POINTER(_f)]),
    "tlhip_timer_start": (_i, [_vp]),
    "tlhip_timer_stop": (_i, [_vp, C.POINTER(_f)]),
}

_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TLHipError(7, f"{LIB_PATH} is missing: run `python -m tensorlogic_amd.build` "
                                "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        msg = lib().tlhip_last_error()
        raise TLHipError(status, msg.decode() if msg else STATUS.get(status, "error"))


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
