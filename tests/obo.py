"""ctypes binding of tests/libobo_driver.so (tests/obo_driver.c): the TL
program debug/chat_demo_with_kvcache.tl run op by op through the C ABI from
C, with no Python between the calls.  Test and benchmark infrastructure."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libobo_driver.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB)
        L.obo_run.restype = C.c_int
        L.obo_run.argtypes = [C.c_char_p, C.POINTER(C.c_int32), C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                              C.c_float, C.c_float, C.POINTER(C.c_int32), C.POINTER(C.c_uint16),
                              C.POINTER(C.c_double)]
        L.obo_error.restype = C.c_char_p
        _lib = L
    return _lib


def run(path: str, prompt, warmup: int, steps: int, max_ctx: int, vocab: int, rope_abs: bool = False,
        eps: float = 1e-6, scale: float = 0.125):
    """Prefill + warmup + steps greedy decode steps from C.  Returns
    (tokens [1 + warmup + steps], last decode logits f16 [vocab],
    prefill ms, ms per timed decode step)."""
    prompt = np.ascontiguousarray(prompt, np.int32)
    toks = np.zeros(1 + warmup + steps, np.int32)
    logits = np.zeros(vocab, np.uint16)
    ms = np.zeros(2, np.float64)
    rc = lib().obo_run(path.encode(), prompt.ctypes.data_as(C.POINTER(C.c_int32)), prompt.size, warmup, steps,
                       max_ctx, int(rope_abs), eps, scale, toks.ctypes.data_as(C.POINTER(C.c_int32)),
                       logits.ctypes.data_as(C.POINTER(C.c_uint16)), ms.ctypes.data_as(C.POINTER(C.c_double)))
    if rc != 0:
        raise RuntimeError(f"obo_run: {lib().obo_error().decode()}")
    return toks, logits.view(np.float16), float(ms[0]), float(ms[1])


def time_legs(S: int = 2048, iters: int = 200):
    """Config 3's rms_norm [S, 2048] and rope [S, 32, 64] / [S, 4, 64] from C:
    us per call of each (hipEvents around back-to-back calls)."""
    L = lib()
    L.obo_time_legs.restype = C.c_int
    L.obo_time_legs.argtypes = [C.c_int, C.c_int, C.POINTER(C.c_double)]
    us = np.zeros(3, np.float64)
    if L.obo_time_legs(S, iters, us.ctypes.data_as(C.POINTER(C.c_double))) != 0:
        raise RuntimeError(f"obo_time_legs: {L.obo_error().decode()}")
    return {"rms_norm_us": float(us[0]), "rope_q_us": float(us[1]), "rope_k_us": float(us[2])}
