"""tensorlogic_amd -- MI355X (gfx950) backend for TensorLogic's quantized-LLM hot path.

The compute lives in libtlhip.so (HIP kernels + C ABI, include/tl_hip.h);
this package holds the ctypes binding, a host-side mirror of the reference's
tensor operator surface, the GGUF writer/reader and the seeded synthetic
model generator.
"""
from ._lib import F16, F32, I32, Q4_0, Q6_K, Q8_0, ROPE_INTERLEAVED, ROPE_NEOX, TLHipError  # noqa: F401
from .tensor import (GGUF, Device, KVCache, Model, Tensor, Timer, attention, bench_copy, bench_linear,  # noqa: F401
                     causal_mask, einsum, embedding, precompute_rope_cos, precompute_rope_sin, temperature_sample)
from .tokenizer import Tokenizer, chat, tinyllama_chat_prompt  # noqa: F401

__all__ = ["Device", "Tensor", "KVCache", "GGUF", "Model", "TLHipError", "einsum", "attention",
           "embedding", "temperature_sample", "causal_mask", "precompute_rope_cos", "precompute_rope_sin", "bench_linear", "bench_copy", "Timer", "F16", "F32", "I32", "Q4_0", "Q8_0", "Q6_K",
           "ROPE_INTERLEAVED", "ROPE_NEOX", "Tokenizer", "chat", "tinyllama_chat_prompt"]
