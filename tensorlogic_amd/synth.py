"""Seeded synthetic inputs for the benchmark configurations.

One generator, splitmix64 in counter mode, feeds every tensor, so the HIP path
and the CPU oracle see identical bytes (the oracle reads the same GGUF files
or arrays).  A stream is keyed by (seed, tensor name, purpose):

    key      = fnv1a64(f"{seed}:{name}:{purpose}")
    z_i      = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)      i = 0, 1, ...
    mix64(z) = z ^= z >> 30; z *= 0xBF58476D1CE4E5B9;
               z ^= z >> 27; z *= 0x94D049BB133111EB; z ^= z >> 31

Derived draws (all arithmetic in float64 unless stated):
    uniform01_i  = (z_i >> 11) * 2**-53                      in [0, 1)
    f16 U[lo,hi) = f16(f32(lo + (hi - lo) * uniform01_i))     (RNE twice)
    f16 N(m, s)  = f16(f32(m + s * sqrt(-2 ln(1 - u_2i)) * cos(2 pi u_2i+1)))
    bytes        = z_i little-endian, 8 per draw (Q4_0 nibbles: 2 per byte)
    int8 U[-127,127] = ((z_i >> 32) * 255 >> 32) - 127
    token id U[0,V)  = (z_i >> 32) * V >> 32

Q4_0 / Q8_0 matrices are returned as packed GGUF blocks (`gguf.rs:68-112`
layout): per block an f16 scale d, then 16 nibble bytes (Q4_0) or 32 int8
(Q8_0).  Configurations follow the benchmark description: Q4_0 scales in
[1e-3, 2e-2), Q8_0 scales in [1e-3, 1e-2), activations N(0, 1), embeddings
and norms N(0, 0.02) (RMSNorm weights in the attention-block test 1+N(0,0.02)).
"""
from __future__ import annotations

import numpy as np

from .gguf import GGML_F16, GGML_F32, GGML_Q4_0, GGML_Q6_K, GGML_Q8_0, GGUFWriter

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def fnv1a64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def stream_key(seed: int, name: str, purpose: str) -> int:
    return fnv1a64(f"{seed}:{name}:{purpose}")


def splitmix64(key: int, n: int, start: int = 0) -> np.ndarray:
    """z_start .. z_{start+n-1} of the counter-mode stream `key` (uint64)."""
    out = np.empty(n, dtype=np.uint64)
    k = np.uint64(key)
    with np.errstate(over="ignore"):
        for c0 in range(0, n, _CHUNK):
            c1 = min(n, c0 + _CHUNK)
            z = np.arange(start + c0 + 1, start + c1 + 1, dtype=np.uint64)
            z *= _GOLDEN
            z += k
            z ^= z >> np.uint64(30)
            z *= _M1
            z ^= z >> np.uint64(27)
            z *= _M2
            z ^= z >> np.uint64(31)
            out[c0:c1] = z
    return out


def uniform01(key: int, n: int) -> np.ndarray:
    return (splitmix64(key, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def uniform_f16(seed: int, name: str, purpose: str, n: int, lo: float, hi: float) -> np.ndarray:
    u = uniform01(stream_key(seed, name, purpose), n)
    return (lo + (hi - lo) * u).astype(np.float32).astype(np.float16)


def normal_f16(seed: int, name: str, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    u = uniform01(stream_key(seed, name, "normal"), 2 * n)
    u1, u2 = u[0::2], u[1::2]
    z = np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * z).astype(np.float32).astype(np.float16).reshape(shape)


def normal_f32(seed: int, name: str, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """The normal_f16 draw kept in f32 (values generally not f16-representable)."""
    n = int(np.prod(shape))
    u = uniform01(stream_key(seed, name, "normal"), 2 * n)
    u1, u2 = u[0::2], u[1::2]
    z = np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * z).astype(np.float32).reshape(shape)


def random_bytes(seed: int, name: str, purpose: str, nbytes: int) -> np.ndarray:
    z = splitmix64(stream_key(seed, name, purpose), (nbytes + 7) // 8)
    return z.view(np.uint8)[:nbytes]


def token_ids(seed: int, name: str, n: int, vocab: int) -> np.ndarray:
    z = splitmix64(stream_key(seed, name, "ids"), n)
    return (((z >> np.uint64(32)) * np.uint64(vocab)) >> np.uint64(32)).astype(np.int32)


def q4_0_blocks(seed: int, name: str, n: int, k: int, dlo: float = 1e-3, dhi: float = 2e-2,
                zero_mean: bool = False) -> np.ndarray:
    """Packed GGUF Q4_0 blocks (uint8, nblocks*18) for W[n, k].

    Codes are uniform in 0..15 (the benchmark configuration), so the
    dequantised weights (q - 8) * d have mean -d/2.  zero_mean draws codes
    uniform in 1..15 instead ((z >> 32) * 15 >> 32, plus 1; element j of a
    block in the low nibble of byte j, element j + 16 in its high nibble):
    weights symmetric about 0, as a trained model's are, so that a deep stack
    with unit RMSNorm gains does not amplify the activations' common mode."""
    if k % 32:
        raise ValueError("K must be a multiple of 32")
    nb = n * k // 32
    d = uniform_f16(seed, name, "d", nb, dlo, dhi)
    if zero_mean:
        z = splitmix64(stream_key(seed, name, "q15"), nb * 32)
        c = ((((z >> np.uint64(32)) * np.uint64(15)) >> np.uint64(32)) + np.uint64(1)).astype(np.uint8)
        c = c.reshape(nb, 32)
        qs = (c[:, :16] | (c[:, 16:] << np.uint8(4))).astype(np.uint8)
    else:
        qs = random_bytes(seed, name, "q", nb * 16).reshape(nb, 16)
    blk = np.empty((nb, 18), dtype=np.uint8)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = qs
    return blk.reshape(-1)


def q8_0_blocks(seed: int, name: str, n: int, k: int, dlo: float = 1e-3, dhi: float = 1e-2) -> np.ndarray:
    """Packed GGUF Q8_0 blocks (uint8, nblocks*34) for W[n, k]."""
    if k % 32:
        raise ValueError("K must be a multiple of 32")
    nb = n * k // 32
    d = uniform_f16(seed, name, "d", nb, dlo, dhi)
    z = splitmix64(stream_key(seed, name, "q"), nb * 32)
    q = ((((z >> np.uint64(32)) * np.uint64(255)) >> np.uint64(32)).astype(np.int16) - 127).astype(np.int8)
    blk = np.empty((nb, 34), dtype=np.uint8)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = q.view(np.uint8).reshape(nb, 32)
    return blk.reshape(-1)


def q6_k_blocks(seed: int, name: str, n: int, k: int, dlo: float = 2e-5, dhi: float = 1e-4,
                smax: int = 100) -> np.ndarray:
    """Packed GGUF Q6_K super-blocks (uint8, nblocks*210) for W[n, k]:
    ql/qh random bytes, int8 scales uniform in [-smax, smax], f16 d."""
    if k % 256:
        raise ValueError("K must be a multiple of 256")
    nb = n * k // 256
    d = uniform_f16(seed, name, "d", nb, dlo, dhi)
    qlh = random_bytes(seed, name, "q", nb * 192).reshape(nb, 192)
    z = splitmix64(stream_key(seed, name, "sc"), nb * 16)
    sc = ((((z >> np.uint64(32)) * np.uint64(2 * smax + 1)) >> np.uint64(32)).astype(np.int16) - smax).astype(np.int8)
    blk = np.empty((nb, 210), dtype=np.uint8)
    blk[:, 0:192] = qlh
    blk[:, 192:208] = sc.view(np.uint8).reshape(nb, 16)
    blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


# ---------------------------------------------------------------------------
# model files
# ---------------------------------------------------------------------------

# keyword arguments of write_llama_gguf / write_phi2_gguf for the full-size models
TINYLLAMA_ARGS = dict(n_layers=22, hidden=2048, inter=5632, n_heads=32, n_kv=4, vocab=32000)
PHI2_ARGS = dict(n_layers=32, hidden=2560, inter=10240, n_heads=32, vocab=51200, rot=32)


def write_llama_gguf(path: str, seed: int, n_layers: int = 22, hidden: int = 2048,
                     inter: int = 5632, n_heads: int = 32, n_kv: int = 4, vocab: int = 32000,
                     eps: float = 1e-5, theta: float = 10000.0, ctx: int = 2048,
                     qtype: int = GGML_Q4_0, norm_mean: float = 0.0, out_qtype: int | None = None,
                     zero_mean: bool = False) -> None:
    """TinyLlama-architecture decoder with random-init weights.

    Linear weights are Q4_0 (or Q8_0, or unquantised F16 / F32 ~ N(0, 0.02);
    the F32 values are not f16-representable, so loading them exercises
    the RNE rounding to f16), `output.weight` the same unless out_qtype says
    otherwise (GGML_Q6_K, as llama.cpp's Q4_0 checkpoints store it),
    embeddings f16 N(0, 0.02) and RMSNorm weights f16 N(norm_mean, 0.02)
    (the benchmark configuration uses norm_mean 0).  zero_mean draws the
    Q4_0 codes symmetric about 8 (see q4_0_blocks); with it, norm_mean 1
    gives a full-depth model whose logits have real top-2 margins.  Tensor
    names follow llama.cpp/GGUF.
    """
    def float_weights(gtype):
        def gen(sd, name, n, k):
            if gtype == GGML_F16:
                return normal_f16(sd, name, (n, k), 0.0, 0.02)
            return normal_f32(sd, name, (n, k), 0.0, 0.02)
        return gen
    def q4(sd, name, n, k):
        return q4_0_blocks(sd, name, n, k, zero_mean=zero_mean)
    qgen = {GGML_Q4_0: q4, GGML_Q8_0: q8_0_blocks, GGML_F16: float_weights(GGML_F16),
            GGML_F32: float_weights(GGML_F32)}[qtype]
    out_qtype = qtype if out_qtype is None else out_qtype
    ogen = {GGML_Q4_0: q4, GGML_Q8_0: q8_0_blocks, GGML_Q6_K: q6_k_blocks,
            GGML_F16: float_weights(GGML_F16), GGML_F32: float_weights(GGML_F32)}[out_qtype]
    hd = hidden // n_heads
    kvd = n_kv * hd
    w = GGUFWriter()
    w.add_str("general.architecture", "llama")
    for key, v in (("block_count", n_layers), ("embedding_length", hidden),
                   ("feed_forward_length", inter), ("attention.head_count", n_heads),
                   ("attention.head_count_kv", n_kv), ("context_length", ctx),
                   ("rope.dimension_count", hd)):
        w.add_u32(f"llama.{key}", v)
    w.add_f32("llama.attention.layer_norm_rms_epsilon", eps)
    w.add_f32("llama.rope.freq_base", theta)
    w.add_tensor("token_embd.weight", GGML_F16, (vocab, hidden),
                 normal_f16(seed, "token_embd.weight", (vocab, hidden), 0.0, 0.02))
    for i in range(n_layers):
        p = f"blk.{i}."
        w.add_tensor(p + "attn_norm.weight", GGML_F16, (hidden,),
                     normal_f16(seed, p + "attn_norm.weight", (hidden,), norm_mean, 0.02))
        for nm, (n, k) in (("attn_q", (hidden, hidden)), ("attn_k", (kvd, hidden)),
                           ("attn_v", (kvd, hidden)), ("attn_output", (hidden, hidden))):
            w.add_tensor(p + nm + ".weight", qtype, (n, k), qgen(seed, p + nm + ".weight", n, k))
        w.add_tensor(p + "ffn_norm.weight", GGML_F16, (hidden,),
                     normal_f16(seed, p + "ffn_norm.weight", (hidden,), norm_mean, 0.02))
        for nm, (n, k) in (("ffn_gate", (inter, hidden)), ("ffn_up", (inter, hidden)),
                           ("ffn_down", (hidden, inter))):
            w.add_tensor(p + nm + ".weight", qtype, (n, k), qgen(seed, p + nm + ".weight", n, k))
    w.add_tensor("output_norm.weight", GGML_F16, (hidden,),
                 normal_f16(seed, "output_norm.weight", (hidden,), norm_mean, 0.02))
    w.add_tensor("output.weight", out_qtype, (vocab, hidden), ogen(seed, "output.weight", vocab, hidden))
    w.write(path)


def write_phi2_gguf(path: str, seed: int, n_layers: int = 32, hidden: int = 2560,
                    inter: int = 10240, n_heads: int = 32, vocab: int = 51200, rot: int = 32,
                    eps: float = 1e-5, theta: float = 10000.0, ctx: int = 2048,
                    qtype: int = GGML_Q8_0, norm_mean: float = 0.0) -> None:
    """Phi-2-architecture decoder with random-init Q8_0 linear weights.

    Fused QKV projection, LayerNorm with bias, NeoX partial rotary on the first
    `rot` dims, GELU MLP in parallel with attention.  Norm weights, biases and
    embeddings are f16 N(0, 0.02) (LayerNorm weights N(norm_mean, 0.02)).
    Names follow llama.cpp's phi2 tensors.
    """
    qgen = q4_0_blocks if qtype == GGML_Q4_0 else q8_0_blocks
    w = GGUFWriter()
    w.add_str("general.architecture", "phi2")
    for key, v in (("block_count", n_layers), ("embedding_length", hidden),
                   ("feed_forward_length", inter), ("attention.head_count", n_heads),
                   ("attention.head_count_kv", n_heads), ("context_length", ctx),
                   ("rope.dimension_count", rot)):
        w.add_u32(f"phi2.{key}", v)
    w.add_f32("phi2.attention.layer_norm_epsilon", eps)
    w.add_f32("phi2.rope.freq_base", theta)

    def vec(name, n, mean=0.0):
        w.add_tensor(name, GGML_F16, (n,), normal_f16(seed, name, (n,), mean, 0.02))

    w.add_tensor("token_embd.weight", GGML_F16, (vocab, hidden),
                 normal_f16(seed, "token_embd.weight", (vocab, hidden), 0.0, 0.02))
    for i in range(n_layers):
        p = f"blk.{i}."
        vec(p + "attn_norm.weight", hidden, norm_mean)
        vec(p + "attn_norm.bias", hidden)
        for nm, (n, k) in (("attn_qkv", (3 * hidden, hidden)), ("attn_output", (hidden, hidden)),
                           ("ffn_up", (inter, hidden)), ("ffn_down", (hidden, inter))):
            w.add_tensor(p + nm + ".weight", qtype, (n, k), qgen(seed, p + nm + ".weight", n, k))
            vec(p + nm + ".bias", n)
    vec("output_norm.weight", hidden, norm_mean)
    vec("output_norm.bias", hidden)
    w.add_tensor("output.weight", qtype, (vocab, hidden), qgen(seed, "output.weight", vocab, hidden))
    vec("output.bias", vocab)
    w.write(path)
