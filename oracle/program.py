"""debug/chat_demo_with_kvcache.tl composed from the oracle's one-builtin
functions -- TEST INFRASTRUCTURE ONLY (the checker of
tensorlogic_amd.program.ChatDemoKVCache, which runs the same sequence on the
device).

Each statement of the program maps to one oracle call, in the program's
order, with its f16 storage points:

    prefill (chat_demo_with_kvcache.tl:130-186)       decode (:208-296)
    embedding(emb, ids)                                embedding(emb, token)
    per layer:                                         per layer:
      rms_norm(x, attn_norm)          eps 1e-6           rms_norm(x, attn_norm)
      Q, K, V = linear(x_norm1, W_*)                     Q = linear; Q_rope = rope(reshape(Q))
      K_rope = rope(reshape(K, [S, Hkv, D]))             K_new, V_new = linear
      cache.set(layer, K_rope, V_heads)                  cache.append(layer, rope(K_new), V_new)
      tinyllama_gqa_attention (:43-89):                  K_full / V_full = cache.get_k / get_v
        rope(Q), rope(K), broadcast_to K / V,            broadcast_to, einsum, * 0.125,
        einsum, * 0.125, apply_attention_mask(           causal_mask(1) broadcast to [1, H, J],
        broadcast causal_mask(S)), softmax, einsum,      apply_attention_mask, softmax,
        linear(W_o)                                      einsum, linear(W_o)
      x1 = x + attn; swiglu_ffn(rms_norm(x1)) (:29-41)   (same)
    slice_last(x, 0), rms_norm, linear(output)         rms_norm, linear(output)
    temperature_sample(logits, T) (greedy here: T = 0, builtin_sampling.rs:170-176)

`rope(x)` has no offset in the program, so rope_mode="program" rotates
prefill row s at position s and every decode row at position 0
(builtin_tensor.rs:531-546); rope_mode="absolute" passes each row's position
as rope(x, offset) allows -- the decoder runner's default.  `eps` is the
rms_norm eps: the builtin default 1e-6 (builtin_nn.rs:84-92) for the program
as written.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8


class ChatDemoKVCache:
    def __init__(self, path: str, rope_mode: str = "program", eps: float = 1e-6, scale: float = 0.125):
        if rope_mode not in ("program", "absolute"):
            raise ValueError(rope_mode)
        g = O.GGUF(path)
        self.n_layers = g.kv_u32("llama.block_count")
        self.hidden = g.kv_u32("llama.embedding_length")
        self.n_heads = g.kv_u32("llama.attention.head_count")
        self.n_kv = g.kv_u32("llama.attention.head_count_kv")
        self.head_dim = self.hidden // self.n_heads
        self.rope_mode, self.eps, self.scale = rope_mode, eps, scale

        def vec(name):
            t, dims, raw = g.tensor(name)
            if t == GGML_F32:
                return np.frombuffer(raw, np.float32).astype(np.float16).reshape(dims)
            assert t == GGML_F16, (name, t)
            return np.frombuffer(raw, np.float16).reshape(dims).copy()

        def lin(name):
            t, dims, raw = g.tensor(name)
            if t in (GGML_Q4_0, GGML_Q8_0):
                return ("q", t, np.frombuffer(raw, np.uint8).copy(), dims[0])
            return ("f", vec(name))

        self.emb = vec("token_embd.weight")
        self.vocab = self.emb.shape[0]
        self.out_norm = vec("output_norm.weight")
        self.out = lin("output.weight")
        self.layers = []
        for i in range(self.n_layers):
            p = f"blk.{i}."
            self.layers.append({k: (vec(p + k + ".weight") if "norm" in k else lin(p + k + ".weight"))
                                for k in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                          "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")})
        g.close()
        self.cache_k = [None] * self.n_layers
        self.cache_v = [None] * self.n_layers
        self.pos = 0

    # -- builtins ------------------------------------------------------------
    @staticmethod
    def linear(x, w):
        if w[0] == "q":
            return O.linear_q(x, w[2], w[1], w[3])
        return O.linear(x, w[1])

    def rms_norm(self, x, w):
        return O.rms_norm(x, w, self.eps)

    def swiglu_ffn(self, x, L):
        gate = self.linear(x, L["ffn_gate"])
        gate_act = O.mul(gate, O.sigmoid(gate))          # silu(x) = x * sigmoid(x)
        up = self.linear(x, L["ffn_up"])
        return self.linear(O.mul(gate_act, up), L["ffn_down"])

    def expand(self, t):
        """reshape [J, Hkv, 1, D] -> broadcast_to [J, Hkv, H/Hkv, D] -> reshape [J, H, D]."""
        J = t.shape[0]
        g = self.n_heads // self.n_kv
        b = O.broadcast_to(t.reshape(J, self.n_kv, 1, self.head_dim), (J, self.n_kv, g, self.head_dim))
        return b.reshape(J, self.n_heads, self.head_dim)

    def attend(self, q_rope, k_exp, v_exp, mask):
        scores = O.einsum_scores(q_rope, k_exp)
        scaled = O.mul_scalar(scores, self.scale)
        p = O.softmax(O.apply_attention_mask(scaled, np.ascontiguousarray(mask)))
        return O.einsum_context(p, v_exp)

    # -- the program ---------------------------------------------------------
    def prefill(self, ids):
        """The prompt pass; returns the logits [1, V] of the last row."""
        S, H, NH, NKV, D = len(ids), self.hidden, self.n_heads, self.n_kv, self.head_dim
        x = O.embedding(self.emb, np.asarray(ids, np.int32))
        for li, L in enumerate(self.layers):
            x_norm1 = self.rms_norm(x, L["attn_norm"])
            Q = self.linear(x_norm1, L["attn_q"])
            K = self.linear(x_norm1, L["attn_k"])
            V = self.linear(x_norm1, L["attn_v"])
            K_rope = O.rope(K.reshape(S, NKV, D))
            self.cache_k[li] = K_rope
            self.cache_v[li] = V.reshape(S, NKV, D)
            # tinyllama_gqa_attention(Q, K, V, W_o)
            Q_rope = O.rope(Q.reshape(S, NH, D))
            K_rope2 = O.rope(K.reshape(S, NKV, D))
            mask = np.broadcast_to(O.causal_mask(S).reshape(S, 1, S), (S, NH, S))
            att = self.attend(Q_rope, self.expand(K_rope2), self.expand(V.reshape(S, NKV, D)), mask)
            attn_out = self.linear(att.reshape(S, H), L["attn_output"])
            x1 = O.add(x, attn_out)
            x = O.add(x1, self.swiglu_ffn(self.rms_norm(x1, L["ffn_norm"]), L))
        self.pos = S
        last = O.slice_last(x, 0).reshape(1, H)
        return self.linear(self.rms_norm(last, self.out_norm), self.out)

    def decode(self, token):
        """One decode step for `token`; returns the logits [1, V]."""
        H, NH, NKV, D = self.hidden, self.n_heads, self.n_kv, self.head_dim
        off = 0 if self.rope_mode == "program" else self.pos
        x = O.embedding(self.emb, np.asarray([token], np.int32))
        for li, L in enumerate(self.layers):
            x_norm1 = self.rms_norm(x, L["attn_norm"])
            Q_rope = O.rope(self.linear(x_norm1, L["attn_q"]).reshape(1, NH, D), off)
            K_new_rope = O.rope(self.linear(x_norm1, L["attn_k"]).reshape(1, NKV, D), off)
            V_new = self.linear(x_norm1, L["attn_v"]).reshape(1, NKV, D)
            self.cache_k[li] = np.concatenate([self.cache_k[li], K_new_rope])
            self.cache_v[li] = np.concatenate([self.cache_v[li], V_new])
            J = self.cache_k[li].shape[0]
            mask = np.broadcast_to(O.causal_mask(1).reshape(1, 1, 1), (1, NH, J))
            att = self.attend(Q_rope, self.expand(self.cache_k[li]), self.expand(self.cache_v[li]), mask)
            x1 = O.add(x, self.linear(att.reshape(1, H), L["attn_output"]))
            x = O.add(x1, self.swiglu_ffn(self.rms_norm(x1, L["ffn_norm"]), L))
        self.pos += 1
        return self.linear(self.rms_norm(x, self.out_norm), self.out)

    def generate(self, prompt, n_decode):
        """Greedy stream (temperature_sample(logits, 0)): 1 + n_decode ids,
        the top-2 margin of each step and the last logits."""
        lg = self.prefill(prompt)[0]
        toks, margins = [], []
        for step in range(n_decode + 1):
            t = O.argmax_last(lg)
            toks.append(t)
            srt = np.sort(lg.astype(np.float32))
            margins.append(float(srt[-1] - srt[-2]))
            if step < n_decode:
                lg = self.decode(t)[0]
        return np.array(toks, np.int32), np.array(margins), lg
