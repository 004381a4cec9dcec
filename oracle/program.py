"""debug/chat_demo_with_kvcache.tl and examples/chat_demo_optimized.tl
composed from the oracle's one-builtin functions -- TEST INFRASTRUCTURE ONLY
(the checker of tensorlogic_amd.program.ChatDemoKVCache / ChatDemoOptimized,
which run the same sequences on the device).

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

ChatDemoOptimized restates examples/chat_demo_optimized.tl's loop
(:200-239): no cache; each step embeds every token so far and runs
transformer_layer (:104-138) over all rows -- rms_norm, linear q/k/v,
tinyllama_gqa_attention (rope with no offset over the full sequence, so row
s at position s; broadcast_to; einsum; * 0.125; the broadcast causal mask;
softmax; einsum; linear W_o), the residual, rms_norm, swiglu_ffn, the
residual -- then slice_last, rms_norm, linear(output) and
temperature_sample, stopping at EOS.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8


class _ChatDemoProgram:
    """The weights and builtins the two chat programs share."""

    def __init__(self, path: str, eps: float = 1e-6, scale: float = 0.125, acc: int = O.ACC_F32):
        self.acc = acc   # ACC_F32_REV: every linear's sums in descending order (the reordered oracle)
        g = O.GGUF(path)
        self.n_layers = g.kv_u32("llama.block_count")
        self.hidden = g.kv_u32("llama.embedding_length")
        self.n_heads = g.kv_u32("llama.attention.head_count")
        self.n_kv = g.kv_u32("llama.attention.head_count_kv")
        self.head_dim = self.hidden // self.n_heads
        self.eps, self.scale = eps, scale

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

    # -- builtins ------------------------------------------------------------
    def linear(self, x, w):
        if w[0] == "q":
            return O.linear_q(x, w[2], w[1], w[3], acc=self.acc)
        return O.linear(x, w[1], acc=self.acc)

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

    def gqa_attention(self, Q, K, V, W_o):
        """tinyllama_gqa_attention (chat_demo_optimized.tl:43-101 /
        chat_demo_with_kvcache.tl:43-89) over S rows."""
        S, NH, NKV, D = Q.shape[0], self.n_heads, self.n_kv, self.head_dim
        Q_rope = O.rope(Q.reshape(S, NH, D))
        K_rope = O.rope(K.reshape(S, NKV, D))
        mask = np.broadcast_to(O.causal_mask(S).reshape(S, 1, S), (S, NH, S))
        att = self.attend(Q_rope, self.expand(K_rope), self.expand(V.reshape(S, NKV, D)), mask)
        return self.linear(att.reshape(S, self.hidden), W_o)

    def head_logits(self, x):
        last = O.slice_last(x, 0).reshape(1, self.hidden)
        return self.linear(self.rms_norm(last, self.out_norm), self.out)


class ChatDemoKVCache(_ChatDemoProgram):
    def __init__(self, path: str, rope_mode: str = "program", eps: float = 1e-6, scale: float = 0.125):
        if rope_mode not in ("program", "absolute"):
            raise ValueError(rope_mode)
        super().__init__(path, eps, scale)
        self.rope_mode = rope_mode
        self.cache_k = [None] * self.n_layers
        self.cache_v = [None] * self.n_layers
        self.pos = 0

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
            attn_out = self.gqa_attention(Q, K, V, L["attn_output"])
            x1 = O.add(x, attn_out)
            x = O.add(x1, self.swiglu_ffn(self.rms_norm(x1, L["ffn_norm"]), L))
        self.pos = S
        return self.head_logits(x)

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


class ChatDemoOptimized(_ChatDemoProgram):
    """examples/chat_demo_optimized.tl's generation loop, no cache."""

    def forward(self, ids):
        """The logits [1, V] of the last row after the n_layers
        transformer_layer calls over every token so far."""
        x = O.embedding(self.emb, np.asarray(ids, np.int32))
        for L in self.layers:
            x_norm1 = self.rms_norm(x, L["attn_norm"])
            Q = self.linear(x_norm1, L["attn_q"])
            K = self.linear(x_norm1, L["attn_k"])
            V = self.linear(x_norm1, L["attn_v"])
            x1 = O.add(x, self.gqa_attention(Q, K, V, L["attn_output"]))
            x = O.add(x1, self.swiglu_ffn(self.rms_norm(x1, L["ffn_norm"]), L))
        return self.head_logits(x)

    def generate(self, prompt, max_steps=10, temperature=0.8, seed=0, eos=2):
        """The program's loop with the draw splitmix64(seed, step) (greedy for
        T <= 1e-4); returns prompt + generated ids, the per-step logits and
        each step's draw."""
        gen = [int(t) for t in np.asarray(prompt, np.int32)]
        logits, draws = [], []
        for step in range(max_steps):
            lg = self.forward(gen)[0]
            logits.append(lg)
            if temperature <= 1e-4:
                t, u = O.argmax_last(lg), None
            else:
                u = O.sample_uniform(seed, step)
                t = O.sample_temperature(lg, temperature, u)
            draws.append(u)
            if t == eos:
                break
            gen.append(t)
        return np.array(gen, np.int32), logits, draws
