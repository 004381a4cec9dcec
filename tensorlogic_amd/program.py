"""debug/chat_demo_with_kvcache.tl and examples/chat_demo_optimized.tl run
unchanged, one TL builtin at a time.

Each statement of the program's prefill (chat_demo_with_kvcache.tl:130-186)
and decode loop (:208-296), and of its helper functions silu / swiglu_ffn /
tinyllama_gqa_attention (:26-89), is one call of the Tensor API, i.e. one
tlhip_* entry point of the C ABI, in the program's order:

    embedding -> per layer: rms_norm -> linear (q, k, v) -> reshape -> rope
    -> KVCache.set / .append -> get_k / get_v -> reshape -> broadcast_to ->
    reshape -> einsum("ihd,jhd->ihj") -> * 0.125 -> causal_mask -> reshape ->
    broadcast_to -> apply_attention_mask -> softmax -> einsum("ihj,jhd->ihd")
    -> reshape -> linear (o) -> + -> rms_norm -> linear (gate) -> sigmoid ->
    * -> linear (up) -> * -> linear (down) -> +; then slice_last -> reshape ->
    rms_norm -> linear (output) -> temperature_sample.

This is what an interpreter calling the C ABI op by op does; the fused
decoder runner (tlhip_model_*) computes the same values in five launches per
layer.  The program's semantics are kept literally by default: rope(x)
without an offset (every decode row rotated as position 0,
builtin_tensor.rs:531-546) and rms_norm at the builtin default eps 1e-6
(builtin_nn.rs:84-92).  rope_mode="absolute" passes each row's position as
rope(x, offset) allows.  Head counts come from the GGUF file where the
program hard-codes TinyLlama's (32 / 4 heads of 64); its literal `* 0.125`
is 1 / sqrt(64), the scale argument.

examples/chat_demo_optimized.tl (ChatDemoOptimized) has no cache: every
step re-embeds the whole token list and runs its transformer_layer
(:104-138) over all rows -- rope(Q_heads) / rope(K_heads) with no offset on
the full sequence rotate row s at position s -- then slice_last, the final
rms_norm, the output linear and temperature_sample(logits, 0.8), stopping
at EOS (id 2) or after 10 steps (:200-239).
"""
from __future__ import annotations

import numpy as np

from .tensor import GGUF, Device, KVCache, Tensor, causal_mask, einsum, embedding, temperature_sample


class _ChatDemoProgram:
    """The weights (get_tensor / model.blk[i].X.weight) and the helper
    functions the two chat programs share."""

    def __init__(self, dev: Device, path: str, eps: float = 1e-6, scale: float = 0.125):
        self.dev, self.eps, self.scale = dev, eps, scale
        g = GGUF(path)
        self.n_layers = g.kv_u32("llama.block_count")
        self.hidden = g.kv_u32("llama.embedding_length")
        self.n_heads = g.kv_u32("llama.attention.head_count")
        self.n_kv = g.kv_u32("llama.attention.head_count_kv")
        self.head_dim = self.hidden // self.n_heads
        # get_tensor(model, name) / model.blk[i].X.weight: packed weights stay packed
        self.emb = g.load_tensor(dev, "token_embd.weight")
        self.out_norm = g.load_tensor(dev, "output_norm.weight")
        self.out = g.load_tensor(dev, "output.weight")
        self.layers = []
        for i in range(self.n_layers):
            p = f"blk.{i}."
            self.layers.append({k: g.load_tensor(dev, p + k + ".weight")
                                for k in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                          "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")})
        g.close()
        self.vocab = self.emb.shape[0]

    # -- the program's helper functions (chat_demo_with_kvcache.tl:26-89) -----
    def rms_norm(self, x: Tensor, w: Tensor) -> Tensor:
        return x.rms_norm([self.hidden], w, self.eps)

    @staticmethod
    def silu(x: Tensor) -> Tensor:
        return x * x.sigmoid()

    def swiglu_ffn(self, x: Tensor, L) -> Tensor:
        gate = x.linear(L["ffn_gate"])
        gate_act = self.silu(gate)
        up = x.linear(L["ffn_up"])
        intermediate = gate_act * up
        return intermediate.linear(L["ffn_down"])

    def expand(self, t: Tensor, n: int) -> Tensor:
        """GQA: reshape [n, Hkv, 1, D] -> broadcast_to [n, Hkv, H/Hkv, D] -> reshape [n, H, D]."""
        g = self.n_heads // self.n_kv
        with_group = t.reshape((n, self.n_kv, 1, self.head_dim))
        bc = with_group.broadcast_to((n, self.n_kv, g, self.head_dim))
        return bc.reshape((n, self.n_heads, self.head_dim))

    def tinyllama_gqa_attention(self, Q: Tensor, K: Tensor, V: Tensor, W_o: Tensor, S: int) -> Tensor:
        NH, NKV, D = self.n_heads, self.n_kv, self.head_dim
        Q_rope = Q.reshape((S, NH, D)).rope()
        K_rope = K.reshape((S, NKV, D)).rope()
        V_heads = V.reshape((S, NKV, D))
        scores = einsum("ihd,jhd->ihj", Q_rope, self.expand(K_rope, S))
        scaled_scores = scores * self.scale
        mask_3d = causal_mask(self.dev, S).reshape((S, 1, S))
        mask_broadcast = mask_3d.broadcast_to((S, NH, S))
        attn_weights = scaled_scores.apply_attention_mask(mask_broadcast).softmax()
        attn_output = einsum("ihj,jhd->ihd", attn_weights, self.expand(V_heads, S))
        return attn_output.reshape((S, self.hidden)).linear(W_o)

    def transformer_layer(self, x: Tensor, L, S: int) -> Tensor:
        """transformer_layer (chat_demo_optimized.tl:104-138)."""
        x_norm1 = self.rms_norm(x, L["attn_norm"])
        Q = x_norm1.linear(L["attn_q"])
        K = x_norm1.linear(L["attn_k"])
        V = x_norm1.linear(L["attn_v"])
        attn_out = self.tinyllama_gqa_attention(Q, K, V, L["attn_output"], S)
        x1 = x + attn_out
        return x1 + self.swiglu_ffn(self.rms_norm(x1, L["ffn_norm"]), L)

    def head_logits(self, x: Tensor) -> Tensor:
        """slice_last(x, 0) -> reshape [1, hidden] -> rms_norm -> linear(output)."""
        last = x.slice_last(0).reshape((1, self.hidden))
        return self.rms_norm(last, self.out_norm).linear(self.out)


class ChatDemoKVCache(_ChatDemoProgram):
    def __init__(self, dev: Device, path: str, max_ctx: int = 512, rope_mode: str = "program",
                 eps: float = 1e-6, scale: float = 0.125):
        if rope_mode not in ("program", "absolute"):
            raise ValueError(rope_mode)
        super().__init__(dev, path, eps, scale)
        self.rope_mode = rope_mode
        self.max_ctx = max_ctx
        self.cache = KVCache(dev, self.n_layers, max_ctx, self.n_kv, self.head_dim)   # KVCache::new_f16(22)
        self.pos = 0

    # -- prefill (:130-186) ------------------------------------------------------
    def prefill(self, ids) -> Tensor:
        """The prompt pass; fills the cache and returns the logits [1, V]."""
        ids = np.asarray(ids, np.int32)
        S, NKV, D = ids.size, self.n_kv, self.head_dim
        if S > self.max_ctx:
            raise ValueError(f"prompt of {S} tokens for a cache of {self.max_ctx}")
        x = embedding(self.emb, ids)
        for li, L in enumerate(self.layers):
            x_norm1 = self.rms_norm(x, L["attn_norm"])
            Q = x_norm1.linear(L["attn_q"])
            K = x_norm1.linear(L["attn_k"])
            V = x_norm1.linear(L["attn_v"])
            K_rope = K.reshape((S, NKV, D)).rope()
            self.cache.set(li, K_rope, V.reshape((S, NKV, D)))
            attn_out = self.tinyllama_gqa_attention(Q, K, V, L["attn_output"], S)
            x1 = x + attn_out
            x = x1 + self.swiglu_ffn(self.rms_norm(x1, L["ffn_norm"]), L)
        self.pos = S
        return self.head_logits(x)

    # -- decode step (:208-296) -----------------------------------------------
    def decode(self, token: int) -> Tensor:
        """One step for `token` against the cache; returns the logits [1, V]."""
        if self.pos >= self.max_ctx:
            raise ValueError("cache full")
        NH, NKV, D = self.n_heads, self.n_kv, self.head_dim
        off = 0 if self.rope_mode == "program" else self.pos
        x = embedding(self.emb, [int(token)])
        for li, L in enumerate(self.layers):
            x_norm1 = self.rms_norm(x, L["attn_norm"])
            Q_rope = x_norm1.linear(L["attn_q"]).reshape((1, NH, D)).rope(off)
            K_new = x_norm1.linear(L["attn_k"])
            V_new = x_norm1.linear(L["attn_v"])
            K_new_rope = K_new.reshape((1, NKV, D)).rope(off)
            self.cache.append(li, K_new_rope, V_new.reshape((1, NKV, D)))
            K_full = self.cache.get_k(li)
            V_full = self.cache.get_v(li)
            J = K_full.shape[0]
            scores = einsum("ihd,jhd->ihj", Q_rope, self.expand(K_full, J))
            scaled_scores = scores * self.scale
            mask_broadcast = causal_mask(self.dev, 1).reshape((1, 1, 1)).broadcast_to((1, NH, J))
            attn_weights = scaled_scores.apply_attention_mask(mask_broadcast).softmax()
            attn_output = einsum("ihj,jhd->ihd", attn_weights, self.expand(V_full, J))
            attn_out = attn_output.reshape((1, self.hidden)).linear(L["attn_output"])
            x1 = x + attn_out
            x = x1 + self.swiglu_ffn(self.rms_norm(x1, L["ffn_norm"]), L)
        self.pos += 1
        return self.rms_norm(x, self.out_norm).linear(self.out)

    def generate(self, prompt, n_decode: int, temperature: float = 0.0, seed: int = 0) -> np.ndarray:
        """prefill then n_decode steps; 1 + n_decode ids chosen by
        temperature_sample(logits, T) (greedy for T <= 1e-4; else the draw
        splitmix64(seed, step))."""
        logits = self.prefill(prompt)
        toks = []
        for step in range(n_decode + 1):
            t = temperature_sample(logits, temperature, seed, step)
            toks.append(t)
            if step < n_decode:
                logits = self.decode(t)
        self.last_logits = logits
        return np.array(toks, np.int32)


class ChatDemoOptimized(_ChatDemoProgram):
    """examples/chat_demo_optimized.tl's generation loop (:200-239), no cache."""

    def forward(self, ids) -> Tensor:
        """embedding of every token so far, the 22 (n_layers) transformer
        layers over all rows, the logits [1, V] of the last row."""
        ids = np.asarray(ids, np.int32)
        x = embedding(self.emb, ids)
        for L in self.layers:
            x = self.transformer_layer(x, L, ids.size)
        return self.head_logits(x)

    def generate(self, prompt, max_steps: int = 10, temperature: float = 0.8, seed: int = 0,
                 eos: int = 2) -> np.ndarray:
        """The program's loop: up to max_steps tokens chosen by
        temperature_sample(logits, T) (draw splitmix64(seed, step)), stopping
        before appending EOS; returns prompt + generated ids."""
        gen = [int(t) for t in np.asarray(prompt, np.int32)]
        self.step_logits = []   # each step's logits tensor (the sampler's input)
        for step in range(max_steps):
            logits = self.forward(gen)
            t = temperature_sample(logits, temperature, seed, step)
            self.step_logits.append(logits)
            self.last_logits = logits
            if t == eos:
                break
            gen.append(t)
        return np.array(gen, np.int32)
