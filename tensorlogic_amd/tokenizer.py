"""Tokenizer and chat loop around the device decoder.

`Tokenizer` mirrors src/tokenizer/mod.rs:9-92: a thin wrapper over the
HuggingFace `tokenizers` library (the reference pins the Rust crate 0.20.4;
the Python package here is the same library), loaded from a tokenizer.json
file, with the same special-token lookups.  `chat` is the generation loop of
examples/chat_demo_optimized.tl:176-262: the TinyLlama chat template,
tokenised without special tokens, `temperature_sample(logits, 0.8)` per
step, stop at the EOS id.  The decoding itself runs on the device
(`Model.set_sampling` + `Model.generate`, one replayed graph per token).
"""
from __future__ import annotations

import numpy as np

from ._lib import TLHipError

INVALID_OPERATION = 3   # tlhip_status TLHIP_ERR_INVALID_OPERATION


class Tokenizer:
    """Tokenizer::from_file / encode / decode / vocab_size / special ids."""

    def __init__(self, inner):
        self.inner = inner

    @classmethod
    def from_file(cls, path: str) -> "Tokenizer":
        from tokenizers import Tokenizer as HFTokenizer
        try:
            return cls(HFTokenizer.from_file(str(path)))
        except Exception as e:  # the library raises its own exception type
            raise TLHipError(INVALID_OPERATION, f"Failed to load tokenizer: {e}") from None

    @classmethod
    def from_pretrained(cls, identifier: str) -> "Tokenizer":
        # mod.rs:36-43: not available; the file must be given
        raise TLHipError(INVALID_OPERATION,
                         "from_pretrained not available in this version. Please download tokenizer file "
                         f"manually from HuggingFace Hub and use from_file: {identifier}")

    def encode(self, text: str, add_special_tokens: bool) -> list[int]:
        try:
            return list(self.inner.encode(text, add_special_tokens=add_special_tokens).ids)
        except Exception as e:
            raise TLHipError(INVALID_OPERATION, f"Failed to encode text: {e}") from None

    def decode(self, ids, skip_special_tokens: bool) -> str:
        try:
            return self.inner.decode([int(i) for i in ids], skip_special_tokens=skip_special_tokens)
        except Exception as e:
            raise TLHipError(INVALID_OPERATION, f"Failed to decode tokens: {e}") from None

    def vocab_size(self) -> int:
        return self.inner.get_vocab_size(with_added_tokens=True)

    def _first_id(self, names):
        for n in names:
            i = self.inner.token_to_id(n)
            if i is not None:
                return i
        return None

    def pad_token_id(self):
        return self._first_id(("<pad>", "[PAD]"))

    def bos_token_id(self):
        return self._first_id(("<s>", "[BOS]", "<bos>"))

    def eos_token_id(self):
        return self._first_id(("</s>", "[EOS]", "<eos>"))


def tinyllama_chat_prompt(system_prompt: str, user_message: str) -> str:
    """The TinyLlama chat template of chat_demo_optimized.tl:184."""
    return "<|system|>\n" + system_prompt + "</s>\n<|user|>\n" + user_message + "</s>\n<|assistant|>\n"


def until_eos(tokens, eos_token_id: int) -> list[int]:
    """The sampled tokens up to (not including) the first EOS, as the chat
    loop breaks on it before appending (chat_demo_optimized.tl:241-247)."""
    out = []
    for t in tokens:
        if int(t) == eos_token_id:
            break
        out.append(int(t))
    return out


def chat(model, tokenizer: Tokenizer, system_prompt: str, user_message: str, max_new_tokens: int = 10,
         temperature: float = 0.8, seed: int = 0, eos_token_id: int = 2, use_graph: bool = True):
    """One assistant turn: returns (text, token ids).  The device decodes
    max_new_tokens steps in one go; tokens after the first EOS are dropped,
    which is what stopping the loop there produces."""
    prompt = tokenizer.encode(tinyllama_chat_prompt(system_prompt, user_message), False)
    model.set_sampling(temperature, seed)
    toks = model.generate(np.asarray(prompt, np.int32), max(max_new_tokens - 1, 0), use_graph=use_graph)
    ids = until_eos(toks[:max_new_tokens], eos_token_id)
    return tokenizer.decode(ids, True), ids
