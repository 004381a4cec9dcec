"""Host-side tokenizer and chat loop (src/tokenizer/mod.rs,
examples/chat_demo_optimized.tl:176-262).  No reference tokenizer file is
available offline: a small byte-level BPE is trained here with the same
`tokenizers` library, with TinyLlama's special-token ids (<unk> 0, <s> 1,
</s> 2) and the chat-template markers as added tokens."""
import numpy as np
import pytest

from tensorlogic_amd import TLHipError, Tokenizer, chat, tinyllama_chat_prompt
from tensorlogic_amd.tokenizer import until_eos

SPECIAL = ["<unk>", "<s>", "</s>", "<|system|>", "<|user|>", "<|assistant|>"]
CORPUS = ["You are a friendly and helpful AI assistant.", "Hello! Tell me a short fun fact about computers.",
          "Computers store numbers in binary, with bits that are zero or one.",
          "The first mechanical computer was designed in the nineteenth century."] * 20


def make_tokenizer_file(path, vocab_size=400):
    from tokenizers import Tokenizer as HF, decoders, models, pre_tokenizers, trainers
    tok = HF(models.BPE(unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=SPECIAL,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(CORPUS, trainer)
    tok.save(str(path))
    return str(path)


@pytest.fixture
def tok(tmp_path):
    return Tokenizer.from_file(make_tokenizer_file(tmp_path / "tokenizer.json"))


def test_encode_decode_round_trip(tok):
    text = "Hello! Tell me a short fun fact about computers."
    ids = tok.encode(text, False)
    assert ids and all(isinstance(i, int) for i in ids)
    assert tok.decode(ids, False) == text
    assert tok.vocab_size() <= 400 + len(SPECIAL)


def test_special_token_ids(tok):
    # mod.rs:72-91 lookups; TinyLlama's EOS id 2 is what the chat loop stops on
    assert (tok.bos_token_id(), tok.eos_token_id(), tok.pad_token_id()) == (1, 2, None)


def test_chat_template_and_special_tokens(tok):
    p = tinyllama_chat_prompt("You are a friendly and helpful AI assistant.",
                              "Hello! Tell me a short fun fact about computers.")
    assert p == ("<|system|>\nYou are a friendly and helpful AI assistant.</s>\n<|user|>\n"
                 "Hello! Tell me a short fun fact about computers.</s>\n<|assistant|>\n")
    ids = tok.encode(p, False)
    for name in ("<|system|>", "<|user|>", "<|assistant|>", "</s>"):
        assert tok.inner.token_to_id(name) in ids
    assert tok.decode(ids, False) == p


def test_errors_are_tensor_errors(tmp_path):
    bad = tmp_path / "bad.json"
    bad.write_text("{not json")
    with pytest.raises(TLHipError) as e:
        Tokenizer.from_file(str(bad))
    assert e.value.kind == "InvalidOperation"
    with pytest.raises(TLHipError) as e:
        Tokenizer.from_pretrained("gpt2")
    assert e.value.kind == "InvalidOperation"


def test_until_eos():
    assert until_eos([5, 6, 2, 7], 2) == [5, 6]
    assert until_eos(np.array([2, 5]), 2) == []
    assert until_eos([5, 6], 2) == [5, 6]


class _FakeModel:
    """Records the calls chat() makes; returns a fixed stream."""

    def __init__(self, stream):
        self.stream = np.asarray(stream, np.int32)
        self.calls = []

    def set_sampling(self, temperature, seed=0):
        self.calls.append(("set_sampling", temperature, seed))

    def generate(self, prompt, n_decode, use_graph=True):
        self.calls.append(("generate", list(prompt), n_decode, use_graph))
        return self.stream[:n_decode + 1]


def test_chat_loop_semantics(tok):
    # up to max_new_tokens draws at temperature 0.8; the first EOS ends the turn
    hello = tok.encode(" fun fact", False)
    m = _FakeModel(hello + [2] + hello)
    text, ids = chat(m, tok, "sys", "hi", max_new_tokens=10, temperature=0.8, seed=3)
    assert ids == hello and text == " fun fact"
    assert m.calls[0] == ("set_sampling", 0.8, 3)
    assert m.calls[1][0] == "generate" and m.calls[1][2] == 9
    assert m.calls[1][1] == tok.encode(tinyllama_chat_prompt("sys", "hi"), False)
