"""CPU-only checks of the product's host side: the C-ABI library loads and
exports every entry point include/tl_hip.h declares, the ctypes binding
declares each of them, and the host-only parts behind the ABI (GGUF header
parsing, argument errors) behave as the reference's loader and error enum
require.  No compute call is made here; device work is in test_gpu_*.py.
"""
import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

from tensorlogic_amd import _lib as L
from tensorlogic_amd import synth as S
from tensorlogic_amd.gguf import GGML_F16, GGML_Q4_0, GGML_Q8_0, GGUFReader, GGUFWriter

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tl_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tlhip_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(L.LIB_PATH)
    names = declared_functions()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared in tl_hip.h but not exported: {missing}"


def test_binding_covers_the_header():
    names = set(declared_functions())
    bound = set(L.SIGNATURES)
    assert not (bound - names), f"bound but not declared: {sorted(bound - names)}"
    assert not (names - bound), f"declared but not bound: {sorted(names - bound)}"


def test_no_oracle_in_the_product():
    """The product library and package never load the CPU oracle."""
    for dirpath, _, files in os.walk(os.path.join(ROOT, "tensorlogic_amd")):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                src = open(os.path.join(dirpath, f), errors="replace").read()
                assert "liboracle" not in src and "from oracle" not in src and "import oracle" not in src, f
    for f in ("_lib.py", "tensor.py"):
        assert "oracle" not in open(os.path.join(ROOT, "tensorlogic_amd", f)).read()


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present; device init is covered by GPU tests")
def test_init_without_a_device_fails_cleanly():
    ctx = C.c_void_p()
    st = L.lib().tlhip_init(0, C.byref(ctx))
    assert st == 7                                   # TLHIP_ERR_DEVICE (TensorError::MetalError)
    assert b"Device" in L.lib().tlhip_last_error()
    assert L.lib().tlhip_sync(None) == 9             # null context -> InvalidArgument


# ---------------------------------------------------------------------------
# GGUF header parsing through the C ABI (host only)
# ---------------------------------------------------------------------------
def _s(b: str) -> bytes:
    e = b.encode()
    return struct.pack("<Q", len(e)) + e


def raw_gguf(kvs, tensors, version=3, align=32, magic=0x46554747, truncate=None, header_offsets=None):
    """Hand-built GGUF: kvs = [(key, type, payload_bytes)], tensors = [(name, dims_rowmajor, gtype, data)].
    header_offsets, when given, replaces the tensor offsets written in the
    tensor table (the data is still laid out at the true offsets)."""
    head = struct.pack("<IIQQ", magic, version, len(tensors), len(kvs))
    for k, t, payload in kvs:
        head += _s(k) + struct.pack("<I", t) + payload
    off, offs = 0, []
    for _, _, _, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + align - 1) // align * align
    for i, ((name, dims, gt, _), o) in enumerate(zip(tensors, offs)):
        head += _s(name) + struct.pack("<I", len(dims))
        for d in reversed(dims):
            head += struct.pack("<Q", d)
        head += struct.pack("<IQ", gt, header_offsets[i] if header_offsets else o)
    head += b"\0" * ((-len(head)) % align)
    body = b""
    for (_, _, _, data), o in zip(tensors, offs):
        body += b"\0" * (o - len(body)) + data
    out = head + body
    return out[:truncate] if truncate else out


def every_kv_type():
    """One value of each GGUF metadata type (u8 i8 u16 i16 u32 i32 f32 bool
    str arr u64 i64 f64).  The reference's skip_metadata_value reads 4 bytes
    for the 1- and 2-byte types (mmap_gguf.rs:329-336); a parser with that
    bug loses its place here."""
    return [
        ("a.u8", 0, struct.pack("<B", 7)), ("a.i8", 1, struct.pack("<b", -7)),
        ("a.u16", 2, struct.pack("<H", 700)), ("a.i16", 3, struct.pack("<h", -700)),
        ("llama.block_count", 4, struct.pack("<I", 22)), ("a.i32", 5, struct.pack("<i", -5)),
        ("llama.rope.freq_base", 6, struct.pack("<f", 10000.0)), ("a.bool", 7, struct.pack("<B", 1)),
        ("general.name", 8, _s("tiny")),
        ("a.arr_u8", 9, struct.pack("<IQ", 0, 3) + bytes([1, 2, 3])),
        ("a.arr_str", 9, struct.pack("<IQ", 8, 2) + _s("x") + _s("yz")),
        ("a.u64", 10, struct.pack("<Q", 1 << 40)), ("a.i64", 11, struct.pack("<q", -(1 << 40))),
        ("a.f64", 12, struct.pack("<d", 0.25)),
    ]


def open_c(path):
    g = C.c_void_p()
    st = L.lib().tlhip_gguf_open(path.encode(), C.byref(g))
    return st, g


def test_gguf_every_kv_type_and_tensor_table(tmp_path, oracle):
    q4 = S.q4_0_blocks(50, "w", 4, 64)
    emb = S.normal_f16(50, "e", (3, 8))
    p = str(tmp_path / "all.gguf")
    open(p, "wb").write(raw_gguf(every_kv_type(), [("w", (4, 64), GGML_Q4_0, q4.tobytes()),
                                                  ("e", (3, 8), GGML_F16, emb.tobytes())]))
    st, g = open_c(p)
    assert st == 0, L.lib().tlhip_last_error()
    lib = L.lib()
    assert lib.tlhip_gguf_n_tensors(g) == 2
    assert {lib.tlhip_gguf_tensor_name(g, i) for i in range(2)} == {b"w", b"e"}
    u, f = C.c_uint32(), C.c_float()
    assert lib.tlhip_gguf_kv_u32(g, b"llama.block_count", C.byref(u)) == 0 and u.value == 22
    assert lib.tlhip_gguf_kv_f32(g, b"llama.rope.freq_base", C.byref(f)) == 0 and f.value == 10000.0
    assert lib.tlhip_gguf_kv_u32(g, b"missing.key", C.byref(u)) != 0
    assert lib.tlhip_gguf_close(g) == 0
    # the numpy reader agrees on the same bytes
    r = GGUFReader(p)
    assert r.kv["a.u16"] == 700 and r.kv["a.arr_str"] == ["x", "yz"] and r.kv["a.f64"] == 0.25
    assert r.tensors["w"].shape == (4, 64) and np.array_equal(r.raw("w"), q4)
    assert np.array_equal(r.raw("e").view(np.float16).reshape(3, 8), emb)
    # and so does the oracle's own reader (tlo_gguf_open), which every
    # oracle model and golden fixture is loaded through
    og = oracle.GGUF(p)
    assert sorted(og.names()) == ["e", "w"]
    assert og.kv_u32("llama.block_count") == 22 and og.kv_f32("llama.rope.freq_base") == 10000.0
    assert og.kv_u32("missing.key") is None
    assert og.tensor("w") == (GGML_Q4_0, (4, 64), q4.tobytes())
    assert og.tensor("e") == (GGML_F16, (3, 8), emb.tobytes())
    og.close()


def test_gguf_general_alignment_is_honoured(tmp_path):
    # the reference always assumes 32 (mmap_gguf.rs:256-257); the spec says
    # general.alignment when present
    data = S.normal_f16(51, "t", (4, 16)).tobytes()
    kvs = [("general.alignment", 4, struct.pack("<I", 64))]
    p = str(tmp_path / "a64.gguf")
    open(p, "wb").write(raw_gguf(kvs, [("t", (4, 16), GGML_F16, data)], align=64))
    st, g = open_c(p)
    assert st == 0, L.lib().tlhip_last_error()
    L.lib().tlhip_gguf_close(g)
    assert GGUFReader(p).raw("t").tobytes() == data


@pytest.mark.parametrize("case", ["magic", "version", "truncated_header", "data_past_eof",
                                  "bad_kv_type", "bad_q_shape", "missing_file", "huge_offset",
                                  "offset_past_eof", "dim_overflow", "dim_overflow_to_zero",
                                  "huge_tensor_count", "huge_kv_count"])
def test_gguf_malformed_is_a_load_error(tmp_path, oracle, case):
    q8 = S.q8_0_blocks(52, "w", 2, 64).tobytes()
    t = [("w", (2, 64), GGML_Q8_0, q8)]
    p = str(tmp_path / f"{case}.gguf")
    if case == "magic":
        blob = raw_gguf([], t, magic=0x12345678)
    elif case == "version":
        blob = raw_gguf([], t, version=9)
    elif case == "truncated_header":
        blob = raw_gguf(every_kv_type(), t, truncate=40)
    elif case == "data_past_eof":
        blob = raw_gguf([], t)[:-10]
    elif case == "bad_kv_type":
        blob = raw_gguf([("x", 99, b"\0" * 8)], t)
    elif case == "bad_q_shape":                     # 48 elements is not a whole number of Q8_0 blocks
        blob = raw_gguf([], [("w", (1, 48), GGML_Q8_0, q8[:51])])
    elif case == "huge_offset":                     # data_off + offset + nbytes wraps past 2^64
        blob = raw_gguf([], t, header_offsets=[(1 << 64) - 64])
    elif case == "offset_past_eof":                 # offset alone beyond the file
        blob = raw_gguf([], t, header_offsets=[1 << 40])
    elif case == "dim_overflow":                    # 2^40 x 2^40 elements: the count wraps 64 bits
        blob = raw_gguf([], [("w", (1 << 40, 1 << 40), GGML_Q8_0, q8)])
    elif case == "dim_overflow_to_zero":            # 2^32 * 2^32 * 2^32 wraps to 0 elements, 0 bytes
        blob = raw_gguf([], [("w", (1 << 32, 1 << 32, 1 << 32), GGML_Q8_0, q8)])
    elif case == "huge_tensor_count":               # 2^24 tensor infos declared over a ~200-byte file
        blob = bytearray(raw_gguf([], t))
        blob[8:16] = struct.pack("<Q", 1 << 24)
    elif case == "huge_kv_count":                   # 2^24 KV pairs declared
        blob = bytearray(raw_gguf([], t))
        blob[16:24] = struct.pack("<Q", 1 << 24)
    if case != "missing_file":
        open(p, "wb").write(blob)
    st, g = open_c(p)
    assert st == 6, (case, st)                       # TLHIP_ERR_LOAD (TensorError::LoadError)
    assert b"LoadError" in L.lib().tlhip_last_error()
    with pytest.raises(ValueError):                  # the oracle's reader refuses the same files
        oracle.GGUF(p)


def test_writer_reader_round_trip_and_reference_parseable_types(tmp_path):
    p = str(tmp_path / "rt.gguf")
    S.write_llama_gguf(p, seed=53, n_layers=1, hidden=64, inter=128, n_heads=4, n_kv=2, vocab=50)
    r = GGUFReader(p)
    # the writer only uses metadata types the reference's own parser sizes
    # correctly (u32 / i32 / f32 / u64 / string), and 32-byte alignment
    raw = open(p, "rb").read()
    assert "general.alignment" not in r.kv
    assert r.tensors["blk.0.attn_k.weight"].shape == (32, 64)
    assert r.tensors["blk.0.ffn_down.weight"].shape == (64, 128)
    assert r.tensors["output.weight"].gtype == GGML_Q4_0
    assert np.array_equal(r.raw("blk.0.attn_q.weight"), S.q4_0_blocks(53, "blk.0.attn_q.weight", 64, 64))
    assert r.data_offset % 32 == 0 and len(raw) >= r.data_offset
    st, g = open_c(p)
    assert st == 0 and L.lib().tlhip_gguf_n_tensors(g) == len(r.tensors)
    L.lib().tlhip_gguf_close(g)
