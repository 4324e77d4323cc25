"""GGUF reader of the device weight registry (host only, no GPU): the native parser (jamhip_gguf_open) on
byte images assembled here field by field from the GGUF v3 layout, on files from qxotic_amd.gguf.write,
and on every malformed case the qxotic reader rejects (gguf/src/main/java/com/qxotic/format/gguf/impl/
ReaderImpl.java:31-380), plus the ones this reader rejects before mapping (unknown types, partial blocks,
data past the end of the file)."""
import struct

import numpy as np
import pytest

from qxotic_amd import gguf as G
from qxotic_amd.ggml import BY_NAME


def s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def header(n_tensors, kvs, version=3, magic=0x46554747):
    return struct.pack("<IIQQ", magic, version, n_tensors, len(kvs)) + b"".join(kvs)


def kv_u32(key, v):
    return s(key) + struct.pack("<II", 4, v)


def tensor(name, dims, ty, off):
    return s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, off)


def image(path, head: bytes, data_offset: int, data: bytes) -> str:
    path.write_bytes(head + b"\0" * (data_offset - len(head)) + data)
    return str(path)


def test_hand_assembled_file(tmp_path):
    """A 2x64 Q8_0 tensor behind general.alignment = 64. Header bytes: 24 (magic, version, counts) + 33
    (key "general.alignment": 8 + 17, type 4, value 4) + 41 (name "w": 8 + 1, n_dims 4, dims 16, type 4,
    offset 8) = 98, so the data region starts at 128."""
    q8 = BY_NAME["Q8_0"].ggml
    head = header(1, [kv_u32("general.alignment", 64)]) + tensor("w", [64, 2], q8, 0)
    assert len(head) == 98
    payload = bytes(range(136))                     # 2 rows x 2 blocks x 34 bytes
    with G.GGUF(image(tmp_path / "a.gguf", head, 128, payload)) as g:
        assert g.alignment == 64 and g.tensor_data_offset == 128
        e = g.tensors["w"]
        assert (e.ggml_type, e.shape, e.offset, e.byte_size) == (q8, (64, 2), 0, 136)
        assert g.data("w").tobytes() == payload
        assert g.find("w") == 0 and g.find("x") == -1


def test_writer_matches_hand_assembled_bytes(tmp_path):
    """qxotic_amd.gguf.write (used by the registry tests and bench.py) emits exactly the hand-assembled
    image of test_hand_assembled_file: header, key, tensor entry, zero padding to 128, then the data."""
    q8 = BY_NAME["Q8_0"].ggml
    payload = bytes(range(136))
    head = header(1, [kv_u32("general.alignment", 64)]) + tensor("w", [64, 2], q8, 0)
    want = head + b"\0" * (128 - len(head)) + payload
    off = G.write(tmp_path / "w.gguf", [("w", q8, (64, 2), np.frombuffer(payload, np.uint8))], alignment=64)
    assert off == 128
    assert (tmp_path / "w.gguf").read_bytes() == want


def test_default_alignment_and_no_tensors(tmp_path):
    head = header(0, [])                            # 24 bytes, padded to 32
    with G.GGUF(image(tmp_path / "e.gguf", head, 24, b"")) as g:
        assert g.alignment == 32 and g.tensor_data_offset == 32 and g.tensors == {}


@pytest.mark.parametrize("alignment", [None, 32, 64, 4096])
def test_writer_round_trip(tmp_path, alignment):
    rng = np.random.default_rng(7)
    q4k, mx, f32, f16 = (BY_NAME[n].ggml for n in ("Q4_K", "MXFP4", "F32", "F16"))
    tensors = [
        ("blk.0.ffn_up.weight", q4k, (512, 24), rng.integers(0, 256, 24 * 2 * 144, dtype=np.uint8)),
        ("blk.0.ffn_gate_exps.weight", mx, (64, 8, 3), rng.integers(0, 256, 3 * 8 * 2 * 17, dtype=np.uint8)),
        ("blk.0.attn_norm.weight", f32, (96,), rng.standard_normal(96).astype(np.float32)),
        ("token_embd.weight", f16, (8, 5), rng.standard_normal(40).astype(np.float16)),
    ]
    meta = [("general.architecture", "string", "llama"), ("llama.block_count", "uint32", 1),
            ("tokenizer.ggml.tokens", "array:string", ["<s>", "a", "b"]),
            ("tokenizer.ggml.scores", "array:float32", [0.0, -1.0, -2.0]), ("x.flag", "bool", True),
            ("x.i64", "int64", -5), ("x.f64", "float64", 0.25)]
    path = tmp_path / "w.gguf"
    data_offset = G.write(path, tensors, meta, alignment)
    align = alignment or 32
    with G.GGUF(path) as g:
        assert g.alignment == align and g.tensor_data_offset == data_offset and data_offset % align == 0
        assert list(g.tensors) == [t[0] for t in tensors]
        for name, ty, shape, data in tensors:
            e = g.tensors[name]
            assert (e.ggml_type, e.shape, e.byte_size) == (ty, tuple(shape), data.nbytes)
            assert e.offset % align == 0
            assert g.data(name).tobytes() == data.tobytes()


def test_limits_accepted(tmp_path):
    """Name of exactly 64 bytes, 4 dimensions, a zero-size tensor."""
    f32 = BY_NAME["F32"].ggml
    tensors = [("n" * 64, f32, (2, 1, 1, 2), np.zeros(4, np.float32)), ("empty", f32, (0, 3), b"")]
    G.write(tmp_path / "l.gguf", tensors)
    with G.GGUF(tmp_path / "l.gguf") as g:
        assert g.tensors["n" * 64].shape == (2, 1, 1, 2)
        assert g.tensors["empty"].byte_size == 0 and g.data("empty").size == 0


F32 = 0
BAD = {
    "magic": (lambda: header(0, [], magic=0x46554746), "magic"),
    "version2": (lambda: header(0, [], version=2), "version 2"),
    "name65": (lambda: header(1, []) + tensor("n" * 65, [4], F32, 0), "too long"),
    "dims5": (lambda: header(1, []) + tensor("t", [1, 1, 1, 1, 4], F32, 0), "too many dimensions"),
    "misaligned": (lambda: header(1, []) + tensor("t", [4], F32, 16), "not aligned"),
    "dup_tensor": (lambda: header(2, []) + tensor("t", [4], F32, 0) + tensor("t", [4], F32, 32), "duplicate tensor"),
    "dup_key": (lambda: header(0, [kv_u32("a.b", 1), kv_u32("a.b", 2)]), "duplicate metadata key"),
    "key_upper": (lambda: header(0, [kv_u32("General.x", 1)]), "invalid metadata key"),
    "key_space": (lambda: header(0, [kv_u32("a b", 1)]), "invalid metadata key"),
    "align_u64": (lambda: header(0, [s("general.alignment") + struct.pack("<IQ", 10, 32)]), "UINT32"),
    "align_48": (lambda: header(0, [kv_u32("general.alignment", 48)]), "power of two"),
    "align_0": (lambda: header(0, [kv_u32("general.alignment", 0)]), "power of two"),
    "array_of_arrays": (lambda: header(0, [s("a.b") + struct.pack("<IIQ", 9, 9, 0)]), "array of arrays"),
    "value_type_13": (lambda: header(0, [s("a.b") + struct.pack("<I", 13)]), "value type"),
    "removed_type": (lambda: header(1, []) + tensor("t", [32], 4, 0), "GGML type"),
    "unknown_type": (lambda: header(1, []) + tensor("t", [32], 99, 0), "GGML type"),
    "partial_block": (lambda: header(1, []) + tensor("t", [100], 12, 0), "whole number of blocks"),
    "past_eof": (lambda: header(1, []) + tensor("t", [64], F32, 0), "past the end"),
    "truncated_header": (lambda: header(1, []) + tensor("t", [4, 4], F32, 0)[:-4], "truncated"),
    "truncated_string": (lambda: header(0, [struct.pack("<Q", 1 << 40)]), "past end of file"),
    "huge_tensor_count": (lambda: header(1 << 40, []) + b"\0" * 64, "count past end of file"),
    "huge_kv_count": (lambda: header(0, []).replace(struct.pack("<QQ", 0, 0), struct.pack("<QQ", 0, 1 << 40)), "count past end of file"),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_rejects(tmp_path, case):
    build, needle = BAD[case]
    p = tmp_path / f"{case}.gguf"
    p.write_bytes(build())
    with pytest.raises(G.GGUFFormatError, match=needle):
        G.GGUF(p)


def test_missing_file(tmp_path):
    with pytest.raises(G.GGUFFormatError, match="cannot open"):
        G.GGUF(tmp_path / "nope.gguf")


def test_null_arguments():
    from qxotic_amd._lib import lib
    L = lib()
    assert L.jamhip_gguf_tensor_count(None) == -1
    assert L.jamhip_gguf_find(None, b"x") == -1
    assert L.jamhip_gguf_pin(None, None, None, None, None) == 1
    assert L.jamhip_gguf_evict(None, None, None, None) == 1
    L.jamhip_gguf_close(None)
