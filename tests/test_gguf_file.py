"""GGUF file reading and writing (tensor_amd.gguf.file), on the CPU.

The reader is pinned by files assembled byte by byte here with ``struct`` from the
public GGUF layout, independently of the module's writer; the writer is then
checked by reading its files back.  Malformed files must fail with GGUFError
before any out-of-range read.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest

from tensor_amd.gguf import file as G
from tensor_amd.gguf import quant as Q


def gstr(text: str) -> bytes:
    data = text.encode()
    return struct.pack("<Q", len(data)) + data


def assemble(kvs: bytes, n_kv: int, infos: bytes, n_tensors: int, data: bytes, *, alignment=32, version=3,
             magic=b"GGUF") -> bytes:
    head = magic + struct.pack("<IQQ", version, n_tensors, n_kv) + kvs + infos
    pad = -len(head) % alignment
    return head + bytes(pad) + data


def test_hand_assembled_file(tmp_path):
    rng = np.random.default_rng(0)
    q4k = Q.sample_weight(2, 512, Q.Q4_K, seed=3)  # 2 rows x 2 blocks x 144 B
    bias = rng.standard_normal(3).astype(np.float32)
    kvs = (gstr("general.architecture") + struct.pack("<I", G.STRING) + gstr("qwen3")
           + gstr("general.alignment") + struct.pack("<I", G.UINT32) + struct.pack("<I", 64)
           + gstr("qwen3.block_count") + struct.pack("<I", G.UINT32) + struct.pack("<I", 36)
           + gstr("tokens") + struct.pack("<I", G.ARRAY) + struct.pack("<IQ", G.STRING, 2) + gstr("a") + gstr("bc")
           + gstr("ids") + struct.pack("<I", G.ARRAY) + struct.pack("<IQ", G.INT32, 3) + struct.pack("<3i", -1, 0, 7)
           + gstr("flag") + struct.pack("<I", G.BOOL) + b"\x01"
           + gstr("eps") + struct.pack("<I", G.FLOAT32) + struct.pack("<f", 1e-6))
    infos = (gstr("blk.0.ffn_gate.weight") + struct.pack("<I", 2) + struct.pack("<2Q", 512, 2)
             + struct.pack("<IQ", 12, 0)
             + gstr("output_norm.bias") + struct.pack("<I", 1) + struct.pack("<Q", 3) + struct.pack("<IQ", 0, 576))
    data = q4k.tobytes() + bias.tobytes()  # 576 = 9 * 64: the bias starts aligned
    path = tmp_path / "hand.gguf"
    path.write_bytes(assemble(kvs, 7, infos, 2, data, alignment=64))
    with G.read(path) as f:
        assert f.version == 3 and f.alignment == 64 and f.data_offset % 64 == 0
        assert f.metadata["general.architecture"] == "qwen3" and f.metadata["qwen3.block_count"] == 36
        assert f.metadata["tokens"] == ["a", "bc"] and f.metadata["flag"] is True
        assert f.metadata["ids"].tolist() == [-1, 0, 7] and abs(f.metadata["eps"] - 1e-6) < 1e-12
        gate = f.tensors["blk.0.ffn_gate.weight"]
        assert (gate.shape, gate.ggml_type, gate.type_name, gate.nbytes) == ((2, 512), 12, "q4_k", 576)
        raw = f.raw("blk.0.ffn_gate.weight")
        assert raw.shape == (2, 288) and raw.dtype == np.uint8 and not raw.flags.writeable
        assert np.array_equal(raw, q4k)
        assert np.array_equal(f.raw("output_norm.bias"), bias)
        del raw


@pytest.mark.parametrize("encoding", ["q4_k", "q6_k", "q8_0", "q4_0"])
def test_writer_round_trip(tmp_path, encoding):
    code = Q.ggml_type(encoding)
    weight = Q.sample_weight(5, 1024, code, seed=7)
    norm = np.linspace(-1, 1, 1024, dtype=np.float32)
    meta = {"general.name": "tiny", "count": 3, "big": -(1 << 40), "ratio": 0.5, "on": False,
            "names": ["x", "yz"], "ids": np.arange(4, dtype=np.int64), "u": G.Value(G.UINT8, 200)}
    path = G.write(tmp_path / "w.gguf", {"w": (code, (1024, 5), weight), "norm": norm,
                                         "h": np.ones((2, 3), np.float16)}, meta, alignment=128)
    with G.read(path) as f:
        assert f.alignment == 128
        assert np.array_equal(f.raw("w"), weight) and f.tensors["w"].shape == (5, 1024)
        assert np.array_equal(f.raw("norm"), norm)
        assert f.raw("h").shape == (2, 3) and f.raw("h").dtype == np.float16
        assert f.metadata["count"] == 3 and f.metadata_types["count"] == G.UINT32
        assert f.metadata["big"] == -(1 << 40) and f.metadata_types["big"] == G.INT64
        assert f.metadata["ratio"] == 0.5 and f.metadata["on"] is False and f.metadata["names"] == ["x", "yz"]
        assert f.metadata["ids"].tolist() == [0, 1, 2, 3] and f.metadata["u"] == 200
        assert all(info.offset % 128 == 0 for info in f.tensors.values())


def test_block_sizes_of_every_known_type():
    # element counts and block bytes of the public GGML layouts
    assert {name: (qk, size) for name, qk, size in G.TENSOR_TYPES.values() if qk > 1} == {
        "q4_0": (32, 18), "q4_1": (32, 20), "q5_0": (32, 22), "q5_1": (32, 24), "q8_0": (32, 34),
        "q8_1": (32, 36), "q2_k": (256, 84), "q3_k": (256, 110), "q4_k": (256, 144), "q5_k": (256, 176),
        "q6_k": (256, 210), "q8_k": (256, 292)}
    for code, (qk, size) in Q.GEOMETRY.items():
        assert G.TENSOR_TYPES[code][1:] == (qk, size)
    assert G.tensor_nbytes(14, (4096, 3)) == 3 * 16 * 210


def test_unknown_tensor_types_are_listed_not_read(tmp_path):
    infos = gstr("iq") + struct.pack("<I", 1) + struct.pack("<Q", 256) + struct.pack("<IQ", 23, 0)
    path = tmp_path / "iq.gguf"
    path.write_bytes(assemble(b"", 0, infos, 1, bytes(64)))
    with G.read(path) as f:
        assert f.tensors["iq"].nbytes is None and f.tensors["iq"].type_name == "type23"
        with pytest.raises(G.GGUFError, match="does not know"):
            f.raw("iq")


def one_tensor(ne=(32,), ggml_type=8, offset=0, name="t"):
    return gstr(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne) + struct.pack("<IQ", ggml_type, offset)


@pytest.mark.parametrize("content,needle", [
    (assemble(b"", 0, b"", 0, b"", magic=b"GGML"), "magic"),
    (assemble(b"", 0, b"", 0, b"", version=1), "version"),
    (b"GGUF" + struct.pack("<IQ", 3, 0), "too small"),
    (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1 << 40), "truncated"),
    (b"GGUF" + struct.pack("<IQQ", 3, 1 << 50, 0) + bytes(8), "larger than the file"),
    (assemble(gstr("k") + struct.pack("<I", 99), 1, b"", 0, b""), "value type"),
    (assemble(gstr("k") + struct.pack("<I", G.BOOL) + b"\x02", 1, b"", 0, b""), "bool"),
    (assemble(gstr("k") + struct.pack("<IIQ", G.ARRAY, G.STRING, 1 << 40), 1, b"", 0, b""), "longer than"),
    (assemble(gstr("k") + struct.pack("<IIQ", G.ARRAY, G.ARRAY, 1) + struct.pack("<IQ", G.UINT8, 0), 1,
              b"", 0, b""), "nested"),
    (assemble((gstr("k") + struct.pack("<I", G.UINT8) + b"\x01") * 2, 2, b"", 0, b""), "duplicate metadata"),
    (assemble(gstr("general.alignment") + struct.pack("<II", G.UINT32, 24), 1, b"", 0, b""), "power-of-two"),
    (assemble(gstr("general.alignment") + struct.pack("<I", G.UINT64) + struct.pack("<Q", 64), 1, b"", 0, b""),
     "power-of-two"),
    (assemble(b"", 0, one_tensor(ne=(32, 1, 1, 1, 1)), 1, bytes(64)), "dimensions"),
    (assemble(b"", 0, one_tensor(ne=(0,)), 1, bytes(64)), "extent"),
    (assemble(b"", 0, one_tensor(ne=(48,)), 1, bytes(64)), "multiple of 32"),
    (assemble(b"", 0, one_tensor(offset=8), 1, bytes(64)), "aligned"),
    (assemble(b"", 0, one_tensor(ne=(64,)), 1, bytes(34)), "past the end"),
    (assemble(b"", 0, one_tensor() + one_tensor(offset=64), 2, bytes(128)), "duplicate tensor"),
])
def test_malformed_files_are_refused(tmp_path, content, needle):
    path = tmp_path / "bad.gguf"
    path.write_bytes(content)
    with pytest.raises(G.GGUFError, match=needle):
        G.read(path)


def test_invalid_utf8_names_are_refused(tmp_path):
    name = b"\xff\xfe"
    infos = struct.pack("<Q", len(name)) + name + struct.pack("<I", 1) + struct.pack("<Q", 32) + struct.pack("<IQ", 8, 0)
    path = tmp_path / "utf8.gguf"
    path.write_bytes(assemble(b"", 0, infos, 1, bytes(64)))
    with pytest.raises(G.GGUFError, match="UTF-8"):
        G.read(path)


def test_writer_refuses_inconsistent_tensors(tmp_path):
    with pytest.raises(G.GGUFError, match="bytes given"):
        G.write(tmp_path / "x.gguf", {"w": (Q.Q4_K, (256, 2), np.zeros(100, np.uint8))})
    with pytest.raises(G.GGUFError, match="multiple of 256"):
        G.write(tmp_path / "x.gguf", {"w": (Q.Q4_K, (200, 1), np.zeros(144, np.uint8))})
    with pytest.raises(G.GGUFError, match="explicit"):
        G.write(tmp_path / "x.gguf", {}, {"empty": []})
    with pytest.raises(G.GGUFError, match="power of two"):
        G.write(tmp_path / "x.gguf", {}, alignment=48)
