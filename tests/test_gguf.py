"""GGUF files parsed by libmx (mx_gguf_open): metadata, tensor infos and the checks that refuse broken files. Host
logic only; the upload into the buffer type is in test_gpu_gguf.py."""
import numpy as np
import pytest

import oracle as O
from gguf_write import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64, as_bytes, gguf_bytes,
                        write_gguf)

KVS = [
    ("general.architecture", STRING, "qwen3-asr"),
    ("speech.layout", U32, 3),
    ("general.alignment", U32, 64),
    ("t.u8", U8, 250), ("t.i8", I8, -7), ("t.u16", U16, 65000), ("t.i16", I16, -300), ("t.i32", I32, -123456),
    ("t.f32", F32, 0.5), ("t.bool", BOOL, True), ("t.u64", U64, 2 ** 40 + 3), ("t.i64", I64, -(2 ** 50)),
    ("t.f64", F64, -1.25e-3),
    ("t.arr_i32", ARRAY, (I32, [1, -2, 3, 1 << 30])),
    ("t.arr_str", ARRAY, (STRING, ["a", "", "speech.cpp"])),
    ("t.empty", ARRAY, (F32, [])),
    ("t.empty_str", STRING, ""),
]


def weights_of(t, N, K, seed):
    return O.quantize_chunk(t, O.fill_normal(seed, N, K, 0.0, 0.02))


def tensor_set():
    """One tensor of each storage speech.cpp writes, plus a Q8_0 and an F16 fallback for rows that are not whole
    256-blocks (storage.cpp:52-89) and a type the device only holds (Q4_0)."""
    out = []
    for i, (name, t, K, N) in enumerate([("blk.0.attn_q.weight", O.TYPE_Q4_K, 512, 6), ("blk.0.ffn_down.weight", O.TYPE_Q6_K, 768, 3),
                          ("blk.0.attn_k.weight", O.TYPE_Q5_K, 256, 5), ("token_embd.weight", O.TYPE_Q8_0, 1024, 7),
                          ("blk.0.attn_norm.weight", O.TYPE_F32, 1024, 1), ("conv.weight", O.TYPE_F16, 96, 4),
                          ("proj.weight", O.TYPE_Q8_0, 160, 3)]):
        out.append((name, t, (K, N), as_bytes(weights_of(t, N, K, 0x5EED2000 + i))))
    out.append(("legacy.weight", 2, (64, 2), bytes(range(2 * 2 * 18))))  # Q4_0: 2 rows of 2 blocks of 18 bytes
    return out


def test_metadata_and_tensor_infos(mx, tmp_path):
    tensors = tensor_set()
    path = tmp_path / "m.gguf"
    data_start = write_gguf(path, KVS, tensors, alignment=64)
    with mx.Gguf(path) as g:
        assert g.keys() == [k for k, _, _ in KVS]
        assert g.get("general.architecture") == "qwen3-asr"
        assert g.get("speech.layout") == 3
        assert g.get("t.u8") == 250 and g.get("t.i8") == -7 and g.get("t.u16") == 65000 and g.get("t.i16") == -300
        assert g.get("t.i32") == -123456 and g.get("t.bool") is True
        assert g.get("t.u64") == 2 ** 40 + 3 and g.get("t.i64") == -(2 ** 50)
        assert g.get("t.f32") == 0.5 and g.get("t.f64") == -1.25e-3
        assert list(g.get("t.arr_i32")) == [1, -2, 3, 1 << 30]
        assert g.get("t.arr_str") == ["a", "", "speech.cpp"]
        assert g.get("t.empty").size == 0 and g.get("t.empty_str") == ""
        assert g.get("absent") is None
        assert g.data_offset == data_start and data_start % 64 == 0
        infos = g.tensors()
        assert [i["name"] for i in infos] == [t[0] for t in tensors]
        for info, (name, t, ne, data) in zip(infos, tensors):
            assert info["type"] == t and info["ne"] == tuple(ne) + (1,) * (4 - len(ne))
            assert info["n_dims"] == len(ne) and info["nbytes"] == len(data) and info["offset"] % 64 == 0
            raw = path.read_bytes()[data_start + info["offset"]:data_start + info["offset"] + info["nbytes"]]
            assert raw == data
        assert g.find_tensor("conv.weight") == 5 and g.find_tensor("nope") == -1


def test_version_2_and_default_alignment(mx, tmp_path):
    tensors = tensor_set()[:2]
    path = tmp_path / "v2.gguf"
    data_start = write_gguf(path, KVS[:2], tensors, version=2)
    with mx.Gguf(path) as g:
        assert g.data_offset == data_start and data_start % 32 == 0
        assert [i["offset"] % 32 for i in g.tensors()] == [0, 0]


def broken(tmp_path, name, blob):
    p = tmp_path / name
    p.write_bytes(blob)
    return p


@pytest.mark.parametrize("case", ["magic", "version", "truncated_header", "data_past_end", "misaligned", "unknown_type",
                                  "partial_block", "alignment", "counts", "string_length", "ndims", "wrapped_shape",
                                  "string_array"])
def test_broken_files_are_refused(mx, tmp_path, case):
    tensors = tensor_set()[:3]
    blob, start = gguf_bytes(KVS[:3], tensors, alignment=64)
    if case == "magic":
        blob = b"GGUX" + blob[4:]
        why = "does not start with GGUF"
    elif case == "version":
        blob = blob[:4] + (1).to_bytes(4, "little") + blob[8:]
        why = "version"
    elif case == "truncated_header":
        blob = blob[:start - 40]
        why = "header"
    elif case == "data_past_end":
        blob = blob[:-10]
        why = "past the end"
    elif case == "misaligned":
        blob, _ = gguf_bytes(KVS[:3], tensors, alignment=64, offsets=[0, 96, 4096])
        why = "not aligned"
    elif case == "unknown_type":
        blob, _ = gguf_bytes(KVS[:3], [(tensors[0][0], 99, tensors[0][2], tensors[0][3])], alignment=64)
        why = "does not know"
    elif case == "partial_block":
        blob, _ = gguf_bytes(KVS[:3], [("w", O.TYPE_Q4_K, (300, 2), bytes(2 * 144))], alignment=64)
        why = "whole blocks"
    elif case == "alignment":
        kv = [("general.alignment", U32, 48)]
        blob, _ = gguf_bytes(kv, tensors, alignment=48)
        why = "power of two"
    elif case == "counts":
        blob = blob[:8] + (1 << 60).to_bytes(8, "little") + blob[16:]
        why = "counts"
    elif case == "string_length":
        blob = blob[:24] + (1 << 50).to_bytes(8, "little") + blob[32:]   # the first key's length
        why = "string"
    elif case == "ndims":
        blob, _ = gguf_bytes(KVS[:3], [("w", O.TYPE_F32, (4, 1, 1, 1, 1), bytes(16))], alignment=64)
        why = "dimensions"
    elif case == "wrapped_shape":
        # 4 * 2^32 * 2^32 * 2^32 * 2^30 bytes is 2^128: exactly 0 in 128-bit arithmetic, so only checked multiplies
        # refuse it
        blob, _ = gguf_bytes(KVS[:3], [("w", O.TYPE_F32, (1 << 32, 1 << 32, 1 << 32, 1 << 30), bytes(64))],
                             alignment=64)
        why = "larger than the file"
    elif case == "string_array":
        # an array of strings whose count fits the remaining bytes but not 8 bytes of length per string
        kv = [("general.architecture", STRING, "x"), ("t.strs", ARRAY, (STRING, ["ab"] * 3))]
        blob, _ = gguf_bytes(kv, tensors[:1], alignment=64)
        at = blob.index(b"t.strs") + len(b"t.strs") + 4 + 4   # past the key, the value type and the element type
        blob = blob[:at] + (len(blob) - at - 16).to_bytes(8, "little") + blob[at + 8:]
        why = "an array runs past the end"
    with pytest.raises(mx.MxError) as e:
        mx.Gguf(broken(tmp_path, case + ".gguf", blob))
    assert why in str(e.value)


def test_missing_file(mx, tmp_path):
    with pytest.raises(mx.MxError) as e:
        mx.Gguf(tmp_path / "absent.gguf")
    assert "cannot open" in str(e.value)
