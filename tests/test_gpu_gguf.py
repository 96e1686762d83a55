"""GGUF files read into the MI355X buffer type (mx_gguf_load_tensor): every storage speech.cpp writes comes back
byte for byte, a tensor larger than one 16 MB piece lands whole, and products on loaded weights match the oracle."""
import os

import numpy as np
import pytest

import oracle as O
from gguf_write import STRING, U32, as_bytes, write_gguf
from helpers import rel_err

pytestmark = pytest.mark.gpu

TIGHT = 2e-5


def weights_of(t, N, K, seed):
    return O.quantize_chunk(t, O.fill_normal(seed, N, K, 0.0, 0.02))


def model_file(tmp_path):
    specs = [("token_embd.weight", O.TYPE_Q8_0, 2048, 8200),   # 17.8 MB: pieces split inside a block
             ("blk.0.attn_q.weight", O.TYPE_Q4_K, 1024, 96), ("blk.0.attn_k.weight", O.TYPE_Q5_K, 1024, 80),
             ("blk.0.ffn_down.weight", O.TYPE_Q6_K, 1536, 40), ("blk.0.attn_norm.weight", O.TYPE_F32, 1024, 1),
             ("audio.conv.weight", O.TYPE_F16, 200, 48),       # rows of 200: no K-quant block fits, F16 fallback
             ("audio.proj.weight", O.TYPE_Q8_0, 160, 64)]      # rows of 160: the Q8_0 fallback
    tensors, host = [], {}
    for i, (name, t, K, N) in enumerate(specs):
        w = weights_of(t, N, K, 0x5EED2100 + i)
        host[name] = (t, K, N, w)
        tensors.append((name, t, (K, N), as_bytes(w)))
    tensors.append(("legacy.weight", 2, (64, 3), bytes(range(3 * 2 * 18))))   # Q4_0, held as bytes
    path = tmp_path / "model.gguf"
    write_gguf(path, [("general.architecture", STRING, "qwen3-asr"), ("speech.layout", U32, 3)], tensors)
    return path, tensors, host


def test_every_tensor_loads_byte_for_byte(mx, be, tmp_path):
    path, tensors, _ = model_file(tmp_path)
    with mx.Gguf(path) as g:
        for name, t, ne, data in tensors:
            T = g.load(be, name)
            assert T.type == t and T.ne[:2] == ne
            got = T.get_bytes()
            assert got.tobytes() == data, name
            T.free()


def test_products_on_loaded_weights(mx, be, tmp_path):
    path, _, host = model_file(tmp_path)
    with mx.Gguf(path) as g:
        for name in ("blk.0.attn_k.weight", "audio.conv.weight", "audio.proj.weight", "blk.0.ffn_down.weight"):
            t, K, N, w = host[name]
            W = g.load(be, name)
            x = O.fill_normal(0xAC702100 + K, 3, K)
            X = be.tensor(mx.F32, (K, 3), x)
            Y = be.tensor(mx.F32, (N, 3))
            be.mul_mat(W, X, Y)
            be.sync()
            assert rel_err(Y.numpy().reshape(3, N), O.mul_mat(t, w, x)) <= TIGHT, name
        t, K, N, tab = host["token_embd.weight"]
        E = g.load(be, "token_embd.weight")
        ids = np.array([0, 8199, 4100], np.int32)
        I = be.tensor(mx.I32, (3,), ids)
        D = be.tensor(mx.F32, (K, 3))
        be.get_rows(E, I, D)
        be.sync()
        assert np.array_equal(D.numpy().reshape(3, K), O.get_rows(t, tab, K, ids))


def test_short_file_is_reported(mx, be, tmp_path):
    """A file cut after it was opened: the load fails with a message naming the tensor and the bytes read, nothing
    aborts."""
    path, tensors, _ = model_file(tmp_path)
    g = mx.Gguf(path)
    try:
        os.truncate(path, os.path.getsize(path) - 100)
        info = g.tensors()[-1]                   # the last tensor's bytes are the ones cut
        T = be.tensor(info["type"], info["ne"])
        with pytest.raises(mx.MxError) as e:
            mx.check(mx.lib().mx_gguf_load_tensor(be.h, g.h, len(tensors) - 1, T.ref()))
        assert "ends past the end of the file" in str(e.value)
        wrong = be.tensor(mx.F32, (4, 4))
        with pytest.raises(mx.MxError):
            mx.check(mx.lib().mx_gguf_load_tensor(be.h, g.h, 0, wrong.ref()))
    finally:
        g.close()
