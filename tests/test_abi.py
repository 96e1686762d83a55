"""The C ABI: libmx.so loads, exports exactly what include/mx.h declares, and its host-side pieces behave (no GPU)."""
import pathlib
import re
import subprocess

import numpy as np
import pytest

import oracle as O

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "mx.h").read_text()
    return sorted(set(re.findall(r"MX_API\s+[\w\s\*]*?\b(mx_\w+)\s*\(", text)))


def test_header_declares_the_binding_list(mx):
    assert declared_symbols() == sorted(mx.EXPORTS)


def test_library_exports_every_declared_symbol(mx):
    out = subprocess.run(["nm", "-D", "--defined-only", str(mx.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = sorted(l.split()[-1] for l in out.splitlines() if " T " in l)
    assert exported == declared_symbols()
    L = mx.lib()
    for s in declared_symbols():
        assert hasattr(L, s)


def test_library_is_built_for_gfx950(mx):
    out = subprocess.run(["strings", str(mx.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    assert "gfx950" in out


def test_no_device_is_reported_cleanly_without_gpu(mx):
    if mx.device_count() > 0:
        pytest.skip("a GPU is visible")
    L = mx.lib()
    assert not L.mx_backend_init(0)
    assert "no device" in L.mx_last_error().decode()


def test_alloc_size_covers_every_plane(mx):
    for t, K, N in [(mx.Q8_0, 1024, 3), (mx.Q4_K, 2048, 5), (mx.Q5_K, 1536, 3), (mx.Q6_K, 6144, 7), (mx.Q6_K, 256, 1)]:
        d = mx.MxTensor()
        d.type = t
        for i, v in enumerate((K, N, 1, 1)):
            d.ne[i] = v
        nb = mx.contiguous_nb(t, (K, N, 1, 1))
        for i in range(4):
            d.nb[i] = nb[i]
        size = mx.lib().mx_tensor_alloc_size(d)
        nbytes = mx.row_size(t, K) * N
        assert nbytes <= size <= nbytes + 4 * 256
        assert size % 256 == 0


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_F16, O.TYPE_F32])
def test_host_quantizer_matches_oracle(mx, t):
    rng = np.random.default_rng(7 + t)
    for std in (0.02, 1.0, 3e-5):
        w = (rng.standard_normal((64, 512)) * std).astype(np.float32)
        w[1] = 0.0
        w[2, :256] = 0.0
        w[3] = np.abs(w[3])
        w[4] = -np.abs(w[4])
        assert np.array_equal(mx.quantize_chunk(t, w), O.quantize_chunk(t, w))


def test_generator_matches_oracle(mx):
    a = mx.fill_normal(0x5EED0010, 7, 1001, 0.0, 0.02)
    assert np.array_equal(a, O.fill_normal(0x5EED0010, 7, 1001, 0.0, 0.02))
    q = mx.quantize_normal(mx.Q6_K, 99, 16, 512, 0.02, nthreads=3)
    assert np.array_equal(q, O.quantize_chunk(O.TYPE_Q6_K, O.fill_normal(99, 16, 512, 0.0, 0.02)))


@pytest.mark.parametrize("name,t", [("q4_K_grid.json", O.TYPE_Q4_K), ("q5_K_grid.json", O.TYPE_Q5_K),
                                    ("q6_K_grid.json", O.TYPE_Q6_K)])
def test_host_quantizer_known_answer_blocks(mx, name, t):
    import json
    f = json.loads((ROOT / "tests" / "golden" / name).read_text())
    x = np.array(f["x"], np.float32)[None]
    assert mx.quantize_chunk(t, x)[0].tobytes().hex() == f["block"]


def test_host_q8_0_exact_blocks(mx):
    import json
    for c in json.loads((ROOT / "tests" / "golden" / "q8_0_exact.json").read_text()):
        assert mx.quantize_chunk(mx.Q8_0, np.array(c["x"], np.float32)[None])[0].tobytes().hex() == c["block"]


def test_supports_op_argmax(mx):
    """ARGMAX: F32 rows (16-byte aligned starts) in, one I32 per row out; anything else is declined (host logic)."""
    def desc(t, ne, nb, data=0x10000):
        d = mx.MxTensor()
        d.type = t
        for i in range(4):
            d.ne[i], d.nb[i] = ne[i], nb[i]
        d.data = data
        return d

    L = mx.lib()
    src = desc(mx.F32, (151936, 2, 1, 1), (4, 4 * 151936, 8 * 151936, 8 * 151936))
    dst = desc(mx.I32, (2, 1, 1, 1), (4, 8, 8, 8))
    assert L.mx_supports_op(mx.OP_ARGMAX, src, None, None, dst) == 1
    odd = desc(mx.F32, (1001, 2, 1, 1), (4, 4004, 8008, 8008))            # rows not 16-byte aligned
    assert L.mx_supports_op(mx.OP_ARGMAX, odd, None, None, dst) == 0
    padded = desc(mx.F32, (1001, 2, 1, 1), (4, 4032, 8064, 8064))
    assert L.mx_supports_op(mx.OP_ARGMAX, padded, None, None, dst) == 1
    wrong_dst = desc(mx.F32, (2, 1, 1, 1), (4, 8, 8, 8))
    assert L.mx_supports_op(mx.OP_ARGMAX, src, None, None, wrong_dst) == 0
    short_dst = desc(mx.I32, (1, 1, 1, 1), (4, 4, 4, 4))
    assert L.mx_supports_op(mx.OP_ARGMAX, src, None, None, short_dst) == 0
    q = desc(mx.Q8_0, (1024, 2, 1, 1), (34, 1088, 2176, 2176))
    assert L.mx_supports_op(mx.OP_ARGMAX, q, None, None, dst) == 0


def desc_contig(mx, t, ne, data=0x10000):
    d = mx.MxTensor()
    d.type = t
    nb = mx.contiguous_nb(t, ne)
    for i in range(4):
        d.ne[i] = ne[i]
        d.nb[i] = nb[i]
    d.data = data
    return d


def test_supports_op_weight_types(mx):
    """Q5_K joins the quantized weights on every op; F16 / F32 weights take MUL_MAT and GET_ROWS (rows of whole
    16-byte loads) but not MUL_MAT_ID, whose experts are quantized (host logic only)."""
    L = mx.lib()
    ok = lambda op, a, b, c, d: L.mx_supports_op(op, a, b, c, d) != 0
    for t, K in [(mx.Q5_K, 512), (mx.F16, 1000), (mx.F32, 1004)]:
        W = desc_contig(mx, t, (K, 48, 1, 1))
        X = desc_contig(mx, mx.F32, (K, 3, 1, 1))
        Y = desc_contig(mx, mx.F32, (48, 3, 1, 1))
        assert ok(mx.OP_MUL_MAT, W, X, None, Y)
        I = desc_contig(mx, mx.I32, (5, 1, 1, 1))
        G = desc_contig(mx, mx.F32, (K, 5, 1, 1))
        assert ok(mx.OP_GET_ROWS, W, I, None, G)
        E = desc_contig(mx, t, (K, 48, 4, 1))
        B = desc_contig(mx, mx.F32, (K, 1, 6, 1))
        ids = desc_contig(mx, mx.I32, (2, 6, 1, 1))
        D = desc_contig(mx, mx.F32, (48, 2, 6, 1))
        assert ok(mx.OP_MUL_MAT_ID, E, B, ids, D) == (t == mx.Q5_K)
    # F16 rows must hold whole 8-element loads, F32 rows whole 4-element ones
    W = desc_contig(mx, mx.F16, (1004, 8, 1, 1))
    X = desc_contig(mx, mx.F32, (1004, 1, 1, 1))
    Y = desc_contig(mx, mx.F32, (8, 1, 1, 1))
    assert not ok(mx.OP_MUL_MAT, W, X, None, Y)
    W = desc_contig(mx, mx.F32, (1004, 8, 1, 1), data=0x10008)   # data not 16-byte aligned
    assert not ok(mx.OP_MUL_MAT, W, X, None, Y)


def test_supports_op_get_rows_row_bound(mx):
    """GET_ROWS indexes its output rows with 32 bits: 2^31 - 1 rows are accepted, 2^31 declined (host logic only)."""
    L = mx.lib()
    W = desc_contig(mx, mx.Q8_0, (64, 10, 1, 1))
    for n, want in [((1 << 31) - 1, 1), (1 << 31, 0)]:
        I = desc_contig(mx, mx.I32, (n, 1, 1, 1))
        G = desc_contig(mx, mx.F32, (64, n, 1, 1))
        assert L.mx_supports_op(mx.OP_GET_ROWS, W, I, None, G) == want
