"""Pins of the CPU oracle (oracle/mx_oracle.c), each against something other than the oracle's own formula.

ggml is not available to run (an empty submodule in the reference), and the reference's own tests of this path need
model files and dumps that are not in its tree, so the oracle is pinned by:
  * IEEE binary16 as numpy implements it (every fp16 value, every midpoint, the overflow edge);
  * known-answer blocks whose bytes follow from the block layout and arithmetic alone (tests/golden/, written by
    tests/golden/make_golden.py without the oracle);
  * an independent numpy decoder of every block layout, compared bit for bit with the oracle's dequantizers;
  * exact float64 brute force over independently decoded values for every dot, MUL_MAT, MUL_MAT_ID and GET_ROWS;
  * invariants (bsums = sums of quants, quantize(dequantize(b)) == b for full-range Q8_0 blocks);
  * mutation checks: a plausible mistake (swapped nibbles, a dropped min term, a wrong scale index) fails the checks;
  * for the K-quant weight quantizers on generic data: every code is the nearest point of its sub-block's grid given
    the packed scales; the packed 6-bit (Q4_K / Q5_K) and int8 (Q6_K) scales and d / dmin are the roundings of the
    sub-block fits; make_qx_quants's fit is the best of its candidate family (evaluated in float64); make_qkx2_quants
    agrees bit for bit with an independent numpy statement, never loses to its min-max start, returns the weighted
    least-squares fit of its own codes (or the start, forced on exact-grid sub-blocks), and returns codes that are the
    rounding onto the start's or a family member's grid with the min in effect (every search path followed in
    float64) -- each with a mutation (another rmin, fewer steps, other weights, an unweighted fit, no min clamp,
    truncated codes, a min that never moves, a max that moves, a narrower family) shown to fail.
Parity unpinned (narrowly): where float32 and float64 differ by less than the float32 rounding -- a value within 2e-4
of a rounding boundary, two candidate errors within 1e-5 -- the float64 checks follow both outcomes, so which way
ggml's float32 loop goes there is fixed only by the two restatements (oracle and numpy). The kernels read whatever
bytes the quantizer wrote, so their parity does not depend on it.
"""
import json
import pathlib

import numpy as np
import pytest

import oracle as O

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def gold(name):
    return json.loads((GOLD / name).read_text())


def h2f(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------------------------- independent decoders
def decode(t, blocks: np.ndarray) -> np.ndarray:
    """Exact values (float64) of ggml blocks, written from ggml-common.h's layout comments."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, O.TSIZE[t])
    if t == O.TYPE_Q8_0:
        d = h2f(b[:, 0:2].copy().view(np.uint16)[:, 0]).astype(np.float64)
        q = b[:, 2:34].view(np.int8).astype(np.float64)
        return (d[:, None] * q).reshape(-1)
    if t == O.TYPE_Q4_K:
        d = h2f(b[:, 0:2].copy().view(np.uint16)[:, 0]).astype(np.float64)
        dmin = h2f(b[:, 2:4].copy().view(np.uint16)[:, 0]).astype(np.float64)
        s = b[:, 4:16].astype(np.int64)
        sc = np.zeros((len(b), 8), np.int64)
        mn = np.zeros((len(b), 8), np.int64)
        sc[:, :4] = s[:, 0:4] & 63
        mn[:, :4] = s[:, 4:8] & 63
        sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
        qs = b[:, 16:144].astype(np.int64)
        out = np.zeros((len(b), 256))
        for e in range(256):
            byte = qs[:, (e // 64) * 32 + e % 32]
            q = (byte >> 4) if (e // 32) % 2 else (byte & 0xF)
            out[:, e] = d * sc[:, e // 32] * q - dmin * mn[:, e // 32]
        return out.reshape(-1)
    if t == O.TYPE_Q5_K:
        d = h2f(b[:, 0:2].copy().view(np.uint16)[:, 0]).astype(np.float64)
        dmin = h2f(b[:, 2:4].copy().view(np.uint16)[:, 0]).astype(np.float64)
        s = b[:, 4:16].astype(np.int64)
        sc = np.zeros((len(b), 8), np.int64)
        mn = np.zeros((len(b), 8), np.int64)
        sc[:, :4] = s[:, 0:4] & 63
        mn[:, :4] = s[:, 4:8] & 63
        sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
        qh = b[:, 16:48].astype(np.int64)
        qs = b[:, 48:176].astype(np.int64)
        out = np.zeros((len(b), 256))
        for e in range(256):
            sub, pos = divmod(e, 32)
            byte = qs[:, (e // 64) * 32 + pos]
            q = ((byte >> 4) if sub % 2 else (byte & 0xF)) + 16 * ((qh[:, pos] >> sub) & 1)
            out[:, e] = d * sc[:, sub] * q - dmin * mn[:, sub]
        return out.reshape(-1)
    if t == O.TYPE_F16:
        return h2f(b.copy().view(np.uint16).reshape(-1)).astype(np.float64)
    if t == O.TYPE_F32:
        return b.copy().view(np.float32).reshape(-1).astype(np.float64)
    if t == O.TYPE_Q6_K:
        ql = b[:, 0:128].astype(np.int64)
        qh = b[:, 128:192].astype(np.int64)
        sc = b[:, 192:208].view(np.int8).astype(np.float64)
        d = h2f(b[:, 208:210].copy().view(np.uint16)[:, 0]).astype(np.float64)
        out = np.zeros((len(b), 256))
        for e in range(256):
            h, r = divmod(e, 128)
            quarter, l = divmod(r, 32)
            lb = ql[:, 64 * h + l + 32 * (quarter & 1)]
            lo = (lb & 0xF) if quarter < 2 else (lb >> 4)
            hb = (qh[:, 32 * h + l] >> (2 * quarter)) & 3
            out[:, e] = d * sc[:, e // 16] * ((lo | (hb << 4)) - 32)
        return out.reshape(-1)
    if t == O.TYPE_Q8_K:
        d = b[:, 0:4].copy().view(np.float32)[:, 0].astype(np.float64)
        q = b[:, 4:260].view(np.int8).astype(np.float64)
        return (d[:, None] * q).reshape(-1)
    raise ValueError(t)


# ------------------------------------------------------------------------------------------------------------- fp16
def test_fp16_to_fp32_every_value():
    L = O.lib()
    for h in range(65536):
        ref = np.array([h], np.uint16).view(np.float16).astype(np.float32)[0]
        got = L.orc_fp16_to_fp32(h)
        if np.isnan(ref):
            assert np.isnan(got)
        else:
            assert np.float32(got).view(np.uint32) == ref.view(np.uint32), hex(h)


def test_fp32_to_fp16_rne_against_numpy():
    L = O.lib()
    finite = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    vals = [finite, -finite]
    # midpoints between consecutive fp16 values (ties go to even) and one fp32 ulp either side of them
    mids = ((finite[:-1].astype(np.float64) + finite[1:].astype(np.float64)) / 2).astype(np.float32)
    vals += [mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0))]
    vals.append(np.array([65504.0, 65519.996, 65520.0, 7e4, 1e-8, 2.9802322e-08, 2.9802326e-08, 5.9604645e-08,
                          np.inf, 1e-40, 3e-38], np.float32))
    rng = np.random.default_rng(0)
    vals.append((rng.standard_normal(200000) * 10.0 ** rng.uniform(-9, 5, 200000)).astype(np.float32))
    x = np.concatenate(vals).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_fp32_to_fp16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------------------------------------ golden fixtures
def test_q8_0_exact_blocks():
    for c in gold("q8_0_exact.json"):
        x = np.array(c["x"], np.float32)[None]
        for r in (O.ROUND_REF, O.ROUND_X86):
            assert O.quantize_rows(O.TYPE_Q8_0, x, r)[0].tobytes().hex() == c["block"]
        blk = np.frombuffer(bytes.fromhex(c["block"]), np.uint8)
        assert np.array_equal(O.dequantize_rows(O.TYPE_Q8_0, blk[None], 32)[0], np.array(c["dequant"], np.float32))


def test_q8_rounding_ties():
    f = gold("q8_ties.json")
    x = np.array(f["x"], np.float32)[None]
    assert O.quantize_rows(O.TYPE_Q8_0, x, O.ROUND_REF)[0].tobytes().hex() == f["ref_block"]
    assert O.quantize_rows(O.TYPE_Q8_0, x, O.ROUND_X86)[0].tobytes().hex() == f["x86_block"]
    q81 = O.quantize_rows(O.TYPE_Q8_1, x, O.ROUND_REF)[0]
    ref = bytes.fromhex(f["ref_block"])
    assert q81[0:2].tobytes() == ref[0:2] and q81[4:].tobytes() == ref[2:]
    s = int(np.frombuffer(ref[2:], np.int8).astype(np.int64).sum())
    assert q81[2:4].view(np.uint16)[0] == np.float32(s * 1.0).astype(np.float16).view(np.uint16)  # s = d * sum, d = 1


def test_q8_K_first_of_tied_maxima():
    f = gold("q8_K_ties.json")
    x = np.array(f["x"], np.float32)[None]
    assert O.quantize_rows(O.TYPE_Q8_K, x)[0].tobytes().hex() == f["block"]
    # mutation: letting the later +3 set the scale flips every sign, which the fixture rejects
    flipped = O.quantize_rows(O.TYPE_Q8_K, -x)[0].tobytes().hex()
    assert flipped != f["block"]


@pytest.mark.parametrize("name,t", [("q4_K_grid.json", O.TYPE_Q4_K), ("q5_K_grid.json", O.TYPE_Q5_K),
                                    ("q6_K_grid.json", O.TYPE_Q6_K)])
def test_k_quant_grid_blocks(name, t):
    f = gold(name)
    x = np.array(f["x"], np.float32)[None]
    blk = np.frombuffer(bytes.fromhex(f["block"]), np.uint8)
    assert O.quantize_rows(t, x)[0].tobytes().hex() == f["block"]
    assert O.quantize_chunk(t, x)[0].tobytes().hex() == f["block"]
    deq = O.dequantize_rows(t, blk[None], 256)[0]
    assert np.array_equal(deq, np.array(f["dequant"], np.float32))
    assert np.array_equal(decode(t, blk), np.array(f["dequant"], np.float64))


def test_q5_K_grid_fixture_rejects_a_dropped_high_bit():
    """Mutation check: the Q5_K grid block without its qh plane (bit 4 of every code) no longer decodes to the grid,
    nor does one whose qh bits are read from the wrong sub-block."""
    f = gold("q5_K_grid.json")
    blk = bytearray.fromhex(f["block"])
    want = np.array(f["dequant"])
    dropped = bytearray(blk)
    dropped[16:48] = bytes(32)
    assert not np.array_equal(decode(O.TYPE_Q5_K, np.frombuffer(bytes(dropped), np.uint8)), want)
    rotated = bytearray(blk)
    rotated[16:48] = bytes(((v << 1) | (v >> 7)) & 0xFF for v in blk[16:48])
    assert not np.array_equal(decode(O.TYPE_Q5_K, np.frombuffer(bytes(rotated), np.uint8)), want)
    assert not np.array_equal(O.dequantize_rows(O.TYPE_Q5_K, np.frombuffer(bytes(dropped), np.uint8)[None], 256)[0],
                              want.astype(np.float32))


def test_f16_conversion_is_ieee_rounding():
    """F16 weights and the F16 activations ggml pairs with them: numpy's IEEE float32 -> float16 rounding."""
    x = np.concatenate([O.fill_normal(33, 4, 512), O.fill_normal(34, 1, 512) * np.float32(1e-6),
                        O.fill_normal(35, 1, 512) * np.float32(3e4)])
    q = O.quantize_rows(O.TYPE_F16, x)
    with np.errstate(over="ignore"):   # the last row runs past 65504 into inf on purpose
        h = x.astype(np.float16)
    assert np.isinf(h).any()
    assert np.array_equal(q.reshape(-1).view(np.uint16), h.view(np.uint16).reshape(-1))
    assert np.array_equal(O.dequantize_rows(O.TYPE_F16, q, 512), h.astype(np.float32))
    assert np.array_equal(O.quantize_rows(O.TYPE_F32, x).reshape(-1).view(np.float32), x.reshape(-1))


def test_grid_fixture_rejects_swapped_nibbles():
    f = gold("q4_K_grid.json")
    blk = bytearray.fromhex(f["block"])
    for i in range(16, 144):
        blk[i] = ((blk[i] & 0xF) << 4) | (blk[i] >> 4)
    assert not np.array_equal(decode(O.TYPE_Q4_K, np.frombuffer(bytes(blk), np.uint8)), np.array(f["dequant"]))


# ------------------------------------------------------------------------------------------ quantizer invariants
def test_q8_K_bsums_and_range():
    x = O.fill_normal(31, 8, 1024)
    x[1] = 0.0
    q = O.quantize_rows(O.TYPE_Q8_K, x).reshape(-1, 292)
    qs = q[:, 4:260].view(np.int8).astype(np.int64)
    bs = q[:, 260:292].copy().view(np.int16).astype(np.int64)
    assert np.array_equal(qs.reshape(-1, 16, 16).sum(axis=2), bs)
    assert qs.min() >= -128 and qs.max() <= 127
    assert np.all(q[4:8, :4].view(np.float32) == 0)  # the zero row's four blocks have d = 0


def test_q8_K_dequantize():
    """ggml's dequantize_row_q8_K (d * q in fp32): a row of k / 128 whose first largest magnitude is -127 / 128
    quantizes to d = 1 / 128, q = k and comes back exactly; random rows match the independent decoder rounded to
    fp32."""
    k = np.concatenate([np.arange(-127, 128), [127]]).astype(np.float32)
    x = (k / 128.0).astype(np.float32)[None]
    q = O.quantize_rows(O.TYPE_Q8_K, x)
    assert q[0, :4].view(np.float32)[0] == np.float32(1.0 / 128)
    assert np.array_equal(q[0, 4:260].view(np.int8), k.astype(np.int8))
    assert np.array_equal(O.dequantize_rows(O.TYPE_Q8_K, q, 256), x)
    y = O.fill_normal(33, 3, 512)
    qy = O.quantize_rows(O.TYPE_Q8_K, y)
    got = O.dequantize_rows(O.TYPE_Q8_K, qy, 512)
    assert np.array_equal(got.reshape(-1).view(np.uint32), decode(O.TYPE_Q8_K, qy.reshape(-1)).astype(np.float32).view(np.uint32))


def test_q8_0_roundtrip_full_range_blocks():
    rng = np.random.default_rng(8)
    q = rng.integers(-127, 128, size=(64, 32))
    q[:, 0] = 127
    d = (2.0 ** rng.integers(-12, 2, size=64)).astype(np.float32)
    blocks = np.concatenate([np.frombuffer(np.float16(di).tobytes(), np.uint8)[None].repeat(1, 0) for di in d])
    raw = np.concatenate([blocks, q.astype(np.int8).view(np.uint8)], axis=1)
    x = O.dequantize_rows(O.TYPE_Q8_0, raw.reshape(1, -1), 64 * 32)
    assert np.array_equal(O.quantize_rows(O.TYPE_Q8_0, x).reshape(-1), raw.reshape(-1))


def test_q8_matches_numpy_restatement():
    """quantize_row_q8_0_ref / _q8_1_ref against vectorized numpy float32 arithmetic."""
    x = np.concatenate([O.fill_normal(41, 16, 512), O.fill_normal(42, 2, 512) * np.float32(1e-5)])
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idf = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
        v = (xb * idf[:, None]).astype(np.float32)
    q_ref = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)   # roundf: half away from zero
    with np.errstate(divide="ignore"):
        idx = np.where(amax != 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
    q_x86 = np.rint((xb * idx[:, None]).astype(np.float32)).astype(np.int8)           # half to even
    dh = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    for r, q in ((O.ROUND_REF, q_ref), (O.ROUND_X86, q_x86)):
        want = np.concatenate([dh, q.view(np.uint8)], axis=1).reshape(-1)
        assert np.array_equal(O.quantize_rows(O.TYPE_Q8_0, x, r).reshape(-1), want)
        s = (q.astype(np.int64).sum(axis=1).astype(np.float32) * d).astype(np.float16).view(np.uint8).reshape(-1, 2)
        want1 = np.concatenate([dh, s, q.view(np.uint8)], axis=1).reshape(-1)
        assert np.array_equal(O.quantize_rows(O.TYPE_Q8_1, x, r).reshape(-1), want1)


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K])
def test_k_quant_weights_reconstruct(t):
    """Validity of the weight quantizers on generic data: field ranges and a reconstruction error of a 4/5/6-bit fit."""
    for std in (0.02, 1.0):
        w = O.fill_normal(50 + t, 32, 1024, 0.0, std)
        w[0] = 0.0
        q = O.quantize_chunk(t, w)
        deq = decode(t, q.reshape(-1))
        assert np.all(deq[:1024] == 0)
        err = np.sqrt(np.mean((deq - w.reshape(-1).astype(np.float64)) ** 2)) / std
        assert err < {O.TYPE_Q4_K: 0.12, O.TYPE_Q5_K: 0.06, O.TYPE_Q6_K: 0.03}[t]
        assert np.array_equal(O.dequantize_rows(t, q, 1024).reshape(-1), deq.astype(np.float32))


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_F16, O.TYPE_F32])
def test_dequantizers_match_independent_decoder(t):
    w = O.fill_normal(60 + t, 16, 512, 0.0, 0.02)
    q = O.quantize_chunk(t, w)
    assert np.array_equal(O.dequantize_rows(t, q, 512).reshape(-1), decode(t, q.reshape(-1)).astype(np.float32))


def test_quantize_chunk_row_offsets():
    w = O.fill_normal(70, 6, 512, 0.0, 0.02)
    for t in (O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_F16, O.TYPE_F32):
        full = O.quantize_chunk(t, w)
        out = np.zeros_like(full)
        L = O.lib()
        rs = O.row_size(t, 512)
        n = L.orc_quantize_chunk(t, w.ctypes.data, out.ctypes.data, 2 * 512, 3, 512)
        assert n == 3 * rs
        assert np.array_equal(out[2:5], full[2:5]) and not out[0].any() and not out[5].any()


# ------------------------------------------------------------------------------------------- dots and ops, brute force
def brute_dot(t, wq, aq):
    return float(np.dot(decode(t, wq), decode(O.VEC_DOT_TYPE[t], aq)))


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_F16, O.TYPE_F32])
def test_vec_dot_against_float64_brute_force(t):
    K = 2048
    w = O.quantize_chunk(t, O.fill_normal(80 + t, 8, K, 0.0, 0.02))
    x = O.fill_normal(90, 4, K)
    a = O.quantize_rows(O.VEC_DOT_TYPE[t], x)
    for i in range(8):
        for j in range(4):
            exact = brute_dot(t, w[i], a[j])
            scale = float(np.abs(decode(t, w[i])) @ np.abs(decode(O.VEC_DOT_TYPE[t], a[j])))
            assert abs(O.vec_dot(t, K, w[i], a[j]) - exact) <= 1e-6 * scale
            # scale products are fp32 in both variants (as ggml forms them): ~6e-8 relative per block
            assert abs(O.vec_dot(t, K, w[i], a[j], exact=True) - exact) <= 2e-7 * scale


def test_brute_force_catches_a_dropped_min_term():
    """Mutation check: the Q4_K dot without its dmin term is far outside the bound the test above uses."""
    K = 512
    w = O.quantize_chunk(O.TYPE_Q4_K, O.fill_normal(81, 1, K, 0.0, 0.02))[0]
    a = O.quantize_rows(O.TYPE_Q8_K, O.fill_normal(91, 1, K))[0]
    wb = bytearray(w.tobytes())
    wb[2:4] = b"\x00\x00"   # dmin = 0 in the first super-block drops its min term
    scale = float(np.abs(decode(O.TYPE_Q4_K, w)) @ np.abs(decode(O.TYPE_Q8_K, a)))
    assert abs(O.vec_dot(O.TYPE_Q4_K, K, np.frombuffer(bytes(wb), np.uint8), a) - brute_dot(O.TYPE_Q4_K, w, a)) > 1e-4 * scale


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_F16, O.TYPE_F32])
def test_mul_mat_is_the_product_of_decoded_operands(t):
    K, N, M = 512, 24, 5
    w = O.quantize_chunk(t, O.fill_normal(100 + t, N, K, 0.0, 0.02))
    x = O.fill_normal(101, M, K)
    y = O.mul_mat(t, w, x)
    W = decode(t, w.reshape(-1)).reshape(N, K)
    X = decode(O.VEC_DOT_TYPE[t], O.quantize_rows(O.VEC_DOT_TYPE[t], x).reshape(-1)).reshape(M, K)
    ref = X @ W.T
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("bcast", [True, False])
def test_mul_mat_id_routes_each_pair(bcast):
    t, K, N, E, k, T = O.TYPE_Q6_K, 256, 16, 5, 2, 4
    w = O.quantize_chunk(t, O.fill_normal(110, E * N, K, 0.0, 0.02)).reshape(E, N, -1)
    B = 1 if bcast else k
    x = O.fill_normal(111, T * B, K).reshape(T, B, K)
    ids = np.array([[4, 0], [1, 1], [2, 3], [0, 4]], np.int32)
    y = O.mul_mat_id(t, w, x, ids)
    for ti in range(T):
        for s in range(k):
            wi = decode(t, w[ids[ti, s]].reshape(-1)).reshape(N, K)
            xi = decode(O.TYPE_Q8_K, O.quantize_rows(O.TYPE_Q8_K, x[ti, s % B][None]).reshape(-1))
            ref = wi @ xi
            assert np.abs(y[ti, s] - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_F16, O.TYPE_F32])
def test_get_rows_is_the_decoded_row(t):
    K, R = 512, 9
    table = O.quantize_chunk(t, O.fill_normal(120 + t, R, K, 0.0, 0.02))
    ids = np.array([8, 0, 3, 3], np.int32)
    out = O.get_rows(t, table, K, ids)
    for i, r in enumerate(ids):
        assert np.array_equal(out[i], decode(t, table[r]).astype(np.float32))
    with pytest.raises(ValueError):
        O.get_rows(t, table, K, np.array([R], np.int32))


def test_cpu_fast_port_agrees_with_oracle():
    if not O.fast().cpf_have_avx2():
        pytest.skip("no AVX2 on this host")
    for t in (O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q6_K):
        w = O.quantize_chunk(t, O.fill_normal(130 + t, 70, 1024, 0.0, 0.02))
        x = O.fill_normal(131, 3, 1024)
        y = O.cpu_fast_mul_mat(t, w, x, 4)
        ref = O.mul_mat(t, w, x, rounding=O.ROUND_X86)
        assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


# ------------------------------------------------------------------------------------------------------------ argmax
def test_argmax_first_of_ties_against_numpy():
    """numpy's argmax also returns the first of equal maxima: on NaN-free rows the two must agree everywhere."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((64, 1003)).astype(np.float32)
    x[1:8, [3, 500, 1002]] = 9.0             # the max three times: the first wins
    x[8, :] = 1.5                            # all equal: index 0
    x[9, :] = -np.inf                        # all -inf: index 0
    x[10, 1002] = np.inf
    x[11, [0, 1]] = [0.0, 7.0]
    x[11, 2] = 7.0
    x[12] = np.round(x[12])                  # many ties among small integers
    assert np.array_equal(O.argmax(x), np.argmax(x, axis=1).astype(np.int32))


def test_argmax_known_answers():
    """NaN never compares greater (first_argmax's `v[i] > v[best]`): the cases numpy would answer differently."""
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    rows = [([nan, 1.0, 2.0, 3.0], 0),       # NaN at index 0: nothing is greater than it
            ([1.0, nan, 3.0, 3.0], 2),       # NaN elsewhere is passed over; the first of the two 3s
            ([nan, nan, nan, nan], 0),
            ([-inf, -inf, -inf, nan], 0),
            ([0.0, -0.0, 0.0, -1.0], 0),     # 0 and -0 are equal: the first
            ([-0.0, 0.0, 5.0, inf], 3),
            ([2.0, 1.0, nan, 2.0], 0)]
    x = np.array([r for r, _ in rows], np.float32)
    assert O.argmax(x).tolist() == [a for _, a in rows]


# ------------------------------------------------------------------ the K-quant candidate searches on generic data
# make_qkx2_quants (Q4_K: nmax 15, rmin -1, rdelta 0.1, 20 steps; Q5_K: nmax 31, rmin -0.5, 15 steps) and
# make_qx_quants (Q6_K) each return the best of a fixed family of candidate fits. On generic data nothing but ggml
# could give their bytes, so these checks pin the searches by optimality instead: the oracle's answer must be the
# best member (within float32 noise) of the family as defined, evaluated independently in float64 numpy, and the
# packed block must be the rounding of those fits. Mutation checks show that a search over a wrong family (another
# rmin, fewer steps, other weights) fails the same check.
QKX2 = {O.TYPE_Q4_K: (15, -1.0, 0.1, 20), O.TYPE_Q5_K: (31, -0.5, 0.1, 15)}


def subblocks(n, size, seed):
    """Sub-blocks of several shapes: normal, shifted so every value is positive or negative, heavy-tailed, small."""
    base = O.fill_normal(seed, n, size, 0.0, 1.0).astype(np.float64)
    out = []
    for i, r in enumerate(base):
        kind = i % 5
        r = {0: r, 1: r + 2.5, 2: r - 2.5, 3: r ** 3, 4: r * 1e-3}[kind]
        out.append(r.astype(np.float32))
    return np.stack(out)


def kquant_weights(x):
    """quantize_row_q4_K_ref's weights of a 32-value sub-block: sqrt(mean of squares) + |x|, summed in order in float32."""
    av = np.sqrt(np.cumsum(x * x, dtype=np.float32)[-1] / np.float32(32))
    return (av + np.abs(x)).astype(np.float32)


def qkx2_numpy(x, w, nmax, rmin, rdelta, nstep, mutate=None):
    """make_qkx2_quants (use_mad = 0) restated in numpy from ggml's description, each candidate's codes vectorized and
    its sums taken in order in float32 (np.cumsum), as the C loop takes them: start from the min-max fit (min clamped
    to <= 0), then for is = 0..nstep round x - min with iscale = (nmax + rmin + rdelta is) / (max - min), fit the
    weighted least-squares (scale, min) of those codes (min > 0: min = 0 and the scale alone), and keep the fit whose
    weighted squared error is smaller -- min and the span max - min follow the fit kept. Returns (scale, min, codes).
    `mutate` plants one mistake, for the tests that must reject it: "fit_unweighted" (the fit ignores the weights),
    "no_clamp" (a positive min is kept), "floor" (codes truncated instead of rounded), "min_fixed" (later candidates
    keep the start's min), "max_moves" (the span's top follows the kept fit too)."""
    f32 = np.float32
    seq = lambda v: np.cumsum(v, dtype=f32)[-1]
    lo, hi = min(f32(x.min()), f32(0)), f32(x.max())
    if hi == lo:
        return f32(0), lo, np.zeros(x.size, np.uint8)
    iscale = f32(nmax) / (hi - lo)
    scale = f32(1) / iscale
    L = np.clip(np.rint(iscale * (x - lo)), 0, nmax).astype(np.uint8)
    best = seq(w * (scale * L.astype(f32) + lo - x) ** 2)
    lo0 = lo
    rnd = np.floor if mutate == "floor" else np.rint
    for i in range(nstep + 1):
        base = lo0 if mutate == "min_fixed" else lo
        isc = (f32(rmin) + f32(rdelta) * f32(i) + f32(nmax)) / (hi - base)
        l = np.clip(rnd(isc * (x - base)), 0, nmax).astype(f32)
        wf = np.ones_like(w) if mutate == "fit_unweighted" else w
        sw, sx = seq(wf), seq(wf * x)
        sl, sl2, sxl = seq(wf * l), seq(wf * l * l), seq(wf * l * x)
        D = sw * sl2 - sl * sl
        if D > 0:
            sc, mn = (sw * sxl - sx * sl) / D, (sl2 * sx - sl * sxl) / D
            if mn > 0 and mutate != "no_clamp":
                mn, sc = f32(0), sxl / sl2
            err = seq(w * (sc * l + mn - x) ** 2)
            if err < best:
                L, best, scale, lo = l.astype(np.uint8), err, sc, mn
                if mutate == "max_moves":
                    hi = f32(sc * f32(nmax) + mn)
    return scale, lo, L


def qkx2_differs(t, xs, search):
    """Indices of the sub-blocks where search(x, w) -> (scale, min, codes) differs from the numpy restatement."""
    nmax, rmin, rdelta, nstep = QKX2[t]
    bad = []
    for i, x in enumerate(xs):
        w = kquant_weights(x)
        s, m, L = search(x, w)
        s2, m2, L2 = qkx2_numpy(x, w, nmax, rmin, rdelta, nstep)
        if not (np.float32(s) == s2 and np.float32(m) == m2 and np.array_equal(L, L2)):
            bad.append(i)
    return bad


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q5_K], ids=["q4_K", "q5_K"])
def test_make_qkx2_quants_matches_a_numpy_restatement(t):
    """The oracle's search and an independent numpy statement of it agree bit for bit on 600 sub-blocks of five
    shapes, and its fit is never worse than the min-max fit it starts from; a search with another rmin, fewer steps
    or uniform weights differs on many of them. (Both statements follow ggml's published algorithm; ggml's own C is
    not here to run, so a misreading shared by both would pass: parity unpinned at that point.)"""
    nmax, rmin, rdelta, nstep = QKX2[t]
    xs = subblocks(600, 32, 0x0A11 + t)
    ours = lambda x, w: O.make_qkx2_quants(x, w, nmax, rmin, rdelta, nstep)
    assert qkx2_differs(t, xs, ours) == []
    for x in xs:
        w = kquant_weights(x)
        s, m, L = ours(x, w)
        lo, hi = min(float(x.min()), 0.0), float(x.max())
        if hi == lo:
            continue
        wd, xd = w.astype(np.float64), x.astype(np.float64)
        l0 = np.clip(np.rint(np.float32(nmax) / np.float32(hi - lo) * (x - np.float32(lo))), 0, nmax)
        e0 = np.sum(wd * ((hi - lo) / nmax * l0 + lo - xd) ** 2)
        assert np.sum(wd * (float(s) * L + float(m) - xd) ** 2) <= e0 * (1 + 1e-5) + 1e-30
    for wrong in (lambda x, w: O.make_qkx2_quants(x, w, nmax, rmin + 0.5, rdelta, nstep),
                  lambda x, w: O.make_qkx2_quants(x, w, nmax, rmin, rdelta, nstep - 5),
                  lambda x, w: O.make_qkx2_quants(x, np.ones_like(w), nmax, rmin, rdelta, nstep)):
        assert len(qkx2_differs(t, xs, wrong)) >= 30


def lsq_fit64(x, w, L):
    """The weighted least-squares (scale, min) of x ~ scale * L + min, in float64 from the normal equations; a positive
    min is set to 0 and the scale fitted alone (make_qkx2_quants' rule: a K-quant min is stored as -min >= 0). None when
    the codes cannot fix two parameters (all equal)."""
    xd, wd, ld = x.astype(np.float64), w.astype(np.float64), L.astype(np.float64)
    sw, sl, sl2 = wd.sum(), (wd * ld).sum(), (wd * ld * ld).sum()
    sx, sxl = (wd * xd).sum(), (wd * ld * xd).sum()
    D = sw * sl2 - sl * sl
    if D <= 1e-12 * sw * sl2:
        return None
    s, m = (sw * sxl - sx * sl) / D, (sl2 * sx - sl * sxl) / D
    if m > 0:
        m, s = 0.0, sxl / sl2
    return s, m


def grid_roundings(v, nmax, tol):
    """Codes clip(rint(v), 0, nmax), and the variants with values lying within tol of a rounding boundary rounded the
    other way (float32 arithmetic may land on either side where float64 is this close)."""
    import itertools
    base = np.clip(np.rint(v), 0, nmax)
    near = np.nonzero(np.abs(v - np.floor(v) - 0.5) < tol)[0]
    out = [base]
    for r in range(1, len(near) + 1):
        for sub in itertools.combinations(near, r):
            L = base.copy()
            for i in sub:
                L[i] = np.clip(np.ceil(v[i]) if base[i] == np.floor(v[i]) else np.floor(v[i]), 0, nmax)
            out.append(L)
    return out


def qkx2_paths(x, w, nmax, rmin, rdelta, nstep, tol_v=2e-4, tol_e=1e-5):
    """Every (kind, codes) make_qkx2_quants can end with on this sub-block, from its definition evaluated in float64:
    kind "start" (the min-max fit, no candidate better) or "fit" (the codes of the last candidate kept). Candidate is
    rounds x - min onto iscale = (nmax + rmin + rdelta is) / (max - min) with the min of the fit kept last (the start's
    min, min(x) clamped to <= 0, before any), and is kept when the weighted squared error of its least-squares fit is
    below the best so far. Where float64 cannot decide how float32 arithmetic goes -- a value within tol_v of a rounding
    boundary, two errors within tol_e of each other -- both outcomes are followed."""
    xd, wd = x.astype(np.float64), w.astype(np.float64)
    lo, hi = min(xd.min(), 0.0), xd.max()
    if hi == lo:
        return [("flat", np.zeros(x.size))]
    states = []
    for L in grid_roundings(nmax / (hi - lo) * (xd - lo), nmax, tol_v):
        states.append((lo, float(np.sum(wd * ((hi - lo) / nmax * L + lo - xd) ** 2)), ("start", L)))
    for i in range(nstep + 1):
        new = []
        for mp, best, src in states:
            isc = (rmin + rdelta * i + nmax) / (hi - mp)
            for L in grid_roundings(isc * (xd - mp), nmax, tol_v):
                f = lsq_fit64(x, w, L)
                if f is None:
                    new.append((mp, best, src))
                    continue
                e = float(np.sum(wd * (f[0] * L + f[1] - xd) ** 2))
                if e <= best * (1 + tol_e):
                    new.append((f[1], e, ("fit", L)))
                if e >= best * (1 - tol_e):
                    new.append((mp, best, src))
        seen, states = set(), []
        for st in new:
            key = (round(st[0], 12), st[2][0], st[2][1].tobytes())
            if key not in seen:
                seen.add(key)
                states.append(st)
        assert len(states) <= 512
    return [st[2] for st in states]


def qkx2_fit_ok(x, w, nmax, s, m, L):
    """Property 1: the returned (scale, min) is the weighted least-squares fit of the returned codes (to float32
    summation: 2e-5 of the scale, 2e-5 of the span for the min), or the min-max start with its own codes."""
    lo, hi = min(float(x.min()), 0.0), float(x.max())
    if hi == lo:
        return float(s) == 0.0 and not L.any()
    f32 = np.float32
    isc0 = f32(nmax) / (f32(hi) - f32(lo))
    L0 = np.clip(np.rint(isc0 * (x - f32(lo))), 0, nmax)
    if np.array_equal(L, L0) and float(m) == lo and float(s) == float(f32(1) / isc0):
        return True
    f = lsq_fit64(x, w, L)
    return f is not None and abs(float(s) - f[0]) <= 2e-5 * abs(f[0]) and abs(float(m) - f[1]) <= 2e-5 * (hi - lo)


def qkx2_codes_ok(x, w, nmax, rmin, rdelta, nstep, L):
    """Property 2: the returned codes are the clamped rounding of x - min onto the start's grid or onto one family
    member's, iscale = (nmax + rmin + rdelta is) / (max - min), with the min in effect when that candidate ran."""
    return any(np.array_equal(L, c) for _, c in qkx2_paths(x, w, nmax, rmin, rdelta, nstep))


def grid_subblocks(n, nmax, seed):
    """Sub-blocks whose values lie on a min-max grid exactly (a multiple of a power of two): the start fit is exact,
    so no candidate can do better and make_qkx2_quants must return it."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        codes = rng.integers(0, nmax + 1, 32)
        codes[0], codes[1] = 0, nmax
        out.append((codes * 2.0 ** -int(rng.integers(4, 9))).astype(np.float32))
    return out


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q5_K], ids=["q4_K", "q5_K"])
def test_make_qkx2_quants_fit_and_codes_properties(t):
    """What the mathematics fixes of make_qkx2_quants, checked in float64 apart from the oracle's float32 loop:
    (1) its (scale, min) is the weighted least-squares fit of its codes (a positive min clamped to 0 and the scale
    refitted), or the min-max start when no candidate was better (exact-grid sub-blocks force that case);
    (2) its codes are the start's rounding or one family member's, taken with the min of the fit kept before it.
    Each property has mutations of the search that it rejects (planted in the numpy restatement, on the CPU). What
    stays open without ggml: which way float32 breaks the near-ties that (2) follows both ways."""
    nmax, rmin, rdelta, nstep = QKX2[t]
    xs = list(subblocks(300, 32, 0x0C11 + t))
    grid = grid_subblocks(20, nmax, 0x0C51 + t)
    for x in xs + grid:
        w = kquant_weights(x)
        s, m, L = O.make_qkx2_quants(x, w, nmax, rmin, rdelta, nstep)
        assert qkx2_fit_ok(x, w, nmax, s, m, L)
        assert qkx2_codes_ok(x, w, nmax, rmin, rdelta, nstep, L)
    for x in grid:
        w = kquant_weights(x)
        s, m, L = O.make_qkx2_quants(x, w, nmax, rmin, rdelta, nstep)
        f32 = np.float32
        isc0 = f32(nmax) / (f32(x.max()) - min(f32(x.min()), f32(0)))
        assert float(s) == float(f32(1) / isc0) and float(m) == min(float(x.min()), 0.0)
        assert np.array_equal(L, np.clip(np.rint(isc0 * (x - min(f32(x.min()), f32(0)))), 0, nmax))
    # teeth: each planted mistake is rejected by the property it breaks, on many sub-blocks
    def rejected(mutate, check):
        n = 0
        for x in xs:
            w = kquant_weights(x)
            s, m, L = qkx2_numpy(x, w, nmax, rmin, rdelta, nstep, mutate=mutate)
            n += not (qkx2_fit_ok(x, w, nmax, s, m, L) if check == 1 else
                      qkx2_codes_ok(x, w, nmax, rmin, rdelta, nstep, L))
        return n
    assert rejected(None, 1) == 0 and rejected(None, 2) == 0
    assert rejected("fit_unweighted", 1) >= 100
    assert rejected("no_clamp", 1) >= 15
    assert rejected("floor", 2) >= 100
    assert rejected("min_fixed", 2) >= 10
    assert rejected("max_moves", 2) >= 10


def qx_objective(x, l):
    """make_qx_quants's figure of merit for codes l (x^2 weights): (sum w x l)^2 / sum w l^2, the weighted error it
    saves with the least-squares scale."""
    xd, ld = x.astype(np.float64), l.astype(np.float64)
    w = xd * xd
    s2 = float(np.sum(w * ld * ld))
    return float(np.sum(w * xd * ld)) ** 2 / s2 if s2 > 0 else 0.0


def qx_best(x, nmax, steps):
    """The best figure of merit over make_qx_quants's candidates iscale = -(nmax + 0.1 is) / max, is in steps, where
    max is the value of largest magnitude and codes are clamped to [-nmax, nmax - 1]."""
    mx = x[np.argmax(np.abs(x))]
    best = 0.0
    for i in steps:
        isc = -(np.float32(nmax) + np.float32(0.1) * np.float32(i)) / mx
        l = np.clip(np.rint(np.float32(isc) * x), -nmax, nmax - 1)
        best = max(best, qx_objective(x, l))
    return best


def test_make_qx_quants_is_the_best_of_its_candidates():
    xs = subblocks(800, 16, 0x0B11)
    steps = range(-9, 10)
    for x in xs:
        s, l = O.make_qx_quants(x, 32)
        assert np.all((l >= -32) & (l <= 31))
        obj = qx_objective(x, l)
        assert obj >= qx_best(x, 32, steps) * (1 - 1e-5)
        xd, ld = x.astype(np.float64), l.astype(np.float64)
        assert abs(float(s) - np.sum(xd ** 3 * ld) / np.sum(xd * xd * ld * ld)) <= 1e-5 * abs(float(s))
    # teeth: the best over a narrower family (is in -5..5) falls short of the full family's on some blocks, so an
    # oracle searching that family would fail the check above
    short = sum(qx_best(x, 32, range(-5, 6)) < qx_best(x, 32, steps) * (1 - 1e-5) for x in xs)
    assert short >= 3


def kquant_fields(t, blocks):
    """Per block of Q4_K / Q5_K / Q6_K bytes: d, dmin (float32 of the fp16 fields), the sub-block scales and mins as
    integers, and the 256 codes, decoded from ggml-common.h's layout."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, O.TSIZE[t])
    n = len(b)
    q = np.zeros((n, 256), np.int64)
    if t == O.TYPE_Q6_K:
        ql, qh = b[:, 0:128].astype(np.int64), b[:, 128:192].astype(np.int64)
        sc = b[:, 192:208].view(np.int8).astype(np.int64)
        d = h2f(b[:, 208:210].copy().view(np.uint16)[:, 0])
        for e in range(256):
            h, r = divmod(e, 128)
            quarter, l = divmod(r, 32)
            lb = ql[:, 64 * h + l + 32 * (quarter & 1)]
            q[:, e] = ((lb & 0xF) if quarter < 2 else (lb >> 4)) | (((qh[:, 32 * h + l] >> (2 * quarter)) & 3) << 4)
        return dict(d=d, sc=sc, q=q)
    d = h2f(b[:, 0:2].copy().view(np.uint16)[:, 0])
    dmin = h2f(b[:, 2:4].copy().view(np.uint16)[:, 0])
    s = b[:, 4:16].astype(np.int64)
    sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)], axis=1)
    mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
    qs = b[:, 16:144].astype(np.int64) if t == O.TYPE_Q4_K else b[:, 48:176].astype(np.int64)
    for e in range(256):
        sub, pos = divmod(e, 32)
        byte = qs[:, (e // 64) * 32 + pos]
        q[:, e] = (byte >> 4) if sub % 2 else (byte & 0xF)
        if t == O.TYPE_Q5_K:
            q[:, e] += 16 * ((b[:, 16 + pos].astype(np.int64) >> sub) & 1)
    return dict(d=d, dmin=dmin, sc=sc, mn=mn, q=q)


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q5_K], ids=["q4_K", "q5_K"])
def test_k_quant_scales_are_the_rounded_subblock_fits(t):
    """Each super-block's 6-bit scales and mins are nearest_int(63 s_j / max s) and nearest_int(63 m_j / max m),
    capped at 63, and d / dmin are fp16(max / 63), where (s_j, -m_j) are make_qkx2_quants's fits of its eight
    sub-blocks with the format's weights and search parameters."""
    nmax, rmin, rdelta, nstep = QKX2[t]
    x = subblocks(48, 256, 0x0C11 + t).reshape(-1)
    f = kquant_fields(t, O.quantize_chunk(t, x.reshape(-1, 256)))
    for i in range(len(f["d"])):
        fits = [O.make_qkx2_quants(xs, kquant_weights(xs), nmax, rmin, rdelta, nstep)
                for xs in x[256 * i:256 * (i + 1)].reshape(8, 32)]
        s = np.array([fit[0] for fit in fits], np.float32)
        m = np.array([-fit[1] for fit in fits], np.float32)
        ms, mm = max(np.float32(0), s.max()), max(np.float32(0), m.max())
        ls = np.minimum(63, np.rint((np.float32(63) / ms if ms > 0 else np.float32(0)) * s)).astype(np.int64)
        lm = np.minimum(63, np.rint((np.float32(63) / mm if mm > 0 else np.float32(0)) * m)).astype(np.int64)
        assert np.array_equal(f["sc"][i], ls) and np.array_equal(f["mn"][i], lm), i
        assert f["d"][i] == np.float32(np.float16(ms / np.float32(63)))
        assert f["dmin"][i] == np.float32(np.float16(mm / np.float32(63)))
        if ms > 0:
            assert ls.max() == 63


def test_q6_K_scales_are_the_rounded_subblock_fits():
    """Q6_K's int8 scales are min(127, nearest_int(-128 s_j / max_scale)) and d = fp16(-max_scale / 128), where s_j
    are make_qx_quants's fits of the sixteen 16-value sub-blocks and max_scale the fit of largest magnitude; that
    sub-block's scale is -128."""
    x = subblocks(48, 256, 0x0D11).reshape(-1)
    f = kquant_fields(O.TYPE_Q6_K, O.quantize_chunk(O.TYPE_Q6_K, x.reshape(-1, 256)))
    for i in range(len(f["d"])):
        s = np.array([O.make_qx_quants(xs, 32)[0] for xs in x[256 * i:256 * (i + 1)].reshape(16, 16)], np.float32)
        ms = s[np.argmax(np.abs(s))]
        isc = np.float32(-128) / ms
        want = np.minimum(127, np.rint(isc * s)).astype(np.int64)
        assert np.array_equal(f["sc"][i], want), i
        assert f["d"][i] == np.float32(np.float16(np.float32(1) / isc))
        assert f["sc"][i].min() == -128


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K], ids=["q4_K", "q5_K", "q6_K"])
def test_k_quant_codes_are_nearest_grid_points(t):
    """Given a block's packed scales, every code is the grid point nearest its value: for Q4_K / Q5_K the grid of
    sub-block j is d sc_j l - dmin m_j (l = 0 .. 15 / 31), for Q6_K d sc_j (l - 32) (l = 0 .. 63). Sub-blocks whose
    scale rounded to zero keep the search's codes and are skipped."""
    x = subblocks(64, 256, 0x0E11 + t).reshape(-1)
    f = kquant_fields(t, O.quantize_chunk(t, x.reshape(-1, 256)))
    x = x.reshape(-1, 256).astype(np.float64)
    sub = 16 if t == O.TYPE_Q6_K else 32
    levels = {O.TYPE_Q4_K: 16, O.TYPE_Q5_K: 32, O.TYPE_Q6_K: 64}[t]
    checked = 0
    for i in range(len(x)):
        for j in range(256 // sub):
            step = float(f["d"][i]) * float(f["sc"][i][j])
            if step == 0:
                continue
            l = np.arange(levels, dtype=np.float64)
            grid = step * (l - 32) if t == O.TYPE_Q6_K else step * l - float(f["dmin"][i]) * float(f["mn"][i][j])
            xs = x[i, sub * j:sub * (j + 1)]
            dist = np.abs(xs[:, None] - grid[None, :])
            got = dist[np.arange(sub), f["q"][i, sub * j:sub * (j + 1)]]
            assert np.all(got <= dist.min(axis=1) + 1e-6 * abs(step)), (i, j)
            checked += 1
    assert checked > 0.9 * len(x) * (256 // sub)
